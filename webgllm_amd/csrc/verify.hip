// Speculative verify's bookkeeping on the device, so that a whole verify
// step (drafts in, the batch's forward, the greedy picks, the accept and
// the rollback) replays as one captured graph with no host decision in it.
//
// The reference's handler keeps the longest prefix of drafts that the picks
// agree with, plus the pick after it (src/handler.ts:1811-1887), and
// Engine.accept moves the cache position on by that count and sets every
// conv layer's state to the state after that many tokens
// (src/engine.ts:8063-8086, the per-prefix states of convPrefixes,
// src/gpu/kernels.ts:1499-1523). Here those decisions read the picks and
// drafts from device memory.
#include "common.h"
#include "pick_core.h"

namespace wg {
namespace {

constexpr int MAX_VERIFY_ROWS = 8;
constexpr int CPT = 8;  // state floats a thread copies (the grid covers max_state with them)

// Rows kept of a batch whose inputs are ids[0..rows) (ids[1..] the drafts)
// and whose greedy picks are picks[0..rows): 1 + the agreeing prefix.
__device__ inline int kept_of(const int32_t *ids, const int32_t *picks, int rows) {
  int kept = 1;
  while (kept < rows && picks[kept - 1] == ids[kept]) kept++;
  return kept;
}

// Workgroup (layer l, slice): the layer's state := its prefix kept - 1
// ((W - 1) x D floats). Workgroup 0 also moves the step on: the accepted
// picks into hist after the position, the last of them into ids[0], the
// position by kept, kept into the log at the cursor, and the cursor on.
// PARTS: the picks are finished here from a head GEMV's pick parts (as
// wg_argmax_parts finishes them; wave w takes row w, its lanes every part
// at once, the first 1024 loaded with the parts' count, not after it: the
// slots past the count are in the array and left out once it arrives),
// and workgroup 0 writes them to picks_out.
constexpr int ACCEPT_THREADS = 64 * MAX_VERIFY_ROWS;
template <bool PARTS>
__global__ __launch_bounds__(ACCEPT_THREADS) void verify_accept_kernel(
    const int32_t *ids_in, const int32_t *picks, int rows, const wg_conv_state *convs,
    int n_conv, int32_t *pos, int32_t *ids, int32_t *hist, int32_t hist_len, int32_t *kept_log,
    int32_t log_len, int32_t *cursor, const char *pick_parts, int32_t *picks_out) {
  __shared__ int32_t p[MAX_VERIFY_ROWS], d[MAX_VERIFY_ROWS];
  if constexpr (PARTS) {
    constexpr int PER = WG_PICK_SLOTS / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = wave;  // (a wave a row: MAX_VERIFY_ROWS waves)
    const uint2 *row =
        reinterpret_cast<const uint2 *>(pick_parts + PICK_HEADER) + (int64_t)min(i, rows - 1) * WG_PICK_SLOTS;
    uint2 raw[16];
#pragma unroll
    for (int k = 0; k < 16; k++) raw[k] = row[lane + 64 * k];
    const int parts = min(*reinterpret_cast<const int *>(pick_parts), WG_PICK_SLOTS);
    PickBest b{PICK_FLOOR, PICK_NONE};
#pragma unroll
    for (int k = 0; k < 16; k++)
      if (lane + 64 * k < parts) b = pick_better(b, PickBest{__uint_as_float(raw[k].x), (int)raw[k].y});
    for (int k0 = 16; k0 < PER && 64 * k0 < parts; k0 += 16) {
#pragma unroll
      for (int k = 0; k < 16; k++) {
        const int at = lane + 64 * (k0 + k);
        raw[k] = at < parts ? row[at]
                            : make_uint2(__float_as_uint(PICK_FLOOR), (uint32_t)PICK_NONE);
      }
#pragma unroll
      for (int k = 0; k < 16; k++)
        b = pick_better(b, PickBest{__uint_as_float(raw[k].x), (int)raw[k].y});
    }
    b = pick_wave_best(b);
    if (lane == 0 && i < rows) p[i] = b.id == PICK_NONE ? 0 : b.id;
    if (threadIdx.x < rows) d[threadIdx.x] = ids_in[threadIdx.x];
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < rows) picks_out[threadIdx.x] = p[threadIdx.x];
  } else {
    if (threadIdx.x < rows) {
      p[threadIdx.x] = picks[threadIdx.x];
      d[threadIdx.x] = ids_in[threadIdx.x];
    }
    __syncthreads();
  }
  const int kept = kept_of(d, p, rows);
  const int l = blockIdx.y;
  if (l < n_conv) {
    // CPT floats a thread, every load issued before the first store (the
    // state and the prefixes are separate arrays, but a loop of single
    // copies had waited for each load in turn)
    const wg_conv_state c = convs[l];
    const int64_t n = (int64_t)(c.width - 1) * c.dim;
    const float *src = c.prefixes + (int64_t)(kept - 1) * n;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n; i0 += CPT * step) {
      float v[CPT];
#pragma unroll
      for (int k = 0; k < CPT; k++) v[k] = i0 + k * step < n ? src[i0 + k * step] : 0.0f;
#pragma unroll
      for (int k = 0; k < CPT; k++)
        if (i0 + k * step < n) c.state[i0 + k * step] = v[k];
    }
  }
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    const int p0 = *pos;
    for (int i = 0; i < kept; i++)
      if (p0 + 1 + i >= 0 && p0 + 1 + i < hist_len) hist[p0 + 1 + i] = p[i];
    const int step = *cursor;
    if (step >= 0 && step < log_len) kept_log[step] = kept;
    *cursor = step + 1;
    *pos = p0 + kept;
    ids[0] = p[kept - 1];
  }
}

// ids[1 .. rows) := row *cursor of the draft table (the last row once the
// cursor is past it).
__global__ void verify_drafts_kernel(int32_t *ids, int rows, const int32_t *table, int n_steps,
                                     const int32_t *cursor) {
  const int i = threadIdx.x;
  if (i < rows - 1) {
    int step = *cursor;
    step = step < 0 ? 0 : (step >= n_steps ? n_steps - 1 : step);
    ids[1 + i] = table[(int64_t)step * (rows - 1) + i];
  }
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

int wg_verify_accept(const int32_t *picks, int32_t rows, const wg_conv_state *convs,
                     int32_t n_conv, int32_t max_state, int32_t *pos, int32_t *ids,
                     int32_t *hist, int32_t hist_len, int32_t *kept_log, int32_t log_len,
                     int32_t *cursor, void *stream) {
  WG_REQUIRE(picks && pos && ids && cursor, "wg_verify_accept: null argument");
  WG_REQUIRE(rows >= 1 && rows <= MAX_VERIFY_ROWS, "wg_verify_accept: %d rows (1 to %d)", rows,
             MAX_VERIFY_ROWS);
  WG_REQUIRE(n_conv >= 0 && (n_conv == 0 || convs), "wg_verify_accept: %d conv layers", n_conv);
  WG_REQUIRE(max_state >= 0, "wg_verify_accept: state of %d floats", max_state);
  WG_REQUIRE(!overlaps(picks, rows * 4, ids, rows * 4),
             "wg_verify_accept: the picks and the batch's ids overlap");
  WG_REQUIRE(hist_len >= 0 && (hist || !hist_len) && log_len >= 0 && (kept_log || !log_len),
             "wg_verify_accept: bad history or log");
  // every conv state (W - 1) x D floats is at most max_state: the grid covers it
  const int per = ACCEPT_THREADS * CPT;
  const unsigned gx = (unsigned)(max_state > 0 ? (max_state + per - 1) / per : 1);
  dim3 grid(gx, (unsigned)(n_conv > 0 ? n_conv : 1));
  // ids is read (the drafts) and written (ids[0]) by the same launch: the
  // kernel reads the drafts into LDS before workgroup 0 writes ids[0]; the
  // other workgroups read ids[1 ..] only
  verify_accept_kernel<false><<<grid, ACCEPT_THREADS, 0, as_stream(stream)>>>(
      ids, picks, rows, convs, n_conv, pos, ids, hist, hist_len, kept_log, log_len, cursor,
      nullptr, nullptr);
  return launched("wg_verify_accept");
}

int wg_verify_accept_parts(const void *pick_parts, int32_t *picks_out, int32_t rows,
                           const wg_conv_state *convs, int32_t n_conv, int32_t max_state,
                           int32_t *pos, int32_t *ids, int32_t *hist, int32_t hist_len,
                           int32_t *kept_log, int32_t log_len, int32_t *cursor, void *stream) {
  WG_REQUIRE(pick_parts && picks_out && pos && ids && cursor,
             "wg_verify_accept_parts: null argument");
  WG_REQUIRE(((uintptr_t)pick_parts & 15) == 0, "wg_verify_accept_parts: parts not 16-byte aligned");
  WG_REQUIRE(rows >= 1 && rows <= MAX_VERIFY_ROWS, "wg_verify_accept_parts: %d rows (1 to %d)",
             rows, MAX_VERIFY_ROWS);
  WG_REQUIRE(n_conv >= 0 && (n_conv == 0 || convs), "wg_verify_accept_parts: %d conv layers",
             n_conv);
  WG_REQUIRE(max_state >= 0, "wg_verify_accept_parts: state of %d floats", max_state);
  WG_REQUIRE(!overlaps(picks_out, rows * 4, ids, rows * 4),
             "wg_verify_accept_parts: the picks and the batch's ids overlap");
  WG_REQUIRE(hist_len >= 0 && (hist || !hist_len) && log_len >= 0 && (kept_log || !log_len),
             "wg_verify_accept_parts: bad history or log");
  const int per = ACCEPT_THREADS * CPT;
  const unsigned gx = (unsigned)(max_state > 0 ? (max_state + per - 1) / per : 1);
  dim3 grid(gx, (unsigned)(n_conv > 0 ? n_conv : 1));
  verify_accept_kernel<true><<<grid, ACCEPT_THREADS, 0, as_stream(stream)>>>(
      ids, nullptr, rows, convs, n_conv, pos, ids, hist, hist_len, kept_log, log_len, cursor,
      (const char *)pick_parts, picks_out);
  return launched("wg_verify_accept_parts");
}

int wg_verify_drafts(int32_t *ids, int32_t rows, const int32_t *table, int32_t n_steps,
                     const int32_t *cursor, void *stream) {
  WG_REQUIRE(ids && table && cursor, "wg_verify_drafts: null argument");
  WG_REQUIRE(rows >= 2 && rows <= MAX_VERIFY_ROWS, "wg_verify_drafts: %d rows (2 to %d)", rows,
             MAX_VERIFY_ROWS);
  WG_REQUIRE(n_steps >= 1, "wg_verify_drafts: an empty draft table");
  verify_drafts_kernel<<<1, 64, 0, as_stream(stream)>>>(ids, rows, table, n_steps, cursor);
  return launched("wg_verify_drafts");
}

}  // extern "C"
