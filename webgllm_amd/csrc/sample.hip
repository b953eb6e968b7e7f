// Sampling candidates on the GPU (the reference's PENALIZED + CHUNK_MAX,
// CHUNK_RANK, CHUNK_BY_RANK and CHUNK_GATHER, src/gpu/kernels.ts:3085-3163,
// :3265-3323, run by Engine.pick, src/engine.ts:8352-8473): the logits of
// the `count` 256-token chunks with the largest penalized logit, so the
// host reads back count x 1 KB a row instead of the vocabulary, and samples
// from them (for top-k with k <= count they hold the k largest: each lies
// in a chunk whose maximum is among the k largest).
//
// Stage 1 (`chunk_max_kernel`): a wave per (row, chunk) reads the chunk's
// 256 logits and mask bytes (4 a lane), penalizes each and
// reduces the maximum. Stage 2 (`chunk_rank_kernel`): a workgroup of 256
// threads per row sorts the chunks by maximum (larger first, ties to the
// lower index: the order the reference's ranks give) and keeps the first
// `count`. Stage 3 (`chunk_gather_kernel`): a workgroup per kept chunk
// writes its penalized logits.
#include "common.h"
#include "dot.h"

namespace wg {
namespace {

constexpr int CHUNK = 256;
constexpr int MAX_SEEN = 16;
constexpr int MAX_TOTAL = 2048;  // chunks a row (vocabularies up to 524,288)

struct Penalty {
  const uint8_t *mask;      // [V]: 0 unseen, 1 prompt, 2 never draw, 3 written
  const int32_t *seen;      // [n_seen][4]: token, state, first row, end row
  int n_seen, row0;
  float penalty, presence;
  const uint32_t *allowed;  // [allowed_rows][ld_allowed] bit per token, or NULL
  int allowed_rows, ld_allowed;
};

// penalized (src/gpu/kernels.ts:3102-3122): token id's logit v (its mask
// byte m) for batch row r, or -1e30 when it may not be drawn.
__device__ inline float penalized(float v, int id, int r, const Penalty &p, int V, int m) {
  if (id >= V) return -1e30f;  // past the vocabulary in the last chunk
  if (p.allowed) {
    const int row = p.allowed_rows == 1 ? 0 : r;
    if (row >= p.allowed_rows) return -1e30f;
    const uint32_t bits = p.allowed[(int64_t)row * p.ld_allowed + (id >> 5)];
    if (!((bits >> (id & 31)) & 1u)) return -1e30f;
  }
  if (m == 2) return -1e30f;
  int state = m;
  for (int k = 0; k < p.n_seen; k++) {
    const int *s = p.seen + 4 * k;
    if (s[0] == id && r >= s[2] && r < s[3]) state = s[1];
  }
  if (state == 1 || state == 3) {
    v = v < 0.0f ? v * p.penalty : v / p.penalty;
    v -= p.presence;
  }
  return v;
}

__global__ __launch_bounds__(256) void chunk_max_kernel(const float *logits, int M, int V,
                                                        int ld, Penalty p, int total,
                                                        float *maxima) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (row, chunk)
  if (w >= (int64_t)M * total) return;
  const int r = (int)(w / total), c = (int)(w % total);
  const float *row = logits + (int64_t)r * ld;
  float mx = -1e30f;
  float v[4];
  int m[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int id = c * CHUNK + 4 * lane + i;
    v[i] = id < V ? row[id] : 0.0f;
    m[i] = id < V && p.mask ? p.mask[id] : 0;
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
    mx = fmaxf(mx, penalized(v[i], c * CHUNK + 4 * lane + i, r + p.row0, p, V, m[i]));
  mx = wave_max(mx);
  if (lane == 0) maxima[w] = mx;
}

constexpr int RANK_THREADS = 256;  // one compare-exchange a thread a pass up to 512 chunks

__global__ __launch_bounds__(RANK_THREADS) void chunk_rank_kernel(int total, const float *maxima,
                                                                 int count, int32_t *chunks_out) {
  __shared__ float sv[MAX_TOTAL];
  __shared__ int si[MAX_TOTAL];
  const int r = blockIdx.x;
  // CHUNK_RANK + CHUNK_BY_RANK: the chunks sorted by maximum, larger first,
  // ties to the lower index (the reference's order), by a bitonic sort in
  // LDS over the next power of two, padded with -inf (every maximum is at
  // least -1e30, so the padding sorts last).
  int n2 = 1;
  while (n2 < total) n2 <<= 1;
  for (int c = threadIdx.x; c < n2; c += RANK_THREADS) {
    sv[c] = c < total ? maxima[(int64_t)r * total + c] : -INFINITY;
    si[c] = c;
  }
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < n2 / 2; t += RANK_THREADS) {
        const int a = 2 * t - (t & (j - 1)), b = a + j;  // pair (a, b), a's bit j clear
        const bool desc = (a & k) == 0;                   // this run sorts best first
        const float va = sv[a], vb = sv[b];
        const int ia = si[a], ib = si[b];
        const bool b_first = vb > va || (vb == va && ib < ia);
        if (b_first == desc) {
          sv[a] = vb;
          sv[b] = va;
          si[a] = ib;
          si[b] = ia;
        }
      }
      __syncthreads();
    }
  }
  for (int k = threadIdx.x; k < count; k += RANK_THREADS)
    chunks_out[(int64_t)r * count + k] = si[k];
}

// CHUNK_GATHER: a workgroup per (ranked chunk, row) writes that chunk's
// penalized logits.
__global__ __launch_bounds__(CHUNK) void chunk_gather_kernel(const float *logits, int V, int ld,
                                                            Penalty p, int count,
                                                            const int32_t *chunks,
                                                            float *cand_out) {
  const int k = blockIdx.x, r = blockIdx.y;
  const int id = chunks[(int64_t)r * count + k] * CHUNK + threadIdx.x;
  const float v = id < V ? logits[(int64_t)r * ld + id] : 0.0f;
  const int m = id < V && p.mask ? p.mask[id] : 0;
  cand_out[((int64_t)r * count + k) * CHUNK + threadIdx.x] = penalized(v, id, r + p.row0, p, V, m);
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

size_t wg_pick_scratch_bytes(int32_t M, int32_t V) {
  return (size_t)M * ((V + CHUNK - 1) / CHUNK) * sizeof(float);
}

int wg_pick_candidates(const float *logits, int32_t M, int32_t V, int32_t ld,
                       const uint8_t *mask, const int32_t *seen_rows, int32_t n_seen,
                       int32_t row0, float penalty, float presence_penalty,
                       const uint32_t *allowed, int32_t allowed_rows, int32_t ld_allowed,
                       int32_t count, int32_t *chunks_out, float *candidates, void *scratch,
                       size_t scratch_bytes, void *stream) {
  WG_REQUIRE(logits && chunks_out && candidates && scratch && M >= 1 && V >= 1 && ld >= V,
             "wg_pick_candidates: bad arguments");
  const int total = (V + CHUNK - 1) / CHUNK;
  WG_REQUIRE(total <= MAX_TOTAL, "wg_pick_candidates: %d chunks a row (at most %d)", total,
             MAX_TOTAL);
  WG_REQUIRE(count >= 1 && count <= 64 && count <= total,
             "wg_pick_candidates: %d chunks asked of %d (1 to 64)", count, total);
  WG_REQUIRE(n_seen >= 0 && n_seen <= MAX_SEEN && (n_seen == 0 || seen_rows),
             "wg_pick_candidates: %d seen rows (at most %d)", n_seen, MAX_SEEN);
  WG_REQUIRE(penalty > 0.0f, "wg_pick_candidates: the repetition penalty must be positive");
  WG_REQUIRE(!allowed || (allowed_rows >= 1 && ld_allowed >= (V + 31) / 32),
             "wg_pick_candidates: the allowed-token bitmap needs rows and %d words a row",
             (V + 31) / 32);
  WG_REQUIRE(scratch_bytes >= wg_pick_scratch_bytes(M, V),
             "wg_pick_candidates: scratch of %zu bytes, %zu needed", scratch_bytes,
             wg_pick_scratch_bytes(M, V));
  Penalty p{mask, seen_rows, n_seen, row0, penalty, presence_penalty, allowed, allowed_rows,
            ld_allowed};
  hipStream_t s = as_stream(stream);
  const int64_t waves = (int64_t)M * total;
  float *maxima = static_cast<float *>(scratch);
  chunk_max_kernel<<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(logits, M, V, ld, p, total,
                                                               maxima);
  int rc = launched("wg_pick_candidates");
  if (rc) return rc;
  chunk_rank_kernel<<<M, RANK_THREADS, 0, s>>>(total, maxima, count, chunks_out);
  rc = launched("wg_pick_candidates");
  if (rc) return rc;
  chunk_gather_kernel<<<dim3(count, M), CHUNK, 0, s>>>(logits, V, ld, p, count, chunks_out,
                                                     candidates);
  return launched("wg_pick_candidates");
}

}  // extern "C"
