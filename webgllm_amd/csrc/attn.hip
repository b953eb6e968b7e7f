// Attention over the fp16 KV cache for decode and speculative verify.
//
// head_prep: the reference's headPrep + values (src/gpu/kernels.ts:2196-2322,
// :3030-3045): per head, optional RMS norm over head_dim, RoPE on the
// rotated dims (dim j pairs with j + R/2 at frequency j; the angle of
// pos = lo + 1024 hi is added from two rows of the table, as
// Engine.ropeTable builds it, src/engine.ts:1292-1312), times 1/sqrt(hd)
// for queries; keys and values go into the cache as halves.
//
// attn_decode: scores / attend / attendPanel (kernels.ts:2386-2579,
// :2803-3027) as split-K flash decoding: a workgroup takes one KV head and a
// chunk of 64 keys for every query row and every query head sharing that KV
// head (GQA: each key and value is read once for all of them), stages the
// K and V tiles in LDS, and writes the chunk's (max, sum of weights,
// weighted sum of values); a combine pass rescales the chunks by their
// running max (attendPanelCombine's online softmax) into half outputs.
// The position comes from device memory so a captured graph replays at any
// position; chunks past the last key leave at once.
#include <mutex>

#include "attn_core.h"
#include "common.h"
#include "dot.h"
#include "lds_load.h"

namespace wg {
namespace {

constexpr int MAX_HD = 256;

__device__ inline uint16_t to_h(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// One wave per (row m, head slot): slots [0, H) queries, [H, H + KV) keys,
// [H + KV, H + 2 KV) values. The row's elements and norm weights (the
// rotation partners' too: lane + 64 i, i < 4, as head_dim <= MAX_HD) load
// with the position, only the rope table and the stores wait for it; the
// arguments those loads need lead the list (the first 14 dwords arrive
// preloaded in scalar registers).
__global__ __launch_bounds__(64) void head_prep_kernel(
    const float *qkv, const int32_t *pos0_dev, const float *q_norm, const float *k_norm, int ldq,
    int H, int KV, int hd, int use_norm, int R, float eps, const float *rope, int rope_rows,
    float *q_out, int ldqo, uint16_t *k_cache, uint16_t *v_cache, int ctx) {
  static_assert(MAX_HD <= 4 * 64, "four elements a lane");
  const int slot = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
  const float *x = qkv + (int64_t)m * ldq + (int64_t)slot * hd;
  const bool is_q = slot < H, is_v = slot >= H + KV;
  const float *nw = is_q ? q_norm : k_norm;
  const int P = R / 2;
  const int pos = *pos0_dev + m;
  float xv[4], wv[4], xp[4], wp[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = lane + 64 * i;
    xv[i] = xp[i] = 0.0f;
    wv[i] = wp[i] = 1.0f;
    if (t < hd) {
      xv[i] = x[t];
      if (!is_v && use_norm) wv[i] = nw[t];
      if (!is_v && t < 2 * P) {
        const int tp = t < P ? t + P : t - P;  // the rotation partner
        xp[i] = x[tp];
        if (use_norm) wp[i] = nw[tp];
      }
    }
  }
  const int kvd = KV * hd;
  if (pos < 0 || pos >= ctx || 1024 + (pos >> 10) >= rope_rows) {
    // A row past the cache has no position: its query is zero, nothing is stored.
    if (slot < H)
      for (int t = lane; t < hd; t += 64) q_out[(int64_t)m * ldqo + (int64_t)slot * hd + t] = 0.0f;
    return;
  }
  if (is_v) {  // values: into the cache as they are
    uint16_t *vo = v_cache + (int64_t)pos * kvd + (int64_t)(slot - H - KV) * hd;
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (lane + 64 * i < hd) vo[lane + 64 * i] = to_h(xv[i]);
    return;
  }
  float inv = 1.0f;
  if (use_norm) {
    // the sum of squares in head_norm_inv's order: lane c < 4 walks dims
    // 32 t + 8 c + e (held by lane (32 t + 8 c + e) % 64, element t / 2)
    const int c = lane & 3;
    float part = 0.0f;
    for (int t = 0; 32 * t < hd; t++) {
      float xs = xv[0];
#pragma unroll
      for (int i = 1; i < 4; i++)
        if (i == (t >> 1)) xs = xv[i];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float x = __shfl(xs, (32 * t + 8 * c + e) & 63, 64);
        part = __builtin_fmaf(x, x, part);
      }
    }
    const float total = (__shfl(part, 0, 64) + __shfl(part, 1, 64)) +
                        (__shfl(part, 2, 64) + __shfl(part, 3, 64));
    inv = head_norm_inv(total, hd, eps);
  }
  const int lo = pos & 1023, hi = 1024 + (pos >> 10);
  const float *r_lo = rope + (int64_t)lo * hd, *r_hi = rope + (int64_t)hi * hd;
  const float scale = is_q ? 1.0f / sqrtf((float)hd) : 1.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = lane + 64 * i;
    if (t >= hd) break;
    float v = xv[i] * (use_norm ? inv * wv[i] : 1.0f);
    float r = v;
    if (t < 2 * P) {
      const bool first = t < P;
      const int f = first ? t : t - P;
      const float p = xp[i] * (use_norm ? inv * wp[i] : 1.0f);
      r = rope_rotate(v, p, first, r_lo[f], r_lo[hd / 2 + f], r_hi[f], r_hi[hd / 2 + f]);
    }
    if (is_q) {
      q_out[(int64_t)m * ldqo + (int64_t)slot * hd + t] = r * scale;
    } else {
      k_cache[(int64_t)pos * kvd + (int64_t)(slot - H) * hd + t] = to_h(r);
    }
  }
}

// Workgroup = (KV head kh, chunk c); chunks past the last key leave at once.
template <int HD>
__global__ __launch_bounds__(256) void attn_chunk_kernel(
    const float *q, int ldq, int M, int H, int KV, const uint16_t *k_cache,
    const uint16_t *v_cache, const int32_t *pos0_dev, int max_keys, float *partial, int chunks) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int pos0 = *pos0_dev;
  // The last row sees keys 0 .. pos0 + M - 1; never more than the cache holds.
  const int n_keys = min(pos0 + M, max_keys);
  if ((int)blockIdx.y * CHUNK >= n_keys) return;
  attn_chunk_item<HD>(q, ldq, M, H, KV, k_cache, v_cache, pos0, n_keys, blockIdx.x, blockIdx.y,
                      partial, chunks, smem);
}

// Decode attention for GM = G * M <= 8 queries per KV head. Workgroup =
// (KV head kh, chunk c of 64 keys), one wave per query (GM waves). Every
// load is issued at the start, straight into LDS: each wave's query (HD
// floats), then the chunk's K and V tiles, 1 KB an instruction, the waves
// taking the instructions in turn, so each key and value crosses the memory
// system once for all GM queries. K row r keeps its 16-byte piece t at slot
// t ^ swz(r): the score loop (lane = key, reading its row piece by piece)
// then touches 16 distinct 16-byte bank groups in any 16 consecutive lanes
// (with 128-byte rows, rows r and r + 8 flip the slot's low bit); V rows are read whole, 16 lanes a
// row, and keep their order. The position is read while the loads fly, and
// the kernel waits for memory once. The chunk's softmax is a wave
// reduction; each V row's weight comes from its lane by a shuffle. The
// chunk's (max, sum of weights, weighted values) go to the scratch for
// attn_combine_kernel. (Combining in the last workgroup to finish a KV
// head costs more here than a second launch: its agent-scope release
// writes an XCD's L2 back once per workgroup.)
constexpr int WK = 64;   // keys a workgroup takes (the partials' chunk)
constexpr int FGM = 8;   // queries per KV head (waves per workgroup) at most

template <int HD>
__global__ __launch_bounds__(FGM * 64) void attn_tile_kernel(
    const float *q, int ldq, int M, int H, int KV, const uint16_t *k_cache,
    const uint16_t *v_cache, const int32_t *pos0_dev, int max_keys, float *partial, int chunks,
    uint16_t *out, int ldo) {
  constexpr int KP = HD / 8;       // 16-byte pieces of a row
  constexpr int ROWB = HD * 2;     // bytes of a row
  constexpr int TILE = WK * ROWB;  // bytes of the K (or V) tile
  constexpr int RPI = 64 / KP;     // rows one 1 KB load instruction covers
  constexpr int NI = WK / RPI;     // load instructions a tile
  constexpr int QOFF = 2 * TILE;   // the queries, HD floats each
  static_assert(HD * 4 <= 1024, "a query fits one load instruction");
  auto swz = [](int r) { return KP == 16 ? (r & 15) : ((r ^ (r >> 3)) & (KP - 1)); };
  __shared__ __align__(16) unsigned char smem[2 * TILE + FGM * HD * 4];
  const int kh = blockIdx.x % KV, c = blockIdx.x / KV;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;  // = G * M
  const int G = H / KV, g = wave % G, m = wave / G;
  const int j0 = c * WK;
  const int kvd = KV * HD;
  // rows at or past max_keys do not exist: their lanes load row j0 again
  // (j0 < max_keys), and the rows are masked below like rows past the position
  const int nk_max = min(WK, max_keys - j0);
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  if (lane < HD / 4)
    dma16(q + (int64_t)m * ldq + (int64_t)(kh * G + g) * HD + lane * 4,
          __builtin_amdgcn_readfirstlane(sbase + QOFF + wave * HD * 4));
  for (int i = wave; i < 2 * NI; i += nw) {
    const bool is_v = i >= NI;
    const int ii = is_v ? i - NI : i;
    const int r = ii * RPI + lane / KP;
    const int slot = lane % KP;
    const int piece = is_v ? slot : (slot ^ swz(r));
    const int rr = r < nk_max ? r : 0;
    dma16((is_v ? v_cache : k_cache) + (int64_t)(j0 + rr) * kvd + kh * HD + piece * 8,
          __builtin_amdgcn_readfirstlane(sbase + (is_v ? TILE : 0) + ii * 1024));
  }
  const int pos0 = *pos0_dev;
  const int n_keys = min(pos0 + M, max_keys);
  // every load has landed before any wave leaves: LDS still being written
  // must not pass to the next workgroup
  wait_vm<0>();
  if (n_keys <= 0) {  // no position in the cache: the output is zero
    if (c == 0) {
      uint16_t *o = out + (int64_t)m * ldo + (int64_t)(kh * G + g) * HD;
      for (int d = lane; d < HD; d += 64) o[d] = 0;
    }
    return;
  }
  if (j0 >= n_keys) return;
  barrier();
  const int nk = min(WK, n_keys - j0);

  // score of key lane: q . k, the query read from LDS (every lane the same
  // address: a broadcast)
  const float4 *ql = reinterpret_cast<const float4 *>(smem + QOFF + wave * HD * 4);
  const unsigned char *krow = smem + lane * ROWB;
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
  for (int i = 0; i < KP; i++) {
    const uint4 kr = *reinterpret_cast<const uint4 *>(krow + ((i ^ swz(lane)) * 16));
    const half2v a = as_h2(kr.x), b = as_h2(kr.y), cc = as_h2(kr.z), dd = as_h2(kr.w);
    const float4 qa = ql[2 * i], qb = ql[2 * i + 1];
    s0 = __builtin_fmaf(qa.x, (float)a.x, s0);
    s1 = __builtin_fmaf(qa.y, (float)a.y, s1);
    s2 = __builtin_fmaf(qa.z, (float)b.x, s2);
    s3 = __builtin_fmaf(qa.w, (float)b.y, s3);
    s0 = __builtin_fmaf(qb.x, (float)cc.x, s0);
    s1 = __builtin_fmaf(qb.y, (float)cc.y, s1);
    s2 = __builtin_fmaf(qb.z, (float)dd.x, s2);
    s3 = __builtin_fmaf(qb.w, (float)dd.y, s3);
  }
  const bool vis = lane < nk && j0 + lane <= pos0 + m;  // causal
  const float sc = vis ? (s0 + s1) + (s2 + s3) : -INFINITY;
  float mx = sc;
  mx = wave_max(mx);
  const float e = (mx == -INFINITY || !vis) ? 0.0f : __expf(sc - mx);
  const float lsum = wave_sum(e);

  // weighted values: lane holds dims d0..d0+7 of rows lane / KP + RPI i;
  // rows past the position may hold any bits (a zero weight times a NaN is
  // NaN): they are read as zero
  const int d0 = (lane % KP) * 8;
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int r = lane / KP + RPI * i;
    uint4 vr = *reinterpret_cast<const uint4 *>(smem + TILE + r * ROWB + (lane % KP) * 16);
    if (r >= nk) vr = make_uint4(0u, 0u, 0u, 0u);
    const float w = __shfl(e, r, 64);
    const uint32_t w4[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const half2v hv = as_h2(w4[t]);
      acc[2 * t] = __builtin_fmaf(w, (float)hv.x, acc[2 * t]);
      acc[2 * t + 1] = __builtin_fmaf(w, (float)hv.y, acc[2 * t + 1]);
    }
  }
#pragma unroll
  for (int t = 0; t < 8; t++) acc[t] = group_reduce<KP>(acc[t], Plus());
  PartialLayout pl{HD, chunks};
  float *po = partial + pl.base(m * H + kh * G + g, c);
  if (lane < KP)
#pragma unroll
    for (int t = 0; t < 8; t++) po[2 + d0 + t] = acc[t];
  if (lane == 0) {
    po[0] = mx;
    po[1] = lsum;
  }
}

// Decode attention in one launch, for GM = G * M <= 8 queries per KV head.
// Workgroup = (KV head kh, split s of 64 * NCH keys), one wave per query.
// All of the split's K and V tiles go to LDS by direct loads issued at the
// start (as in attn_tile_kernel); each wave then runs the online softmax
// over the NCH chunks (attendPanel's running max and sum) and publishes its
// (max, sum of weights, weighted values) with coherent stores (sc1: they
// reach the point where every compute unit sees them, with no write-back of
// the L2). Once those stores are done, one relaxed atomic per workgroup
// counts the KV head's live splits in; the workgroup that completes the
// count resets the counter to zero for the next call and does
// attendPanelCombine for the KV head's queries, reading every partial at
// once with coherent vector loads. No workgroup waits on another, so the
// launch always drains.
//
// The XCD-grouped form (XL) gives each XCD whole KV heads: KV head kh
// belongs to XCD kh mod 8 (KV a multiple of 8), and the workgroup with
// blockIdx b, on XCD x (its hardware XCC id), takes split (b / 8) mod
// splits of head x + 8 (b / 8 / splits). Workgroups are handed to the XCDs
// round-robin, so the 8 with the same b / 8 run one on each XCD and every
// XCD holds grid / 8 of them. One counter per XCD (on its own 256-byte
// line) counts its workgroups in, and the last one resets it and combines
// every query of the XCD's heads: one serial combine an XCD instead of one
// a KV head. Since every workgroup of the exchange shares the XCD's L2, the
// partials, the count and the combine's loads stay in it (store_part and
// load_part with LOCAL; checked bit for bit against the coherent exchange
// over thousands of launches of changing queries and positions, eager and
// in graphs).
constexpr int MAX_KV_COUNTERS = 64;       // counters at the scratch's start
// then one 256-byte line of counters per XCD (the XCD-grouped form's), so no
// two XCDs' L2s ever hold the same counter line
constexpr int XCDS = 8;
constexpr int XCD_LINE = 64;              // ints: 256 bytes
constexpr int COUNTER_INTS = MAX_KV_COUNTERS + XCDS * XCD_LINE;
constexpr int COUNTER_BYTES = COUNTER_INTS * 4;
constexpr int MAX_FUSED_KEYS = 1 << 20;   // keys the one-launch form takes
// partition partials a split workgroup merges in LDS: G M (P - 1) <= 12
// with G M P <= 16 and P <= 4
constexpr int MERGE_ROWS = 12;

// A split's partial for one query: max, sum, 2 floats of padding, then the
// HD weighted values, so that the values start 16-byte aligned.
__host__ __device__ constexpr int split_row(int hd) { return hd + 4; }

// How split partials pass from the workgroups that write them to the one
// that combines them. Across XCDs (LOCAL false): 16-byte stores with sc1
// (through to memory: the XCDs' L2s are not coherent with each other) and
// the count at agent scope. Within one XCD (LOCAL true: every workgroup of
// the exchange runs on it): plain stores, which the vector L1 writes
// through to the XCD's L2, and the count as an L2 atomic (workgroup
// scope). Loads with sc1 either way: they pass the L1 and take the line
// from the XCD's L2 when it has it (measured on the MI355X: a plain or sc0
// load keeps returning a line the CU's L1 holds, even after a workgroup on
// the same XCD has stored to it and counted itself in; an sc1 load sees
// the store every time, and takes a line the L2 holds in the L2 hit's
// time). The loads are buffer loads whose cache-policy bits the compiler
// sees, so that it places the waits for their results itself.
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f2v __attribute__((ext_vector_type(2)));
template <bool LOCAL>
__device__ inline void store_part(float *p, f4v v) {
  if constexpr (LOCAL)
    asm volatile("global_store_dwordx4 %0, %1, off" ::"v"(p), "v"(v) : "memory");
  else
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
// A buffer resource over [base, base + 2^31) (raw 32-bit loads).
__device__ inline __amdgpu_buffer_rsrc_t rsrc_of(const float *base) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
}
// a buffer load's cache policy: sc1 (bit 4)
template <bool LOCAL>
constexpr int part_policy() { return 16; }
template <bool LOCAL>
__device__ inline f4v load_part(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(
      f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, part_policy<LOCAL>()));
}
template <bool LOCAL>
__device__ inline f2v load2_part(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(
      f2v, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, part_policy<LOCAL>()));
}
// Counts a workgroup's partials in; true for the one that completes the
// count (`expect` arrivals), which also puts the counter back to zero.
template <bool LOCAL>
__device__ inline bool count_in(int *count, int expect) {
  if constexpr (LOCAL) {
    if (__hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) !=
        expect - 1)
      return false;
    __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  } else {
    if (__hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) !=
        expect - 1)
      return false;
    __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return true;
}

// The XCD this workgroup runs on (hardware register XCC_ID, bits 3:0).
__device__ inline int xcd_id() {
  return (int)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);
}

// attendPanelCombine of one query's `live` split partials (rows of
// split_row(HD) floats from pr, written with coherent stores) into its HD
// output halves at op: the wave's lanes, every load of a batch issued
// before the first use.
template <int HD, bool LOCAL>
__device__ inline void combine_splits(const float *pr, int live, uint16_t *op) {
  constexpr int SR = split_row(HD);
  const int lane = threadIdx.x & 63;
  // BT splits at a time: lane
  // (t, h) with t = lane / LPS and h = lane % LPS holds dims 4h..4h+3 of
  // split t + TS i; lane t < BT holds split t's max and sum. Every load of
  // a batch is issued before the wait.
  constexpr int LPS = HD / 4;      // lanes a split's values take
  constexpr int TS = 64 / LPS;     // splits one load instruction covers
  constexpr int BT = 4096 / HD;    // splits a batch (16 value loads a lane)
  constexpr int NL = BT / TS;      // value loads a lane issues a batch
  const int th = lane / LPS, dh = (lane % LPS) * 4;
  float gmax = -INFINITY, ltot = 0.0f;
  f4v o = {0.0f, 0.0f, 0.0f, 0.0f};
  const __amdgpu_buffer_rsrc_t rs = rsrc_of(pr);
  for (int t0 = 0; t0 < live; t0 += BT) {
    const int n = min(BT, live - t0);
    f4v v[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int t = t0 + min(th + TS * i, n - 1);
      v[i] = load_part<LOCAL>(rs, (t * SR + 4 + dh) * 4);
    }
    const f2v ml = load2_part<LOCAL>(rs, (t0 + min(lane, n - 1)) * SR * 4);
    const float mt = lane < n ? ml.x : -INFINITY;
    float bmax = mt;
    bmax = wave_max(bmax);
    const float nmax = fmaxf(gmax, bmax);
    if (nmax == -INFINITY) continue;  // nothing visible yet
    const float alpha = gmax == -INFINITY ? 0.0f : __expf(gmax - nmax);
    const float w = mt == -INFINITY ? 0.0f : __expf(mt - nmax);
    ltot = ltot * alpha + wave_sum(w * (lane < n ? ml.y : 0.0f));
    o.x *= alpha;
    o.y *= alpha;
    o.z *= alpha;
    o.w *= alpha;
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int t = th + TS * i;  // < 64
      // every lane takes part in the shuffle: a lane whose split is past
      // the batch must not leave its source lanes inactive
      const float ws = __shfl(w, t, 64);
      const float wt = t < n ? ws : 0.0f;
      o.x = __builtin_fmaf(wt, v[i].x, o.x);
      o.y = __builtin_fmaf(wt, v[i].y, o.y);
      o.z = __builtin_fmaf(wt, v[i].z, o.z);
      o.w = __builtin_fmaf(wt, v[i].w, o.w);
    }
    gmax = nmax;
  }
  // lanes holding the same dims (different splits) add up
  o.x = group_reduce<LPS>(o.x, Plus());
  o.y = group_reduce<LPS>(o.y, Plus());
  o.z = group_reduce<LPS>(o.z, Plus());
  o.w = group_reduce<LPS>(o.w, Plus());
  const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
  if (lane < LPS) {
    op += dh;
    const uint32_t lo = (uint32_t)half_bits(o.x * inv) | ((uint32_t)half_bits(o.y * inv) << 16);
    const uint32_t hi = (uint32_t)half_bits(o.z * inv) | ((uint32_t)half_bits(o.w * inv) << 16);
    *reinterpret_cast<uint2 *>(op) = make_uint2(lo, hi);
  }
}

// The same combine for several queries at once, when they have few splits:
// lane (query slot lane / (HD / 4), dims 4 h .. 4 h + 3 with h = lane % (HD
// / 4)) walks its own query's splits (CU at a time, every load of a batch
// issued before the first use: 6 CU registers), so a wave takes 64 / (HD /
// 4) queries in one memory round trip and needs no cross-lane reduction.
// qrow: the lane's query row of the partials (rows of `splits` partials
// from `partial`); op: its output, written when `valid`.
template <int HD, bool LOCAL, int CU>
__device__ inline void combine_lanes(const float *partial, int qrow, int splits, int live,
                                     uint16_t *op, bool valid) {
  constexpr int SR = split_row(HD);
  const int dh = ((threadIdx.x & 63) % (HD / 4)) * 4;
  const __amdgpu_buffer_rsrc_t rs = rsrc_of(partial);
  const int row0 = (valid ? qrow : 0) * splits;
  float gmax = -INFINITY, ltot = 0.0f;
  f4v o = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int t0 = 0; t0 < live; t0 += CU) {
    f4v v[CU];
    f2v ml[CU];
#pragma unroll
    for (int i = 0; i < CU; i++) {
      const int t = row0 + min(t0 + i, live - 1);
      v[i] = load_part<LOCAL>(rs, (t * SR + 4 + dh) * 4);
      ml[i] = load2_part<LOCAL>(rs, t * SR * 4);
    }
#pragma unroll
    for (int i = 0; i < CU; i++) {
      const float mt = t0 + i < live ? ml[i].x : -INFINITY;
      const float nmax = fmaxf(gmax, mt);
      const float a = gmax == -INFINITY ? (nmax == -INFINITY ? 1.0f : 0.0f) : __expf(gmax - nmax);
      const float w = mt == -INFINITY ? 0.0f : __expf(mt - nmax);
      ltot = ltot * a + w * ml[i].y;
      o = o * a + v[i] * w;
      gmax = nmax;
    }
  }
  const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
  if (valid) {
    const uint32_t lo = (uint32_t)half_bits(o.x * inv) | ((uint32_t)half_bits(o.y * inv) << 16);
    const uint32_t hi = (uint32_t)half_bits(o.z * inv) | ((uint32_t)half_bits(o.w * inv) << 16);
    *reinterpret_cast<uint2 *>(op + dh) = make_uint2(lo, hi);
  }
}

// Whether combine_lanes<CU> takes nq queries of `live` splits in fewer
// memory round trips than combine_splits, nw waves sharing them either way.
template <int HD, int CU>
__device__ inline bool lanes_combine_pays(int nq, int nw, int live) {
  const int per = 64 / (HD / 4);  // queries a wave takes at once
  const int lanes_trips = (nq + nw * per - 1) / (nw * per) * ((live + CU - 1) / CU);
  const int split_trips = (nq + nw - 1) / nw * ((live + 4096 / HD - 1) / (4096 / HD));
  return lanes_trips < split_trips;
}

template <int HD, int NCH, bool XL = false>
__global__ __launch_bounds__(1024) void attn_split_kernel(
    const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0_dev, const float *q,
    int max_keys, int splits, int M, int H, int KV, int nw, int ldq, float *partial,
    int *counters, uint16_t *out, int ldo) {
  constexpr int KP = HD / 8;       // 16-byte pieces of a row
  constexpr int ROWB = HD * 2;     // bytes of a row
  constexpr int TILE = WK * ROWB;  // bytes of a chunk's K (or V) tile
  constexpr int RPI = 64 / KP;     // rows one 1 KB load instruction covers
  constexpr int NI = WK / RPI;     // load instructions a tile
  constexpr int QOFF = 2 * NCH * TILE;
  constexpr int SPLIT = WK * NCH;  // keys a workgroup takes
  constexpr int SR = split_row(HD);
  static_assert(HD * 4 <= 1024, "a query fits one load instruction");
  auto swz = [](int r) { return KP == 16 ? (r & 15) : ((r ^ (r >> 3)) & (KP - 1)); };
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int last;
  int kh = blockIdx.x % KV, s = blockIdx.x / KV, xcd = 0;
  if constexpr (XL) {
    xcd = xcd_id() & (XCDS - 1);  // (0..7 on an 8-XCD part)
    const int rank = blockIdx.x / XCDS;  // < KV / 8 * splits: the grid is KV * splits
    kh = xcd + XCDS * (rank / splits);
    s = rank % splits;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // G M queries, each taken by P waves (chunks p, p + P, ... of the split);
  // nw = blockDim.x / 64 = G M P, passed among the preloaded arguments
  const int G = H / KV, GM = G * M, P = nw / GM;
  const int qi = wave % GM, p = wave / GM;
  const int g = qi % G, m = qi / G;
  const int j0 = s * SPLIT;  // < max_keys: s < splits
  const int kvd = KV * HD;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  // (an XCC id past 7 would name a head past the last: such a workgroup
  // loads nothing and computes nothing, and its XCD's count never completes)
  const bool here = !XL || kh < KV;
  // rows at or past max_keys do not exist: their lanes load row j0 again,
  // and they are masked below like rows past the position
  for (int i = wave; here && i < 2 * NI * NCH; i += nw) {
    const int c = i / (2 * NI), ic = i % (2 * NI);
    const bool is_v = ic >= NI;
    const int ii = is_v ? ic - NI : ic;
    const int r = ii * RPI + lane / KP;
    const int slot = lane % KP;
    const int piece = is_v ? slot : (slot ^ swz(r));
    const int row = j0 + c * WK + r;
    const int rr = row < max_keys ? row : j0;
    dma16((is_v ? v_cache : k_cache) + (int64_t)rr * kvd + kh * HD + piece * 8,
          __builtin_amdgcn_readfirstlane(sbase + c * 2 * TILE + (is_v ? TILE : 0) + ii * 1024));
  }
  // the query after the keys and values (ldq is not among the preloaded
  // arguments: its fetch then delays no key load)
  if (here && p == 0 && lane < HD / 4)
    dma16(q + (int64_t)m * ldq + (int64_t)(kh * G + g) * HD + lane * 4,
          __builtin_amdgcn_readfirstlane(sbase + QOFF + qi * HD * 4));
  const int pos0 = *pos0_dev;
  const int n_keys = min(pos0 + M, max_keys);
  // every load has landed before any wave leaves
  wait_vm<0>();
  if constexpr (!XL) {
    if (n_keys <= 0) {  // no position in the cache: the output is zero
      if (s == 0 && p == 0) {
        uint16_t *o = out + (int64_t)m * ldo + (int64_t)(kh * G + g) * HD;
        for (int d = lane; d < HD; d += 64) o[d] = 0;
      }
      return;
    }
  }
  // splits holding a visible key (none: the combine writes zeros)
  const int live = n_keys > 0 ? (n_keys + SPLIT - 1) / SPLIT : 0;
  if (!XL && s >= live) return;
  barrier();
  if (!XL || (here && s < live)) {

  const float4 *ql = reinterpret_cast<const float4 *>(smem + QOFF + qi * HD * 4);
  const int d0 = (lane % KP) * 8;
  float mrun = -INFINITY, lrun = 0.0f;
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = p; c < NCH; c += P) {
    const int jc = j0 + c * WK;
    if (jc >= n_keys) break;
    const int nk = min(WK, n_keys - jc);
    const unsigned char *kt = smem + c * 2 * TILE;
    const unsigned char *krow = kt + lane * ROWB;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
    for (int i = 0; i < KP; i++) {
      const uint4 kr = *reinterpret_cast<const uint4 *>(krow + ((i ^ swz(lane)) * 16));
      const half2v a = as_h2(kr.x), b = as_h2(kr.y), cc = as_h2(kr.z), dd = as_h2(kr.w);
      const float4 qa = ql[2 * i], qb = ql[2 * i + 1];
      s0 = __builtin_fmaf(qa.x, (float)a.x, s0);
      s1 = __builtin_fmaf(qa.y, (float)a.y, s1);
      s2 = __builtin_fmaf(qa.z, (float)b.x, s2);
      s3 = __builtin_fmaf(qa.w, (float)b.y, s3);
      s0 = __builtin_fmaf(qb.x, (float)cc.x, s0);
      s1 = __builtin_fmaf(qb.y, (float)cc.y, s1);
      s2 = __builtin_fmaf(qb.z, (float)dd.x, s2);
      s3 = __builtin_fmaf(qb.w, (float)dd.y, s3);
    }
    const bool vis = lane < nk && jc + lane <= pos0 + m;  // causal
    const float sc = vis ? (s0 + s1) + (s2 + s3) : -INFINITY;
    float cmax = sc;
    cmax = wave_max(cmax);
    const float mnew = fmaxf(mrun, cmax);
    if (mnew == -INFINITY) continue;  // nothing visible to this row yet
    const float alpha = mrun == -INFINITY ? 0.0f : __expf(mrun - mnew);
    const float e = vis ? __expf(sc - mnew) : 0.0f;
    lrun = lrun * alpha + wave_sum(e);
#pragma unroll
    for (int t = 0; t < 8; t++) acc[t] *= alpha;
    // weighted values: lane holds dims d0..d0+7 of rows lane / KP + RPI i;
    // rows past the position may hold any bits: read as zero
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int r = lane / KP + RPI * i;
      uint4 vr = *reinterpret_cast<const uint4 *>(kt + TILE + r * ROWB + (lane % KP) * 16);
      if (r >= nk) vr = make_uint4(0u, 0u, 0u, 0u);
      const float w = __shfl(e, r, 64);
      const uint32_t w4[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const half2v hv = as_h2(w4[t]);
        acc[2 * t] = __builtin_fmaf(w, (float)hv.x, acc[2 * t]);
        acc[2 * t + 1] = __builtin_fmaf(w, (float)hv.y, acc[2 * t + 1]);
      }
    }
    mrun = mnew;
  }
#pragma unroll
  for (int t = 0; t < 8; t++) acc[t] = group_reduce<KP>(acc[t], Plus());
  if (P > 1) {
    // the query's P partitions meet in LDS (past the tiles and queries):
    // partitions p > 0 leave (max, sum, values), partition 0 merges them
    float *mg = reinterpret_cast<float *>(smem + QOFF + FGM * HD * 4);
    if (p > 0) {
      float *e = mg + (qi * (P - 1) + p - 1) * SR;
      if (lane < KP) {
        *reinterpret_cast<f4v *>(e + 4 + d0) = f4v{acc[0], acc[1], acc[2], acc[3]};
        *reinterpret_cast<f4v *>(e + 8 + d0) = f4v{acc[4], acc[5], acc[6], acc[7]};
      } else if (lane == KP) {
        e[0] = mrun;
        e[1] = lrun;
      }
    }
    __syncthreads();
    if (p == 0) {
      for (int j = 1; j < P; j++) {
        const float *e = mg + (qi * (P - 1) + j - 1) * SR;
        const float m2 = e[0], l2 = e[1];
        const float mx = fmaxf(mrun, m2);
        const float a1 = mrun == -INFINITY ? 0.0f : __expf(mrun - mx);
        const float a2 = m2 == -INFINITY ? 0.0f : __expf(m2 - mx);
        lrun = lrun * a1 + l2 * a2;
        if (lane < KP)
#pragma unroll
          for (int t = 0; t < 8; t++) acc[t] = acc[t] * a1 + e[4 + d0 + t] * a2;
        mrun = mx;
      }
    }
  }
  const int qrow = m * H + kh * G + g;
  float *po = partial + ((int64_t)qrow * splits + s) * SR;
  if (p == 0 && lane < KP) {
    store_part<XL>(po + 4 + d0, f4v{acc[0], acc[1], acc[2], acc[3]});
    store_part<XL>(po + 8 + d0, f4v{acc[4], acc[5], acc[6], acc[7]});
  } else if (p == 0 && lane == KP) {
    store_part<XL>(po, f4v{mrun, lrun, 0.0f, 0.0f});
  }
  }  // the split's work
  asm volatile("" ::: "memory");
  wait_vm<0>();  // this wave's stores are done
  __syncthreads();
  int *count = XL ? counters + MAX_KV_COUNTERS + xcd * XCD_LINE : counters + kh;
  // XL: every workgroup of the XCD; else the head's live splits
  const int expect = XL ? (int)(gridDim.x / XCDS) : live;
  if (threadIdx.x == 0) last = count_in<XL>(count, expect);
  __syncthreads();
  if (!last) return;

  if constexpr (XL) {
    // every query of the XCD's heads: several a wave at once when that
    // takes fewer memory round trips, else a wave each
    const int GM = G * M, nq = (KV / XCDS) * GM;
    if (lanes_combine_pays<HD, 8>(nq, nw, live)) {
      constexpr int PER = 64 / (HD / 4);
      for (int j0 = wave * PER; j0 < nq; j0 += nw * PER) {
        const int j = min(j0 + lane / (HD / 4), nq - 1);
        const int kj = xcd + XCDS * (j / GM), gj = j % GM % G, mj = j % GM / G;
        combine_lanes<HD, true, 8>(partial, mj * H + kj * G + gj, splits, live,
                                out + (int64_t)mj * ldo + (int64_t)(kj * G + gj) * HD,
                                j0 + lane / (HD / 4) < nq);
      }
    } else {
      for (int j = wave; j < nq; j += nw) {
        const int kj = xcd + XCDS * (j / GM), gj = j % GM % G, mj = j % GM / G;
        combine_splits<HD, true>(partial + (int64_t)(mj * H + kj * G + gj) * splits * SR, live,
                                 out + (int64_t)mj * ldo + (int64_t)(kj * G + gj) * HD);
      }
    }
  } else {
    combine_splits<HD, false>(partial + (int64_t)(m * H + kh * G + g) * splits * SR, live,
                              out + (int64_t)m * ldo + (int64_t)(kh * G + g) * HD);
  }
}

// Decode attention in one launch on MFMA, for any number of queries per KV
// head (G M: a decode step's G heads, or a verify batch's G M). Workgroup
// = (KV head kh, group qg of 16 of its queries, split s of AW CPW chunks of
// 32 keys); its AW waves each take CPW consecutive chunks and run
// attendPanel's online softmax over them alone:
//  - a chunk's K and V tiles go to the wave's own LDS by direct loads (16-byte
//    pieces of row r at slot piece ^ swz(r), for both), the lane offsets
//    computed once, the chunk's row in a scalar base;
//  - scores as S^T = K Q^T (v_mfma_f32_16x16x32_f16): A = 16 key rows of the
//    K tile, B = the group's 16 queries, each split into hi = half(q) and lo
//    = half(q - hi) (two MFMAs: the scores keep ~22 bits). Lane l then holds
//    keys 4 (l / 16) .. + 3 of a 16-key tile for query l % 16, so a query's
//    max and sum are in-lane plus two lane swaps;
//  - weighted values as O^T = V^T P^T: A = V^T, 16 dims by 32 keys, read by
//    two transposing LDS loads (ds_read_b64_tr_b16: lane i of each 16 gets
//    element i % 4 of the 8 bytes lane 4 j + i / 4 addresses, as its element
//    j), B = the weights split hi / lo, through a small per-wave LDS buffer;
//  - the waves' (max, sum, values) merge in LDS; the workgroup publishes the
//    split's partial, one relaxed atomic counts it in, and the workgroup
//    that completes the count combines the group's queries, several a wave
//    at once (combine_lanes) when the splits are few, else a wave each
//    (combine_splits), as attn_split_kernel does;
//  - XG (KV * QG a multiple of 8): unit u's workgroups all run on XCD u mod
//    8 (ranked as the XCD-grouped split form ranks them), and the exchange
//    stays in that XCD's L2 (LOCAL).
// K rows past the cache read the chunk's first row; V rows at or past the
// last position are zeroed in LDS (a zero weight times a NaN is NaN); the
// keys past a query's position are masked.
// The arguments that place the workgroup and address its first chunk (the
// caches, the position, the query, the key count, the split shape) lead the
// list, within the 14 dwords that arrive preloaded in scalar registers; the
// split kernel's list is ordered the same way.
constexpr int AW = 4;    // waves a workgroup
constexpr int AWK = 32;  // keys a wave's chunk

template <int HD>
__host__ __device__ constexpr int amfma_wave_bytes() {
  return 2 * AWK * HD * 2 + 16 * 36 * 4;  // K and V tiles, the weights (16 x 36 floats)
}

// (PREP) What head_prep_kernel takes besides the rows: the attention then
// prepares its own heads from the q|k|v rows.
struct AttnPrep {
  const float *q_norm, *k_norm;  // (use_norm) the heads' norm weights
  const float *rope;             // rope_rows rows of hd floats
  uint16_t *k_cache, *v_cache;   // the new rows' destination (the caches read)
  float *q_out;                  // (or null) the prepared queries, as head_prep writes them
  int ld_q_out;
  float eps;
  int use_norm, rope_rows, ctx;
};

// (PREP) A lane's rope values for the position of its row: cos and sin of
// the low (c1, s1) and high (c2, s2) table rows at the lane's frequencies
// 32 t + 8 c4 + e (t < HD / 64, c4 = lane / 16 % 4). Returns whether the
// position has rows (in the cache and the table); where it has not, the
// values are row 0's and unused, as head_prep_kernel stores nothing there.
template <int HD>
struct RopeLane {
  float c1[HD / 64][8], s1[HD / 64][8], c2[HD / 64][8], s2[HD / 64][8];
};

template <int HD>
__device__ inline bool rope_lane_load(const AttnPrep &pp, int pos, RopeLane<HD> &r) {
  const bool in = pos >= 0 && pos < pp.ctx && 1024 + (pos >> 10) < pp.rope_rows;
  const int p = in ? pos : 0;
  const int c4 = (threadIdx.x >> 4) & 3;
  const float *r_lo = pp.rope + (int64_t)(p & 1023) * HD;
  const float *r_hi = pp.rope + (int64_t)(1024 + (p >> 10)) * HD;
#pragma unroll
  for (int t = 0; t < HD / 64; t++) {
    const int f = 32 * t + 8 * c4;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      *reinterpret_cast<float4 *>(r.c1[t] + 4 * h) = *reinterpret_cast<const float4 *>(r_lo + f + 4 * h);
      *reinterpret_cast<float4 *>(r.s1[t] + 4 * h) =
          *reinterpret_cast<const float4 *>(r_lo + HD / 2 + f + 4 * h);
      *reinterpret_cast<float4 *>(r.c2[t] + 4 * h) = *reinterpret_cast<const float4 *>(r_hi + f + 4 * h);
      *reinterpret_cast<float4 *>(r.s2[t] + 4 * h) =
          *reinterpret_cast<const float4 *>(r_hi + HD / 2 + f + 4 * h);
    }
  }
  return in;
}

// (PREP) One head row as head_prep_kernel makes it, for a lane holding
// dims 32 t + 8 c4 + e (the 4 lanes of a row are lane % 16 + 16 c4): x the
// raw values, w their norm weights, r the rope values of the row's
// position (`in`: it has rows); every dim rotated (its partner, dim +- hd /
// 2, is in the same lane at t ^ QS / 2). The norm's sum runs in
// head_norm_inv's order (the lane's dims, then the lanes as (S0 + S1) +
// (S2 + S3)). Every lane of the wave calls it; out is written where `in`.
template <int HD>
__device__ inline void prep_head_lane(const float (&x)[HD / 32][8], const float (&w)[HD / 32][8],
                                      bool in, const RopeLane<HD> &r, const AttnPrep &pp,
                                      float scale, float (&out)[HD / 32][8]) {
  constexpr int QS = HD / 32, HQ = QS / 2;
  float inv = 1.0f;
  if (pp.use_norm) {
    float part = 0.0f;
#pragma unroll
    for (int t = 0; t < QS; t++)
#pragma unroll
      for (int e = 0; e < 8; e++) part = __builtin_fmaf(x[t][e], x[t][e], part);
    part = part + xor16(part);
    part = part + xor32(part);
    inv = head_norm_inv(part, HD, pp.eps);
  }
  if (!in) return;
  float v[QS][8];
#pragma unroll
  for (int t = 0; t < QS; t++)
#pragma unroll
    for (int e = 0; e < 8; e++) v[t][e] = x[t][e] * (pp.use_norm ? inv * w[t][e] : 1.0f);
#pragma unroll
  for (int t = 0; t < HQ; t++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float c1 = r.c1[t][e], s1 = r.s1[t][e], c2 = r.c2[t][e], s2 = r.s2[t][e];
      out[t][e] = rope_rotate(v[t][e], v[t + HQ][e], true, c1, s1, c2, s2) * scale;
      out[t + HQ][e] = rope_rotate(v[t + HQ][e], v[t][e], false, c1, s1, c2, s2) * scale;
    }
}

template <int HD, bool XG, bool PREP = false>
__global__ __launch_bounds__(AW * 64) void attn_mfma_kernel(
    const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0_dev, const float *q,
    int max_keys, int splits, int cpw, int M, int H, int KV, int ldq, float *partial,
    int *counters, uint16_t *out, int ldo, const AttnPrep pp) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef _Float16 half4 __attribute__((ext_vector_type(4)));
  typedef short short4v __attribute__((ext_vector_type(4)));
  constexpr int KP = HD / 8, ROWB = HD * 2, TILE = AWK * ROWB, RPI = 64 / KP, NI = AWK / RPI;
  constexpr int QS = HD / 32;  // 32-dim steps of the scores
  constexpr int DT = HD / 16;  // 16-dim tiles of the values
  constexpr int SR = split_row(HD);
  constexpr int WB = amfma_wave_bytes<HD>();
  constexpr int PS = 36;  // weights row stride (floats)
  auto swz = [](int r) { return KP == 16 ? (r & 15) : ((r ^ (r >> 3)) & (KP - 1)); };
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int last;
  const int G = H / KV, GM = G * M;
  const int QG = (GM + 15) / 16;
  // XG: the units (KV * QG, a multiple of 8) go to XCDs by unit % 8, each
  // XCD's workgroups (ranked by blockIdx / 8: workgroups are dispatched to
  // the XCDs in turn) taking its units' splits, so that a unit's partials
  // meet in one L2
  const int u = XG ? (xcd_id() & (XCDS - 1)) + XCDS * ((int)(blockIdx.x / XCDS) / splits)
                   : (int)(blockIdx.x % (KV * QG));
  const int s = XG ? (int)(blockIdx.x / XCDS) % splits : (int)(blockIdx.x / (KV * QG));
  const int kh = u % KV, qg = u / KV;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, c4 = lane >> 4;
  const int kvd = KV * HD;
  unsigned char *wbase = smem + wave * WB;
  unsigned char *kt = wbase, *vt = wbase + TILE;
  float *pbuf = reinterpret_cast<float *>(wbase + 2 * TILE);
  const uint32_t wlds = (uint32_t)(uintptr_t)wbase;
  const int SPLIT = AW * cpw * AWK;  // keys a workgroup takes
  const int j0w = s * SPLIT + wave * cpw * AWK;

  // This lane's byte offset, from a chunk's first row, of its piece of each
  // load instruction (K and V alike): row ii RPI + lane / KP, piece
  // (lane % KP) ^ swz(row).
  uint32_t loff[NI];
#pragma unroll
  for (int ii = 0; ii < NI; ii++) {
    const int r = ii * RPI + lane / KP;
    loff[ii] = (uint32_t)(r * kvd + ((lane % KP) ^ swz(r)) * 8) * 2u;
  }
  auto issue = [&](int j0) {  // chunk j0's K and V tiles, 2 NI instructions
    if (j0 + AWK <= max_keys) {
      const uint16_t *kb = k_cache + (int64_t)j0 * kvd + kh * HD;
      const uint16_t *vb = v_cache + (int64_t)j0 * kvd + kh * HD;
#pragma unroll
      for (int ii = 0; ii < NI; ii++) dma16(kb, loff[ii], wlds + ii * 1024);
#pragma unroll
      for (int ii = 0; ii < NI; ii++) dma16(vb, loff[ii], wlds + TILE + ii * 1024);
    } else {  // the cache's last, partial chunk: rows past it read row j0
#pragma unroll
      for (int i = 0; i < 2 * NI; i++) {
        const bool is_v = i >= NI;
        const int ii = is_v ? i - NI : i;
        const int r = ii * RPI + lane / KP;
        const int piece = (lane % KP) ^ swz(r);
        const int row = j0 + r < max_keys ? j0 + r : j0;
        dma16((is_v ? v_cache : k_cache) + (int64_t)row * kvd + kh * HD + piece * 8,
              wlds + (is_v ? TILE : 0) + ii * 1024);
      }
    }
  };
  // this lane's query (column n16 of every tile)
  const int qi = qg * 16 + n16;
  const bool qvalid = qi < GM;
  const int qm = qvalid ? qi / G : 0, qh = qvalid ? qi % G : 0;
  // the wave's first chunk goes out before the position is read; every
  // exit below waits for it (LDS still being written must not pass to the
  // next workgroup)
  if (j0w < max_keys) issue(j0w);
  // the query's loads go out with the chunk's, ahead of the position
  // (PREP: the raw query of the q|k|v row, and its norm weights)
  float4 qraw[QS][2];
  float qw[PREP ? QS : 1][8];
  {
    const float *qp = q + (int64_t)qm * ldq + (int64_t)(kh * G + qh) * HD + 8 * c4;
#pragma unroll
    for (int t = 0; t < QS; t++) {
      qraw[t][0] = qraw[t][1] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (qvalid) {
        qraw[t][0] = *reinterpret_cast<const float4 *>(qp + 32 * t);
        qraw[t][1] = *reinterpret_cast<const float4 *>(qp + 32 * t + 4);
      }
    }
    if constexpr (PREP)
#pragma unroll
      for (int t = 0; t < QS; t++)
#pragma unroll
        for (int e = 0; e < 8; e++) qw[t][e] = pp.use_norm ? pp.q_norm[32 * t + 8 * c4 + e] : 1.0f;
  }
  // (PREP) the lane's new row j = n16 of the batch: its raw key and the key
  // norm's weights go out with the query's (64 dims: before the position
  // is read; 128: with the rope values, to spare registers)
  constexpr bool EARLY = PREP && HD == 64;
  float xk[PREP ? QS : 1][8], wk[PREP ? QS : 1][8];
  auto load_key = [&]() {
    const float *kp = q + (int64_t)(n16 < M ? n16 : 0) * ldq + (int64_t)(H + kh) * HD + 8 * c4;
#pragma unroll
    for (int t = 0; t < QS; t++) {
      const float4 k0 = *reinterpret_cast<const float4 *>(kp + 32 * t);
      const float4 k1 = *reinterpret_cast<const float4 *>(kp + 32 * t + 4);
      const float ka[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        xk[t][e] = ka[e];
        wk[t][e] = pp.use_norm ? pp.k_norm[32 * t + 8 * c4 + e] : 1.0f;
      }
    }
  };
  if constexpr (EARLY) load_key();
  const int pos0 = *pos0_dev;
  const int n_keys = min(pos0 + M, max_keys);
  const int live = n_keys <= 0 ? 0 : (n_keys + SPLIT - 1) / SPLIT;  // splits with a visible key
  if (n_keys <= 0) {  // no position in the cache: the output is zero
    wait_vm<0>();
    if (s == 0 && qvalid && c4 == 0) {
      uint16_t *o = out + (int64_t)qm * ldo + (int64_t)(kh * G + qh) * HD;
      for (int d = 0; d < HD; d++) o[d] = 0;
    }
    return;
  }
  if (s >= live) {
    wait_vm<0>();
    return;
  }
  const int nch = max(0, min(cpw, (n_keys - j0w + AWK - 1) / AWK));  // this wave's chunks

  // PREP: the batch's new keys and values (rows j < M of the q|k|v rows, at
  // positions pos0 + j) are made here as head_prep_kernel makes them, by
  // the waves whose chunks hold them (into their K and V tiles after each
  // load) and by one wave of the head's first query group and split (into
  // the caches): lane (j = lane % 16, c4) holds row j's dims 32 t + 8 c4 ..
  // + 7 as halves.
  const bool patch = PREP && j0w < n_keys && j0w + nch * AWK > pos0;
  bool knew = false;
  uint4 kh4[PREP ? QS : 1], vh4[PREP ? QS : 1];
  if constexpr (PREP) {
    const bool writer = qg == 0 && s == 0 && wave == 0;
    const bool keys = writer || patch;  // (uniform in the wave)
    // the rope values of the query's position and of the new row's, and
    // the new row's raw value (and key where not loaded yet), all at once
    RopeLane<HD> rq, rk;
    const bool qin = rope_lane_load<HD>(pp, pos0 + qm, rq);
    bool kin = false;
    float xv[QS][8];
    if (keys) {
      kin = rope_lane_load<HD>(pp, pos0 + n16, rk);
      if constexpr (!EARLY) load_key();
      const float *vp =
          q + (int64_t)(n16 < M ? n16 : 0) * ldq + (int64_t)(H + KV + kh) * HD + 8 * c4;
#pragma unroll
      for (int t = 0; t < QS; t++) {
        const float4 v0 = *reinterpret_cast<const float4 *>(vp + 32 * t);
        const float4 v1 = *reinterpret_cast<const float4 *>(vp + 32 * t + 4);
        const float va[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) xv[t][e] = va[e];
      }
    }
    if (keys) {
      float kr[QS][8];
      prep_head_lane<HD>(xk, wk, kin, rk, pp, 1.0f, kr);
      knew = kin && n16 < M;
      if (knew) {
#pragma unroll
        for (int t = 0; t < QS; t++) {
          uint32_t kw[4], vw[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            kw[e] = (uint32_t)to_h(kr[t][2 * e]) | ((uint32_t)to_h(kr[t][2 * e + 1]) << 16);
            vw[e] = (uint32_t)to_h(xv[t][2 * e]) | ((uint32_t)to_h(xv[t][2 * e + 1]) << 16);
          }
          kh4[t] = make_uint4(kw[0], kw[1], kw[2], kw[3]);
          vh4[t] = make_uint4(vw[0], vw[1], vw[2], vw[3]);
        }
        if (writer) {
          const int64_t row = (int64_t)(pos0 + n16) * kvd + (int64_t)kh * HD + 8 * c4;
#pragma unroll
          for (int t = 0; t < QS; t++) {
            *reinterpret_cast<uint4 *>(pp.k_cache + row + 32 * t) = kh4[t];
            *reinterpret_cast<uint4 *>(pp.v_cache + row + 32 * t) = vh4[t];
          }
        }
      }
    }
    // the query as head_prep_kernel makes it (zero where its position has
    // no row)
    float xq[QS][8], oq[QS][8];
#pragma unroll
    for (int t = 0; t < QS; t++) {
      const float4 a = qraw[t][0], b = qraw[t][1];
      const float qa[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) xq[t][e] = qa[e];
    }
    prep_head_lane<HD>(xq, qw, qin, rq, pp, 1.0f / sqrtf((float)HD), oq);
#pragma unroll
    for (int t = 0; t < QS; t++) {
      qraw[t][0] = qraw[t][1] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (qvalid && qin) {
        qraw[t][0] = make_float4(oq[t][0], oq[t][1], oq[t][2], oq[t][3]);
        qraw[t][1] = make_float4(oq[t][4], oq[t][5], oq[t][6], oq[t][7]);
      }
    }
    if (pp.q_out && s == 0 && qvalid) {  // each query once: its group's first split
      float *qo = pp.q_out + (int64_t)qm * pp.ld_q_out + (int64_t)(kh * G + qh) * HD + 8 * c4;
#pragma unroll
      for (int t = 0; t < QS; t++) {
        *reinterpret_cast<float4 *>(qo + 32 * t) = qraw[t][0];
        *reinterpret_cast<float4 *>(qo + 32 * t + 4) = qraw[t][1];
      }
    }
  }

  // the queries as B operands, hi and lo halves: dims 32 t + 8 c4 .. + 7
  half8 qhi[QS], qlo[QS];
  {
#pragma unroll
    for (int t = 0; t < QS; t++) {
      const float4 a = qraw[t][0], b = qraw[t][1];
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const _Float16 hi = (_Float16)v[e];
        qhi[t][e] = hi;
        qlo[t][e] = (_Float16)(v[e] - (float)hi);
      }
    }
  }
  const int q_last = pos0 + qm;  // the last key this query sees
  float m_run = -INFINITY, l_run = 0.0f;
  f4v o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; dt++) o[dt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

  for (int ci = 0; ci < nch; ci++) {
    const int j0 = j0w + ci * AWK;
    wait_vm<0>();
    asm volatile("" ::: "memory");
    if (j0 + AWK > n_keys) {  // V rows at or past the last position read as zero
      const int nv = n_keys - j0;
      for (int idx = nv * KP + lane; idx < AWK * KP; idx += 64)
        *reinterpret_cast<uint4 *>(vt + idx * 16) = make_uint4(0u, 0u, 0u, 0u);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      asm volatile("" ::: "memory");
    }
    if constexpr (PREP) {
      if (patch) {  // the new rows in this chunk: their pieces over the loaded ones
        const int r = pos0 + n16 - j0;
        if (knew && r >= 0 && r < AWK && pos0 + n16 < n_keys) {
#pragma unroll
          for (int t = 0; t < QS; t++) {
            const int at = r * ROWB + (((4 * t + c4) ^ swz(r)) * 16);
            *reinterpret_cast<uint4 *>(kt + at) = kh4[t];
            *reinterpret_cast<uint4 *>(vt + at) = vh4[t];
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        asm volatile("" ::: "memory");
      }
    }
    float sc[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int kt2 = 0; kt2 < 2; kt2++) {
      f4v st = {0.0f, 0.0f, 0.0f, 0.0f};
      const int r = 16 * kt2 + n16;
#pragma unroll
      for (int t = 0; t < QS; t++) {
        const half8 ka =
            *reinterpret_cast<const half8 *>(kt + r * ROWB + (((4 * t + c4) ^ swz(r)) * 16));
        st = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[t], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[t], st, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = j0 + 16 * kt2 + 4 * c4 + i;
        const bool vis = qvalid && key <= q_last && key < max_keys;
        sc[kt2][i] = vis ? st[i] : -INFINITY;
        tmax = fmaxf(tmax, sc[kt2][i]);
      }
    }
    tmax = fmaxf(tmax, xor16(tmax));
    tmax = fmaxf(tmax, xor32(tmax));
    const float m_new = fmaxf(m_run, tmax);
    float psum = 0.0f;
    const float corr = m_run == -INFINITY ? 0.0f : __expf(m_run - m_new);
#pragma unroll
    for (int kt2 = 0; kt2 < 2; kt2++) {
      f4v pv;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pv[i] = sc[kt2][i] == -INFINITY ? 0.0f : __expf(sc[kt2][i] - m_new);
        psum += pv[i];
      }
      *reinterpret_cast<f4v *>(pbuf + n16 * PS + 16 * kt2 + 4 * c4) = pv;
    }
    psum += xor16(psum);
    psum += xor32(psum);
    if (m_new != -INFINITY) {
      l_run = l_run * corr + psum;
#pragma unroll
      for (int dt = 0; dt < DT; dt++) o[dt] *= corr;
    }
    m_run = m_new;
    // every lane's weights are in LDS before any lane reads another's
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("" ::: "memory");
    {
      const f4v pa = *reinterpret_cast<const f4v *>(pbuf + n16 * PS + 8 * c4);
      const f4v pb = *reinterpret_cast<const f4v *>(pbuf + n16 * PS + 8 * c4 + 4);
      half8 phi, plo;
      const float pw[8] = {pa[0], pa[1], pa[2], pa[3], pb[0], pb[1], pb[2], pb[3]};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const _Float16 hi = (_Float16)pw[e];
        phi[e] = hi;
        plo[e] = (_Float16)(pw[e] - (float)hi);
      }
#pragma unroll
      for (int dt = 0; dt < DT; dt++) {
        half8 va;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          // source lane n16 of this 16: row 8 c4 + 4 hh + n16 / 4, dims
          // 16 dt + 4 (n16 % 4) .. + 3
          const int r = 8 * c4 + 4 * hh + (n16 >> 2);
          const int col = 16 * dt + 4 * (n16 & 3);
          const unsigned char *a = vt + r * ROWB + (((col >> 3) ^ swz(r)) * 16) + (col & 7) * 2;
          const short4v t4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) short4v *)(uint32_t)(uintptr_t)a);
          const half4 h4 = __builtin_bit_cast(half4, t4);
#pragma unroll
          for (int e = 0; e < 4; e++) va[4 * hh + e] = h4[e];
        }
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, phi, o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, plo, o[dt], 0, 0, 0);
      }
    }
    // the next chunk's loads may overwrite the tiles: every read of them is done
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("" ::: "memory");
    if (ci + 1 < nch) issue(j0 + AWK);
  }

  // The waves' partials merge in LDS (the tiles are free): wave w > 0 leaves
  // its lane's (max, sum) and DT value quads; wave 0 merges them.
  constexpr int MW = 64 * (4 * DT + 2);  // floats a wave leaves
  static_assert((AW - 1) * MW * 4 <= WB * AW, "merge area");
  float *mrg = reinterpret_cast<float *>(smem);
  wait_vm<0>();  // a first chunk past the position was loaded and not read
  __builtin_amdgcn_s_waitcnt(0xc07f);
  barrier();
  if (wave > 0) {
    float *mw = mrg + (wave - 1) * MW;
    mw[lane] = m_run;
    mw[64 + lane] = l_run;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
      *reinterpret_cast<f4v *>(mw + 128 + (dt * 64 + lane) * 4) = o[dt];
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  barrier();
  float *po = partial + ((int64_t)(qm * H + kh * G + qh) * splits + s) * SR;
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < AW; w++) {
      const float *mw = mrg + (w - 1) * MW;
      const float m2 = mw[lane], l2 = mw[64 + lane];
      const float mx = fmaxf(m_run, m2);
      const float a1 = m_run == -INFINITY ? 0.0f : __expf(m_run - mx);
      const float a2 = m2 == -INFINITY ? 0.0f : __expf(m2 - mx);
      l_run = l_run * a1 + l2 * a2;
#pragma unroll
      for (int dt = 0; dt < DT; dt++)
        o[dt] = o[dt] * a1 + *reinterpret_cast<const f4v *>(mw + 128 + (dt * 64 + lane) * 4) * a2;
      m_run = mx;
    }
    if (qvalid) {  // lane (query, c4) holds dims 16 dt + 4 c4 .. + 3
#pragma unroll
      for (int dt = 0; dt < DT; dt++) store_part<XG>(po + 4 + 16 * dt + 4 * c4, o[dt]);
      if (c4 == 0) store_part<XG>(po, f4v{m_run, l_run, 0.0f, 0.0f});
    }
    wait_vm<0>();  // this wave's coherent stores are done
  }
  __syncthreads();
  // XG: the counter on its XCD's own line (after the split form's)
  int *count = XG ? counters + MAX_KV_COUNTERS + (u % XCDS) * XCD_LINE + 1 + u / XCDS
                  : counters + u;
  if (threadIdx.x == 0) last = count_in<XG>(count, live);
  __syncthreads();
  if (!last) return;
  const int nq = min(16, GM - qg * 16);  // the group's queries
  // several queries a wave at once, a lane group each, 8 or 16 splits a
  // batch (the smaller when it holds them all)
  const bool by8 = live <= 8 && lanes_combine_pays<HD, 8>(nq, AW, live);
  if (by8 || lanes_combine_pays<HD, 16>(nq, AW, live)) {
    constexpr int PER = 64 / (HD / 4);
    for (int k0 = wave * PER; k0 < nq; k0 += AW * PER) {
      const int k = k0 + lane / (HD / 4);
      const int qk = qg * 16 + min(k, nq - 1);
      const int mk = qk / G, gk = qk % G;
      uint16_t *op = out + (int64_t)mk * ldo + (int64_t)(kh * G + gk) * HD;
      if (by8)
        combine_lanes<HD, XG, 8>(partial, mk * H + kh * G + gk, splits, live, op, k < nq);
      else
        combine_lanes<HD, XG, 16>(partial, mk * H + kh * G + gk, splits, live, op, k < nq);
    }
    return;
  }
  // a wave each in turn
  for (int k = wave; k < nq; k += AW) {
    const int qk = qg * 16 + k;
    const int mk = qk / G, gk = qk % G;
    combine_splits<HD, XG>(partial + (int64_t)(mk * H + kh * G + gk) * splits * SR, live,
                       out + (int64_t)mk * ldo + (int64_t)(kh * G + gk) * HD);
  }
}

// The chunks' online-softmax combine (attendPanelCombine): one wave per
// (query head h, row m, slice of 16 dims), 4 per workgroup, lane = chunk
// (c, c + 64, ... up to 256 chunks). A lane loads its chunks' max, sum and
// 16 values at once (one memory round trip); the global max, the weights
// exp(m_c - max), the total and the 16 weighted sums are wave reductions.
// Many small waves rather than a few wide ones: the loads spread over many
// compute units instead of queueing in a few.
constexpr int MAX_CH = 256;  // chunks of 64 keys the combine holds (16384 keys)
constexpr int CSL = 16;      // dims a combine wave takes

template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *partial, int M, int H,
                                                           int chunks,
                                                           const int32_t *pos0_dev,
                                                           int max_keys, uint16_t *out,
                                                           int ldo) {
  constexpr int NS = HD / CSL;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= H * M * NS) return;  // whole waves
  const int sl = wid % NS, h = (wid / NS) % H, m = wid / (NS * H);
  const int lane = threadIdx.x & 63;
  uint16_t *o = out + (int64_t)m * ldo + (int64_t)h * HD + sl * CSL;
  const PartialLayout pl{HD, chunks};
  const float *pr = partial + pl.base(m * H + h, 0);
  // every load first (all within the scratch), then the position
  float cm[MAX_CH / 64], cl[MAX_CH / 64];
  float4 cv[MAX_CH / 64][CSL / 4];
#pragma unroll
  for (int t = 0; t < MAX_CH / 64; t++) {
    const int c = lane + 64 * t;
    const bool ok = c < chunks;
    const float *p = pr + (int64_t)c * (HD + 2);
    cm[t] = ok ? p[0] : -INFINITY;
    cl[t] = ok ? p[1] : 0.0f;
#pragma unroll
    for (int u = 0; u < CSL / 4; u++) {
      const float *pv = p + 2 + sl * CSL + 4 * u;
      cv[t][u] = ok ? make_float4(pv[0], pv[1], pv[2], pv[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const int nk = min(*pos0_dev + m + 1, max_keys);  // keys row m sees
  if (nk <= 0) {
    if (lane < CSL) o[lane] = 0;
    return;
  }
  const int used = (nk + CHUNK - 1) / CHUNK;
  float gmax = -INFINITY;
#pragma unroll
  for (int t = 0; t < MAX_CH / 64; t++)
    if (lane + 64 * t < used) gmax = fmaxf(gmax, cm[t]);
  gmax = wave_max(gmax);
  float ltot = 0.0f, acc[CSL];
#pragma unroll
  for (int d = 0; d < CSL; d++) acc[d] = 0.0f;
#pragma unroll
  for (int t = 0; t < MAX_CH / 64; t++) {
    // chunks past the position (or holding stale bits) weigh exactly zero
    const bool live = lane + 64 * t < used && cm[t] != -INFINITY;
    const float w = live ? __expf(cm[t] - gmax) : 0.0f;
    ltot += live ? w * cl[t] : 0.0f;
#pragma unroll
    for (int u = 0; u < CSL / 4; u++) {
      acc[4 * u] += live ? w * cv[t][u].x : 0.0f;
      acc[4 * u + 1] += live ? w * cv[t][u].y : 0.0f;
      acc[4 * u + 2] += live ? w * cv[t][u].z : 0.0f;
      acc[4 * u + 3] += live ? w * cv[t][u].w : 0.0f;
    }
  }
  ltot = wave_sum(ltot);
#pragma unroll
  for (int d = 0; d < CSL; d++) acc[d] = wave_sum(acc[d]);
  const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
  if (lane == 0) {
    uint32_t hw[CSL / 2];
#pragma unroll
    for (int d = 0; d < CSL / 2; d++)
      hw[d] = (uint32_t)half_bits(acc[2 * d] * inv) |
              ((uint32_t)half_bits(acc[2 * d + 1] * inv) << 16);
    uint4 *o4 = reinterpret_cast<uint4 *>(o);
    o4[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    o4[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
  }
}


// Prefill attention (the reference's chunked scores / attend for a prompt
// batch, Engine.attention src/engine.ts:6359-6630) as flash attention: a
// workgroup per (KV head kh, block of BR query rows) holds the block's
// GM = G * BR <= 32 queries (the KV head's G query heads for each row) and
// walks the keys in chunks of 64 up to the block's last visible key, with an
// online softmax, so it needs no partials and no combine pass. Four waves;
// wave w owns query slots w, w + 4, ..., 8 of them.
//  - each chunk's K and V tiles go to LDS by direct loads, K rows swizzled
//    as in attn_tile_kernel;
//  - scores: lane = key, its K row in registers, each query read from LDS
//    as a broadcast;
//  - per query the chunk's max and sum are DPP wave reductions; the
//    running max, sum and output are rescaled as the max grows;
//  - weighted values: lane = dim (HD / 64 of them), the weights of four
//    keys read from LDS at once as a broadcast.
// Keys past a row's position are masked; value rows past the block's last
// visible key are read as zero (stale bits times a zero weight could be NaN).
constexpr int PF_Q = 32;    // query slots a workgroup
constexpr int PF_QPW = 8;   // query slots a wave

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const float *q, int ldq, int M, int H, int KV, int BR, const uint16_t *k_cache,
    const uint16_t *v_cache, const int32_t *pos0_dev, int max_keys, uint16_t *out, int ldo) {
  constexpr int KP = HD / 8, ROWB = HD * 2, TILE = WK * ROWB, RPI = 64 / KP, NI = WK / RPI;
  constexpr int DPL = HD / 64;  // value dims a lane
  static_assert(DPL == 1 || DPL == 2, "head_dim 64 or 128");
  constexpr int QOFF = 2 * TILE, POFF = QOFF + PF_Q * HD * 4;
  __shared__ __align__(16) unsigned char smem[POFF + 4 * PF_QPW * WK * 4];
  auto swz = [](int r) { return KP == 16 ? (r & 15) : ((r ^ (r >> 3)) & (KP - 1)); };
  const int kh = blockIdx.x % KV, blk = blockIdx.x / KV;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = H / KV, GM = G * BR;
  const int m0 = blk * BR;
  const int m_last = min(M, m0 + BR) - 1;
  const int kvd = KV * HD;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  const int pos0 = *pos0_dev;
  // the block's queries: slot qi = (row m0 + qi / G, head kh G + qi % G)
  for (int k = 0; k < PF_QPW; k++) {
    const int qi = wave + 4 * k;
    const int m = m0 + qi / G;
    if (qi < GM && m < M) {
      constexpr int LPQ = HD / 4;  // lanes a query (16 bytes each)
      if (lane < LPQ)
        dma16(q + (int64_t)m * ldq + (int64_t)(kh * G + qi % G) * HD + lane * 4,
              __builtin_amdgcn_readfirstlane(sbase + QOFF + qi * HD * 4));
    }
  }
  const int last_key = min(pos0 + m_last, max_keys - 1);  // the block's last visible key
  const int nchunks = last_key < 0 ? 0 : last_key / WK + 1;
  float m_run[PF_QPW], l_run[PF_QPW], acc[PF_QPW][DPL];
#pragma unroll
  for (int k = 0; k < PF_QPW; k++) {
    m_run[k] = -INFINITY;
    l_run[k] = 0.0f;
#pragma unroll
    for (int t = 0; t < DPL; t++) acc[k][t] = 0.0f;
  }
  float *pw = reinterpret_cast<float *>(smem + POFF) + wave * PF_QPW * WK;
  for (int c = 0; c < nchunks; c++) {
    const int j0 = c * WK;
    const int nk_max = min(WK, max_keys - j0);
    for (int i = wave; i < 2 * NI; i += 4) {
      const bool is_v = i >= NI;
      const int ii = is_v ? i - NI : i;
      const int r = ii * RPI + lane / KP;
      const int slot = lane % KP;
      const int piece = is_v ? slot : (slot ^ swz(r));
      const int rr = r < nk_max ? r : 0;
      dma16((is_v ? v_cache : k_cache) + (int64_t)(j0 + rr) * kvd + kh * HD + piece * 8,
            __builtin_amdgcn_readfirstlane(sbase + (is_v ? TILE : 0) + ii * 1024));
    }
    wait_vm<0>();
    barrier();
    // this lane's key row
    uint4 kr[KP];
    const unsigned char *krow = smem + lane * ROWB;
#pragma unroll
    for (int i = 0; i < KP; i++)
      kr[i] = *reinterpret_cast<const uint4 *>(krow + ((i ^ swz(lane)) * 16));
    const int jg = j0 + lane;
    float corr[PF_QPW];
#pragma unroll
    for (int k = 0; k < PF_QPW; k++) {
      const int qi = wave + 4 * k;
      const int m = m0 + qi / G;
      corr[k] = 1.0f;
      if (qi >= GM || m >= M) continue;  // wave-uniform
      const float4 *ql = reinterpret_cast<const float4 *>(smem + QOFF + qi * HD * 4);
      float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
      for (int i = 0; i < KP; i++) {
        const half2v a = as_h2(kr[i].x), b = as_h2(kr[i].y), cc = as_h2(kr[i].z),
                     dd = as_h2(kr[i].w);
        const float4 qa = ql[2 * i], qb = ql[2 * i + 1];
        s0 = __builtin_fmaf(qa.x, (float)a.x, s0);
        s1 = __builtin_fmaf(qa.y, (float)a.y, s1);
        s2 = __builtin_fmaf(qa.z, (float)b.x, s2);
        s3 = __builtin_fmaf(qa.w, (float)b.y, s3);
        s0 = __builtin_fmaf(qb.x, (float)cc.x, s0);
        s1 = __builtin_fmaf(qb.y, (float)cc.y, s1);
        s2 = __builtin_fmaf(qb.z, (float)dd.x, s2);
        s3 = __builtin_fmaf(qb.w, (float)dd.y, s3);
      }
      const bool vis = lane < nk_max && jg <= pos0 + m;
      const float sc = vis ? (s0 + s1) + (s2 + s3) : -INFINITY;
      const float m_new = fmaxf(m_run[k], wave_max_u(sc));
      const float p = (!vis || m_new == -INFINITY) ? 0.0f : __expf(sc - m_new);
      corr[k] = m_run[k] == -INFINITY ? 0.0f : __expf(m_run[k] - m_new);
      l_run[k] = l_run[k] * corr[k] + wave_sum_u(p);
      m_run[k] = m_new;
      pw[k * WK + lane] = p;
    }
    // weighted values: lane = dim(s); rows at or past nkv read as zero
    const int nkv = min(WK, last_key - j0 + 1);
#pragma unroll
    for (int k = 0; k < PF_QPW; k++)
#pragma unroll
      for (int t = 0; t < DPL; t++) acc[k][t] *= corr[k];
    const unsigned char *vrow = smem + TILE + lane * DPL * 2;
    for (int jb = 0; jb < (nkv + 3) / 4; jb++) {
      float v[4][DPL];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int j = 4 * jb + u;
        if constexpr (DPL == 2) {
          const half2v hv = as_h2(*reinterpret_cast<const uint32_t *>(vrow + j * ROWB));
          v[u][0] = j < nkv ? (float)hv.x : 0.0f;
          v[u][1] = j < nkv ? (float)hv.y : 0.0f;
        } else {
          const _Float16 hv = *reinterpret_cast<const _Float16 *>(vrow + j * ROWB);
          v[u][0] = j < nkv ? (float)hv : 0.0f;
        }
      }
#pragma unroll
      for (int k = 0; k < PF_QPW; k++) {
        const int qi = wave + 4 * k;
        if (qi >= GM || m0 + qi / G >= M) continue;  // wave-uniform
        const float4 p4 = reinterpret_cast<const float4 *>(pw + k * WK)[jb];
#pragma unroll
        for (int t = 0; t < DPL; t++) {
          float a = acc[k][t];
          a = __builtin_fmaf(p4.x, v[0][t], a);
          a = __builtin_fmaf(p4.y, v[1][t], a);
          a = __builtin_fmaf(p4.z, v[2][t], a);
          a = __builtin_fmaf(p4.w, v[3][t], a);
          acc[k][t] = a;
        }
      }
    }
    barrier();  // every wave is done with this chunk's tiles
  }
  wait_vm<0>();  // (no chunk: the query loads must still land before the workgroup ends)
#pragma unroll
  for (int k = 0; k < PF_QPW; k++) {
    const int qi = wave + 4 * k;
    const int m = m0 + qi / G;
    if (qi >= GM || m >= M) continue;
    const float inv = l_run[k] > 0.0f ? 1.0f / l_run[k] : 0.0f;
    uint16_t *o = out + (int64_t)m * ldo + (int64_t)(kh * G + qi % G) * HD + lane * DPL;
#pragma unroll
    for (int t = 0; t < DPL; t++) o[t] = to_h(acc[k][t] * inv);
  }
}

// The same prompt attention on MFMA (v_mfma_f32_32x32x16_f16, f32
// accumulation). A wave owns 32 queries (slots of the workgroup's rows x the
// KV head's G query heads) and walks the keys 32 at a time:
//  - scores as S^T = K Q^T: A = 32 key rows of the K tile (16-byte pieces,
//    swizzled as in attn_tile_kernel), B = the wave's queries. The queries
//    are f32; each is split into hi = half(q) and lo = half(q - hi), two
//    MFMAs, so the scores keep ~22 bits (the keys are halves already);
//  - in that orientation lane i holds 16 keys of query i % 32 (keys
//    8 (j / 4) + 4 (i / 32) + j % 4 of the tile), so the softmax max and sum
//    are in-lane plus one exchange between the half-waves;
//  - weighted values as O^T = V^T P^T: B = the lane's own weights (slice s
//    of 16 keys = registers 8 s .. 8 s + 7, split hi / lo like the queries),
//    A = the values of those keys (k-index 8 h + t = key 16 s + 8 (t / 4) +
//    4 h + t % 4) read from LDS; O^T keeps every output of a lane in its
//    query, so the online-softmax rescale is per lane.
// K and V rows past the block's last visible key (or the cache) are loaded
// from the chunk's first row instead: stale bits never reach an MFMA.
template <int HD, int NW>
__global__ __launch_bounds__(NW * 64) void attn_prefill_mfma_kernel(
    const float *q, int ldq, int M, int H, int KV, int R, const uint16_t *k_cache,
    const uint16_t *v_cache, const int32_t *pos0_dev, int max_keys, uint16_t *out, int ldo) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef float float16v __attribute__((ext_vector_type(16)));
  constexpr int KP = HD / 8, ROWB = HD * 2, TILE = WK * ROWB, RPI = 64 / KP, NI = WK / RPI;
  constexpr int KS = HD / 16, DT = HD / 32;
  __shared__ __align__(16) unsigned char smem[2 * TILE];
  auto swz = [](int r) { return KP == 16 ? (r & 15) : ((r ^ (r >> 3)) & (KP - 1)); };
  const int kh = blockIdx.x % KV, blk = blockIdx.x / KV;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = lane >> 5, c32 = lane & 31;
  const int G = H / KV, GM = G * R;
  const int m0 = blk * R;
  const int m_last = min(M, m0 + R) - 1;
  const int kvd = KV * HD;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  const int pos0 = *pos0_dev;
  // this lane's query (slot qs) and the wave's last visible key
  const int qs = wave * 32 + c32;
  const int qm = m0 + qs / G;
  const bool qvalid = qs < GM && qm < M;
  const int q_last = pos0 + qm;  // the last key this query sees
  const int wlast_slot = min(wave * 32 + 31, GM - 1);
  const int w_row = min(m0 + wlast_slot / G, m_last);
  const bool w_any = wave * 32 < GM && m0 + (wave * 32) / G <= m_last;
  const int w_last_key = min(pos0 + w_row, max_keys - 1);
  const int last_key = min(pos0 + m_last, max_keys - 1);
  const int nchunks = last_key < 0 ? 0 : last_key / WK + 1;
  half8 qb_hi[KS], qb_lo[KS];
  {
    const float *qp = q + (int64_t)(qvalid ? qm : 0) * ldq + (int64_t)(kh * G + qs % G) * HD + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
      if (qvalid) {
        a = *reinterpret_cast<const float4 *>(qp + 16 * ks);
        b = *reinterpret_cast<const float4 *>(qp + 16 * ks + 4);
      }
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const _Float16 hi = (_Float16)v[t];
        qb_hi[ks][t] = hi;
        qb_lo[ks][t] = (_Float16)(v[t] - (float)hi);
      }
    }
  }
  float m_run = -INFINITY, l_run = 0.0f;
  float16v o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int j = 0; j < 16; j++) o[dt][j] = 0.0f;
  for (int c = 0; c < nchunks; c++) {
    const int j0 = c * WK;
    const int nk_load = min(WK, last_key - j0 + 1);  // rows worth loading (>= 1)
    for (int i = wave; i < 2 * NI; i += NW) {
      const bool is_v = i >= NI;
      const int ii = is_v ? i - NI : i;
      const int r = ii * RPI + lane / KP;
      const int slot = lane % KP;
      const int piece = is_v ? slot : (slot ^ swz(r));
      const int rr = r < nk_load ? r : 0;
      dma16((is_v ? v_cache : k_cache) + (int64_t)(j0 + rr) * kvd + kh * HD + piece * 8,
            __builtin_amdgcn_readfirstlane(sbase + (is_v ? TILE : 0) + ii * 1024));
    }
    wait_vm<0>();
    barrier();
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      const int kb = j0 + 32 * kt;
      if (!w_any || kb > w_last_key) continue;  // wave-uniform
      float16v st;
#pragma unroll
      for (int j = 0; j < 16; j++) st[j] = 0.0f;
      const int r = 32 * kt + c32;
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        const half8 ka = *reinterpret_cast<const half8 *>(smem + r * ROWB +
                                                         (((2 * ks + hh) ^ swz(r)) * 16));
        st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb_hi[ks], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb_lo[ks], st, 0, 0, 0);
      }
      float p[16];
      float tmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const int key = kb + 8 * (j >> 2) + 4 * hh + (j & 3);
        const bool vis = qvalid && key <= q_last && key < max_keys;
        p[j] = vis ? st[j] : -INFINITY;
        tmax = fmaxf(tmax, p[j]);
      }
      tmax = fmaxf(tmax, xor32(tmax));
      const float m_new = fmaxf(m_run, tmax);
      const float corr = m_new == -INFINITY ? 1.0f : __expf(m_run - m_new);
      float psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        p[j] = p[j] == -INFINITY ? 0.0f : __expf(p[j] - m_new);
        psum += p[j];
      }
      psum += xor32(psum);
      l_run = l_run * corr + psum;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int j = 0; j < 16; j++) o[dt][j] *= corr;
#pragma unroll
      for (int sl = 0; sl < 2; sl++) {
        half8 pb_hi, pb_lo;
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const _Float16 hi = (_Float16)p[8 * sl + t];
          pb_hi[t] = hi;
          pb_lo[t] = (_Float16)(p[8 * sl + t] - (float)hi);
        }
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
          half8 va;
#pragma unroll
          for (int t = 0; t < 8; t++) {
            const int vr = 32 * kt + 16 * sl + 8 * (t >> 2) + 4 * hh + (t & 3);
            va[t] = *reinterpret_cast<const _Float16 *>(smem + TILE + vr * ROWB +
                                                        (32 * dt + c32) * 2);
          }
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb_hi, o[dt], 0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb_lo, o[dt], 0, 0, 0);
        }
      }
    }
    barrier();  // every wave is done with this chunk's tiles
  }
  wait_vm<0>();
  if (qvalid) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    uint16_t *op = out + (int64_t)qm * ldo + (int64_t)(kh * G + qs % G) * HD;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int j = 0; j < 16; j++)
        op[32 * dt + 8 * (j >> 2) + 4 * hh + (j & 3)] = to_h(o[dt][j] * inv);
  }
}

}  // namespace

// The no-allocation entry point's scratch (the chunks' partial results):
// one array per GPU, held while the process lives. Every call on a GPU
// shares it, so calls that overlap on one GPU race.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

__global__ void clear_ints_kernel(int *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// The device address of `scratch` on the current device, looked up once per
// device (each GPU holds its own copy at its own address; the array's name
// is no device address in host code). The first lookup on a device also
// clears the one-launch attention's counters at the array's start (static
// storage starts zeroed; the clear, a kernel on the caller's stream, makes
// sure of it without a memset).
static int noalloc_scratch(void **out, hipStream_t stream) {
  static std::mutex mu;
  static void *ptrs[64];
  int dev = 0;
  WG_HIP(hipGetDevice(&dev));
  WG_REQUIRE(dev >= 0 && dev < 64, "no-allocation scratch: device %d", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(WG_ERR_DEVICE, "no-allocation scratch on device %d: %s", dev,
                  hipGetErrorString(e));
    clear_ints_kernel<<<1, COUNTER_INTS, 0, stream>>>((int *)p, COUNTER_INTS);
    int rc = launched("no-allocation scratch (counters)");
    if (rc) return rc;
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return WG_OK;
}

// The XCD-grouped forms take for granted that the dispatcher deals
// workgroups to 8 XCDs round-robin: the 8 workgroups b = 8r .. 8r + 7 run
// one on each XCD (the whole MI355X in its single-partition mode). On a
// partitioned device, one with another XCD count, or under a CU mask, a
// workgroup would take a (KV head, split) pair another one also takes and
// leave one untaken, so the grouped forms run only where the device says it
// has 8 XCDs and a probe launch has seen every such group of 8 land on 8
// distinct XCDs.
constexpr int PROBE_BLOCKS = 8 * 256;
static __device__ int xcd_probe_ids[PROBE_BLOCKS];

__global__ void xcd_probe_kernel(int *ids) {
  if (threadIdx.x == 0) ids[blockIdx.x] = xcd_id();
}

// Whether the XCD-grouped forms may run on the current device: decided once
// a device, by the first call not made while the stream is being captured
// (the probe waits for its own launch); a call under capture before then
// takes the ungrouped forms.
static bool xcd_grouping(hipStream_t stream) {
  static std::mutex mu;
  static signed char known[64];  // 0 unknown, 1 grouped forms allowed, -1 not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::lock_guard<std::mutex> lock(mu);
  if (known[dev]) return known[dev] > 0;
  int xccs = 0;
  if (hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
      xccs != XCDS) {
    (void)hipGetLastError();
    known[dev] = -1;
    return false;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return false;
  }
  void *d = nullptr;
  if (hipGetSymbolAddress(&d, HIP_SYMBOL(xcd_probe_ids)) != hipSuccess || !d) {
    (void)hipGetLastError();
    known[dev] = -1;
    return false;
  }
  static int ids[PROBE_BLOCKS];
  xcd_probe_kernel<<<PROBE_BLOCKS, 64, 0, stream>>>((int *)d);
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(ids, d, sizeof ids, hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess) {
    (void)hipGetLastError();
    known[dev] = -1;
    return false;
  }
  bool ok = true;
  for (int g = 0; ok && g < PROBE_BLOCKS / XCDS; g++) {
    int seen = 0;
    for (int j = 0; j < XCDS; j++) {
      const int x = ids[g * XCDS + j];
      if (x < 0 || x >= XCDS) ok = false;
      else seen |= 1 << x;
    }
    ok = ok && seen == (1 << XCDS) - 1;
  }
  known[dev] = ok ? 1 : -1;
  return ok;
}

// The MFMA decode attention's launch: cpw chunks a wave, as few as keep
// about one workgroup a compute unit; grouped by XCD where the units are a
// multiple of 8 and `group`. PREP: the heads prepared in the kernel.
template <bool PREP>
static int launch_amfma(const float *q, int M, int ldq, int H, int KV, int hd,
                        const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0,
                        int max_keys, uint16_t *out, int ldo, float *partial, int *counters,
                        const AttnPrep &pp, bool group, hipStream_t s) {
  const int QG = ((H / KV) * M + 15) / 16;  // groups of 16 queries a KV head
  const int cus = persistent_grid(1 << 30, 1);
  const int units = KV * QG;
  const int wchunks = (max_keys + AWK - 1) / AWK;  // 32-key chunks
  int cpw = (int)(((int64_t)wchunks * units + (int64_t)AW * cus - 1) / ((int64_t)AW * cus));
  cpw = cpw < 1 ? 1 : cpw;
  const int splits = (wchunks + AW * cpw - 1) / (AW * cpw);
  const size_t lds = (size_t)AW * (hd == 64 ? amfma_wave_bytes<64>() : amfma_wave_bytes<128>());
  const dim3 grid((unsigned)(units * splits));
  const bool xg = units % XCDS == 0 && group && xcd_grouping(s);
#define WG_AMFMA_LAUNCH(HDV, XGV)                                                                \
  do {                                                                                           \
    int rc_ = raise_lds((const void *)attn_mfma_kernel<HDV, XGV, PREP>, (int)lds);               \
    if (rc_) return rc_;                                                                         \
    attn_mfma_kernel<HDV, XGV, PREP><<<grid, AW * 64, lds, s>>>(                                 \
        k_cache, v_cache, pos0, q, max_keys, splits, cpw, M, H, KV, ldq, partial, counters, out, \
        ldo, pp);                                                                                \
  } while (0)
  if (hd == 64) {
    if (xg) WG_AMFMA_LAUNCH(64, true);
    else WG_AMFMA_LAUNCH(64, false);
  } else {
    if (xg) WG_AMFMA_LAUNCH(128, true);
    else WG_AMFMA_LAUNCH(128, false);
  }
#undef WG_AMFMA_LAUNCH
  return launched("wg_attn_decode");
}

}  // namespace wg

using namespace wg;

extern "C" {

int wg_head_prep(const float *qkv, int32_t M, int32_t ldq, const wg_attn_shape *sh,
                 const float *q_norm, const float *k_norm, const float *rope, int32_t rope_rows,
                 const int32_t *pos0, float *q_out, int32_t ldqo, uint16_t *k_cache,
                 uint16_t *v_cache, int32_t ctx, void *stream) {
  WG_REQUIRE(sh && qkv && rope && pos0 && q_out && k_cache && v_cache,
             "wg_head_prep: null argument");
  WG_REQUIRE(M >= 1 && M <= 65535, "wg_head_prep: %d rows", M);
  WG_REQUIRE(sh->kv_heads > 0 && sh->heads % sh->kv_heads == 0,
             "wg_head_prep: %d query heads over %d KV heads", sh->heads, sh->kv_heads);
  WG_REQUIRE(sh->head_dim >= 2 && sh->head_dim <= MAX_HD && sh->head_dim % 2 == 0,
             "wg_head_prep: head_dim %d", sh->head_dim);
  WG_REQUIRE(sh->rotated_dims >= 0 && sh->rotated_dims <= sh->head_dim &&
                 sh->rotated_dims % 2 == 0,
             "wg_head_prep: rotated dims %d", sh->rotated_dims);
  WG_REQUIRE(!sh->use_norm || (q_norm && k_norm), "wg_head_prep: norm weights missing");
  WG_REQUIRE(ctx >= 1 && rope_rows >= 1024 + (ctx + 1023) / 1024,
             "wg_head_prep: a rope table of %d rows for a %d-position cache (needs %d)",
             rope_rows, ctx, 1024 + (ctx + 1023) / 1024);
  int slots = sh->heads + 2 * sh->kv_heads;
  WG_REQUIRE(ldq >= slots * sh->head_dim && ldqo >= sh->heads * sh->head_dim,
             "wg_head_prep: strides too small");
  head_prep_kernel<<<dim3(slots, M), 64, 0, as_stream(stream)>>>(
      qkv, pos0, q_norm, k_norm, ldq, sh->heads, sh->kv_heads, sh->head_dim, sh->use_norm,
      sh->rotated_dims, sh->eps, rope, rope_rows, q_out, ldqo, k_cache, v_cache, ctx);
  return launched("wg_head_prep");
}

size_t wg_attn_scratch_bytes(int32_t M, int32_t heads, int32_t head_dim, int32_t max_keys) {
  int64_t chunks = (max_keys + CHUNK - 1) / CHUNK;
  // rows of split_row(head_dim) floats hold either form's partials
  return COUNTER_BYTES + (size_t)M * heads * chunks * split_row(head_dim) * sizeof(float);
}

int wg_attn_prefill(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *sh,
                    const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0,
                    int32_t max_keys, uint16_t *out, int32_t ldo, void *stream) {
  WG_REQUIRE(sh && q && k_cache && v_cache && pos0 && out, "wg_attn_prefill: null argument");
  int H = sh->heads, KV = sh->kv_heads, hd = sh->head_dim;
  WG_REQUIRE(KV > 0 && H % KV == 0 && H / KV <= PF_Q,
             "wg_attn_prefill: %d query heads over %d KV heads", H, KV);
  WG_REQUIRE(hd == 64 || hd == 128, "wg_attn_prefill: head_dim %d (64 or 128)", hd);
  WG_REQUIRE(M >= 1 && max_keys >= 1, "wg_attn_prefill: %d rows, %d keys", M, max_keys);
  WG_REQUIRE(ldq >= H * hd && ldo >= H * hd, "wg_attn_prefill: strides too small");
  WG_REQUIRE(((uintptr_t)q & 15) == 0 && ldq % 4 == 0,
             "wg_attn_prefill: queries must be 16-byte aligned with a stride of 4k floats");
  hipStream_t s = as_stream(stream);
  if (const int nw = tuning("attn_prefill_mfma")) {  // waves (32 queries each) a workgroup
    const int R = nw * 32 / (H / KV);
    WG_REQUIRE(R >= 1, "wg_attn_prefill: %d query heads a KV head", H / KV);
    const int64_t blocks = (int64_t)KV * ((M + R - 1) / R);
    WG_REQUIRE(blocks <= 0x7fffffff, "wg_attn_prefill: %d rows", M);
#define WG_PF_LAUNCH(NWP)                                                                      \
  do {                                                                                         \
    if (hd == 64)                                                                              \
      attn_prefill_mfma_kernel<64, NWP><<<(unsigned)blocks, NWP * 64, 0, s>>>(                 \
          q, ldq, M, H, KV, R, k_cache, v_cache, pos0, max_keys, out, ldo);                    \
    else                                                                                       \
      attn_prefill_mfma_kernel<128, NWP><<<(unsigned)blocks, NWP * 64, 0, s>>>(                \
          q, ldq, M, H, KV, R, k_cache, v_cache, pos0, max_keys, out, ldo);                    \
  } while (0)
    if (nw == 1) WG_PF_LAUNCH(1);
    else if (nw == 4) WG_PF_LAUNCH(4);
    else WG_PF_LAUNCH(2);
#undef WG_PF_LAUNCH
    return launched("wg_attn_prefill");
  }
  const int BR = PF_Q / (H / KV);
  const int64_t blocks = (int64_t)KV * ((M + BR - 1) / BR);
  WG_REQUIRE(blocks <= 0x7fffffff, "wg_attn_prefill: %d rows", M);
  if (hd == 64)
    attn_prefill_kernel<64><<<(unsigned)blocks, 256, 0, s>>>(q, ldq, M, H, KV, BR, k_cache,
                                                            v_cache, pos0, max_keys, out, ldo);
  else
    attn_prefill_kernel<128><<<(unsigned)blocks, 256, 0, s>>>(q, ldq, M, H, KV, BR, k_cache,
                                                             v_cache, pos0, max_keys, out, ldo);
  return launched("wg_attn_prefill");
}

int wg_attn_decode(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *sh,
                   const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0,
                   int32_t max_keys, uint16_t *out, int32_t ldo, void *scratch,
                   size_t scratch_bytes, void *stream) {
  WG_REQUIRE(sh && q && k_cache && v_cache && pos0 && out && scratch,
             "wg_attn_decode: null argument");
  int H = sh->heads, KV = sh->kv_heads, hd = sh->head_dim;
  WG_REQUIRE(KV > 0 && H % KV == 0, "wg_attn_decode: %d query heads over %d KV heads", H, KV);
  WG_REQUIRE(M >= 1 && (H / KV) * M <= 64,
             "wg_attn_decode: %d rows x %d heads per KV head (at most 64)", M, H / KV);
  WG_REQUIRE(hd == 64 || hd == 128, "wg_attn_decode: head_dim %d (64 or 128)", hd);
  // The one-launch form's last-arriver combine costs about as much as the
  // second launch it saves at 2048 cached keys, more past that (measured at
  // 4096 keys: 14.3 us against 8.4 + 4.7), less below: it is taken up to
  // 1024 keys and past the two-launch form's 16384 (attn_fused 2 always
  // takes it, 0 never).
  const int fused_knob = tuning("attn_fused");
  const bool fits = (H / KV) * M <= FGM && KV <= MAX_KV_COUNTERS;
  const bool fused = fits && (fused_knob == 2 ||
                              (fused_knob == 1 && (max_keys <= 1024 || max_keys > MAX_CH * CHUNK)));
  // the one-launch forms combine any number of splits; the two-launch
  // combine holds MAX_CH chunks
  // Which form, from layer-by-layer timings in captured graphs (us a layer;
  // 32 query heads over 8 of 128 dims / of 64 dims):
  //   rows keys       XCD-grouped    MFMA          two-launch
  //   1    1024       8.3 / 6.7      8.6 / 7.2     9.3 / 8.1
  //   1    2048       8.6 / 7.2      9.0 / 7.5     9.8 / 8.3
  //   1    4096      10.8 / 8.4     10.2 / 8.2    11.6 / 9.1
  //   1    8192      16.9 / 11.2    14.7 / 10.2   15.2 / 11.2
  //   2    1024       9.0 / 7.6      8.3 / 6.7     9.7 / 8.5
  //   2    4096      13.4 / 10.3    11.8 / 9.7    13.6 / 10.4
  // and with 14 query heads over 2 (not a multiple of 8, no XCD grouping;
  // 64 dims, one row): MFMA 7.2 at 1024 and 2048 keys against 7.7 / 7.8
  // two-launch, 9.6 / 11.1 at 4096 / 8192 against 8.4 / 8.9. So, by
  // default: MFMA past 8 queries a KV head (a verify batch), from 16384
  // keys on, and, with KV heads a multiple of 8, everywhere but the
  // XCD-grouped form's range (up to 4 queries a KV head below 4096 keys),
  // otherwise up to 2048 keys; the chunk and combine kernels in between.
  // attn_mfma 2 always takes the MFMA form, 0 never; attn_xcd 2 always
  // takes the XCD-grouped form where it applies, 0 never (nor groups the
  // MFMA form by XCD).
  const int GMq = (H / KV) * M;
  hipStream_t s = as_stream(stream);
  const int xcd_knob = tuning("attn_xcd");
  // (the XCD-grouped forms only where the dispatch they assume is checked)
  const bool groupable = KV % XCDS == 0 && xcd_grouping(s);
  const int mfma_knob = tuning("attn_mfma");
  const bool xl_range = groupable && GMq <= 4 && max_keys < 4096 && xcd_knob != 0;
  const bool amfma = KV * ((GMq + 15) / 16) <= MAX_KV_COUNTERS &&
                     (mfma_knob == 2 ||
                      (mfma_knob == 1 && (GMq > FGM || max_keys >= 16384 ||
                                          (groupable ? !xl_range : max_keys <= 2048))));
  const bool xl = !amfma && GMq <= FGM && groupable &&
                  (xcd_knob == 2 || (xcd_knob == 1 && max_keys < 4096));
  const int key_cap = fused || amfma || xl ? MAX_FUSED_KEYS : MAX_CH * CHUNK;
  WG_REQUIRE(max_keys >= M && max_keys <= key_cap,
             "wg_attn_decode: max_keys %d (rows %d; at most %d)", max_keys, M, key_cap);
  WG_REQUIRE(ldq >= H * hd && ldo >= H * hd, "wg_attn_decode: strides too small");
  WG_REQUIRE(((uintptr_t)out & 15) == 0 && ldo % 8 == 0,
             "wg_attn_decode: the output must be 16-byte aligned with a stride of 8k halves");
  WG_REQUIRE(scratch_bytes >= wg_attn_scratch_bytes(M, H, hd, max_keys),
             "wg_attn_decode: scratch of %zu bytes, %zu needed", scratch_bytes,
             wg_attn_scratch_bytes(M, H, hd, max_keys));
  int *counters = (int *)scratch;
  float *partial = (float *)((char *)scratch + COUNTER_BYTES);
  const int chunks = (max_keys + CHUNK - 1) / CHUNK;
  const int QG = ((H / KV) * M + 15) / 16;  // groups of 16 queries a KV head
  if (amfma)  // (attn_xcd 0: never grouped by XCD)
    return launch_amfma<false>(q, M, ldq, H, KV, hd, k_cache, v_cache, pos0, max_keys, out, ldo,
                               partial, counters, AttnPrep{}, xcd_knob != 0, s);
  if (fused || xl) {
    // one launch: 64 * nch keys a workgroup, the smallest nch (1, 2, 4) that
    // keeps the grid to about one workgroup a compute unit
    int nch = tuning("attn_split_chunks");
    if (nch == 3) nch = 4;
    if (!nch) {
      const int cus = persistent_grid(1 << 30, 1);
      nch = KV * chunks <= cus ? 1 : KV * ((chunks + 1) / 2) <= cus ? 2 : 4;
    }
    const int splits = (chunks + nch - 1) / nch;
    // P waves a query, each taking every P-th chunk of the split (up to 16
    // waves), their partials merged in LDS (MERGE_ROWS rows past the queries)
    const int GMq = (H / KV) * M;
    int P = nch < 16 / GMq ? nch : 16 / GMq;
    if (tuning("attn_split_waves") == 0) P = 1;
    const size_t lds = (size_t)2 * nch * WK * hd * 2 + (size_t)FGM * hd * 4 +
                       (P > 1 ? (size_t)MERGE_ROWS * split_row(hd) * 4 : 0);
    dim3 grid((unsigned)(KV * splits));
    const unsigned threads = 64 * GMq * P;
#define WG_SPLIT_LAUNCH1(HDV, NCHV, XLV)                                                        \
  do {                                                                                          \
    int rc_ = raise_lds((const void *)attn_split_kernel<HDV, NCHV, XLV>, (int)lds);              \
    if (rc_) return rc_;                                                                        \
    attn_split_kernel<HDV, NCHV, XLV><<<grid, threads, lds, s>>>(                               \
        k_cache, v_cache, pos0, q, max_keys, splits, M, H, KV, (int)(threads / 64), ldq,       \
        partial, counters, out, ldo);                                                           \
  } while (0)
#define WG_SPLIT_LAUNCH(HDV, NCHV)                                                              \
  do {                                                                                          \
    if (xl) WG_SPLIT_LAUNCH1(HDV, NCHV, true);                                                  \
    else WG_SPLIT_LAUNCH1(HDV, NCHV, false);                                                    \
  } while (0)
    if (hd == 64) {
      if (nch == 1) WG_SPLIT_LAUNCH(64, 1);
      else if (nch == 2) WG_SPLIT_LAUNCH(64, 2);
      else WG_SPLIT_LAUNCH(64, 4);
    } else {
      if (nch == 1) WG_SPLIT_LAUNCH(128, 1);
      else if (nch == 2) WG_SPLIT_LAUNCH(128, 2);
      else WG_SPLIT_LAUNCH(128, 4);
    }
#undef WG_SPLIT_LAUNCH
#undef WG_SPLIT_LAUNCH1
    return launched("wg_attn_decode");
  }
  if ((H / KV) * M <= FGM) {
    dim3 grid((unsigned)(KV * chunks));
    if (hd == 64)
      attn_tile_kernel<64><<<grid, 64 * (H / KV) * M, 0, s>>>(
          q, ldq, M, H, KV, k_cache, v_cache, pos0, max_keys, partial, chunks, out, ldo);
    else
      attn_tile_kernel<128><<<grid, 64 * (H / KV) * M, 0, s>>>(
          q, ldq, M, H, KV, k_cache, v_cache, pos0, max_keys, partial, chunks, out, ldo);
  } else {
    size_t lds = attn_lds_bytes((H / KV) * M, hd);
    int rc = raise_lds((const void *)attn_chunk_kernel<64>, 160 * 1024);  // past 64 KiB
    if (!rc) rc = raise_lds((const void *)attn_chunk_kernel<128>, 160 * 1024);
    if (rc) return rc;
    if (hd == 64)
      attn_chunk_kernel<64><<<dim3(KV, chunks), 256, lds, s>>>(
          q, ldq, M, H, KV, k_cache, v_cache, pos0, max_keys, partial, chunks);
    else
      attn_chunk_kernel<128><<<dim3(KV, chunks), 256, lds, s>>>(
          q, ldq, M, H, KV, k_cache, v_cache, pos0, max_keys, partial, chunks);
  }
  int rc = launched("wg_attn_decode");
  if (rc) return rc;
  unsigned cgrid = (unsigned)((H * M * (hd / CSL) + 3) / 4);
  if (hd == 64)
    attn_combine_kernel<64><<<cgrid, 256, 0, s>>>(partial, M, H, chunks, pos0, max_keys, out,
                                                  ldo);
  else
    attn_combine_kernel<128><<<cgrid, 256, 0, s>>>(partial, M, H, chunks, pos0, max_keys, out,
                                                   ldo);
  return launched("wg_attn_decode (combine)");
}

int wg_attn_decode_prep(const float *qkv, int32_t M, int32_t ldqkv, const wg_attn_shape *sh,
                        const float *q_norm, const float *k_norm, const float *rope,
                        int32_t rope_rows, int32_t ctx, uint16_t *k_cache, uint16_t *v_cache,
                        const int32_t *pos0, int32_t max_keys, float *q_out, int32_t ld_q_out,
                        uint16_t *out, int32_t ldo, void *scratch, size_t scratch_bytes,
                        void *stream) {
  WG_REQUIRE(sh && qkv && rope && k_cache && v_cache && pos0 && out && scratch,
             "wg_attn_decode_prep: null argument");
  const int H = sh->heads, KV = sh->kv_heads, hd = sh->head_dim;
  WG_REQUIRE(KV > 0 && H % KV == 0, "wg_attn_decode_prep: %d query heads over %d KV heads", H,
             KV);
  WG_REQUIRE(hd == 64 || hd == 128, "wg_attn_decode_prep: head_dim %d (64 or 128)", hd);
  WG_REQUIRE(M >= 1 && (H / KV) * M <= 64,
             "wg_attn_decode_prep: %d rows x %d heads per KV head (at most 64)", M, H / KV);
  WG_REQUIRE(!sh->use_norm || (q_norm && k_norm), "wg_attn_decode_prep: norm weights missing");
  WG_REQUIRE(ctx >= 1 && rope_rows >= 1024 + (ctx + 1023) / 1024,
             "wg_attn_decode_prep: a rope table of %d rows for a %d-position cache", rope_rows,
             ctx);
  WG_REQUIRE(max_keys >= M && max_keys <= ctx && max_keys <= MAX_FUSED_KEYS,
             "wg_attn_decode_prep: max_keys %d (rows %d, cache %d)", max_keys, M, ctx);
  WG_REQUIRE(ldqkv >= (H + 2 * KV) * hd && ldqkv % 4 == 0 && ((uintptr_t)qkv & 15) == 0 &&
                 ((uintptr_t)rope & 15) == 0 && ((uintptr_t)k_cache & 15) == 0 &&
                 ((uintptr_t)v_cache & 15) == 0,
             "wg_attn_decode_prep: the q|k|v rows, rope table and caches must be 16-byte "
             "aligned (row stride a multiple of 4 floats, at least the heads' width)");
  WG_REQUIRE(!q_out || (ld_q_out >= H * hd && ld_q_out % 4 == 0 && ((uintptr_t)q_out & 15) == 0),
             "wg_attn_decode_prep: q_out stride or alignment");
  WG_REQUIRE(ldo >= H * hd && ((uintptr_t)out & 15) == 0 && ldo % 8 == 0,
             "wg_attn_decode_prep: the output must be 16-byte aligned with a stride of 8k halves");
  WG_REQUIRE(scratch_bytes >= wg_attn_scratch_bytes(M, H, hd, max_keys),
             "wg_attn_decode_prep: scratch of %zu bytes, %zu needed", scratch_bytes,
             wg_attn_scratch_bytes(M, H, hd, max_keys));
  // the form that prepares its heads: the MFMA one, every dim rotated, up
  // to 16 rows (a lane group's new key each)
  const int QG = ((H / KV) * M + 15) / 16;
  if (sh->rotated_dims != hd || M > 16 || KV * QG > MAX_KV_COUNTERS)
    return fail(WG_ERR_UNSUPPORTED,
                "wg_attn_decode_prep: %d rows, %d of %d dims rotated: not for this shape", M,
                sh->rotated_dims, hd);
  int *counters = (int *)scratch;
  float *partial = (float *)((char *)scratch + COUNTER_BYTES);
  AttnPrep pp{q_norm, k_norm, rope, k_cache, v_cache, q_out, ld_q_out,
              sh->eps, sh->use_norm, rope_rows, ctx};
  return launch_amfma<true>(qkv, M, ldqkv, H, KV, hd, k_cache, v_cache, pos0, max_keys, out, ldo,
                            partial, counters, pp, tuning("attn_xcd") != 0, as_stream(stream));
}

int wg_attn_decode_noalloc(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *sh,
                           const uint16_t *k_cache, const uint16_t *v_cache,
                           const int32_t *pos0, int32_t max_keys, uint16_t *out, int32_t ldo,
                           void *stream) {
  WG_REQUIRE(sh, "wg_attn_decode_noalloc: null argument");
  WG_REQUIRE(M >= 1 && max_keys >= 1 && sh->heads >= 1 && sh->head_dim >= 1,
             "wg_attn_decode_noalloc: %d rows, %d heads of %d, %d keys", M, sh->heads,
             sh->head_dim, max_keys);
  const size_t need = wg_attn_scratch_bytes(M, sh->heads, sh->head_dim, max_keys);
  WG_REQUIRE(need <= NOALLOC_SCRATCH_BYTES,
             "wg_attn_decode_noalloc: %d rows x %d heads of %d over %d keys need %zu bytes of "
             "scratch; the built-in scratch holds %zu",
             M, sh->heads, sh->head_dim, max_keys, need, NOALLOC_SCRATCH_BYTES);
  void *p = nullptr;
  int rc = noalloc_scratch(&p, as_stream(stream));
  if (rc) return rc;
  return wg_attn_decode(q, M, ldq, sh, k_cache, v_cache, pos0, max_keys, out, ldo, p,
                        NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
