// Gated DeltaNet, the linear-attention layers of Qwen3.5 (the reference's
// Engine.linearAttend, src/engine.ts:6646-6825, and its lin* passes,
// src/gpu/kernels.ts:1544-1862; the math in src/delta-rule.ts:38-62).
//
// Per head h, with q^ and k^ the row's q and k over their L2 norms (q^ also
// over sqrt(dk)), beta = sigmoid(b) and a = exp(A softplus(a_in + dt_bias)):
//   d = beta (v - a S^T k^),  S <- a S + k^ d^T,  o = a S^T q^ + (q^.k^) d.
//
// `delta_rule_kernel` runs the gates, the q/k prep and the recurrence of a
// batch of rows in one launch (LIN_GATES + LIN_PREP + LIN_DELTA + LIN_STATE
// per token, or LIN_DELTA_FUSED at one). The columns of a head's state are
// independent given q^, k^ and the gates, so a workgroup takes one head and
// CB state columns (16 for short batches, 64 for long ones), and the 512 / CB
// threads of a column split its dk rows: each thread keeps its rows' state
// values in registers for the whole batch, so the state is read and written
// once a launch, whatever the row count. Per row, two barriers that wait on
// LDS only: one after q, k and the gates are in LDS, one after the partial
// S^T k^ and S^T q^ are; the next row's inputs load across them.
#include "common.h"
#include "epilogue.h"

namespace wg {
namespace {

constexpr int DW = 8;        // waves a recurrence workgroup
constexpr int MAX_DK = 256;  // key dims a head (DW * 32 rows)
constexpr int MAX_CONV = 16; // convolution taps

struct DeltaArgs {
  const float *qkv;  // [M][ldq]: q (H dk) | k (H dk) | v (H dv)
  int ldq;
  const float *ba;  // [M][ldba]: b (H) | a (H)
  int ldba;
  const float *A, *dt;  // [H]
  int H, dk, dv, M;
  float *state;  // [H][dk][dv]
  float *snap;   // the state after row save_at, or null
  int save_at;
  float *out;  // [M][ldo]: H dv
  int ldo;
};

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// A workgroup barrier that waits for this wave's LDS operations only: the
// next row's global loads, issued before it, stay in flight across it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One row's inputs for this thread: q[t], k[t] (threads t < MAX_DK), v at
// this thread's column, b and a of the head (thread MAX_DK).
struct RowIn {
  float q, k, v, b, a;
};

__device__ inline RowIn load_row(const DeltaArgs &a, int m, int h, int j, bool col) {
  const float *row = a.qkv + (int64_t)m * a.ldq;
  const int t = threadIdx.x, K = a.H * a.dk;
  RowIn r{0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (t < a.dk) {
    r.q = row[h * a.dk + t];
    r.k = row[K + h * a.dk + t];
  } else if (t == MAX_DK) {
    const float *g = a.ba + (int64_t)m * a.ldba;
    r.b = g[h];
    r.a = g[a.H + h];
  }
  if (col) r.v = row[2 * K + h * a.dv + j];
  return r;
}

// CB state columns a workgroup, one a thread; the 512 / CB threads of a
// column split its dk rows, ROWS each.
template <int ROWS, int CB>
__global__ __launch_bounds__(64 * DW) void delta_rule_kernel(DeltaArgs a) {
  constexpr int RG = 64 * DW / CB;  // row groups
  static_assert(ROWS * RG <= MAX_DK, "rows a thread");
  // By row parity, so a row's writes never meet the previous row's reads.
  __shared__ float qn[2][MAX_DK], kn[2][MAX_DK];  // raw q, k (0 past dk)
  __shared__ float part[2][3][4];                 // sums of q^2, k^2, q k per wave
  __shared__ float gate[2][2];                    // beta, decay
  __shared__ float redk[2][DW][CB], redq[2][DW][CB];
  const int h = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = threadIdx.x % CB, rg = threadIdx.x / CB;
  const int j = blockIdx.x * CB + c;
  const bool col = j < a.dv;
  const int i0 = rg * ROWS;
  const float scale = 1.0f / sqrtf((float)a.dk);
  float *Sh = a.state + (int64_t)h * a.dk * a.dv;
  float s[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++)
    s[r] = col && i0 + r < a.dk ? Sh[(int64_t)(i0 + r) * a.dv + j] : 0.0f;
  RowIn in = load_row(a, 0, h, j, col);
  for (int m = 0; m < a.M; m++) {
    const int p = m & 1;
    const int t = threadIdx.x;
    if (t < MAX_DK) {  // waves 0-3: the head's q and k, their squares and products
      qn[p][t] = in.q;
      kn[p][t] = in.k;
      const float x0 = wave_sum(in.q * in.q), x1 = wave_sum(in.k * in.k);
      const float x2 = wave_sum(in.q * in.k);
      if (lane == 0) {
        part[p][0][w] = x0;
        part[p][1][w] = x1;
        part[p][2][w] = x2;
      }
    } else if (t == MAX_DK) {  // LIN_GATES for this head
      const float x = in.a + a.dt[h];
      const float softplus = fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
      gate[p][0] = 1.0f / (1.0f + expf(-in.b));
      gate[p][1] = expf(a.A[h] * softplus);
    }
    const float vj = in.v;
    if (m + 1 < a.M) in = load_row(a, m + 1, h, j, col);
    lds_barrier();
    const float sq = part[p][0][0] + part[p][0][1] + part[p][0][2] + part[p][0][3];
    const float sk = part[p][1][0] + part[p][1][1] + part[p][1][2] + part[p][1][3];
    const float sqk = part[p][2][0] + part[p][2][1] + part[p][2][2] + part[p][2][3];
    const float invq = scale / sqrtf(sq + 1e-6f), invk = 1.0f / sqrtf(sk + 1e-6f);
    float pk = 0.0f, pq = 0.0f;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      pk = fmaf(s[r], kn[p][i0 + r], pk);
      pq = fmaf(s[r], qn[p][i0 + r], pq);
    }
#pragma unroll
    for (int off = CB; off < 64; off <<= 1) {  // the wave's row groups of this column
      pk += __shfl_xor(pk, off, 64);
      pq += __shfl_xor(pq, off, 64);
    }
    if (lane < CB) {
      redk[p][w][c] = pk * invk;
      redq[p][w][c] = pq * invq;
    }
    lds_barrier();
    float kvs = 0.0f, qss = 0.0f;
#pragma unroll
    for (int u = 0; u < DW; u++) {
      kvs += redk[p][u][c];
      qss += redq[p][u][c];
    }
    const float beta = gate[p][0], decay = gate[p][1];
    const float d = beta * (vj - decay * kvs);
    if (rg == 0 && col)
      a.out[(int64_t)m * a.ldo + h * a.dv + j] = decay * qss + sqk * invq * invk * d;
#pragma unroll
    for (int r = 0; r < ROWS; r++) s[r] = fmaf(decay, s[r], kn[p][i0 + r] * invk * d);
    if (a.snap && m + 1 == a.save_at && col) {
      float *Sn = a.snap + (int64_t)h * a.dk * a.dv;
#pragma unroll
      for (int r = 0; r < ROWS; r++)
        if (i0 + r < a.dk) Sn[(int64_t)(i0 + r) * a.dv + j] = s[r];
    }
  }
  if (col) {
#pragma unroll
    for (int r = 0; r < ROWS; r++)
      if (i0 + r < a.dk) Sh[(int64_t)(i0 + r) * a.dv + j] = s[r];
  }
}

template <int CB>
void launch_delta_rule(const DeltaArgs &a, hipStream_t s) {
  constexpr int RG = 64 * DW / CB;
  const dim3 grid((a.dv + CB - 1) / CB, a.H);
  const int rows = (a.dk + RG - 1) / RG;
  if (rows <= 1 && RG <= MAX_DK)
    delta_rule_kernel<1, CB><<<grid, 64 * DW, 0, s>>>(a);
  else if (rows <= 2 && 2 * RG <= MAX_DK)
    delta_rule_kernel<(2 * RG <= MAX_DK ? 2 : 1), CB><<<grid, 64 * DW, 0, s>>>(a);
  else if (rows <= 4 && 4 * RG <= MAX_DK)
    delta_rule_kernel<(4 * RG <= MAX_DK ? 4 : 1), CB><<<grid, 64 * DW, 0, s>>>(a);
  else if (rows <= 8 && 8 * RG <= MAX_DK)
    delta_rule_kernel<(8 * RG <= MAX_DK ? 8 : 1), CB><<<grid, 64 * DW, 0, s>>>(a);
  else if (rows <= 16 && 16 * RG <= MAX_DK)
    delta_rule_kernel<(16 * RG <= MAX_DK ? 16 : 1), CB><<<grid, 64 * DW, 0, s>>>(a);
  else
    delta_rule_kernel<(32 * RG <= MAX_DK ? 32 : 1), CB><<<grid, 64 * DW, 0, s>>>(a);
}

// LIN_CONV + LIN_CONV_STATE: a thread per output (row, channel), then per
// state (row, channel).
__global__ __launch_bounds__(256) void delta_conv_kernel(const float *in, int ldi, int M, int C,
                                                         int W, const float *taps,
                                                         const float *state, float *state_out,
                                                         float *out, int ldo) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)(M + W - 1) * C) return;
  const int m = (int)(idx / C), c = (int)(idx % C);
  if (m < M) {
    float x[MAX_CONV];
    for (int k = 0; k < W; k++) {
      const int t = m - (W - 1) + k;
      x[k] = t >= 0 ? in[(int64_t)t * ldi + c] : state[(int64_t)(W - 1 + t) * C + c];
    }
    float acc = 0.0f;
    for (int k = 0; k < W; k++) acc = fmaf(taps[(int64_t)c * W + k], x[k], acc);
    out[(int64_t)m * ldo + c] = acc / (1.0f + expf(-acc));
  } else {
    const int i = m - M, t = M - (W - 1) + i;
    state_out[(int64_t)i * C + c] =
        t >= 0 ? in[(int64_t)t * ldi + c] : state[(int64_t)(M + i) * C + c];
  }
}

// LIN_NORM: a wave per (row, head), up to 4 values a lane.
__global__ __launch_bounds__(256) void delta_norm_kernel(const float *o, int ldo, int M, int H,
                                                         int dv, const float *z, int ldz,
                                                         const float *wt, float eps,
                                                         uint16_t *out16, int ldh) {
  const int lane = threadIdx.x & 63;
  const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= (int64_t)M * H) return;
  const int m = (int)(wv / H), h = (int)(wv % H);
  const float *oh = o + (int64_t)m * ldo + h * dv;
  const float *zh = z + (int64_t)m * ldz + h * dv;
  float x[4], ss = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int i = lane + 64 * u;
    x[u] = i < dv ? oh[i] : 0.0f;
    ss = fmaf(x[u], x[u], ss);
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)dv + eps);
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int i = lane + 64 * u;
    if (i < dv) {
      const float zz = zh[i];
      out16[(int64_t)m * ldh + h * dv + i] =
          half_bits(x[u] * inv * wt[i] * (zz / (1.0f + expf(-zz))));
    }
  }
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

int wg_delta_rule(const float *qkv, int32_t M, int32_t ldq, const float *ba, int32_t ldba,
                  const float *A, const float *dt_bias, const wg_delta_shape *shape,
                  float *state, float *snapshot, int32_t save_at, float *out, int32_t ldo,
                  void *stream) {
  WG_REQUIRE(qkv && ba && A && dt_bias && shape && state && out && M >= 1,
             "wg_delta_rule: bad arguments");
  const int H = shape->heads, dk = shape->key_dim, dv = shape->value_dim;
  WG_REQUIRE(H >= 1 && dk >= 1 && dk <= MAX_DK && dv >= 1,
             "wg_delta_rule: %d heads of %d key and %d value dims (key dims 1 to %d)", H, dk,
             dv, MAX_DK);
  WG_REQUIRE(ldq >= 2 * H * dk + H * dv && ldba >= 2 * H && ldo >= H * dv,
             "wg_delta_rule: row strides too short for the heads");
  WG_REQUIRE(save_at >= 0 && save_at <= M && (save_at == 0 || snapshot),
             "wg_delta_rule: save_at %d of %d rows needs a snapshot buffer", save_at, M);
  const size_t state_bytes = (size_t)H * dk * dv * sizeof(float);
  WG_REQUIRE(!snapshot || !overlaps(snapshot, state_bytes, state, state_bytes),
             "wg_delta_rule: the snapshot overlaps the state");
  DeltaArgs a{qkv, ldq, ba, ldba, A, dt_bias, H, dk, dv, M, state, snapshot, save_at, out, ldo};
  // Short batches: 16 columns a workgroup (128 workgroups at 16 heads of
  // 128), so more CUs read the state; long ones: 64 (fewer shuffles a row).
  if (M <= tuning("delta_narrow_rows"))
    launch_delta_rule<16>(a, as_stream(stream));
  else
    launch_delta_rule<64>(a, as_stream(stream));
  return launched("wg_delta_rule");
}

int wg_delta_conv(const float *in, int32_t M, int32_t ldi, int32_t C, int32_t W,
                  const float *taps, const float *state, float *state_out, float *out,
                  int32_t ldo, void *stream) {
  WG_REQUIRE(in && taps && out && M >= 1 && C >= 1 && W >= 1 && W <= MAX_CONV,
             "wg_delta_conv: bad arguments (%d taps, 1 to %d)", W, MAX_CONV);
  WG_REQUIRE(ldi >= C && ldo >= C, "wg_delta_conv: row strides shorter than %d channels", C);
  const size_t sb = (size_t)(W - 1) * C * sizeof(float);
  WG_REQUIRE(W == 1 || (state && state_out && !overlaps(state, sb, state_out, sb)),
             "wg_delta_conv: %d taps need a state and a separate state_out", W);
  const int64_t n = (int64_t)(M + W - 1) * C;
  delta_conv_kernel<<<(unsigned)((n + 255) / 256), 256, 0, as_stream(stream)>>>(
      in, ldi, M, C, W, taps, state, state_out, out, ldo);
  return launched("wg_delta_conv");
}

int wg_delta_norm(const float *o, int32_t M, int32_t ldo, const wg_delta_shape *shape,
                  const float *z, int32_t ldz, const float *weight, float eps, uint16_t *out16,
                  int32_t ldh, void *stream) {
  WG_REQUIRE(o && shape && z && weight && out16 && M >= 1, "wg_delta_norm: bad arguments");
  const int H = shape->heads, dv = shape->value_dim;
  WG_REQUIRE(H >= 1 && dv >= 1 && dv <= 256, "wg_delta_norm: %d value dims (1 to 256)", dv);
  WG_REQUIRE(ldo >= H * dv && ldz >= H * dv && ldh >= H * dv,
             "wg_delta_norm: row strides shorter than %d", H * dv);
  const int64_t waves = (int64_t)M * H;
  delta_norm_kernel<<<(unsigned)((waves + 3) / 4), 256, 0, as_stream(stream)>>>(
      o, ldo, M, H, dv, z, ldz, weight, eps, out16, ldh);
  return launched("wg_delta_norm");
}

}  // extern "C"
