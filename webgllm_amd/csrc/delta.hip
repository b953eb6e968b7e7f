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
    if constexpr (CB < 64) {  // the wave's row groups of this column
      pk = group_reduce<CB>(pk, Plus());
      pq = group_reduce<CB>(pq, Plus());
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

// ---------------------------------------------------- the chunked form
//
// deltaChunked (src/delta-rule.ts:73-166; the reference's linCum, linGram,
// linSolve, linUW, linQO, linChunkOut and linChunkState passes): rows in
// chunks of CH (a first chunk of `first` rows, so that one ends at a
// snapshot), G the running sum of the log-decays within a chunk:
//   A[r][s] = beta_r e^{G_r - G_s} k^_r.k^_s (s < r), T = (I + A)^-1,
//   U = T diag(beta) V, W = T diag(beta e^G) K^, P[r][s] = e^{G_r - G_s} q^_r.k^_s,
//   Oi = P U, Q' = e^G Q^ - P W, K~_s = e^{G_last - G_s} k^_s;
// then from each chunk's starting state S: D = U - W S, O = Oi + Q' S,
// S <- e^{G_last} S + K~^T D. `delta_chunk_prep_kernel` does the first
// part for every (head, chunk) at once; `delta_chunk_chain_kernel` the
// state chain, a workgroup per (head, 16 state columns).

constexpr int CH = 64;        // rows a chunk
constexpr int CMAX = 128;     // key and value dims the chunked form takes
constexpr int RS = CMAX + 4;  // LDS row stride (floats) of the row tiles
constexpr int AS = CH + 4;    // LDS row stride of A (then T) and P
constexpr int CBW = 16;       // state columns a chain workgroup
constexpr size_t PREP_LDS = (3 * CH * RS + 2 * CH * AS + 3 * CH) * sizeof(float);
constexpr size_t CHAIN_LDS = (CMAX * CBW + 3 * CH * RS + CH * CBW) * sizeof(float);

struct ChunkArgs {
  const float *qkv;
  int ldq;
  const float *ba;
  int ldba;
  const float *A, *dt;
  int H, dk, dv, M, first, nch;
  float *U, *W, *Oi, *Qp, *Kt, *eg;  // [H][nch][CH][dv or dk]; eg [H][nch]
  float *state, *snap;
  int save_at;
  float *out;
  int ldo;
};

__device__ inline void chunk_rows(const ChunkArgs &a, int c, int &c0, int &n) {
  c0 = c == 0 ? 0 : a.first + (c - 1) * CH;
  n = min(c == 0 ? a.first : CH, a.M - c0);
}

__device__ inline float dot4(float4 x, float4 y) {
  return fmaf(x.x, y.x, fmaf(x.y, y.y, fmaf(x.z, y.z, x.w * y.w)));
}

__global__ __launch_bounds__(256) void delta_chunk_prep_kernel(ChunkArgs a) {
  extern __shared__ __align__(16) float sm[];
  float *sq = sm, *sk = sq + CH * RS, *sv = sk + CH * RS;  // q^, k^, v rows (0 past n, dims)
  float *sA = sv + CH * RS, *sP = sA + CH * AS;             // A (then T) and P
  float *sG = sP + CH * AS, *sB = sG + CH, *sE = sB + CH;  // G, beta, e^G
  const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x, lane = t & 63;
  int c0, n;
  chunk_rows(a, c, c0, n);
  const int K = a.H * a.dk, dk = a.dk, dv = a.dv;
  {  // every load issued before the first store: thread t takes column t % 128 of rows 2u + t / 128
    const int i = t & (CMAX - 1), r0 = t >> 7;
    float rq[CH / 2], rk[CH / 2], rv[CH / 2];
#pragma unroll
    for (int u = 0; u < CH / 2; u++) {
      const int r = 2 * u + r0;
      const float *row = a.qkv + (int64_t)(c0 + r) * a.ldq;
      const bool in = r < n;
      rq[u] = in && i < dk ? row[h * dk + i] : 0.0f;
      rk[u] = in && i < dk ? row[K + h * dk + i] : 0.0f;
      rv[u] = in && i < dv ? row[2 * K + h * dv + i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < CH / 2; u++) {
      const int r = 2 * u + r0;
      sq[r * RS + i] = rq[u];
      sk[r * RS + i] = rk[u];
      sv[r * RS + i] = rv[u];
    }
  }
  if (t < CH) {  // wave 0: the gates (LIN_GATES) and G by a shuffle scan (linCum)
    float beta = 0.0f, g = 0.0f;
    if (t < n) {
      const float *gb = a.ba + (int64_t)(c0 + t) * a.ldba;
      const float x = gb[a.H + h] + a.dt[h];
      beta = 1.0f / (1.0f + expf(-gb[h]));
      g = a.A[h] * (fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))));
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(g, off, 64);
      if (lane >= off) g += y;
    }
    sB[t] = beta;
    sG[t] = g;
    sE[t] = expf(g);
  }
  lds_barrier();
  {  // LIN_PREP: four threads a row
    const int r = t >> 2, part = t & 3;
    float ssq = 0.0f, ssk = 0.0f;
    for (int i = part; i < dk; i += 4) {
      ssq = fmaf(sq[r * RS + i], sq[r * RS + i], ssq);
      ssk = fmaf(sk[r * RS + i], sk[r * RS + i], ssk);
    }
    ssq = quad_sum(ssq);
    ssk = quad_sum(ssk);
    const float invq = 1.0f / sqrtf((float)dk) / sqrtf(ssq + 1e-6f);
    const float invk = 1.0f / sqrtf(ssk + 1e-6f);
    for (int i = part; i < dk; i += 4) {
      sq[r * RS + i] *= invq;
      sk[r * RS + i] *= invk;
    }
  }
  lds_barrier();
  {  // linGram: a 4 x 4 block of (row, key) pairs a thread, lower triangle only
    const int rb = t >> 4, sb = t & 15;
    float kk[4][4] = {}, qk[4][4] = {};
    if (sb <= rb) {
      for (int i = 0; i < dk; i += 4) {
        float4 kr[4], qr[4], ks[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
          kr[u] = *reinterpret_cast<const float4 *>(&sk[(4 * rb + u) * RS + i]);
          qr[u] = *reinterpret_cast<const float4 *>(&sq[(4 * rb + u) * RS + i]);
          ks[u] = *reinterpret_cast<const float4 *>(&sk[(4 * sb + u) * RS + i]);
        }
#pragma unroll
        for (int x = 0; x < 4; x++)
#pragma unroll
          for (int y = 0; y < 4; y++) {
            kk[x][y] += dot4(kr[x], ks[y]);
            qk[x][y] += dot4(qr[x], ks[y]);
          }
      }
    }
#pragma unroll
    for (int x = 0; x < 4; x++)
#pragma unroll
      for (int y = 0; y < 4; y++) {
        const int r = 4 * rb + x, s = 4 * sb + y;
        const bool ok = r < n && s <= r;
        const float e = ok ? expf(sG[r] - sG[s]) : 0.0f;
        sA[r * AS + s] = ok && s < r ? sB[r] * e * kk[x][y] : 0.0f;
        sP[r * AS + s] = ok ? e * qk[x][y] : 0.0f;
      }
  }
  const float gl = sG[n - 1];
  const int64_t base = (int64_t)(h * a.nch + c) * CH;
  for (int idx = t; idx < n * dk; idx += 256) {
    const int r = idx / dk, i = idx % dk;
    a.Kt[(base + r) * dk + i] = expf(gl - sG[r]) * sk[r * RS + i];
  }
  if (t == 0) a.eg[h * a.nch + c] = expf(gl);
  lds_barrier();
  if (t < 64) {  // linSolve: T = (I + A)^-1 by forward substitution, lane = column
    float Tc[CH];
#pragma unroll
    for (int r = 0; r < CH; r++) {
      float acc[4] = {lane == r ? 1.0f : 0.0f, 0.0f, 0.0f, 0.0f};  // 4 chains, not one
#pragma unroll
      for (int s = 0; s < r; s++) acc[s & 3] = fmaf(-sA[r * AS + s], Tc[s], acc[s & 3]);
      Tc[r] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
#pragma unroll
    for (int r = 0; r < CH; r++) sA[r * AS + lane] = Tc[r];
  }
  lds_barrier();
  // linUW, then linQO: 4 rows x 8 columns (16 apart) a thread
  const int rb = t >> 4, jb = t & 15;
  const int smax = min(4 * rb + 3, n - 1);
  float u[4][8] = {}, w[4][8] = {};
#pragma unroll 2
  for (int s = 0; s <= smax; s++) {
    const float bs = sB[s], be = bs * sE[s];
    float tr[4];
#pragma unroll
    for (int x = 0; x < 4; x++) tr[x] = sA[(4 * rb + x) * AS + s];
#pragma unroll
    for (int y = 0; y < 8; y++) {
      const float vv = sv[s * RS + jb + 16 * y] * bs, kv = sk[s * RS + jb + 16 * y] * be;
#pragma unroll
      for (int x = 0; x < 4; x++) {
        u[x][y] = fmaf(tr[x], vv, u[x][y]);
        w[x][y] = fmaf(tr[x], kv, w[x][y]);
      }
    }
  }
  lds_barrier();  // every read of v and k^ is done: U and W take their places
#pragma unroll
  for (int x = 0; x < 4; x++) {
    const int r = 4 * rb + x;
#pragma unroll
    for (int y = 0; y < 8; y++) {
      const int j = jb + 16 * y;
      sv[r * RS + j] = u[x][y];
      sk[r * RS + j] = w[x][y];
      if (r < n && j < dv) a.U[(base + r) * dv + j] = u[x][y];
      if (r < n && j < dk) a.W[(base + r) * dk + j] = w[x][y];
    }
  }
  lds_barrier();
  float o[4][8] = {}, qp[4][8];
#pragma unroll
  for (int x = 0; x < 4; x++)
#pragma unroll
    for (int y = 0; y < 8; y++) qp[x][y] = sE[4 * rb + x] * sq[(4 * rb + x) * RS + jb + 16 * y];
#pragma unroll 2
  for (int s = 0; s <= smax; s++) {
    float pr[4];
#pragma unroll
    for (int x = 0; x < 4; x++) pr[x] = sP[(4 * rb + x) * AS + s];
#pragma unroll
    for (int y = 0; y < 8; y++) {
      const float us = sv[s * RS + jb + 16 * y], ws = sk[s * RS + jb + 16 * y];
#pragma unroll
      for (int x = 0; x < 4; x++) {
        o[x][y] = fmaf(pr[x], us, o[x][y]);
        qp[x][y] = fmaf(-pr[x], ws, qp[x][y]);
      }
    }
  }
#pragma unroll
  for (int x = 0; x < 4; x++) {
    const int r = 4 * rb + x;
    if (r >= n) continue;
#pragma unroll
    for (int y = 0; y < 8; y++) {
      const int j = jb + 16 * y;
      if (j < dv) a.Oi[(base + r) * dv + j] = o[x][y];
      if (j < dk) a.Qp[(base + r) * dk + j] = qp[x][y];
    }
  }
}

constexpr int CT = 512;                   // chain threads
constexpr int CG = CT / CBW;              // their groups (32)
constexpr int DROWS = CH / CG;            // D and O rows a thread
constexpr int SROWS = CMAX / CG;          // state rows a thread
constexpr int SPT = CH * CMAX / 4 / CT;   // float4 of each staged tile a thread

__device__ __forceinline__ void chain_fetch(const ChunkArgs &a, int c, int h, int t, int g,
                                            int jj, bool col, float4 (&pw)[SPT],
                                            float4 (&pq)[SPT], float4 (&pk)[SPT],
                                            float (&pu)[DROWS], float (&po)[DROWS],
                                            float &pe) {
  int c0, n;
  chunk_rows(a, c, c0, n);
  const int64_t base = (int64_t)(h * a.nch + c) * CH;
  const int dk = a.dk, dv = a.dv;
#pragma unroll
  for (int u = 0; u < SPT; u++) {
    const int idx = t + CT * u, r = idx / (CMAX / 4), i = (idx % (CMAX / 4)) * 4;
    pw[u] = pq[u] = pk[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (r < n && i < dk) {  // (a select of the two would put the zero in memory)
      pw[u] = *reinterpret_cast<const float4 *>(&a.W[(base + r) * dk + i]);
      pq[u] = *reinterpret_cast<const float4 *>(&a.Qp[(base + r) * dk + i]);
      pk[u] = *reinterpret_cast<const float4 *>(&a.Kt[(base + r) * dk + i]);
    }
  }
#pragma unroll
  for (int x = 0; x < DROWS; x++) {
    const int r = DROWS * g + x;
    const bool in = r < n && col;
    pu[x] = in ? a.U[(base + r) * dv + jj] : 0.0f;
    po[x] = in ? a.Oi[(base + r) * dv + jj] : 0.0f;
  }
  pe = a.eg[h * a.nch + c];
}

__global__ __launch_bounds__(CT) void delta_chunk_chain_kernel(ChunkArgs a) {
  extern __shared__ __align__(16) float sm[];
  float *sS = sm;                                           // [CMAX][CBW] state block
  float *sW = sS + CMAX * CBW, *sQ = sW + CH * RS, *sK = sQ + CH * RS;  // [CH][RS]
  float *sD = sK + CH * RS;                                 // [CH][CBW]
  // blockIdx.x is the head: the workgroups of one head (consecutive in
  // blockIdx.y, H apart in launch order) land on one XCD, whose L2 then
  // serves the head's tiles to all of them.
  const int h = blockIdx.x, t = threadIdx.x, j = t & (CBW - 1), g = t / CBW;
  const int jj = blockIdx.y * CBW + j;
  const bool col = jj < a.dv;
  const int dk = a.dk, dv = a.dv;
  float *Sh = a.state + (int64_t)h * dk * dv;
  for (int i = g; i < CMAX; i += CG) sS[i * CBW + j] = col && i < dk ? Sh[(int64_t)i * dv + jj] : 0.0f;
  // A chunk's W, Q', K~ tiles and this thread's U and Oi, fetched into
  // registers one chunk ahead.
  float4 pw[SPT], pq[SPT], pk[SPT];
  float pu[DROWS], po[DROWS], pe;
  chain_fetch(a, 0, h, t, g, jj, col, pw, pq, pk, pu, po, pe);
  for (int c = 0; c < a.nch; c++) {
    int c0, n;
    chunk_rows(a, c, c0, n);
#pragma unroll
    for (int u = 0; u < SPT; u++) {
      const int idx = t + CT * u, r = idx / (CMAX / 4), i = (idx % (CMAX / 4)) * 4;
      *reinterpret_cast<float4 *>(&sW[r * RS + i]) = pw[u];
      *reinterpret_cast<float4 *>(&sQ[r * RS + i]) = pq[u];
      *reinterpret_cast<float4 *>(&sK[r * RS + i]) = pk[u];
    }
    float d[DROWS], o[DROWS];
#pragma unroll
    for (int x = 0; x < DROWS; x++) {
      d[x] = pu[x];
      o[x] = po[x];
    }
    const float e = pe;
    lds_barrier();
    if (c + 1 < a.nch)  // in flight while this chunk computes
      chain_fetch(a, c + 1, h, t, g, jj, col, pw, pq, pk, pu, po, pe);
    // linChunkOut: D = U - W S, O = Oi + Q' S, rows DROWS g ..
    for (int i = 0; i < dk; i += 8) {  // dk is a multiple of 4: the operands of two steps first
      float sv[8];
      float4 wv[2][DROWS], qv[2][DROWS];
#pragma unroll
      for (int q = 0; q < 8; q++) sv[q] = sS[(i + q) * CBW + j];  // rows dk.. (< 128) are 0
#pragma unroll
      for (int q = 0; q < 2; q++)
#pragma unroll
        for (int x = 0; x < DROWS; x++) {
          wv[q][x] = *reinterpret_cast<const float4 *>(&sW[(DROWS * g + x) * RS + i + 4 * q]);
          qv[q][x] = *reinterpret_cast<const float4 *>(&sQ[(DROWS * g + x) * RS + i + 4 * q]);
        }
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const float4 s4 = make_float4(sv[4 * q], sv[4 * q + 1], sv[4 * q + 2], sv[4 * q + 3]);
#pragma unroll
        for (int x = 0; x < DROWS; x++) {
          d[x] -= dot4(wv[q][x], s4);
          o[x] += dot4(qv[q][x], s4);
        }
      }
    }
#pragma unroll
    for (int x = 0; x < DROWS; x++) {
      const int r = DROWS * g + x;
      sD[r * CBW + j] = r < n ? d[x] : 0.0f;
      if (r < n && col) a.out[(int64_t)(c0 + r) * a.ldo + h * dv + jj] = o[x];
    }
    lds_barrier();
    // linChunkState: S <- e^{G_last} S + K~^T D, state rows g + CG u
    float acc[SROWS];
#pragma unroll
    for (int u = 0; u < SROWS; u++) acc[u] = e * sS[(g + CG * u) * CBW + j];
    for (int r = 0; r < n; r += 4) {  // rows past n hold D = 0 and K~ = 0
      float dr[4], kv[4][SROWS];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        dr[q] = sD[(r + q) * CBW + j];
#pragma unroll
        for (int u = 0; u < SROWS; u++) kv[q][u] = sK[(r + q) * RS + g + CG * u];
      }
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int u = 0; u < SROWS; u++) acc[u] = fmaf(kv[q][u], dr[q], acc[u]);
    }
#pragma unroll
    for (int u = 0; u < SROWS; u++) {
      const int i = g + CG * u;
      sS[i * CBW + j] = acc[u];
      if (a.snap && c0 + n == a.save_at && col && i < dk)
        a.snap[(int64_t)h * dk * dv + (int64_t)i * dv + jj] = acc[u];
    }
    lds_barrier();
  }
  if (col)
    for (int i = g; i < dk; i += CG) Sh[(int64_t)i * dv + jj] = sS[i * CBW + j];
}

// Chunks of a batch of M rows whose first chunk has `first` rows.
inline int chunk_count(int M, int first) { return M <= first ? 1 : 1 + (M - first + CH - 1) / CH; }

// The first chunk's rows: shorter, so that a chunk ends at save_at
// (Engine.recurrenceChunks' rule), else CH.
inline int first_rows(int save_at) { return save_at > 0 && save_at % CH ? save_at % CH : CH; }

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

size_t wg_delta_chunk_scratch_bytes(int32_t M, const wg_delta_shape *shape, int32_t save_at) {
  if (!shape || M < 1) return 0;
  const size_t nch = (size_t)chunk_count(M, first_rows(save_at));
  return sizeof(float) * ((size_t)shape->heads * nch * CH *
                              (2 * (size_t)shape->value_dim + 3 * (size_t)shape->key_dim) +
                          (size_t)shape->heads * nch);
}

int wg_delta_rule_chunked(const float *qkv, int32_t M, int32_t ldq, const float *ba,
                          int32_t ldba, const float *A, const float *dt_bias,
                          const wg_delta_shape *shape, float *state, float *snapshot,
                          int32_t save_at, float *out, int32_t ldo, void *scratch,
                          size_t scratch_bytes, void *stream) {
  WG_REQUIRE(qkv && ba && A && dt_bias && shape && state && out && scratch && M >= 1,
             "wg_delta_rule_chunked: bad arguments");
  const int H = shape->heads, dk = shape->key_dim, dv = shape->value_dim;
  WG_REQUIRE(H >= 1 && dk >= 4 && dk <= CMAX && dk % 4 == 0 && dv >= 1 && dv <= CMAX,
             "wg_delta_rule_chunked: %d key and %d value dims (key dims a multiple of 4, "
             "both at most %d)", dk, dv, CMAX);
  WG_REQUIRE(ldq >= 2 * H * dk + H * dv && ldba >= 2 * H && ldo >= H * dv,
             "wg_delta_rule_chunked: row strides too short for the heads");
  WG_REQUIRE(save_at >= 0 && save_at <= M && (save_at == 0 || snapshot),
             "wg_delta_rule_chunked: save_at %d of %d rows needs a snapshot buffer", save_at, M);
  const size_t state_bytes = (size_t)H * dk * dv * sizeof(float);
  WG_REQUIRE(!snapshot || !overlaps(snapshot, state_bytes, state, state_bytes),
             "wg_delta_rule_chunked: the snapshot overlaps the state");
  const size_t need = wg_delta_chunk_scratch_bytes(M, shape, save_at);
  WG_REQUIRE(scratch_bytes >= need, "wg_delta_rule_chunked: scratch of %zu bytes, %zu needed",
             scratch_bytes, need);
  WG_REQUIRE(((uintptr_t)scratch & 15) == 0, "wg_delta_rule_chunked: scratch not 16-byte aligned");
  int rc = raise_lds((const void *)delta_chunk_prep_kernel, (int)PREP_LDS);
  if (!rc) rc = raise_lds((const void *)delta_chunk_chain_kernel, (int)CHAIN_LDS);
  if (rc) return rc;
  const int first = first_rows(save_at), nch = chunk_count(M, first);
  const size_t rows = (size_t)H * nch * CH;
  float *f = static_cast<float *>(scratch);
  ChunkArgs a{qkv, ldq, ba, ldba, A, dt_bias, H, dk, dv, M, first, nch,
              f, f + rows * dv, f + rows * (dv + dk), f + rows * (2 * dv + dk),
              f + rows * (2 * dv + 2 * dk), f + rows * (2 * dv + 3 * dk),
              state, snapshot, save_at, out, ldo};
  hipStream_t s = as_stream(stream);
  delta_chunk_prep_kernel<<<dim3(nch, H), 256, PREP_LDS, s>>>(a);
  rc = launched("wg_delta_rule_chunked");
  if (rc) return rc;
  delta_chunk_chain_kernel<<<dim3(H, (dv + CBW - 1) / CBW), CT, CHAIN_LDS, s>>>(a);
  return launched("wg_delta_rule_chunked");
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
