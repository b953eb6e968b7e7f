// Persistent batch-1 decode: the attention layers of one token in one
// launch (the reference's Engine.forwardBatch at one row,
// src/engine.ts:8875-9303, which issues a pass per matmul, attention step and
// norm).
//
// Why one launch: at batch 1 every layer is a chain of small dependent
// steps (qkv 16 MB, attention 17 MB, o 10 MB, gate|up 73 MB, down 37 MB at
// the Llama-3-8B shape). As separate kernels each pays a launch, a ramp up
// to full bandwidth and a drain, ~4-5 us a kernel, which is as long as the
// o matrix takes to stream. Here a persistent workgroup per compute-unit
// slot runs the phases in order with a grid barrier between them. Before it
// waits at a barrier it issues the loads of its first weights of the next
// phase (weights never depend on the previous phase), so HBM keeps
// streaming while the slowest workgroup finishes and the barrier resolves.
//
// Phases of a layer (a GEMV phase is the streaming GEMV of gemv.hip with a
// runtime K split, computing exactly what wg_q4_gemv computes):
//   qkv (RoPE + KV write) | attention | o (+ residual, next norm input) |
//   gate|up (SwiGLU) | down (+ residual, next layer's norm input)
// Attention is split-K over (KV head, 64-key chunk) items; the last item of
// a KV head to finish (an arrival counter) combines the head's chunks, so
// the combine needs no barrier of its own.
//
// Barriers: a workgroup per compute unit, grouped by the XCD it runs on
// (the hardware's XCC id). Workgroups are dispatched to the 8 XCDs
// round-robin from wherever the previous launch left off, so with a grid
// that is a multiple of 8 each XCD holds grid / 8 of them; any other
// spread leaves an XCD's count short, its wait runs out and the error is
// reported, never a silent result. Every wave waits for its own stores, so they sit in
// its XCD's L2; the last workgroup of an XCD to arrive writes that L2 back
// (an agent-scope release) and arrives at the top counter; the last XCD
// flips the generation; each workgroup then acquires at agent scope. One
// L2 writeback per XCD instead of one per workgroup, and counters on their
// own cache lines, keep a barrier near the hardware's round-trip latency.
// Every wait is bounded: past the poll limit it sets an error flag that
// ends every later wait at once, so the kernel always drains; the host
// reads the flag with wg_decode_status. The grid never exceeds what the
// occupancy calculator says fits at once, so all workgroups are resident.
#include <vector>

#include "attn_core.h"
#include "common.h"
#include "dot.h"
#include "epilogue.h"
#include "gemv_core.h"
#include "kernels.h"

namespace wg {
namespace {

constexpr int MAX_KV = 64;
constexpr int MAX_CTX = 16384;
constexpr int MAX_G = 8;
constexpr int NT = 512, WAVES = NT / 64;  // threads and waves of a workgroup
constexpr int XCDS = 8;
constexpr int LINE = 64;  // 32-bit words in 256 bytes: one counter per line

struct Phase {
  wg_gemv_call c;
  int ks;  // K split: waves of a workgroup that share a row group
};

struct LayerDesc {
  Phase ph[4];  // qkv, o, gate_up, down
};

// Barrier and attention counters, each on its own line.
struct Sync {
  unsigned sub[XCDS][LINE];         // arrivals per XCD
  unsigned top[LINE];               // XCDs arrived
  unsigned gen[LINE];               // barrier generation
  int error[LINE];                  // 1: a wait ran out; 2: an XCC id past 7
  unsigned kv_count[MAX_KV][LINE];  // per KV head: attention items finished
};

struct DecodeArgs {
  const LayerDesc *layers;
  int n_layers;
  float *partial;
  int chunks;
  Sync *sync;
  int spin_limit;
};

__device__ inline unsigned ld_agent(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline unsigned add_agent(unsigned *p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void set_error(Sync *s, int code) {
  __hip_atomic_store(&s->error[0], code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The XCD this workgroup runs on (hardware register XCC_ID, bits 3:0).
__device__ inline int xcc_id() {
  return (int)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);
}

// ---------------------------------------------------------------- barrier
// Every wave's stores complete (into its XCD's L2) before the workgroup
// arrives; returns the generation to wait past (thread 0). xcd is the
// workgroup's XCD (0..7).
__device__ inline unsigned barrier_arrive(Sync *s, int xcd) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  unsigned gen = 0;
  if (threadIdx.x == 0) {
    const unsigned members = gridDim.x / XCDS;
    gen = ld_agent(&s->gen[0]);
    if (add_agent(&s->sub[xcd][0]) == members - 1) {
      st_agent(&s->sub[xcd][0], 0u);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // this XCD's L2 written back
      if (add_agent(&s->top[0]) == XCDS - 1) {
        st_agent(&s->top[0], 0u);
        __hip_atomic_fetch_add(&s->gen[0], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  return gen;
}

__device__ inline void barrier_wait(Sync *s, unsigned gen, int limit) {
  if (threadIdx.x == 0) {
    int n = 0;
    while (ld_agent(&s->gen[0]) == gen) {
      if ((n & 63) == 0 &&
          __hip_atomic_load(&s->error[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        break;
      if (++n >= limit) {
        set_error(s, 1);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

// ------------------------------------------------------------ GEMV phases
struct Geo {
  int part, slot, rgw, B, G, b0, b_end;
};

__device__ inline Geo geometry(const Phase &P) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KS = P.ks;
  Geo o;
  o.rgw = WAVES / KS;
  o.part = wave % KS;
  o.slot = wave / KS;
  o.B = P.c.w.K / 32;
  o.G = P.c.w.N / 4;
  const int BP = (o.B + KS - 1) / KS;
  o.b0 = o.part * BP + lane;
  o.b_end = min(o.B, (o.part + 1) * BP);
  return o;
}

// This wave's first unit of a phase (no dependence on any earlier phase).
template <int ZK, int NB>
__device__ inline void phase_first(const Phase &P, Unit<ZK, NB> &u) {
  const Geo o = geometry(P);
  const int g = blockIdx.x * o.rgw + o.slot;
  load_unit<ZK, NB>(u, (const uint4 *)P.c.w.quants, (const uint16_t *)P.c.w.scales,
                    P.c.w.zeros, g, o.B, o.b0, o.b_end, g < o.G);
}

// The streaming GEMV of gemv_stream_kernel for one token, starting from the
// prefetched first unit.
template <int ZK, int NB, int MODE>
__device__ void gemv_phase(const Phase &P, const Unit<ZK, NB> &first, float (*red)[WAVES][4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Geo o = geometry(P);
  const int KS = P.ks;
  const wg_epilogue &e = P.c.ep;
  const uint4 *quants = (const uint4 *)P.c.w.quants;
  const uint16_t *scales = (const uint16_t *)P.c.w.scales;
  const void *zeros = P.c.w.zeros;
  const int stride = gridDim.x * o.rgw;
  int g = blockIdx.x * o.rgw + o.slot;
  Unit<ZK, NB> next = first;
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pnext = {};
  if (o.part == 0) epi_prefetch<1, MODE>(e, g, o.G, pos0, pnext);

  uint4 a[1][NB][4];
  float sa[1][NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    int b = o.b0 + 64 * j;
    if (b < o.b_end) {
      const uint4 *xp = reinterpret_cast<const uint4 *>(P.c.x + b * 32);
      a[0][j][0] = xp[0];
      a[0][j][1] = xp[1];
      a[0][j][2] = xp[2];
      a[0][j][3] = xp[3];
    } else {
      a[0][j][0] = a[0][j][1] = a[0][j][2] = a[0][j][3] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  float scale[1];
  input_scales<1>(e, scale);
#pragma unroll
  for (int j = 0; j < NB; j++) sa[0][j] = block_sum(a[0][j]) * 0x1p-24f;

  int it = 0;
  for (int g0 = blockIdx.x * o.rgw; g0 < o.G; g0 += stride, g += stride, it ^= 1) {
    Unit<ZK, NB> u = next;
    load_unit<ZK, NB>(next, quants, scales, zeros, g + stride, o.B, o.b0, o.b_end,
                      g + stride < o.G);
    const EpiPre pe = pnext;
    if (o.part == 0) epi_prefetch<1, MODE>(e, g + stride, o.G, pos0, pnext);
    float acc[4][1] = {{0.0f}, {0.0f}, {0.0f}, {0.0f}};
    accumulate_unit<1, ZK, NB>(u, a, sa, acc);
    const int row = wave_sum4_row();
    float tot[1] = {wave_sum4(acc[0][0], acc[1][0], acc[2][0], acc[3][0])};
    if (KS > 1) {
      if ((lane & 15) == 0 && o.part > 0) red[it][wave][row] = tot[0];
      __syncthreads();
      if (o.part == 0)
        for (int p = 1; p < KS; p++) tot[0] += red[it][wave + p][row];
    }
    if (o.part == 0) finish<1, MODE>(e, g, o.G, tot, scale, P.c.y, P.c.ldy, pe, pos0);
  }
}

// ------------------------------------------------------------- attention
// Items (KV head kh, chunk c) over the workgroups; the last item of each KV
// head combines its query heads into the o matrix's input.
template <int HD>
__device__ void attention_phase(const wg_epilogue &qe, uint16_t *out, int ldo,
                                const DecodeArgs &p, unsigned char *smem, int *flag) {
  const int H = qe.heads, KV = qe.kv_heads;
  const int pos0 = *qe.pos0;
  const int n_keys = min(pos0 + 1, qe.ctx);
  if (n_keys <= 0) {  // no position in the cache: the output is zero
    if (blockIdx.x == 0)
      for (int i = threadIdx.x; i < H * HD; i += NT) out[i] = 0;
    return;
  }
  const int used = (n_keys + CHUNK - 1) / CHUNK;
  const int items = KV * used;
  for (int it = blockIdx.x; it < items; it += gridDim.x) {
    const int kh = it % KV, c = it / KV;
    attn_chunk_item<HD, NT>(qe.q_out, qe.ld_q_out, 1, H, KV, qe.k_cache, qe.v_cache, pos0,
                            n_keys, kh, c, p.partial, p.chunks, smem);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const unsigned old = add_agent(&p.sync->kv_count[kh][0]);
      const int last = old == (unsigned)(used - 1);
      if (last) {
        st_agent(&p.sync->kv_count[kh][0], 0u);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
      *flag = last;
    }
    __syncthreads();
    if (*flag)
      attn_combine_group<HD, NT>(p.partial, p.chunks, 1, H, KV, kh, pos0, qe.ctx, out, ldo,
                                 reinterpret_cast<float *>(smem));
    __syncthreads();  // smem and flag are reused by the next item
  }
}

template <int HD>
constexpr size_t decode_smem() {
  return attn_lds_bytes(MAX_G, HD) > (size_t)(2 * MAX_G * (MAX_CTX / CHUNK) + MAX_G) * 4
             ? attn_lds_bytes(MAX_G, HD)
             : (size_t)(2 * MAX_G * (MAX_CTX / CHUNK) + MAX_G) * 4;
}

template <int ZK, int HD, int NBD>
__global__ __launch_bounds__(NT, 2) void decode_kernel(const DecodeArgs p) {
  __shared__ __align__(16) unsigned char smem[decode_smem<HD>()];
  __shared__ float red[2][WAVES][4];
  __shared__ int flag;
  Unit<ZK, 1> u1;
  Unit<ZK, NBD> u2;
  const int limit = p.spin_limit;
  int xcd = xcc_id();
  if (xcd >= XCDS) {
    if (threadIdx.x == 0) set_error(p.sync, 2);
    xcd &= XCDS - 1;
  }
  phase_first<ZK, 1>(p.layers[0].ph[0], u1);
  for (int l = 0; l < p.n_layers; l++) {
    const LayerDesc &L = p.layers[l];
    gemv_phase<ZK, 1, WG_EPI_ROPE_KV>(L.ph[0], u1, red);
    unsigned gen = barrier_arrive(p.sync, xcd);
    phase_first<ZK, 1>(L.ph[1], u1);  // o's weights, held through attention
    barrier_wait(p.sync, gen, limit);
    attention_phase<HD>(L.ph[0].c.ep, const_cast<uint16_t *>(L.ph[1].c.x), L.ph[1].c.ldx, p,
                        smem, &flag);
    gen = barrier_arrive(p.sync, xcd);
    barrier_wait(p.sync, gen, limit);
    gemv_phase<ZK, 1, WG_EPI_STORE>(L.ph[1], u1, red);
    gen = barrier_arrive(p.sync, xcd);
    phase_first<ZK, 1>(L.ph[2], u1);
    barrier_wait(p.sync, gen, limit);
    gemv_phase<ZK, 1, WG_EPI_SWIGLU>(L.ph[2], u1, red);
    gen = barrier_arrive(p.sync, xcd);
    phase_first<ZK, NBD>(L.ph[3], u2);
    barrier_wait(p.sync, gen, limit);
    gemv_phase<ZK, NBD, WG_EPI_STORE>(L.ph[3], u2, red);
    if (l + 1 < p.n_layers) {
      gen = barrier_arrive(p.sync, xcd);
      phase_first<ZK, 1>(p.layers[l + 1].ph[0], u1);
      barrier_wait(p.sync, gen, limit);
    }
  }
}

typedef void (*Launcher)(const DecodeArgs &, int, hipStream_t);

template <int ZK, int HD, int NBD>
void launch_decode(const DecodeArgs &a, int grid, hipStream_t s) {
  decode_kernel<ZK, HD, NBD><<<grid, NT, 0, s>>>(a);
}

template <int ZK, int HD, int NBD>
const void *decode_fn() {
  return (const void *)decode_kernel<ZK, HD, NBD>;
}

template <int ZK, int HD>
void pick_nbd(int nbd, Launcher *l, const void **fn) {
  if (nbd == 1) {
    *l = launch_decode<ZK, HD, 1>;
    *fn = decode_fn<ZK, HD, 1>();
  } else {
    *l = launch_decode<ZK, HD, 2>;
    *fn = decode_fn<ZK, HD, 2>();
  }
}

template <int ZK>
void pick_hd(int hd, int nbd, Launcher *l, const void **fn) {
  if (hd == 64) pick_nbd<ZK, 64>(nbd, l, fn);
  else pick_nbd<ZK, 128>(nbd, l, fn);
}

// The smallest K split (1, 2 or 4 waves) that leaves a wave at most 64 *
// nb_max blocks.
int split_for(int K, int nb_max) {
  int B = K / 32;
  for (int ks = 1; ks <= 4; ks *= 2)
    if ((B + ks - 1) / ks <= 64 * nb_max) return ks;
  return 0;
}

// The checks wg_q4_gemv makes of one call, at M = 1.
int check_call(const wg_gemv_call &c, const char *what) {
  int rc = check_matrix(&c.w, "wg_decode_plan_create");
  if (rc) return rc;
  if (c.w.layout != WG_LAYOUT_ROWGROUP)
    return fail(WG_ERR_UNSUPPORTED, "wg_decode_plan_create: %s: row-group matrices only", what);
  WG_REQUIRE(c.x && c.ldx >= c.w.K && c.ldx % 8 == 0 && ((uintptr_t)c.x & 15) == 0,
             "wg_decode_plan_create: %s: activations (16-byte aligned, ldx >= K)", what);
  if ((rc = check_epilogue(&c.w, 1, c.y, c.ldy, c.ep))) return rc;
  if (c.y)
    WG_REQUIRE(!overlaps(c.x, (size_t)c.w.K * 2, c.y, (size_t)c.w.N * 4),
               "wg_decode_plan_create: %s: activations and output overlap", what);
  if (c.ep.out16)
    WG_REQUIRE(!overlaps(c.x, (size_t)c.w.K * 2, c.ep.out16,
                         (size_t)(c.ep.mode == WG_EPI_SWIGLU ? c.w.N / 2 : c.w.N) * 2),
               "wg_decode_plan_create: %s: activations and half output overlap", what);
  return WG_OK;
}

}  // namespace
}  // namespace wg

using namespace wg;

struct wg_decode_plan {
  LayerDesc *descs = nullptr;
  float *partial = nullptr;
  Sync *sync = nullptr;
  int n_layers = 0, chunks = 0, grid = 0, spin_limit = 1 << 20;
  Launcher launch = nullptr;
};

extern "C" {

int wg_decode_plan_destroy(wg_decode_plan *plan) {
  if (!plan) return WG_OK;
  if (plan->descs) (void)hipFree(plan->descs);
  if (plan->partial) (void)hipFree(plan->partial);
  if (plan->sync) (void)hipFree(plan->sync);
  delete plan;
  return WG_OK;
}

int wg_decode_plan_create(const wg_decode_layer *layers, int32_t n_layers, wg_decode_plan **out) {
  WG_REQUIRE(out && layers && n_layers >= 1, "wg_decode_plan_create: no layers");
  *out = nullptr;
  const wg_decode_layer &f = layers[0];
  const int zk = f.qkv.w.zero, hd = f.qkv.ep.head_dim;
  const int H = f.qkv.ep.heads, KV = f.qkv.ep.kv_heads;
  int nbd = 0, ctx_max = 0;
  std::vector<LayerDesc> descs((size_t)n_layers);
  for (int l = 0; l < n_layers; l++) {
    const wg_decode_layer &L = layers[l];
    const wg_gemv_call *calls[4] = {&L.qkv, &L.o, &L.gate_up, &L.down};
    const char *names[4] = {"qkv", "o", "gate_up", "down"};
    const int modes[4] = {WG_EPI_ROPE_KV, WG_EPI_STORE, WG_EPI_SWIGLU, WG_EPI_STORE};
    for (int i = 0; i < 4; i++) {
      int rc = check_call(*calls[i], names[i]);
      if (rc) return rc;
      WG_REQUIRE(calls[i]->ep.mode == modes[i],
                 "wg_decode_plan_create: layer %d: %s has epilogue mode %d, not %d", l, names[i],
                 calls[i]->ep.mode, modes[i]);
      if (calls[i]->w.zero != zk) {
        fail(WG_ERR_UNSUPPORTED, "wg_decode_plan_create: layer %d: %s: mixed zero kinds", l,
             names[i]);
        return WG_ERR_UNSUPPORTED;
      }
    }
    const wg_epilogue &qe = L.qkv.ep;
    const int D = L.qkv.w.K;
    if (qe.head_dim != hd || qe.heads != H || qe.kv_heads != KV ||
        !(hd == 64 || hd == 128) || H / KV > MAX_G || KV > MAX_KV || qe.ctx > MAX_CTX) {
      fail(WG_ERR_UNSUPPORTED,
           "wg_decode_plan_create: layer %d: %d heads over %d KV heads of %d, ctx %d "
           "(head_dim 64 or 128, at most %d heads per KV head, %d KV heads, ctx %d; all layers "
           "alike)",
           l, qe.heads, qe.kv_heads, qe.head_dim, qe.ctx, MAX_G, MAX_KV, MAX_CTX);
      return WG_ERR_UNSUPPORTED;
    }
    WG_REQUIRE(L.o.w.K == H * hd && L.o.w.N == D && L.gate_up.w.K == D && L.down.w.N == D &&
                   L.down.w.K == L.gate_up.w.N / 2,
               "wg_decode_plan_create: layer %d: matrix shapes do not chain", l);
    WG_REQUIRE(L.gate_up.ep.out16 == L.down.x,
               "wg_decode_plan_create: layer %d: gate_up's SwiGLU output must be down's input",
               l);
    WG_REQUIRE(!overlaps(qe.q_out, (size_t)H * hd * 4, L.o.x, (size_t)H * hd * 2),
               "wg_decode_plan_create: layer %d: queries and attention output overlap", l);
    ctx_max = ctx_max > qe.ctx ? ctx_max : qe.ctx;
    for (int i = 0; i < 3; i++) {
      int ks = split_for(calls[i]->w.K, 1);
      if (!ks) {
        fail(WG_ERR_UNSUPPORTED, "wg_decode_plan_create: layer %d: %s: K %d over 8192", l,
             names[i], calls[i]->w.K);
        return WG_ERR_UNSUPPORTED;
      }
      descs[l].ph[i].ks = ks;
    }
    int ks = split_for(L.down.w.K, 2);
    if (!ks) {
      fail(WG_ERR_UNSUPPORTED, "wg_decode_plan_create: layer %d: down K %d over 16384", l,
           L.down.w.K);
      return WG_ERR_UNSUPPORTED;
    }
    int nb = (L.down.w.K / 32 + ks - 1) / ks > 64 ? 2 : 1;
    if (l == 0) nbd = nb;
    if (nb != nbd) {
      fail(WG_ERR_UNSUPPORTED, "wg_decode_plan_create: layers of different down widths");
      return WG_ERR_UNSUPPORTED;
    }
    descs[l].ph[3].ks = ks;
    for (int i = 0; i < 4; i++) descs[l].ph[i].c = *calls[i];
  }

  Launcher launch = nullptr;
  const void *fn = nullptr;
  switch (zk) {
    case WG_ZERO_8: pick_hd<WG_ZERO_8>(hd, nbd, &launch, &fn); break;
    case WG_ZERO_U8: pick_hd<WG_ZERO_U8>(hd, nbd, &launch, &fn); break;
    default: pick_hd<WG_ZERO_F16>(hd, nbd, &launch, &fn); break;
  }
  int dev = 0, cus = 0, occ = 0;
  WG_HIP(hipGetDevice(&dev));
  WG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  WG_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, NT, 0));
  int per_cu = tuning("decode_wg_per_cu");
  per_cu = per_cu < occ ? per_cu : occ;
  if (per_cu < 1 || cus < 1 || (cus * per_cu) % XCDS) {
    fail(WG_ERR_UNSUPPORTED, "wg_decode_plan_create: %d compute units x %d workgroups (needs a "
                             "multiple of %d)", cus, per_cu, XCDS);
    return WG_ERR_UNSUPPORTED;
  }

  wg_decode_plan *p = new wg_decode_plan();
  p->n_layers = n_layers;
  p->chunks = (ctx_max + CHUNK - 1) / CHUNK;
  p->grid = cus * per_cu;
  p->launch = launch;
  size_t partial_bytes = (size_t)H * p->chunks * (hd + 2) * sizeof(float);
  if (hipMalloc((void **)&p->descs, sizeof(LayerDesc) * n_layers) != hipSuccess ||
      hipMalloc((void **)&p->partial, partial_bytes) != hipSuccess ||
      hipMalloc((void **)&p->sync, sizeof(Sync)) != hipSuccess) {
    (void)hipGetLastError();
    wg_decode_plan_destroy(p);
    fail(WG_ERR_OOM, "wg_decode_plan_create: out of device memory");
    return WG_ERR_OOM;
  }
  if (hipMemcpy(p->descs, descs.data(), sizeof(LayerDesc) * n_layers, hipMemcpyHostToDevice) !=
          hipSuccess ||
      hipMemset(p->sync, 0, sizeof(Sync)) != hipSuccess) {
    wg_decode_plan_destroy(p);
    fail(WG_ERR_DEVICE, "wg_decode_plan_create: %s", hipGetErrorString(hipGetLastError()));
    return WG_ERR_DEVICE;
  }
  *out = p;
  return WG_OK;
}

int wg_decode_run(wg_decode_plan *plan, void *stream) {
  WG_REQUIRE(plan, "wg_decode_run: null plan");
  DecodeArgs a{plan->descs, plan->n_layers, plan->partial, plan->chunks, plan->sync,
               plan->spin_limit};
  plan->launch(a, plan->grid, as_stream(stream));
  return launched("wg_decode_run");
}

int wg_decode_status(wg_decode_plan *plan) {
  WG_REQUIRE(plan, "wg_decode_status: null plan");
  int err = 0;
  WG_HIP(hipMemcpy(&err, &plan->sync->error[0], sizeof(int), hipMemcpyDeviceToHost));
  if (err) {
    WG_HIP(hipMemset(plan->sync, 0, sizeof(Sync)));
    if (err == 2)
      fail(WG_ERR_DEVICE, "wg_decode_run: a workgroup ran on an XCD past %d; the results of "
                          "that run are undefined",
           XCDS - 1);
    else
      fail(WG_ERR_DEVICE, "wg_decode_run: a grid barrier wait ran past %d polls; the results "
                          "of that run are undefined",
           plan->spin_limit);
    return WG_ERR_DEVICE;
  }
  return WG_OK;
}

int wg_decode_set_spin_limit(wg_decode_plan *plan, int32_t polls) {
  WG_REQUIRE(plan && polls >= 1, "wg_decode_set_spin_limit: bad arguments");
  plan->spin_limit = polls;
  return WG_OK;
}

}  // extern "C"
