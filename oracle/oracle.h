/*
 * CPU oracle for webgllm's Q4 decode/prefill hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the
 * arithmetic of the reference (webgllm, packages/webgllm/src/...) so that the
 * HIP kernels can be checked against it. Only tests/, the smoke check in
 * __graft_entry__.py and bench.py's CPU-baseline leg may load it. The product
 * (webgllm_amd/) never calls it and has no CPU fallback.
 *
 * Every function cites the reference file:line it follows. Paths are
 * relative to packages/webgllm/ of the reference.
 */
#ifndef WEBGLLM_ORACLE_H
#define WEBGLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (src/half.ts) ---- */
uint16_t orc_to_half(double v);         /* half.ts:7-32 */
float orc_from_half(uint16_t h);        /* half.ts:37-55 */

/* ---- QuantMatrix (src/weights.ts:1-31, :153-178) ----
 * quants word index ((g*blocks+b)*4+r)*4+w; scales/zeros index (g*blocks+b)*4+r.
 * zeros == NULL and zero_halves == NULL means zero point 8. raw != NULL means
 * the quants are MatMulNBits rows [N][K/32][16] kept as they are. */
typedef struct {
  int N, K;
  uint32_t *quants;
  uint16_t *scales;
  uint8_t *zeros;
  uint16_t *zero_halves;
  const uint8_t *raw;
} orc_qm;

/* Index of row n, block b's scale (weights.ts:18-22). */
static inline size_t orc_si(int N_unused, int blocks, int n, int b) {
  (void)N_unused;
  return ((size_t)(n >> 2) * blocks + b) * 4 + (n & 3);
}

int orc_pack_q4_0(orc_qm *m, int row0, const uint8_t *src, size_t src_len, int rows,
                  const int32_t *src_rows);                       /* repack.ts:60-88 */
int orc_pack_q4_k(orc_qm *m, int row0, const uint8_t *src, size_t src_len, int rows,
                  const int32_t *src_rows);                       /* repack.ts:100-168 */
int orc_pack_nbits(orc_qm *m, int row0, const uint8_t *quant, const uint8_t *scale_bytes,
                   const uint8_t *zp, int rows, const int32_t *src_rows); /* repack.ts:342-390 */
int orc_pack_nbits_scales(orc_qm *m, int row0, const uint8_t *scale_bytes, const uint8_t *zp,
                          int rows);                              /* repack.ts:312-337 */
void orc_quants_from_raw(const uint8_t *raw, int N, int K, uint32_t *out); /* repack.ts:216-245 */
void orc_matrix_row(const orc_qm *m, int n, float *out);          /* repack.ts:865-891 */
void orc_matrix_dense(const orc_qm *m, float *out, int threads);
void orc_dequantize_q4_k(const uint8_t *src, int rows, int K, float *out); /* repack.ts:474-511 */
void orc_dequantize_nbits_row(int K, const uint8_t *quant, const uint8_t *scales,
                              const uint8_t *zp, int n, float *out); /* load-onnx.ts:471-501 */
void orc_half_bytes_f32(const float *src, size_t n, uint16_t *out); /* load-onnx.ts:450-462 */

/* Synthetic quantizers used to make the workloads' weights. */
void orc_quantize_q4_0(const float *w, int rows, int K, uint8_t *out);  /* ggml quantize_row_q4_0_ref */
void orc_quantize_nbits(const float *w, int rows, int K, const uint8_t *zp_per_block,
                        uint8_t *quant, uint16_t *scales, uint8_t *zp_packed);

/* ---- 8-bit and Q6_K matrices (src/weights.ts:9-11, :23-30) ----
 * 8-bit: codes at bytes 32 si .. 32 si + 31, half scales at si =
 * (g*blocks+b)*4+r. Q6_K: 208-byte records and half d at (g*supers+s)*4+r. */
int orc_pack_q8_0(uint8_t *quants, uint16_t *scales, int N, int K, int row0, const uint8_t *src,
                  size_t src_len, int rows, const int32_t *src_rows);  /* repack.ts:174-200 */
int orc_quantize_q8(uint8_t *quants, uint16_t *scales, int N, int K, int row0,
                    const float *values, int rows);                   /* repack.ts:634-704 */
int orc_pack_q6_k(uint8_t *quants, uint16_t *scales, int N, int K, int row0, const uint8_t *src,
                  size_t src_len, int rows, const int32_t *src_rows);  /* repack.ts:706-728 */
void orc_dequantize_q8_0(const uint8_t *src, int rows, int K, float *out); /* repack.ts:514-528 */
void orc_dequantize_q4_1(const uint8_t *src, int rows, int K, float *out); /* repack.ts:447-466 */
void orc_dequantize_q5_k(const uint8_t *src, int rows, int K, float *out); /* repack.ts:535-572 */
void orc_dequantize_q6_k(const uint8_t *src, int rows, int K, float *out); /* repack.ts:405-440 */
void orc_q8_row(const uint8_t *quants, const uint16_t *scales, int K, int n, float *out);
                                                                   /* repack.ts:873-876 */
void orc_q6k_row(const uint8_t *quants, const uint16_t *scales, int K, int n, float *out);
                                                                   /* kernels.ts:3376-3390 */
void orc_matmul_q8(const uint8_t *quants, const uint16_t *scales, int N, int K,
                   const uint16_t *x16, int M, float *y, int threads, int split_fragments,
                   int max_split);                                 /* kernels.ts:219-246 */
void orc_matmul_q6k(const uint8_t *quants, const uint16_t *scales, int N, int K,
                    const uint16_t *x16, int M, float *y, int threads); /* kernels.ts:3593-3686 */

/* ---- matmul ---- */
/* y[m][n] = sum_k W[n][k] * x[m][k], W as orc_matrix_row dequantizes it, in fp64. */
void orc_gemv_f64(const orc_qm *m, const float *x, int M, double *y, int threads);
/* The split matmul's block form (kernels.ts:163-296 with split, :744-895): per block
 * acc += d * (sum q*a - z * sum a), fp32, activations as halves, slices by the
 * engine's split rule (engine.ts:5316-5327), slice partials summed as pf does
 * (kernels.ts:69-79). x16 is [M][K] half bits. */
void orc_matmul_split(const orc_qm *m, const uint16_t *x16, int M, float *y, int threads,
                      int split_fragments, int max_split);

/* ---- elementwise / norms ---- */
void orc_f32_to_h2(const float *x, size_t n, uint16_t *out);      /* packH2 kernels.ts:32-36 */
void orc_rms_norm(const float *x, const float *w, int M, int D, float eps, float *out); /* kernels.ts:1195-1242 */
void orc_swiglu(const float *gu, int M, int F, float *out);       /* kernels.ts:1066-1077 */

/* ---- attention ---- */
void orc_rope_table(double theta, int head_dim, int rotated_dims, int freq_dims, int context,
                    float *table);                                 /* engine.ts:1292-1312 */
int orc_rope_rows(int context);
void orc_head_prep(const float *x, const float *norm_w, const float *rope, int head_dim,
                   int rotated_dims, int pos, float eps, float scale, int use_norm, float *out);
                                                                   /* kernels.ts:2196-2322 */
void orc_attention_f64(const float *q, const uint16_t *kc, const uint16_t *vc, int heads,
                       int kv_heads, int head_dim, int keys, int kv_stride, double *out);
                                                                   /* attention-check.ts:48-92 */
void orc_attention_f32(const float *q, const uint16_t *kc, const uint16_t *vc, int heads,
                       int kv_heads, int head_dim, int keys, int kv_stride, float *out,
                       int threads);                      /* kernels.ts:2386-2579, float32 */

/* ---- short convolution (kernels.ts:1380-1523) ---- */
void orc_short_conv(const float *bcx, int M, int D, int W, const float *taps, const float *state,
                    float *out, float *new_state, float *prefixes);

/* ---- sampling candidates (kernels.ts:3085-3163, :3265-3323) ---- */
void orc_pick_candidates(const float *logits, int M, int V, const uint8_t *mask,
                         const int32_t *seen, int n_seen, int row0, float penalty,
                         float presence, const uint32_t *allowed, int allowed_rows,
                         int ld_allowed, int count, int32_t *chunks_out, float *cand_out);

/* ---- Gated DeltaNet (delta-rule.ts:38-166; kernels.ts:1544-1862) ---- */
void orc_delta_sequential(int dk, int dv, int T, const double *q, const double *k,
                          const double *v, const double *beta, const double *g, double *S,
                          double *o);                               /* delta-rule.ts:38-62 */
void orc_delta_chunked(int dk, int dv, int T, const double *q, const double *k,
                       const double *v, const double *beta, const double *g, double *S,
                       double *o, int chunk, int first, int save_at, double *snap);
                                                                   /* delta-rule.ts:73-166 */
void orc_delta_gates(const float *ba, int ldba, int H, const float *A, const float *dt,
                     double *beta, double *log_decay);            /* kernels.ts:1544-1562 */
void orc_delta_prep(const float *x, int dk, int is_q, double *out); /* kernels.ts:1646-1665 */
void orc_delta_rule(const float *qkv, int ldq, const float *ba, int ldba, const float *A,
                    const float *dt, int H, int dk, int dv, int M, double *state, int save_at,
                    double *snap, double *out);
void orc_delta_conv(const float *in, int ldi, int M, int C, int W, const float *w,
                    const float *state, double *out, float *state_out);
                                                                   /* kernels.ts:1564-1641 */
void orc_delta_norm(const float *o, int ldo, int M, int H, int dv, const float *z, int ldz,
                    const float *w, float eps, double *out);     /* kernels.ts:1836-1860 */

/* ---- greedy pick (kernels.ts:3169-3246) ---- */
int orc_argmax(const float *logits, int V, float *top);

/* ---- timing helpers ---- */
double orc_now(void);

#ifdef __cplusplus
}
#endif
#endif
