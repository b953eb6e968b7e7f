/*
 * webgllm_hip: the MI355X (gfx950) backend for webgllm's Q4 decode/prefill
 * hot path, as a C ABI. Plain pointers and sizes; no torch or HIP types in
 * the signatures (streams are passed as void*, a hipStream_t or NULL for the
 * context's own stream).
 *
 * Two layers, as the reference's GPU-backend contract has them:
 *  1. The backend object (reference: class Gpu, src/gpu/gl.ts:47, and the
 *     PacedGpu contract, src/gpu/paced.ts:11-22): a context per device, device
 *     buffers standing in for textures, asynchronous readback behind fences.
 *  2. Typed kernels, one per family of the reference's GLSL generators
 *     (src/gpu/kernels.ts), the way WebGpu.nativeProgram(spec) adds native
 *     kernels beside compiled shaders (src/gpu/webgpu.ts:39-46, :413).
 *
 * Every call returns WG_OK (0) or a negative status; wg_last_error() gives
 * the message (thread-local). Statuses map to the reference's GpuError kinds
 * (src/gpu/gl.ts:110-113, :160-170, :271-275, :502-522).
 *
 * Paths cited are relative to packages/webgllm/ of the reference.
 */
#ifndef WEBGLLM_HIP_H
#define WEBGLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------- statuses */
#define WG_OK 0
#define WG_ERR_INVALID (-1)     /* bad shape, layout or argument (GpuError "limits") */
#define WG_ERR_OOM (-2)         /* device allocation failed (Gpu.outOfMemory, gl.ts:440-446) */
#define WG_ERR_DEVICE (-3)      /* HIP error: the device is unusable (context lost, gl.ts:502) */
#define WG_ERR_ALIASED (-4)     /* an op reads and writes one buffer (gl.ts:521-522) */
#define WG_ERR_DISPOSED (-5)    /* use after wg_ctx_destroy / wg_buf_delete */
#define WG_ERR_UNSUPPORTED (-6) /* no kernel for this variant (a program that won't compile) */

const char *wg_last_error(void);
const char *wg_version(void);

/* Launch-shape knobs, as the reference's TUNING table (src/engine.ts:147-625):
 * "gemv_wg_per_cu", "gemv_wg_per_cu_small" (1024 row groups or fewer),
 * "gemv_wg_per_cu_deep" (4096 to 16383), "gemv_wg_per_cu_wide" (16384+),
 * "q4k_wg_per_cu", "wide_wg_per_cu" (8-bit and Q6_K matrices: persistent
 * GEMV workgroups per compute unit) and
 * "gemv_min_waves" (below this many waves a GEMV splits K inside a
 * workgroup) and "gemm_tile" (prefill GEMM tile: 1 64 x 128, 2 128 x 128,
 * 3 128 x 256, or 0 to choose by shape) and "gemm_pingpong" (its 128 x 256
 * tiles with two wave groups half a K step apart, 1, or in lock-step, 0,
 * the default: the lock-step form runs two workgroups a compute unit).
 * Process-wide; results never depend on them. */
int wg_tuning_set(const char *name, int32_t value);
int wg_tuning_get(const char *name, int32_t *value);

/* ---------------------------------------------- 1. backend object layer */
typedef struct wg_ctx wg_ctx;
typedef struct wg_buf wg_buf;
typedef struct wg_fence wg_fence;

typedef struct {
  int32_t device;
  int32_t compute_units;
  int64_t global_bytes;
  int64_t max_alloc_bytes;
  int32_t lds_bytes_per_block;
  int32_t wave_size;
} wg_limits;

/* new Gpu(canvas) / dispose (gl.ts:316-331): a context on `device`, with
 * its own stream and a pool of pinned host staging slots for writes and
 * reads. Destroy waits for the stream, frees every buffer it still holds
 * and cancels its outstanding reads. Every handle of a deleted buffer, a
 * finished or cancelled read or a destroyed context makes later calls
 * return WG_ERR_DISPOSED (the reference's lost-context GpuError, gl.ts:502).
 * A context is used from one thread at a time, as the reference's Gpu is. */
int wg_ctx_create(int device, wg_ctx **out);
int wg_ctx_destroy(wg_ctx *ctx);
/* Gpu.limits (gl.ts:131-140). */
int wg_ctx_limits(wg_ctx *ctx, wg_limits *out);
/* The context's stream (a hipStream_t), for callers that launch typed kernels on it. */
void *wg_ctx_stream(wg_ctx *ctx);

/* Gpu.texture (gl.ts:263-305): a device buffer, optionally initialised. */
int wg_buf_create(wg_ctx *ctx, size_t bytes, const void *init, wg_buf **out);
/* Gpu.write (gl.ts:354-374): bytes into [offset, offset + bytes), queued on
 * the context's stream; `src` is copied into pinned staging before the
 * call returns (the caller may reuse it at once) and nothing waits. */
int wg_buf_write(wg_ctx *ctx, wg_buf *buf, size_t offset, const void *src, size_t bytes);
/* Gpu.zero (gl.ts:710-726). */
int wg_buf_zero(wg_ctx *ctx, wg_buf *buf);
/* Gpu.delete (gl.ts:448-461): the handle dies at once (and leaves
 * wg_bytes_live); the memory is freed once the work queued before the
 * delete has finished. */
int wg_buf_delete(wg_ctx *ctx, wg_buf *buf);
void *wg_buf_ptr(wg_buf *buf);
size_t wg_buf_size(wg_buf *buf);
/* Gpu.bytes: device bytes the context holds. */
size_t wg_bytes_live(wg_ctx *ctx);

/* Gpu.readStart (gl.ts:740-782): a copy of [offset, offset + bytes) queued
 * behind the work already issued; wg_fence_ready polls it, wg_read_finish
 * waits, copies into dst and frees the fence, wg_read_cancel frees it
 * unread (PendingRead.cancel). */
int wg_read_start(wg_ctx *ctx, wg_buf *buf, size_t offset, size_t bytes, wg_fence **out);
/* PacedGpu.fence (src/gpu/paced.ts:11-22): a fence behind the work queued
 * on the context's stream so far, with no read; wg_fence_ready polls it,
 * wg_read_finish waits for it (dst ignored) and releases it, wg_read_cancel
 * releases it without waiting (deleteFence). */
int wg_fence_record(wg_ctx *ctx, wg_fence **out);
/* The bytes a fence's read copies into wg_read_finish's dst (0 for a plain
 * fence or a released handle). */
size_t wg_fence_bytes(wg_fence *f);
int wg_fence_ready(wg_fence *f); /* 1 ready, 0 pending, < 0 error */
int wg_read_finish(wg_fence *f, void *dst);
int wg_read_cancel(wg_fence *f);
/* Gpu.readNow (gl.ts:658-700): the same, blocking. */
int wg_read_now(wg_ctx *ctx, wg_buf *buf, size_t offset, size_t bytes, void *dst);
/* Gpu.flush (gl.ts:729-732) and PacedGpu.finish. */
int wg_flush(wg_ctx *ctx);
int wg_finish(wg_ctx *ctx);
/* The context's pinned staging pool: slots and their bytes (slots are
 * reused; the pool grows only while more copies are in flight than it
 * holds, to at most 16 uploads in flight). No reference counterpart: it
 * accounts for the host memory the readbacks and writes above use. */
int wg_ctx_staging(wg_ctx *ctx, int32_t *slots, size_t *bytes);

/* ------------------------------------------------ 2. quantized matrices */

/* Device layouts of a quantized matrix.
 * WG_LAYOUT_ROWGROUP is the reference's QuantMatrix layout (src/weights.ts:1-31,
 * :153-178): rows in groups of 4, blocks of 32 along K, 16 bytes a block row
 * in Q4_0 nibble order (byte j: weight j low, weight j + 16 high); word
 * index ((g * blocks + b) * 4 + r) * 4 + w; scales (half bits) and zero
 * points at (g * blocks + b) * 4 + r. Weight = scale * (q - zero).
 * WG_LAYOUT_Q4K is GGUF Q4_K super-blocks (256 weights: fp16 d, fp16 dmin,
 * 12 bytes of 6-bit scales and mins, 128 nibble bytes) kept at 0.5625
 * bytes a weight and regrouped by rows of 4: record (g * supers + s) * 4 + r
 * of 144 bytes; the kernels rebuild packQ4_K's per-32 (d', z')
 * (src/repack.ts:100-168) in registers.
 * WG_LAYOUT_Q8 is the reference's 8-bit QuantMatrix (src/weights.ts:9-11,
 * :24-25): the same row groups and blocks of 32, a block row 32 signed
 * bytes (weight j in byte j), byte index ((g * blocks + b) * 4 + r) * 32 +
 * j, half scales at (g * blocks + b) * 4 + r; weight = scale * q.
 * WG_LAYOUT_Q6K is the reference's 6-bit QuantMatrix (src/weights.ts:23-30):
 * GGUF Q6_K super-blocks of 256 weights kept as they are, a row's
 * super-block 208 bytes (ql[128], qh[64], int8 scales[16]) at byte
 * ((g * supers + s) * 4 + r) * 208, its half d in `scales` at (g * supers
 * + s) * 4 + r; weight = d * scales[sub-block of 16] * (q - 32) as
 * dequantize_row_q6_K. `zero` is WG_ZERO_8 (unused) for both. */
#define WG_LAYOUT_ROWGROUP 0
#define WG_LAYOUT_Q4K 1
#define WG_LAYOUT_Q8 2
#define WG_LAYOUT_Q6K 3

/* Zero points of WG_LAYOUT_ROWGROUP: none (8, Q4_0), one u8 a block
 * (MatMulNBits), or one half a block (Q4_K repacked: QuantMatrix.zeroHalves).
 * WG_ZERO_Q4K keeps Q4_K's own scales instead of per-block halves, at the
 * file's 0.5625 bytes a weight: quants as above (a block whose d' below is
 * 0 holds 15s, as packQ4_K writes it), no zeros array, and in `scales` one
 * 64-byte record a row group and super-block of 256 columns, at byte (g *
 * K / 256 + s) * 64: bytes 0-15 the 4 rows' (half d, half dmin), bytes
 * 16-63 the 8 blocks' 6-bit scales and mins (get_scale_min_k4), blocks 2i
 * and 2i + 1 in the 96 bits of dwords 4 + 3i .. 6 + 3i (block 2i in bits
 * 0-47), a block's row r at bits 12r (scale) and 12r + 6 (min). Dequant
 * rebuilds packQ4_K's (d', z') bit for bit (d' = half(d sc), z' =
 * half(dmin m / d'), src/repack.ts:100-168); the GEMVs weigh a block as d'
 * q - dmin m (the zero term without z's half rounding: within 2^-11 of
 * it); the prefill GEMM takes (d', z') rebuilt into a workspace. K a
 * multiple of 256. */
#define WG_ZERO_8 0
#define WG_ZERO_U8 1
#define WG_ZERO_F16 2
#define WG_ZERO_Q4K 3

/* A quantized matrix of any layout above (the name is historical: 8- and
 * 6-bit layouts use the same descriptor). */
typedef struct {
  int32_t N;      /* output rows, a multiple of 4 */
  int32_t K;      /* inputs per row, a multiple of 32 (256 for WG_LAYOUT_Q4K, Q6K, WG_ZERO_Q4K) */
  int32_t layout; /* WG_LAYOUT_* */
  int32_t zero;   /* WG_ZERO_* (WG_LAYOUT_ROWGROUP only) */
  const void *quants; /* ROWGROUP: N*K/2 bytes; Q4K: N*K/256*144; Q8: N*K; Q6K: N*K/256*208 */
  const void *scales; /* ROWGROUP, Q8: N*K/32 halves (WG_ZERO_Q4K: N*K/256*16 bytes of
                         records); Q6K: N*K/256 halves; Q4K: unused */
  const void *zeros;  /* ROWGROUP: N*K/32 u8 or halves, or NULL for WG_ZERO_8, WG_ZERO_Q4K */
} wg_q4_matrix;

/* Bytes of device memory each array of a matrix needs. */
int wg_q4_sizes(int32_t N, int32_t K, int32_t layout, int32_t zero, size_t *quant_bytes,
                size_t *scale_bytes, size_t *zero_bytes);

/* Load-time repacking on the GPU (the reference does these on the CPU while
 * loading; src/load-gguf.ts, src/load-onnx.ts). Inputs are device copies of
 * the file's bytes; `rows` rows go to rows row0.. of `dst` (row0 and rows
 * multiples of 4); src_rows (device int32[rows]) may pick each row's source
 * row, as the packers' srcRows does, or be NULL. */
/* packQ4_0 (src/repack.ts:60-88): GGUF Q4_0 blocks (18 bytes) -> ROWGROUP, WG_ZERO_8. */
int wg_repack_q4_0(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream);
/* packQ4_K (src/repack.ts:100-168): Q4_K super-blocks -> ROWGROUP, WG_ZERO_F16,
 * bit-exact to the reference's (d', z') chain; or, into a WG_ZERO_Q4K
 * matrix, the same quants with the file's d, dmin and 6-bit scales and mins
 * regrouped into its records. */
int wg_repack_q4_k(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream);
/* packQ4_K's half scales and zero points of a WG_ZERO_Q4K matrix (N*K/32
 * halves each, at the WG_ZERO_F16 indices), bit for bit what
 * wg_repack_q4_k writes into a WG_ZERO_F16 matrix of the same rows: with
 * the same quants they make that matrix, which the prefill GEMM reads
 * without rebuilding them each call. No reference counterpart (a caller
 * keeping Q4_K records for decode and halves for prompts). */
int wg_q4k_record_halves(const wg_q4_matrix *m, uint16_t *scales, uint16_t *zeros, void *stream);
/* Q4_K super-blocks -> WG_LAYOUT_Q4K (a regrouping copy). */
int wg_repack_q4_k_native(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const void *src,
                          const int32_t *src_rows, void *stream);
/* packMatMulNBits (src/repack.ts:342-390; the raw path's quantsFromRaw
 * :216-245 + packMatMulNBitsScales :312-337): MatMulNBits quant bytes
 * [rows][K/32][16], fp16 scale bytes [rows][K/32], zero points
 * [rows][ceil(K/64)] (NULL: 8) -> ROWGROUP with WG_ZERO_U8 (or WG_ZERO_8). */
int wg_repack_nbits(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const void *quant,
                    const void *scales, const void *zp, const int32_t *src_rows, void *stream);
/* packQ8_0 (src/repack.ts:171-200): GGUF Q8_0 blocks (34 bytes: half scale,
 * 32 int8) -> WG_LAYOUT_Q8, bytes as they are. */
int wg_repack_q8_0(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream);
/* quantizeQ8 (src/repack.ts:634-704): float32 rows [rows][K] (device) ->
 * WG_LAYOUT_Q8, bit-exact: per block of 32, scale = toHalf(max |v| / 127)
 * and q = clamp(floor(v / scale + 0.5), -127, 127) with the quotient in
 * doubles (q = 0 where the scale is 0); the path the reference's GGUF
 * loader takes for every tensor it does not keep in its own format
 * (packRows, src/load-gguf.ts:509-555). */
int wg_quantize_q8(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const float *src,
                   void *stream);
/* packQ6_K (src/repack.ts:706-728): GGUF Q6_K super-blocks (210 bytes)
 * -> WG_LAYOUT_Q6K, the first 208 bytes of each as they are and its half d
 * into the scales. */
int wg_repack_q6_k(const wg_q4_matrix *dst, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream);

/* ---------------------------------------------------- GGUF files
 * readGgufHeader (src/gguf.ts:276-328) over a read-only memory map of the
 * file: metadata and tensor infos; the tensor bytes stay in the map (copy
 * them to the device and repack them there). Values and names point into
 * the reader and live until wg_gguf_close. */
typedef struct wg_gguf wg_gguf;

typedef struct {
  const char *name;    /* NUL-terminated */
  int32_t n_dims;
  int64_t dims[4];     /* ggml order: dims[0] is the contiguous one */
  int32_t type;        /* a ggml type (src/gguf.ts:27-48) */
  uint64_t offset;     /* absolute file offset of the data */
  uint64_t bytes;      /* data bytes; 0 for a type the reader does not know */
  const void *data;    /* the mapped bytes, or NULL with bytes == 0 */
} wg_gguf_tensor_info;

typedef struct {
  const char *key;     /* NUL-terminated */
  int32_t type;        /* a GGUF value type (src/gguf.ts:9-23): 8 string, 9 array */
  int32_t elem_type;   /* arrays: the elements' type */
  uint64_t length;     /* arrays: elements; strings: bytes of s */
  int64_t i;           /* integers and booleans (floats truncated) */
  double f;            /* floats (integers converted) */
  const char *s;       /* strings: `length` bytes, not NUL-terminated */
  uint64_t offset;     /* file offset of the value (arrays: first element) */
} wg_gguf_value;

int wg_gguf_open(const char *path, wg_gguf **out);
int wg_gguf_close(wg_gguf *g);
int32_t wg_gguf_version(const wg_gguf *g);
int64_t wg_gguf_data_offset(const wg_gguf *g);
int64_t wg_gguf_tensor_count(const wg_gguf *g);
int64_t wg_gguf_meta_count(const wg_gguf *g);
/* Index of a tensor or key, or -1. */
int64_t wg_gguf_find_tensor(const wg_gguf *g, const char *name);
int64_t wg_gguf_find_meta(const wg_gguf *g, const char *key);
int wg_gguf_tensor(const wg_gguf *g, int64_t i, wg_gguf_tensor_info *out);
int wg_gguf_meta(const wg_gguf *g, int64_t i, wg_gguf_value *out);
/* Element j of array key i (readGgufArray, src/gguf.ts:346-360). */
int wg_gguf_meta_element(const wg_gguf *g, int64_t i, uint64_t j, wg_gguf_value *out);

/* ---------------------------------------------------- ONNX files
 * parseOnnxModel (src/onnx.ts:71-282) over a read-only memory map of a
 * ModelProto: the graph's nodes and initializers. Inline tensor bytes
 * stay in the map; external ones are named by location, offset and
 * length (the loader reads them from that file). Names and arrays point
 * into the reader and live until wg_onnx_close. */
typedef struct wg_onnx wg_onnx;

typedef struct {
  const char *name;
  int32_t n_dims;
  int64_t dims[8];
  int32_t data_type;         /* TensorProto.DataType (src/onnx.ts:8-25) */
  const uint8_t *raw;        /* raw_data in the map, or NULL */
  uint64_t raw_bytes;
  const char *location;      /* external data file, or NULL when inline */
  int64_t offset, length;    /* in that file (length -1 when absent) */
  const int64_t *int64_data; /* the typed fields small constants use */
  int64_t n_int64;
  const float *float_data;
  int64_t n_float;
} wg_onnx_tensor_info;

typedef struct {
  const char *name, *op_type, *domain;
  int32_t n_inputs, n_outputs, n_attrs;
} wg_onnx_node_info;

typedef struct {
  const char *name;
  int32_t type;              /* AttributeProto.AttributeType: 1 float, 2 int, 3 string, 4 tensor, 6 floats, 7 ints, 8 strings */
  float f;
  int64_t i;
  const char *s;             /* `s_len` bytes, not NUL-terminated */
  uint64_t s_len;
  const int64_t *ints;
  int64_t n_ints;
  const float *floats;
  int64_t n_floats;
  int64_t n_strings;
  int64_t tensor;            /* its tensor's index (wg_onnx_tensor), or -1 */
} wg_onnx_attr;

int wg_onnx_open(const char *path, wg_onnx **out);
int wg_onnx_close(wg_onnx *f);
const char *wg_onnx_graph_name(const wg_onnx *f);
int64_t wg_onnx_node_count(const wg_onnx *f);
/* Tensors: the initializers (0 .. wg_onnx_init_count - 1), then the
 * attributes' tensors (a Constant node's value). */
int64_t wg_onnx_tensor_count(const wg_onnx *f);
int64_t wg_onnx_init_count(const wg_onnx *f);
/* Index of an initializer, or -1. */
int64_t wg_onnx_find_init(const wg_onnx *f, const char *name);
int wg_onnx_tensor(const wg_onnx *f, int64_t i, wg_onnx_tensor_info *out);
int wg_onnx_node(const wg_onnx *f, int64_t i, wg_onnx_node_info *out);
/* Input or output j of node i, or NULL. */
const char *wg_onnx_node_input(const wg_onnx *f, int64_t i, int32_t j);
const char *wg_onnx_node_output(const wg_onnx *f, int64_t i, int32_t j);
int wg_onnx_node_attr(const wg_onnx *f, int64_t i, int32_t j, wg_onnx_attr *out);

/* rowsToFloats (src/load-gguf.ts:557-580) on the GPU: `rows` rows of K
 * weights of ggml type `type` (device bytes as the file has them) to
 * float32, bit-exact to the reference's dequantizers: F32, F16, Q8_0
 * (repack.ts:514-528), Q4_1 (:447-466), Q4_K (:474-511), Q5_K (:535-572)
 * and Q6_K (:405-440); other types return WG_ERR_UNSUPPORTED. The loader
 * feeds them to wg_quantize_q8 for tensors it keeps in 8 bits. */
int wg_rows_to_floats(int32_t type, const void *src, int32_t rows, int32_t K, float *out,
                      void *stream);

/* matrixRow (src/repack.ts:865-891) on the GPU: rows [row0, row0 + rows)
 * dequantized to float32, bit-exact: fp32(d * (q - z)) with the difference
 * and product in doubles, as the reference computes them; 8-bit: fp32(d *
 * q); 6-bit: fp32(d * sc * (q - 32)) as dequantizeQ6_K (src/repack.ts:405-440)
 * on the same bytes. */
int wg_q4_dequant(const wg_q4_matrix *m, int32_t row0, int32_t rows, float *out, void *stream);

/* ------------------------------------------------------------ matmul */

/* What a GEMV does with its sums (the reference folds the same steps into
 * its matmul and add passes: the "prescaled" normed matmul, addScaled,
 * rmsOfAdd and REDUCE_SWIGLU, src/gpu/kernels.ts:744-895, :1169-1361,
 * :1066-1077; headPrep + values, :2196-2322, :3030-3045).
 *
 * Input side: with norm_parts, row m of the result is multiplied by
 * norm_mult / sqrt(sum of norm_parts[m][0 .. n_parts) / norm_count + eps):
 * the activations were stored as half(x * w / norm_mult) by the producer,
 * and the parts are the sums of squares of x it wrote (one a row group).
 * row_scale[m], if given, multiplies as well.
 *
 * Output side, by mode:
 *  WG_EPI_STORE: y[m][n] = (residual ? residual[m][n] : 0) + s_m * acc; with
 *    out16, out16[m][n] = half(y[m][n] * out16_w[n] / norm_mult_out) (the
 *    next norm's input, prescaled); with parts_out, parts_out[m][g] = the sum
 *    of squares of y[m][4g .. 4g + 3]. residual may equal y (in-place add).
 *  WG_EPI_SWIGLU: rows come in groups of 4 as (gate 2i, gate 2i + 1, up 2i,
 *    up 2i + 1); out16[m][2i + j] = half(silu(gate) * up); y is not written.
 *  WG_EPI_ROPE_KV: the matrix is a q|k|v projection whose q and k rows come
 *    in groups of 4 as (j, j + hd/2, j + 1, j + 1 + hd/2) of a head (all dims
 *    rotated); q goes to q_out (rotated, times 1/sqrt(hd)), k (rotated) and
 *    v to the caches as halves at row *pos0 + m (see wg_head_prep).
 *  WG_EPI_SHORT_CONV: the matrix is a short-conv in_proj of N = 3 D rows,
 *    B | C | x (D a multiple of 16); the GEMV's float32 outputs go straight
 *    into wg_short_conv's computation (same results, bit for bit, as
 *    wg_q4_gemv with WG_EPI_STORE then wg_short_conv over those rows):
 *    out16[m][c] = half(C_m[c] * sum_k conv_taps[c][k] y[m - (W-1) + k])
 *    with y_t = B_t[c] x_t[c] (earlier tokens' y from conv_state, W - 1
 *    rows of D, oldest first), the state after the M tokens to
 *    conv_state_out (may equal conv_state), and with conv_prefixes the
 *    state after each prefix ([M][W - 1][D]). W = conv_width, 2 to 4; y
 *    is not written. Taken by the streaming and the MFMA GEMVs on 4-bit
 *    row-group matrices (one to eight tokens); elsewhere the
 *    call returns WG_ERR_UNSUPPORTED and the caller makes the two calls
 *    (LFM2's convolve: src/engine.ts:5806-5899, src/gpu/kernels.ts:1447-1523). */
/* With pick_parts (WG_EPI_STORE, no residual; the head GEMV), the GEMV also
 * runs CHUNK_MAX_AT's reduction (src/gpu/kernels.ts:3169-3205) over the
 * values it stores: each workgroup's (largest value, lowest row holding it)
 * of every row m (strict > from -3e38, so NaN never enters), into
 * pick_parts (wg_pick_parts_bytes(M), 16-byte aligned); wg_argmax_parts then
 * finishes the pick from them, reading no logit again. The 4-bit row-group
 * GEMVs (MFMA and streaming) take it; elsewhere the call returns
 * WG_ERR_UNSUPPORTED having launched nothing (then wg_q4_gemv without it
 * and wg_argmax_rows over y). */
#define WG_EPI_STORE 0
#define WG_EPI_SWIGLU 1
#define WG_EPI_ROPE_KV 2
#define WG_EPI_SHORT_CONV 3

typedef struct {
  int32_t mode;
  /* input normalisation */
  const float *norm_parts;
  int32_t n_parts, ld_parts_in;
  int32_t norm_count;
  float eps, norm_mult;
  const float *row_scale;
  /* WG_EPI_STORE */
  const float *residual;
  int32_t ld_residual;
  uint16_t *out16;
  int32_t ld_out16;
  const float *out16_w;
  float norm_mult_out;
  float *parts_out;
  int32_t ld_parts_out;
  /* WG_EPI_ROPE_KV */
  int32_t heads, kv_heads, head_dim, ctx, rope_rows;
  const float *rope;
  const int32_t *pos0;
  float *q_out;
  int32_t ld_q_out;
  uint16_t *k_cache, *v_cache;
  /* WG_EPI_SHORT_CONV */
  const float *conv_taps;
  const float *conv_state;
  float *conv_state_out;
  float *conv_prefixes;
  int32_t conv_width;
  /* WG_EPI_STORE without residual: the greedy pick's first stage */
  void *pick_parts;
} wg_epilogue;

/* Decode / few-token GEMV (matmulSplitRgba4 and the split matmul,
 * src/gpu/kernels.ts:744-895, :163-296, dispatched by Engine.splitPartials,
 * engine.ts:5241-5377): y[m][n] = sum_k W[n][k] x[m][k] for M <= 8 rows of
 * half activations x ([M][ldx], natural order), fp32 out. One or two
 * tokens stream on the vector units (128-bit loads of nibbles, dequant in
 * registers, wavefront reductions); 3 to 8 tokens of a 4-bit row-group
 * matrix run on MFMA (16x16x32 f16, nibbles unpacked to exact halves,
 * f32 sums). Every layout: 8-bit matrices as the 8-bit split matmul sums
 * them (per block acc += d * sum q a, kernels.ts:219-246), Q6_K as the Q6_K
 * head does (per super-block acc += d * sum_sub sc * sum (q - 32) a,
 * kernels.ts:3593-3686), with every epilogue. */
int wg_q4_gemv(const wg_q4_matrix *w, const uint16_t *x, int32_t M, int32_t ldx, float *y,
               int32_t ldy, const wg_epilogue *ep, void *stream);

/* Prefill GEMM (Engine.matmul -> matmulQuad, or dequant + matmulF16,
 * kernels.ts:370-429, :436-735; Engine.f16Plan, engine.ts:980-995):
 * C[m][n] = (residual ? residual[m][n] : 0) + sum_k A[m][k] W[n][k] for M
 * tokens of half activations A ([M][lda], 16-byte aligned) and a 4-bit
 * row-group or an 8-bit matrix (N and K multiples of 64); float32 C
 * [M][ldc]. Weights are dequantized in registers to halves, d (q - z) (or d
 * q) rounded once as dequantOut does (kernels.ts:436-597), and multiplied
 * on MFMA (v_mfma_f32_32x32x16_f16)
 * with float32 accumulation. residual may equal C. row_scale (or NULL)
 * multiplies row m's sums before the residual is added (a prescaled norm's
 * 32 / RMS, see wg_norm_to_h2). col_of (or NULL for n -> n) maps the
 * matrix's stored row n to its output column: a matrix uploaded with a row
 * order (the loaders' srcRows, stored row n = logical row col_of[n]) then
 * comes out in logical order; entries outside 0..N-1 are not written.
 * Where tiles are fewer than the compute units, K is split 2 or 4 ways and
 * the partial sums are added in a fixed pairwise order (bits independent of
 * which split ends last), in a workspace the library keeps per stream and
 * grows on demand; launches on one stream run in turn. A launch made while
 * its stream is being captured into a graph runs unsplit (the graph holds
 * no workspace, so it may replay on any stream and beside eager GEMMs), and
 * so its sums may differ in the last bits from an eager launch's.
 * A WG_ZERO_Q4K matrix's (d', z') halves are rebuilt first, bit for bit as
 * packQ4_K makes them, into a second workspace of the same kind (one more
 * launch; N*K/8 bytes), so its results are a WG_ZERO_F16 matrix's; such a
 * call made while the stream is being captured returns WG_ERR_UNSUPPORTED
 * before any launch. */
int wg_q4_gemm(const wg_q4_matrix *w, const uint16_t *A, int32_t M, int32_t lda, float *C,
               int32_t ldc, const float *residual, int32_t ldr, const float *row_scale,
               const int32_t *col_of, void *stream);

/* The gate|up GEMM with the SwiGLU folded into it, for prompt batches (the
 * fused FFN passes of the reference's WebGPU kernels, src/gpu/native.ts:33,
 * and REDUCE_SWIGLU, kernels.ts:1066-1077): the matrix's rows come in
 * groups of 4 as (gate 2i, gate 2i + 1, up 2i, up 2i + 1), as for
 * WG_EPI_SWIGLU; out16[m][i] = half(silu(g) * u) of the float32 sums
 * (times row_scale[m] when given), N / 2 columns, no float32 product
 * written. Equals wg_q4_gemm (with the matrix's column map) followed by
 * wg_swiglu, bit for bit. */
int wg_q4_gemm_swiglu(const wg_q4_matrix *w, const uint16_t *A, int32_t M, int32_t lda,
                      uint16_t *out16, int32_t ldo, const float *row_scale, void *stream);

/* float32 -> half activations, clamped to +-65504 (packH2, kernels.ts:32-36). */
int wg_f32_to_f16(const float *x, uint16_t *out, int64_t n, void *stream);

/* ---------------------------------------------- residual-stream glue */

/* RMS norm into half activations (RMS_SCALE + NORM_TO_H2,
 * src/gpu/kernels.ts:1195-1242): out[m][i] = half(x[m][i] * w[i] / sqrt(mean_i
 * x[m][i]^2 + eps)), clamped to +-65504; rs_out[m] = the 1 / RMS (or NULL). */
int wg_rms_norm(const float *x, int32_t M, int32_t D, int32_t ldx, const float *w, float eps,
                uint16_t *out, int32_t ldo, float *rs_out, void *stream);
/* The prescaled form the reference's matmuls read (NORM_TO_H2 with PRESCALE
 * 32, src/gpu/kernels.ts:89, :1195-1242): out[m][i] = half(x[m][i] * w[i] /
 * 32), clamped to +-65504, and row_scale[m] = 32 / sqrt(mean_i x[m][i]^2 +
 * eps), the factor a product over out takes afterwards (the GEMV's and
 * GEMM's row scale). */
int wg_norm_to_h2(const float *x, int32_t M, int32_t D, int32_t ldx, const float *w, float eps,
                  uint16_t *out, int32_t ldo, float *row_scale, void *stream);

/* SwiGLU (REDUCE_SWIGLU / SWIGLU_F16, kernels.ts:1066-1077, :1256-1264):
 * out[m][i] = half(silu(gu[m][i]) * gu[m][F + i]) (gate rows, then up rows). */
int wg_swiglu(const float *gu, int32_t M, int32_t F, int32_t ldg, uint16_t *out, int32_t ldo,
              void *stream);

/* Embedding rows (embed / embedFold, kernels.ts:1092-1149, :985-1041): h[m] =
 * row ids[m] of the quantized embedding, dequantized as matrixRow does
 * (src/repack.ts:865-891; a Q6_K embedding as dequantizeQ6_K, src/repack.ts:405-440);
 * an id outside [0, N) embeds as zeros. With ep
 * (its STORE outputs out16 and parts_out), also layer 0's prescaled half
 * input and the sums of squares of each 4 values, as embedFold draws them. */
int wg_embed(const wg_q4_matrix *emb, const int32_t *ids, int32_t M, float *h, int32_t ldh,
             const wg_epilogue *ep, void *stream);
/* wg_verify_drafts and wg_embed in one launch: row 0 embeds ids[0], row
 * m >= 1 entry m - 1 of table row *cursor (the last row once the cursor is
 * past n_steps), which it also writes to ids[m] for the accept. */
int wg_embed_drafts(const wg_q4_matrix *emb, int32_t *ids, int32_t rows, const int32_t *table,
                    int32_t n_steps, const int32_t *cursor, float *h, int32_t ldh,
                    const wg_epilogue *ep, void *stream);

/* -------------------------------------------------------- attention */

typedef struct {
  int32_t heads;        /* query heads */
  int32_t kv_heads;     /* KV heads (heads % kv_heads == 0: GQA) */
  int32_t head_dim;
  int32_t rotated_dims; /* dims RoPE rotates (the loaders put them first) */
  float eps;            /* QK RMS norm epsilon */
  int32_t use_norm;     /* 1: RMS-normalise q and k per head (headPrep norm: true) */
} wg_attn_shape;

/* headPrep + values (kernels.ts:2196-2322, :3030-3045): qkv rows hold heads
 * * head_dim queries, then kv_heads * head_dim keys, then values. Queries go
 * to q_out (float32, times 1/sqrt(head_dim)); keys and values to the caches
 * ([ctx][kv_heads * head_dim] halves) at row *pos0 + m. `rope` is the table
 * Engine.ropeTable builds (src/engine.ts:1292-1312): rope_rows rows of
 * head_dim/2 cosines then head_dim/2 sines, rows 0..1023 positions 0..1023,
 * row 1024 + i position 1024 i. *pos0 is read on the device (a graph
 * replays at any position); rows outside [0, ctx) store nothing. */
int wg_head_prep(const float *qkv, int32_t M, int32_t ldq, const wg_attn_shape *shape,
                 const float *q_norm, const float *k_norm, const float *rope, int32_t rope_rows,
                 const int32_t *pos0, float *q_out, int32_t ldqo, uint16_t *k_cache,
                 uint16_t *v_cache, int32_t ctx, void *stream);

/* Prefill attention for a prompt batch: the reference's chunked scores /
 * attend plan for many query rows (Engine.attention, engine.ts:6359-6630).
 * q [M][ldq] f32 (as wg_head_prep writes it), rows at positions *pos0 + m,
 * each row m seeing keys 0 .. *pos0 + m of the caches (rows < max_keys);
 * out [M][ldo] halves. Scores and softmax in f32 with an online softmax
 * over 64-key chunks; no scratch. head_dim 64 or 128, at most 32 query
 * heads per KV head, q 16-byte aligned with ldq % 4 == 0. */
int wg_attn_prefill(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *shape,
                    const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0,
                    int32_t max_keys, uint16_t *out, int32_t ldo, void *stream);
/* Decode / verify attention (scores, attend, attendPanel + attendPanelCombine,
 * kernels.ts:2386-2579, :2803-3027): row m's query at position *pos0 + m
 * attends keys 0..*pos0 + m (causal) of its KV head; half output. max_keys
 * is how many rows the caches hold (the position is clamped to it).
 * scratch holds wg_attn_scratch_bytes(M, heads, head_dim, max_keys) bytes:
 * counters (wg_attn_scratch_bytes(0, heads, head_dim, 0) bytes), then
 * per-chunk partial results. The counters must be zero before the first
 * call (a zeroed allocation); every call leaves them zero. Calls that share
 * a scratch must not overlap.
 * With heads / kv_heads * M <= 8 and kv_heads a multiple of 8 it is one
 * launch (max_keys up to 2^20): a workgroup per (KV head, split of 64, 128
 * or 256 keys), a wave per query; each of the 8 XCDs takes the KV heads
 * congruent to its id mod 8, and its last workgroup to finish combines
 * them from the XCD's L2. Other shapes of up to 8 queries a KV head: one
 * launch whose last workgroup of a KV head combines its splits (up to 1024
 * keys and past 16384), else two launches (an LDS-staged workgroup per
 * 64-key chunk, then the online-softmax combine). More queries a KV head:
 * one launch on MFMA. */
size_t wg_attn_scratch_bytes(int32_t M, int32_t heads, int32_t head_dim, int32_t max_keys);
int wg_attn_decode(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *shape,
                   const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0,
                   int32_t max_keys, uint16_t *out, int32_t ldo, void *scratch,
                   size_t scratch_bytes, void *stream);
/* wg_head_prep then wg_attn_decode in one launch, the heads prepared in the
 * attention kernel (headPrep + attention, kernels.ts:2196-2322, :2803-3027):
 * qkv [M][ldqkv] f32 rows q | k | v as wg_head_prep takes them; each
 * workgroup makes its queries (norm, rotation at *pos0 + m, 1/sqrt(hd)),
 * and the batch's new keys and values (rows *pos0 + m, k normed and
 * rotated) go into the K and V tiles of the workgroups that read them and,
 * from one workgroup a KV head, into the caches (ctx rows; rows outside
 * [0, ctx) or the rope table store nothing, their queries are zero, as
 * wg_head_prep does). q_out (or NULL) receives the queries as wg_head_prep
 * writes them. The same bits as wg_head_prep then wg_attn_decode on the
 * MFMA form (attn_mfma 2). Every dim rotated, up to 16 rows: other shapes
 * return WG_ERR_UNSUPPORTED before any launch (then the two calls).
 * qkv, rope and the caches 16-byte aligned; max_keys <= ctx. */
int wg_attn_decode_prep(const float *qkv, int32_t M, int32_t ldqkv, const wg_attn_shape *shape,
                        const float *q_norm, const float *k_norm, const float *rope,
                        int32_t rope_rows, int32_t ctx, uint16_t *k_cache, uint16_t *v_cache,
                        const int32_t *pos0, int32_t max_keys, float *q_out, int32_t ld_q_out,
                        uint16_t *out, int32_t ldo, void *scratch, size_t scratch_bytes,
                        void *stream);
/* wg_attn_decode with no scratch argument and no allocation of any kind:
 * no counterpart in the reference. It is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The partial results go to a 16 MiB
 * array built into the library, one per GPU, held until the process ends;
 * a request needing more (wg_attn_scratch_bytes(M, heads, head_dim,
 * max_keys) > 16 MiB, e.g. 8 rows of 32 heads of 128 past 7,936 keys) is
 * rejected with WG_ERR_INVALID before anything runs. Every call on a GPU
 * shares that array: calls that overlap on one GPU (other streams, other
 * threads) race. Same results as wg_attn_decode, bit for bit. */
int wg_attn_decode_noalloc(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *shape,
                           const uint16_t *k_cache, const uint16_t *v_cache,
                           const int32_t *pos0, int32_t max_keys, uint16_t *out, int32_t ldo,
                           void *stream);

/* ------------------------------------------------ short convolution */

/* convFused + convPrefixes (kernels.ts:1447-1523; Engine.convolve,
 * engine.ts:5806-5899): bcx rows B | C | x (3 D floats, src/weights.ts:180-190),
 * taps [D][W] (tap W-1 is the current token), state [W-1][D] (oldest
 * first). out[t] = half(C_t * sum_k taps[c][k] * y[t-(W-1)+k]) with y = B * x;
 * state_out = the last W-1 y rows (may be state itself); prefixes
 * [M][W-1][D], or NULL, = the state after each prefix of the batch. */
int wg_short_conv(const float *bcx, int32_t M, int32_t D, int32_t ldb, int32_t W,
                  const float *taps, const float *state, float *state_out, float *prefixes,
                  uint16_t *out, int32_t ldo, void *stream);
/* Engine.accept's rollback (engine.ts:8063-8086, COPY_ROWS kernels.ts:2177-2183):
 * state <- the state after the first `kept` of `rows` tokens. */
int wg_conv_accept(const float *prefixes, int32_t kept, int32_t rows, int32_t D, int32_t W,
                   float *state, void *stream);

/* ---------------------------------------------- speculative verify on the device
 * The reference's verify loop (src/handler.ts:1811-1887) reads each batch's
 * picks back and decides on the host; these two calls take the decision on
 * the device, so that a verify step (drafts in, forward of the batch,
 * greedy picks, accept, rollback) replays as one captured graph. */

/* A conv layer's rollback operands: prefixes [rows][width - 1][dim] (the
 * state after each prefix of the batch, wg_short_conv) and its state
 * [width - 1][dim]. */
typedef struct {
  float *prefixes;
  float *state;
  int32_t dim;
  int32_t width;
} wg_conv_state;

/* Engine.accept after a verify batch (engine.ts:8063-8086) with the
 * handler's rule for what to keep (handler.ts:1811-1887): the batch's
 * inputs are ids[0 .. rows) (ids[1 ..] the drafts) and picks[0 .. rows)
 * its greedy picks; kept = 1 + the longest prefix i with picks[i] ==
 * ids[i + 1]. Then every conv layer's state := its prefix kept - 1 (convs:
 * a device array of n_conv wg_conv_state, each (width - 1) * dim <=
 * max_state floats), hist[*pos + 1 + i] = picks[i] for i < kept (within
 * hist_len), kept_log[*cursor] = kept (within log_len), *cursor += 1,
 * *pos += kept, ids[0] = picks[kept - 1]. One launch. */
int wg_verify_accept(const int32_t *picks, int32_t rows, const wg_conv_state *convs,
                     int32_t n_conv, int32_t max_state, int32_t *pos, int32_t *ids,
                     int32_t *hist, int32_t hist_len, int32_t *kept_log, int32_t log_len,
                     int32_t *cursor, void *stream);
/* The drafts of a verify step from a device table (the reference's draft
 * lookup, src/draft.ts:15-45, runs on the host; a table lets a whole run
 * of steps replay without it): ids[1 .. rows) := table row *cursor of
 * rows - 1 ids (the last row once the cursor is past n_steps). */
int wg_verify_drafts(int32_t *ids, int32_t rows, const int32_t *table, int32_t n_steps,
                     const int32_t *cursor, void *stream);
/* wg_argmax_parts and wg_verify_accept in one launch: the batch's picks
 * finished from a head GEMV's pick_parts (the same ids wg_argmax_parts
 * gives), written to picks_out, then the accept as wg_verify_accept. */
int wg_verify_accept_parts(const void *pick_parts, int32_t *picks_out, int32_t rows,
                           const wg_conv_state *convs, int32_t n_conv, int32_t max_state,
                           int32_t *pos, int32_t *ids, int32_t *hist, int32_t hist_len,
                           int32_t *kept_log, int32_t log_len, int32_t *cursor, void *stream);

/* ------------------------------------------------- Gated DeltaNet */

/* A Gated DeltaNet layer's shape (Qwen3.5's linear attention,
 * src/load-gguf.ts:715-726): as many key as value heads (the reference
 * refuses others), key_dim at most 256. */
typedef struct {
  int32_t heads, key_dim, value_dim;
} wg_delta_shape;

/* Engine.linearAttend's recurrence for M rows (engine.ts:6697-6815): per row
 * LIN_GATES, LIN_PREP, LIN_DELTA, LIN_STATE (kernels.ts:1544-1862; one row:
 * LIN_DELTA_FUSED), in one launch. qkv rows: the convolution's output q
 * (heads * key_dim) | k | v (heads * value_dim); ba rows: b (heads) | a
 * (heads); A = -exp(A_log) and dt_bias per head. Per head, beta =
 * sigmoid(b), decay = exp(A softplus(a + dt_bias)), q^ = q / sqrt(|q|^2 +
 * 1e-6) / sqrt(key_dim), k^ = k / sqrt(|k|^2 + 1e-6); d = beta (v - decay
 * S^T k^), S <- decay S + k^ d^T, out = S^T q^. state [heads][key_dim]
 * [value_dim] float32, updated in place; with save_at in 1..M, snapshot (its
 * size, not overlapping) receives the state after row save_at (the
 * reference's saveAt). */
int wg_delta_rule(const float *qkv, int32_t M, int32_t ldq, const float *ba, int32_t ldba,
                  const float *A, const float *dt_bias, const wg_delta_shape *shape,
                  float *state, float *snapshot, int32_t save_at, float *out, int32_t ldo,
                  void *stream);
/* The same recurrence in chunks of 64 rows, as Engine.recurrenceChunks
 * runs prompt batches (engine.ts:6950-7050; delta-rule.ts:73-166): per
 * chunk the gates, q/k prep, A = beta e^(G_r - G_s) k.k, T = (I + A)^-1,
 * U, W, P, Oi, Q' for all chunks at once, then the state chain, two steps
 * a chunk. The first chunk is shorter when save_at is not a multiple of
 * 64, so that a chunk ends there. key_dim a multiple of 4, key_dim and
 * value_dim at most 128; scratch (16-byte aligned) of
 * wg_delta_chunk_scratch_bytes(M, shape, save_at) bytes. Otherwise as
 * wg_delta_rule. */
size_t wg_delta_chunk_scratch_bytes(int32_t M, const wg_delta_shape *shape, int32_t save_at);
int wg_delta_rule_chunked(const float *qkv, int32_t M, int32_t ldq, const float *ba,
                          int32_t ldba, const float *A, const float *dt_bias,
                          const wg_delta_shape *shape, float *state, float *snapshot,
                          int32_t save_at, float *out, int32_t ldo, void *scratch,
                          size_t scratch_bytes, void *stream);
/* LIN_CONV + LIN_CONV_STATE (kernels.ts:1564-1641): out[m][c] = silu(sum_k
 * taps[c][k] * x[m - (W-1) + k][c]) over the first C channels of each in
 * row (W at most 16; tap W-1 the current row), earlier rows from state
 * [W-1][C] (oldest first); state_out (apart from state) = the last W-1 raw
 * rows. */
int wg_delta_conv(const float *in, int32_t M, int32_t ldi, int32_t C, int32_t W,
                  const float *taps, const float *state, float *state_out, float *out,
                  int32_t ldo, void *stream);
/* LIN_NORM (kernels.ts:1836-1860): out16[m][h dv + i] = half(o * w[i] *
 * silu(z) / sqrt(mean of the head's o^2 + eps)), out_proj's input (value_dim
 * at most 256). */
int wg_delta_norm(const float *o, int32_t M, int32_t ldo, const wg_delta_shape *shape,
                  const float *z, int32_t ldz, const float *weight, float eps, uint16_t *out16,
                  int32_t ldh, void *stream);

/* ------------------------------------------------------ greedy pick */

/* CHUNK_MAX_AT + CHUNK_ARGMAX_ROWS (kernels.ts:3169-3246): ids[m] = the lowest
 * id holding row m's largest logit (strict > from -3e38 at id 0: NaN never
 * wins); tops[m] its logit (or NULL). */
size_t wg_argmax_scratch_bytes(int32_t M, int32_t V);
int wg_argmax_rows(const float *logits, int32_t M, int32_t V, int32_t ld, int32_t *ids,
                   float *tops, void *scratch, size_t scratch_bytes, void *stream);
/* One greedy decode step's pick and advance, on the device: the pick of one
 * row of V logits (as wg_argmax_rows, same scratch size for M = 1), then
 * ids[0] = the pick, hist[*pos + 1] = the pick when 0 <= *pos + 1 < hist_len
 * (hist may be NULL with hist_len 0), *pos += 1. A captured decode step
 * thereby replays at successive positions, its input the previous pick, as
 * the reference's guessed forward reads CHUNK_ARGMAX's pick from the ids
 * texture without the host (Engine.forwardGuess, engine.ts:8095-8110,
 * Engine.argmax guess, :8318-8336). */
int wg_argmax_advance(const float *logits, int32_t V, int32_t *ids, int32_t *pos, int32_t *hist,
                      int32_t hist_len, float *tops, void *scratch, size_t scratch_bytes,
                      void *stream);

/* The pick finished from a head GEMV's pick_parts (see wg_epilogue): ids[m]
 * and tops[m] (or NULL) as wg_argmax_rows gives them over the GEMV's y,
 * bit for bit. With pos (M = 1), the advance of wg_argmax_advance as well.
 * One launch; for one decode step the GEMV's own reduction replaces
 * wg_argmax_advance's first. */
#define WG_PICK_SLOTS 4096 /* workgroups a GEMV may write parts for */
size_t wg_pick_parts_bytes(int32_t M);
int wg_argmax_parts(const void *pick_parts, int32_t M, int32_t *ids, float *tops, int32_t *pos,
                    int32_t *hist, int32_t hist_len, void *stream);

/* -------------------------------------------------- sampling candidates */

/* Engine.pick (src/engine.ts:8352-8473; PENALIZED, CHUNK_MAX, CHUNK_RANK,
 * CHUNK_BY_RANK, CHUNK_GATHER, src/gpu/kernels.ts:3085-3163, :3265-3323):
 * for each of M rows of V logits, the `count` (1..64) 256-token chunks with
 * the largest penalized logit, in rank order (ties to the lower chunk), and
 * their penalized logits: chunks_out [M][count] chunk indices, candidates
 * [M][count][256] (token chunk * 256 + t; past V, -1e30). Penalized as the
 * reference does for batch row r = row0 + m:
 *  - -1e30 where the allowed bitmap (allowed [allowed_rows][ld_allowed]
 *    words, bit id % 32 of word id / 32 of row r, or row 0 when
 *    allowed_rows is 1; rows past allowed_rows allow nothing), if given,
 *    has the bit clear, or where mask[id] is 2 (never draw);
 *  - the token's state, mask[id] (0 unseen, 1 in the window from the
 *    prompt, 3 written; mask may be NULL for all 0), replaced by the last
 *    of seen_rows [n_seen][4] (token, state, first row, end row: at most 16)
 *    that covers row r;
 *  - a seen token (state 1 or 3): v < 0 ? v * penalty : v / penalty, then
 *    minus presence_penalty.
 * scratch: wg_pick_scratch_bytes(M, V) bytes (calls sharing it must not
 * overlap). The host samples from the candidates (see webgllm_amd/sampler.py,
 * the reference's createSampler with penalize = false); for top-k with k <=
 * count they hold the k largest penalized logits. */
size_t wg_pick_scratch_bytes(int32_t M, int32_t V);
int wg_pick_candidates(const float *logits, int32_t M, int32_t V, int32_t ld,
                       const uint8_t *mask, const int32_t *seen_rows, int32_t n_seen,
                       int32_t row0, float penalty, float presence_penalty,
                       const uint32_t *allowed, int32_t allowed_rows, int32_t ld_allowed,
                       int32_t count, int32_t *chunks_out, float *candidates, void *scratch,
                       size_t scratch_bytes, void *stream);

/* The host sampler (createSampler's distribution, draw, drawAt:
 * src/sampler.ts:27-242), over candidates the pick read back: settings as
 * the reference's Sampling (doubles, as JavaScript numbers). */
typedef struct {
  double temperature; /* <= 0: greedy */
  double top_p;       /* 1: off */
  double min_p;       /* 0: off */
  int32_t top_k;      /* <= 0: every candidate */
} wg_sampling;

/* distribution(logits, penalize = false): the kept candidates (ids_out,
 * from ids_in[i], or i when ids_in is NULL) and their probabilities, after
 * top-k (a min-heap of slots: the reference's order), top-p, min-p and the
 * temperature, with its float32 stores; *n_out of them (1 when greedy).
 * ids_out and p_out hold n entries. Host code; no device work. */
int wg_sample_distribution(const wg_sampling *s, const float *logits, const int32_t *ids_in,
                           int32_t n, int32_t *ids_out, float *p_out, int32_t *n_out);
/* draw (src/sampler.ts:188-200): the token a uniform u in [0, 1) picks,
 * candidates in their slot order. */
int32_t wg_sample_draw(const int32_t *ids, const float *p, int32_t n, double u);
/* drawAt (src/sampler.ts:227-242): the same, candidates in ascending id
 * order (seeded sampling). */
int32_t wg_sample_draw_at(const int32_t *ids, const float *p, int32_t n, double u);

#ifdef __cplusplus
}
#endif
#endif
