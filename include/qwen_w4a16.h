/*
 * qwen_w4a16.h -- C-ABI of the MI355X (gfx950) W4A16 quantized-matmul path.
 *
 * Plain C: device pointers, sizes and status codes only. `stream` is a
 * hipStream_t passed as void* (NULL = the null stream). Every call that
 * launches work is asynchronous on that stream, never synchronizes and never
 * allocates, so it can be captured into a hipGraph; the *_alloc / *_free calls
 * are the only ones that allocate or free.
 *
 * Each entry point names the reference interface it replaces
 * (patrickbdevaney/qwen38-3090-cuda-server, path:line). The reference aborts on
 * bad input; these return a status code instead, and the C++ layer in
 * qwen_w4a16.hpp turns a non-zero code into a message plus abort() so existing
 * reference callers keep their behaviour.
 *
 * Weight format accepted: INT4, asymmetric, group 128, stored nibbles 0..15
 * (w = (q - zp) * scale). Shapes: out_f % 64 == 0, in_f % 128 == 0.
 */
#ifndef QWEN_W4A16_H
#define QWEN_W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
enum {
  QW4_OK = 0,
  QW4_ERR_NULL = 1,        /* a required pointer is NULL                         */
  QW4_ERR_SHAPE = 2,       /* out_f % 64, in_f % 128, row offset or M invalid    */
  QW4_ERR_GROUP = 3,       /* group_size other than 128                          */
  QW4_ERR_M = 4,           /* M outside the range the entry point supports       */
  QW4_ERR_SCRATCH = 5,     /* scratch / workspace too small for this call        */
  QW4_ERR_ALIGN = 6,       /* activation / output pointer not 16-byte aligned    */
  QW4_ERR_HIP = 7,         /* a HIP runtime call failed (see qw4_last_hip_error)  */
  QW4_ERR_NOMEM = 8,       /* device allocation failed                           */
  QW4_ERR_LAYOUT = 9,      /* unknown source layout id                           */
  QW4_ERR_IO = 10,         /* file cannot be opened, mapped or parsed            */
  QW4_ERR_NOTFOUND = 11    /* tensor absent from a safetensors file              */
};

const char* qw4_status_string(int status);
int qw4_last_hip_error(void);   /* hipError_t of the last QW4_ERR_HIP, this thread */
int qw4_version(void);

/* ------------------------------------------------------------- weights
 * Device-resident repacked weights (the reference's W4A16Weights,
 * src/kernels/gemv_w4a16.cuh:50-60). The internal layout is private to the
 * library; its three buffers are separate allocations, each freeable with
 * hipFree, as the reference's callers do (src/model/model.cu:111, :204).
 */
typedef struct qw4_weights {
  uint32_t* qweight;   /* packed nibbles, tile-major                   */
  uint16_t* scale;     /* bf16, per (row, group)                        */
  uint16_t* zeros;     /* 4-bit zero points, 4 rows per u16             */
  int32_t out_f, in_f, group_size, num_groups;
} qw4_weights;

size_t qw4_weights_bytes(const qw4_weights* w);   /* device bytes held */

/* Repacked-layout sizes (the library asserts it uses these): output rows per
 * tile, and bytes of one (tile, group) scale record (64 bf16 scales + 16
 * zero-point words). */
#define QW4_TILE_ROWS 64
#define QW4_META_BYTES 160

/* awq_alloc_fused (src/kernels/gemv_w4a16.cuh:81-82; .cu:308-315). */
int qw4_weights_alloc(qw4_weights* w, int out_f, int in_f, int group_size, void* stream);
/* awq_free (gemv_w4a16.cuh:86; .cu:331-334). */
int qw4_weights_free(qw4_weights* w);

/* awq_repack_into (gemv_w4a16.cuh:83-85; .cu:317-323): compressed-tensors
 * pack-quantized source (src/loader/w4a16_unpack.h:1-18)
 *   packed [out_f][in_f/8] u32, scale [out_f][G] bf16, zp [out_f/8][G] u32,
 * written at destination rows [row_offset, row_offset + out_f) (row_offset % 64 == 0). */
int qw4_repack_ct_into(qw4_weights* w, int row_offset, const uint32_t* packed,
                       const uint16_t* scale, const uint32_t* zp, int out_f, void* stream);
/* awq_repack (gemv_w4a16.cuh:70-75; .cu:325-329) = alloc + repack_into(0). */
int qw4_repack_ct(qw4_weights* w, const uint32_t* packed, const uint16_t* scale,
                  const uint32_t* zp, int out_f, int in_f, int group_size, void* stream);

/* AWQ-order sources (no reference counterpart: the benchmark's input format).
 *   QW4_LAYOUT_AWQ_K: qweight [in_f/8][out_f] u32 packed along K,
 *   QW4_LAYOUT_AWQ_N: qweight [in_f][out_f/8] u32 packed along N (AutoAWQ GEMM),
 * both with nibble order {0,2,4,6,1,3,5,7}, scales [G][out_f] bf16 and
 * zeros [G][out_f/8] u32 in the same nibble order along N. */
enum { QW4_LAYOUT_AWQ_K = 1, QW4_LAYOUT_AWQ_N = 2 };
int qw4_repack_awq_into(qw4_weights* w, int row_offset, const uint32_t* qweight,
                        const uint16_t* scales, const uint32_t* zeros, int out_f,
                        int layout, void* stream);

/* w4a16_dequant_rows (src/kernels/gemm_w4a16.cuh:45-48; .cu:56-61):
 * dst [nrows][in_f] bf16 row-major = RNE((q - zp) * s) for rows row0.. */
int qw4_dequant_rows(uint16_t* dst, const qw4_weights* w, int row0, int nrows,
                     void* stream);

/* ------------------------------------------------------------- scratch
 * GemvScratch (gemv_w4a16.cuh:94-110): split-K partials and the self-resetting
 * counters of the skinny kernels. Counters start at zero and every call leaves
 * them at zero, so calls may be graph-captured; two calls that share one
 * scratch must not run concurrently.
 */
typedef struct qw4_scratch {
  float* partial;          /* split-K capacity of the reference (unused here)  */
  uint32_t* counters;      /* fused-argmax arrival counters (65 lines)       */
  uint64_t* keys;          /* fused-argmax keys: 64 groups x 16 rows         */
  size_t partial_elems;
  int32_t max_in, max_out, max_m, max_tiles;
} qw4_scratch;

/* gemv_scratch_alloc (gemv_w4a16.cuh:106-107; .cu:344-355). */
int qw4_scratch_alloc(qw4_scratch* s, int max_in, int max_out, int min_group, int max_m);
/* gemv_scratch_free (gemv_w4a16.cuh:108; .cu:368-371). */
int qw4_scratch_free(qw4_scratch* s);
/* gemv_partial_check (gemv_w4a16.cuh:109-110; .cu:359-366), as a status code. */
int qw4_partial_check(const qw4_scratch* s, int splits, int out_f, int M);
/* gemv_choose_splits (gemv_w4a16.cuh:134; .cu:289-306): cross-workgroup
 * K-splits the skinny kernels use for this shape. Always 1: every workgroup
 * owns whole output rows over all of K. On MI355X every K split measured
 * (partials exchanged between workgroups as tagged agent-scope words, or
 * summed by a second kernel as the reference does) was slower than whole
 * rows at the decode and verify shapes. */
int qw4_choose_splits(int out_f, int num_groups);

/* TEST-ONLY tuning overrides: not part of the product interface (no reference
 * counterpart). The benchmark and the tests use them to force every kernel
 * form; a product caller never needs them and must not call them while other
 * threads launch, since they are process-wide atomics read at each launch.
 * qw4_tune_decode, the skinny launches: mode 0 the library's measured policy;
 * 1 the bf16 skinny kernel (k_rows) instead of the integer-MFMA decode kernel
 * at M = 1, S (1, 2, 4 row quads per unit) and D (2..4) forcing its unit size
 * and LDS-DMA depth; 2 k_rows with items in
 * registers for every M, S (1, 2, 4 row quads per unit) and W (8, 16 waves)
 * forcing its shape; 3 the decode kernel with unit size S, W waves and D items
 * per wave (0 = the policy's value); 4 the policy with the M > 1 activations
 * never staged in LDS and never shared by a workgroup's units (loaded with
 * each item); 5 the policy without the group-major M > 1 kernel. P > 0 forces
 * the decode kernel's workgroup count. */
int qw4_tune_decode(int mode, int S, int W, int D, int P);
/* qw4_tune_gemm: the prefill schedule, -1 the cost model (default), 0 one
 * workgroup per tile, 1 stream-K, 2 hybrid, 3 split-K (every tile cut into the
 * same k-slices; at most CUs / 2 tiles) (split schedules need a workspace);
 * variant 0 the default kernel (4 waves, each on a whole 64-row weight tile
 * against all 256 activation rows), 1 8 waves on 32-row tile halves, 2 8 waves
 * on whole tiles against 128 rows; the variants' results are bitwise equal. */
int qw4_tune_gemm(int schedule, int variant);
/* qw4_tune_linear: max_t of qw4_linear for every weight, 0 = the measured rule
 * (the role of the reference's QWEN_MMA_MAX_T environment variable). */
int qw4_tune_linear(int max_t);

/* ------------------------------------------------------- decode / verify
 * y [M][out_f] = x [M][in_f] @ W^T, bf16 row-major, fp32 accumulation.
 * x must be 16-byte aligned; y 8-byte aligned (16 for fp32).
 */
/* gemv_w4a16 (gemv_w4a16.cuh:130-131; .cu:464-469), M = 1. */
int qw4_gemv(uint16_t* y, const qw4_weights* w, const uint16_t* x, qw4_scratch* s,
             void* stream);
/* gemv_w4a16_f32 (gemv_w4a16.cuh:132-133; .cu:456-462), M = 1, fp32 output. */
int qw4_gemv_f32(float* y, const qw4_weights* w, const uint16_t* x, qw4_scratch* s,
                 void* stream);
/* gemm_small_w4a16 (gemv_w4a16.cuh:124-125; .cu:396-454), 1 <= M <= 16. */
int qw4_gemm_small(uint16_t* y, const qw4_weights* w, const uint16_t* x, int M,
                   qw4_scratch* s, void* stream);
/* gemm_mma_w4a16 (gemv_w4a16.cuh:187-188; .cu:842-865), 1 <= M <= 16. */
int qw4_gemm_mma(uint16_t* y, const qw4_weights* w, const uint16_t* x, int M,
                 qw4_scratch* s, void* stream);

/* lm_head GEMV fused with an fp32 row-argmax (lowest index on ties). Replaces
 * head() + argmax / model_apply_head() + argmax_rows (src/model/model.cu:796-815,
 * :1009-1051; src/kernels/elementwise.cuh:39-43) without writing logits.
 * idx [M] int32, 1 <= M <= 16. */
int qw4_gemv_argmax(int32_t* idx, const qw4_weights* w, const uint16_t* x, int M,
                    qw4_scratch* s, void* stream);
/* qw4_gemv_argmax without allocation. No counterpart in the reference: for
 * callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same results as
 * qw4_gemv_argmax; its scratch (argmax keys and arrival counters, 16.5 KiB) is
 * a file-scope device array the library holds per GPU until the process ends,
 * so no scratch argument. M in 1..16 (QW4_ERR_M beyond). Calls that overlap on
 * one GPU (several streams or threads at once) share that array and race:
 * serialize them. Calls nothing that allocates. */
int qw4_gemv_argmax_noalloc(int32_t* idx, const qw4_weights* w, const uint16_t* x, int M,
                            void* stream);

/* ------------------------------------------------------------- prefill
 * GemmWorkspace (src/kernels/gemm_w4a16.cuh:30-35). The fused kernel needs no
 * dequantized-weight buffer; a workspace of at least 2 x CUs x 256 KiB
 * (128 MiB on MI355X; the reference allocates 256 MiB, model.cu:440) lets it
 * split tiles across workgroups (stream-K, hybrid, or split-K when there are
 * at most CUs / 2 tiles) when whole tiles would leave CUs idle. The workspace
 * then holds fp32 partial tiles: calls that share one must be stream-ordered.
 * NULL or smaller: one workgroup per tile. */
typedef struct qw4_workspace {
  void* buf;
  size_t bytes;
} qw4_workspace;

/* gemm_workspace_alloc / _free (gemm_w4a16.cuh:37-38; .cu:42-54). */
int qw4_workspace_alloc(qw4_workspace* ws, size_t bytes);
int qw4_workspace_free(qw4_workspace* ws);
/* gemm_w4a16 (gemm_w4a16.cuh:40-43; .cu:63-88): C [M][out_f] bf16 =
 * A [M][in_f] bf16 @ W^T with W dequantized to bf16 (RNE((q-zp)*s)), bf16 MFMA,
 * fp32 accumulation. Any M >= 1 with M * in_f * 2 < 2^32. A 16-byte aligned,
 * C 8-byte aligned. Results are bitwise reproducible for a given shape and
 * workspace size. */
int qw4_gemm(uint16_t* C, const qw4_weights* w, const uint16_t* A, int M,
             qw4_workspace* ws, void* stream);

/* -------------------------------------------------------------- argmax
 * argmax / argmax_rows over bf16 logits (src/kernels/elementwise.cuh:34-43;
 * .cu:96-158, :184-194), lowest index on ties. argmax's scratch holds
 * >= 512 int32 (the reference's 256 (idx, val) pairs). */
int qw4_argmax(int32_t* out, const uint16_t* x, int n, int32_t* scratch, void* stream);
int qw4_argmax_rows(int32_t* out, const uint16_t* x, int rows, int n, void* stream);

/* ------------------------------------------------- layer steps either side
 * The elementwise steps around the projections in the reference's layer
 * (src/kernels/elementwise.cuh:8-22, .cu:8-49; called at
 * src/model/model.cu:697, :772-785). Data bf16, 16-byte aligned.
 *
 * rmsnorm: out [rows][dim] = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)),
 * fp32 throughout (elementwise.cuh:8-13). dim % 8 == 0. */
int qw4_rmsnorm(uint16_t* out, const uint16_t* x, const uint16_t* w, int rows, int dim,
                float eps, void* stream);
/* residual_add: out[i] = bf16(out[i] + x[i]), i < n (elementwise.cuh:15-17). */
int qw4_residual_add(uint16_t* out, const uint16_t* x, size_t n, void* stream);
/* swiglu: out [rows][inter] = bf16(silu(g) * u) of a fused [rows][gate | up]
 * buffer, silu(g) = g / (1 + exp(-g)) (elementwise.cuh:19-22). inter % 8 == 0. */
int qw4_swiglu(uint16_t* out, const uint16_t* fused, int rows, int inter, void* stream);

/* The same steps fused into the decode / verify GEMV (1 <= M <= 16), with the
 * reference's roundings (each projection output rounded to bf16 first):
 *
 * linear then residual_add (model.cu:779-784): h [M][out_f] = bf16(h + bf16(x @ W^T)). */
int qw4_gemv_residual(uint16_t* h, const qw4_weights* w, const uint16_t* x, int M,
                      qw4_scratch* s, void* stream);
/* linear over the fused [gate | up] weight (out_f = 2 * inter, inter % 64 == 0),
 * then swiglu (model.cu:776-778): y [M][inter]. For M <= 2 (or tmp NULL) the
 * intermediate [M][2 inter] is never written; for M > 2 with tmp
 * ([M][2 inter] bf16) the projection goes through tmp and a separate swiglu,
 * which is faster there. Same results either way. */
int qw4_gemv_swiglu(uint16_t* y, const qw4_weights* w, const uint16_t* x, int M, uint16_t* tmp,
                    qw4_scratch* s, void* stream);
/* rmsnorm then linear (model.cu:697-700, :773-777): y [M][out_f] = rmsnorm(h) @ W^T
 * with norm weight norm_w [in_f]. The normalized rows are formed in LDS and
 * never written. When they do not fit (M > 1 with M * in_f * 2 beyond the
 * staging limit), tmp ([M][in_f] bf16) receives them and the plain GEMV
 * follows; without tmp such a call returns QW4_ERR_SHAPE. At M = 1 beyond what
 * the decode kernel stages beside its other LDS, a given tmp takes the same
 * two-step path (the faster one), and without tmp the bf16 skinny kernel
 * normalizes the row in LDS itself (within the GEMV tolerance of the two-step
 * result, not bitwise equal to it). Otherwise results equal qw4_rmsnorm +
 * qw4_gemm_small bit for bit. tmp may be NULL. */
int qw4_gemv_rmsnorm(uint16_t* y, const qw4_weights* w, const uint16_t* h,
                     const uint16_t* norm_w, float eps, int M, uint16_t* tmp, qw4_scratch* s,
                     void* stream);

/* ------------------------------------------------------------ dispatch
 * linear() with lin_path() (src/model/model.cu:522-565, :643-658): T rows of
 * x through the GEMV (T = 1), the skinny kernel in chunks of up to 16 rows
 * (2 <= T <= max_t), or the prefill GEMM (T > max_t). max_t is the crossover
 * measured on MI355X for this weight's size (qw4_linear_max_t: 48 rows for
 * a 93 MB projection, 112 for an 11 MB one); qw4_tune_linear overrides it,
 * as QWEN_MMA_MAX_T does in the reference. ws may be NULL. */
int qw4_linear(uint16_t* y, const qw4_weights* w, const uint16_t* x, int T, qw4_scratch* s,
               qw4_workspace* ws, void* stream);
int qw4_linear_max_t(const qw4_weights* w);

/* quantize_w4a16_raw (src/model/model.cu:174-186, kernel k_quant_i4 :140-172):
 * a bf16 [out_f][in_f] matrix (device, 16-byte aligned; the reference's
 * lm_head ablation, --lm-head-bits 4) quantized to INT4 group-128 asymmetric
 * (per row and group: s = (max - min) / 15, z = clamp(rint(-min / s), 0, 15),
 * q = clamp(rint(v / s) + z, 0, 15); bf16 scale) straight into the repacked
 * layout; allocates w like qw4_weights_alloc. */
int qw4_quantize_w4a16(qw4_weights* w, const uint16_t* src, int out_f, int in_f, int group_size,
                       void* stream);

/* ------------------------------------------------------ 8-bit weights
 * W8A16Weights (src/kernels/gemv_w4a16.cuh:141-154), the reference's default
 * lm_head format: per (row, 128-group) a bf16 scale and int8 q in [-127, 127].
 * Private device layout: 64-row tiles x 128-k groups, 8 KiB blocks, q stored
 * as q + 128. qweight (out_f * in_f bytes) and scale (out_f * G * 2 bytes) are
 * separate hipMalloc allocations. */
typedef struct qw4_w8_weights {
  uint8_t* qweight;
  uint16_t* scale;
  int32_t out_f, in_f, group_size, num_groups;
} qw4_w8_weights;

/* quantize_w8a16 (gemv_w4a16.cuh:156-157; .cu:478-495, :616-623): allocates w
 * and quantizes the bf16 source src [out_f][in_f] (16-byte aligned) on the
 * stream: s = bf16(max|w| / 127), q = clamp(rint(w * 127 / max|w|), +-127). */
int qw4_w8_quantize(qw4_w8_weights* w, const uint16_t* src, int out_f, int in_f,
                    int group_size, void* stream);
/* w8a16_free (gemv_w4a16.cuh:164). */
int qw4_w8_free(qw4_w8_weights* w);
size_t qw4_w8_bytes(const qw4_w8_weights* w);   /* W8A16Weights::total_bytes */
/* dst [nrows][in_f] bf16 = RNE(q * s); no reference counterpart (the 8-bit
 * analogue of w4a16_dequant_rows, for bit-exact checks). */
int qw4_w8_dequant_rows(uint16_t* dst, const qw4_w8_weights* w, int row0, int nrows,
                        void* stream);
/* gemv_w8a16 (gemv_w4a16.cuh:158-159; .cu:624-636), M = 1, and
 * gemm_small_w8a16 (gemv_w4a16.cuh:163-164; .cu:551-614), 1 <= M <= 16:
 * y [M][out_f] bf16, the same kernel as qw4_gemv / qw4_gemm_small. */
int qw4_w8_gemv(uint16_t* y, const qw4_w8_weights* w, const uint16_t* x, qw4_scratch* s,
                void* stream);
int qw4_w8_gemm_small(uint16_t* y, const qw4_w8_weights* w, const uint16_t* x, int M,
                      qw4_scratch* s, void* stream);
/* The 8-bit lm_head fused with the fp32 row-argmax: head() with lm_head_bits 8
 * (src/model/model.cu:796-815, :1044-1047) without writing logits. */
int qw4_w8_gemv_argmax(int32_t* idx, const qw4_w8_weights* w, const uint16_t* x, int M,
                       qw4_scratch* s, void* stream);

/* ---------------------------------------------------------- checkpoints
 * mmap'd safetensors reader (src/loader/safetensors.h:44-75; C++ API in
 * qwen_safetensors.hpp) and the compressed-tensors -> repacked loader.
 * Host code only: a qw4_st_tensor's data points into the read-only mapping and
 * stays valid until qw4_st_close. dtype uses the safetensors dtype order
 * BF16, F16, F32, F64, I8, U8, I16, I32, I64, BOOL, F8_E4M3, F8_E5M2 = 0..11. */
typedef struct qw4_st qw4_st;
typedef struct qw4_st_tensor {
  int32_t dtype;
  int32_t ndim;            /* dims beyond 8 are not reported */
  int64_t shape[8];
  const void* data;
  size_t nbytes;
} qw4_st_tensor;

/* SafeTensors::open_files / open_dir (safetensors.h:53-55). */
int qw4_st_open(qw4_st** st, const char* const* paths, int npaths);
int qw4_st_open_dir(qw4_st** st, const char* dir);
int qw4_st_close(qw4_st* st);
int qw4_st_count(const qw4_st* st);
/* SafeTensors::find (safetensors.h:60); QW4_ERR_NOTFOUND if absent. */
int qw4_st_find(const qw4_st* st, const char* name, qw4_st_tensor* out);
/* Message of the last QW4_ERR_IO / _NOTFOUND / _SHAPE from these calls (this thread). */
const char* qw4_st_last_error(void);
/* fuse() (src/model/model.cu:103-128): allocate w for the sum of the parts'
 * rows and repack each part's <prefix>.weight_packed (I32 [rows][in_f/8]),
 * .weight_scale (BF16 [rows][G]) and .weight_zero_point (I32 [rows/8][G]) at
 * consecutive row offsets (each part's rows % 64 == 0). Synchronizes the
 * stream (the uploaded sources are freed before returning). */
int qw4_load_ct_fused(qw4_weights* w, const qw4_st* st, const char* const* prefixes,
                      int nparts, int in_f, int group_size, void* stream);

/* ------------------------------------------------- synthetic inputs
 * Device-side generator for the benchmark (no reference counterpart). The
 * counter-based spec is documented with the generator kernel:
 *   kind 0: x = bf16(N(0,1)), kind 1: scale = bf16(|N(0,0.02)| + 1e-4).
 * qw4_gen_awq_k writes one tensor in QW4_LAYOUT_AWQ_K form from streams
 * tensor*8 + {0: q, 1: zp, 2: scale}. */
int qw4_gen_bf16(uint16_t* out, size_t count, uint64_t seed, uint64_t stream_id,
                 uint64_t offset, int kind, void* stream);
int qw4_gen_awq_k(uint32_t* qweight, uint16_t* scales, uint32_t* zeros, int out_f,
                  int in_f, uint64_t seed, uint64_t tensor, void* stream);

/* Streaming-read microbenchmark (no reference counterpart; the intent of the
 * reference's bench/microbench.cu "streaming read"): reads `bytes` (multiple of
 * 16) with 16-byte loads and writes one XOR per workgroup to sink[blocks]. */
int qw4_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream);

/* MFMA peak microbenchmark (no reference counterpart; the intent of the
 * reference's bench/microbench.cu peak measurement, used as the measured
 * denominator next to the published bf16 peak): `blocks` workgroups of 4
 * waves, each wave `iters` x 8 v_mfma_f32_32x32x16_bf16 (32768 flop each) on
 * random operands; writes one word per workgroup to sink[blocks]. */
int qw4_mfma_peak(uint32_t* sink, int blocks, int iters, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* QWEN_W4A16_H */
