/*
 * CPU oracle for the W4A16 quantized-matmul path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as the
 * checker; the product library never links or calls it.
 *
 * Every function restates the reference's host-side algorithm; the citation
 * next to each names the reference file:line it follows (paths relative to the
 * reference repository root).
 *
 * Logical weight tensor (one per projection), shared by every layout:
 *   q[n][k]  in 0..15   the STORED nibble   (reference: signed q + 8)
 *   zp[n][g] in 0..15   the STORED nibble   (reference: signed zp + 8)
 *   s[n][g]  bf16 bits
 *   w[n][k] = float(q - zp) * float(s)      (src/loader/w4a16_unpack.h:14,
 *             tests/gate_dequant.cpp:73-76; offsets cancel, gemv_w4a16.cuh:32-37)
 */
#ifndef QW4_ORACLE_H
#define QW4_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 helpers (tests/gate_gemv.cu:23-29: RNE, matches __float2bfloat16) */
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);

/* ---- deterministic synthetic inputs (counter-based; no reference analogue:
 *      the reference's mt19937 + normal_distribution is implementation-defined,
 *      so the same spec is implemented here and in the HIP generator).
 *  draw(key, i) = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)
 *  key          = mix64(seed * 0xD1B54A32D192ED03 + stream)
 *  u4(i)        = draw(i) >> 60
 *  normal(i)    = Irwin-Hall(12): sum of the twelve 16-bit fields of
 *                 draw(3i), draw(3i+1), draw(3i+2) -> (S + 6) / 65536 - 6
 *                 (exact in fp32; mean 0, variance 1, support +-6)
 *  kind 0: x     = bf16(normal)
 *  kind 1: scale = bf16(|normal * 0.02f| + 1e-4f)
 */
uint64_t or_mix64(uint64_t z);
uint64_t or_key(uint64_t seed, uint64_t stream);
void or_gen_u4(uint8_t* out, size_t count, uint64_t seed, uint64_t stream, uint64_t offset);
void or_gen_bf16(uint16_t* out, size_t count, uint64_t seed, uint64_t stream,
                 uint64_t offset, int kind);
float or_normal(uint64_t key, uint64_t i);

/* ---- packed layouts ---------------------------------------------------------
 * A0  compressed-tensors pack-quantized (the reference's on-disk format,
 *     src/loader/w4a16_unpack.h:1-18):
 *       packed [N][K/8] u32, element e of a row at bits 4*(e%8) of word e/8
 *       scale  [N][G]   bf16
 *       zp     [N/8][G] u32, row n at nibble n%8 of word [n/8][g]
 * A1  BASELINE layout: qweight [K/8][N] u32 packed along K, nibble slot i of
 *     word [r][n] holds k = 8r + AWQ_ORDER[i]; scales [G][N] bf16;
 *     zeros [G][N/8] u32, slot i of word [g][c] holds n = 8c + AWQ_ORDER[i]
 * A2  AutoAWQ GEMM layout: qweight [K][N/8] u32, slot i of word [k][c] holds
 *     n = 8c + AWQ_ORDER[i]; scales [G][N]; zeros [G][N/8] as A1
 *  AWQ_ORDER = {0,2,4,6,1,3,5,7}
 */
void or_pack_ct(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                int group, uint32_t* packed, uint16_t* scale, uint32_t* zpw);
void or_unpack_ct(const uint32_t* packed, const uint16_t* scale, const uint32_t* zpw,
                  int N, int K, int group, uint8_t* q, uint8_t* zp, uint16_t* s);
void or_pack_awq_k(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                   int group, uint32_t* qweight, uint16_t* scales, uint32_t* zeros);
void or_unpack_awq_k(const uint32_t* qweight, const uint16_t* scales, const uint32_t* zeros,
                     int N, int K, int group, uint8_t* q, uint8_t* zp, uint16_t* s);
void or_pack_awq_n(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                   int group, uint32_t* qweight, uint16_t* scales, uint32_t* zeros);
void or_unpack_awq_n(const uint32_t* qweight, const uint16_t* scales, const uint32_t* zeros,
                     int N, int K, int group, uint8_t* q, uint8_t* zp, uint16_t* s);

/* Signed reference accessors on A0 (restates w4a16_unpack.h:25-42 exactly). */
int32_t or_ct_q(const uint32_t* packed, int64_t in_features, int64_t o, int64_t i);
int32_t or_ct_zp(const uint32_t* zpw, int64_t num_groups, int64_t o, int64_t g);

/* ---- dequant (gemm_w4a16.cu:26-36: fp32 (q - z) * s, then RNE to bf16) */
void or_dequant_f32(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                    int group, int row0, int nrows, float* w);
void or_dequant_bf16(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                     int group, int row0, int nrows, uint16_t* w);

/* ---- matmul references -------------------------------------------------------
 * y[m][n] = sum_k x[m][k] * w[n][k], fp64 accumulation (tests/gate_gemv.cu:96-115,
 * tests/gate_gemm.cu:73-90), computed for every (m, n), nthreads workers. */
void or_matmul_f64(const uint16_t* x, int M, const uint8_t* q, const uint8_t* zp,
                   const uint16_t* s, int N, int K, int group, double* y, int nthreads);
/* Same product with the weights first rounded to bf16 (the prefill semantics:
 * dequant to bf16, then an fp32-accumulated bf16 GEMM, gemm_w4a16.cu:63-88). */
void or_matmul_bf16w_f64(const uint16_t* x, int M, const uint8_t* q, const uint8_t* zp,
                         const uint16_t* s, int N, int K, int group, double* y,
                         int nthreads);

/* CPU baseline: the reference's host dequant+matmul over the A0 packed tensors,
 * fp32 accumulation, bf16 output, threads over N (gate_gemm.cu:73-90 with fp32
 * accumulation and every row computed). Returns the thread count used. */
int or_cpu_w4a16_matmul(const uint16_t* x, int M, const uint32_t* packed,
                        const uint16_t* scale, const uint32_t* zpw, int N, int K,
                        int group, uint16_t* y, int nthreads);

/* ---- W8A16 (the reference's lm_head format, src/kernels/gemv_w4a16.cuh:141-166).
 * Quantizer, k_quant_w8 (src/kernels/gemv_w4a16.cu:478-495): for each (row n,
 * group g) of the bf16 source w[N][K], mx = max |w|, s = bf16(mx / 127),
 * inv = mx > 0 ? 127 / mx : 0 (fp32, from mx, not from the rounded s),
 * q = clamp(rint(w * inv), -127, 127). Dequantized weight: q * float(s). */
void or_w8_quantize(const uint16_t* w, int N, int K, int group, int8_t* q, uint16_t* s);
/* k_quant_i4 (src/model/model.cu:140-172): INT4 g128 asymmetric, A0 tensors. */
void or_quant_i4(const uint16_t* w, int N, int K, int group, uint32_t* packed, uint16_t* scale,
                 uint32_t* zp);
/* y[m][n] = sum_k x[m][k] * q[n][k] * s[n][k / group], fp64 (k_gemv8,
 * src/kernels/gemv_w4a16.cu:498-523, with fp64 accumulation). */
void or_w8_matmul_f64(const uint16_t* x, int M, const int8_t* q, const uint16_t* s, int N,
                      int K, int group, double* y, int nthreads);

/* ---- argmax: lowest index on ties (elementwise.cu:103-104, :111-112).
 * margin[m] = best - second best (distinct indices), for near-tie reporting. */
void or_argmax_rows_f64(const double* v, int rows, int n, int32_t* idx, double* margin);
void or_argmax_rows_f32(const float* v, int rows, int n, int32_t* idx);
void or_argmax_rows_bf16(const uint16_t* v, int rows, int n, int32_t* idx);

#ifdef __cplusplus
}
#endif
#endif
