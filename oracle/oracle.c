/*
 * CPU oracle for the W4A16 path -- TEST INFRASTRUCTURE, never shipped or called by
 * the product library. Declarations and layout definitions are in oracle.h.
 *
 * Parity pins (checked by tests/test_oracle.py):
 *   or_unpack_ct / or_ct_q / or_ct_zp / or_dequant_f32 : the reference's
 *       compressed-tensors fixtures (tests/fixtures/dequant, copied under
 *       tests/golden/ct_dequant) bit-exact, and oracle/_ref (the reference's
 *       own w4a16_unpack.h compiled) on random words.
 *   or_pack_awq_k / or_pack_awq_n : hand-computed AutoAWQ known answers
 *       (0x75316420 for elements 0..7) and round trips through A0.
 *   or_matmul_f64 : closed forms (column pick, q == zp, constant x, rank-1),
 *       numpy float64 brute force on tiny shapes.
 *   or_argmax_* : numpy argmax (lowest index on ties) and constructed ties.
 *   or_gen_* : moments of the distributions and fixed known values.
 *   or_cpu_w4a16_matmul : agreement with or_matmul_f64 within fp32 error.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static const int kAwqOrder[8] = {0, 2, 4, 6, 1, 3, 5, 7};

/* ------------------------------------------------------------------ bf16 */
float or_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* tests/gate_gemv.cu:23-29 -- round to nearest even on the top 16 bits. */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t r = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + r) >> 16);
}

/* ------------------------------------------------------------- generator */
uint64_t or_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t or_key(uint64_t seed, uint64_t stream) {
  return or_mix64(seed * 0xD1B54A32D192ED03ull + stream);
}

static inline uint64_t draw(uint64_t key, uint64_t i) {
  return or_mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

void or_gen_u4(uint8_t* out, size_t count, uint64_t seed, uint64_t stream, uint64_t offset) {
  const uint64_t key = or_key(seed, stream);
  for (size_t i = 0; i < count; ++i) out[i] = (uint8_t)(draw(key, offset + i) >> 60);
}

float or_normal(uint64_t key, uint64_t i) {
  uint32_t s = 0;
  for (int t = 0; t < 3; ++t) {
    const uint64_t r = draw(key, 3 * i + (uint64_t)t);
    s += (uint32_t)(r & 0xffff) + (uint32_t)((r >> 16) & 0xffff) +
         (uint32_t)((r >> 32) & 0xffff) + (uint32_t)(r >> 48);
  }
  return ((float)s + 6.0f) * (1.0f / 65536.0f) - 6.0f;
}

void or_gen_bf16(uint16_t* out, size_t count, uint64_t seed, uint64_t stream,
                 uint64_t offset, int kind) {
  const uint64_t key = or_key(seed, stream);
  for (size_t i = 0; i < count; ++i) {
    const float v = or_normal(key, offset + i);
    out[i] = kind == 0 ? or_f32_to_bf16(v) : or_f32_to_bf16(fabsf(v * 0.02f) + 1e-4f);
  }
}

/* --------------------------------------------------------- A0 (reference) */
/* src/loader/w4a16_unpack.h:25-29, :32-34 */
int32_t or_ct_q(const uint32_t* packed, int64_t in_features, int64_t o, int64_t i) {
  const uint32_t w = packed[o * (in_features >> 3) + (i >> 3)];
  return (int32_t)((w >> ((i & 7) * 4)) & 0xFu) - 8;
}

/* src/loader/w4a16_unpack.h:38-42: zero points packed down the OUTPUT axis. */
int32_t or_ct_zp(const uint32_t* zpw, int64_t num_groups, int64_t o, int64_t g) {
  const uint32_t w = zpw[(o >> 3) * num_groups + g];
  return (int32_t)((w >> ((o & 7) * 4)) & 0xFu) - 8;
}

void or_pack_ct(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                int group, uint32_t* packed, uint16_t* scale, uint32_t* zpw) {
  const int G = K / group, W = K / 8;
  memset(packed, 0, sizeof(uint32_t) * (size_t)N * W);
  memset(zpw, 0, sizeof(uint32_t) * (size_t)(N / 8) * G);
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k)
      packed[(size_t)n * W + k / 8] |= (uint32_t)(q[(size_t)n * K + k] & 0xF) << (4 * (k % 8));
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < G; ++g) {
      scale[(size_t)n * G + g] = s[(size_t)n * G + g];
      zpw[(size_t)(n / 8) * G + g] |= (uint32_t)(zp[(size_t)n * G + g] & 0xF) << (4 * (n % 8));
    }
}

void or_unpack_ct(const uint32_t* packed, const uint16_t* scale, const uint32_t* zpw,
                  int N, int K, int group, uint8_t* q, uint8_t* zp, uint16_t* s) {
  const int G = K / group;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) q[(size_t)n * K + k] = (uint8_t)(or_ct_q(packed, K, n, k) + 8);
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < G; ++g) {
      zp[(size_t)n * G + g] = (uint8_t)(or_ct_zp(zpw, G, n, g) + 8);
      s[(size_t)n * G + g] = scale[(size_t)n * G + g];
    }
}

/* ------------------------------------------------ A1 / A2 (AWQ nibble order) */
static void pack_zeros_awq(const uint8_t* zp, int N, int G, uint32_t* zeros) {
  memset(zeros, 0, sizeof(uint32_t) * (size_t)G * (N / 8));
  for (int g = 0; g < G; ++g)
    for (int c = 0; c < N / 8; ++c) {
      uint32_t w = 0;
      for (int i = 0; i < 8; ++i) w |= (uint32_t)(zp[(size_t)(8 * c + kAwqOrder[i]) * G + g] & 0xF) << (4 * i);
      zeros[(size_t)g * (N / 8) + c] = w;
    }
}

static void unpack_zeros_awq(const uint32_t* zeros, int N, int G, uint8_t* zp) {
  for (int g = 0; g < G; ++g)
    for (int c = 0; c < N / 8; ++c) {
      const uint32_t w = zeros[(size_t)g * (N / 8) + c];
      for (int i = 0; i < 8; ++i) zp[(size_t)(8 * c + kAwqOrder[i]) * G + g] = (uint8_t)((w >> (4 * i)) & 0xF);
    }
}

static void transpose_scales(const uint16_t* s, int N, int G, uint16_t* scales) {
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < G; ++g) scales[(size_t)g * N + n] = s[(size_t)n * G + g];
}

static void untranspose_scales(const uint16_t* scales, int N, int G, uint16_t* s) {
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < G; ++g) s[(size_t)n * G + g] = scales[(size_t)g * N + n];
}

void or_pack_awq_k(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                   int group, uint32_t* qweight, uint16_t* scales, uint32_t* zeros) {
  const int G = K / group;
  for (int r = 0; r < K / 8; ++r)
    for (int n = 0; n < N; ++n) {
      uint32_t w = 0;
      for (int i = 0; i < 8; ++i) w |= (uint32_t)(q[(size_t)n * K + 8 * r + kAwqOrder[i]] & 0xF) << (4 * i);
      qweight[(size_t)r * N + n] = w;
    }
  transpose_scales(s, N, G, scales);
  pack_zeros_awq(zp, N, G, zeros);
}

void or_unpack_awq_k(const uint32_t* qweight, const uint16_t* scales, const uint32_t* zeros,
                     int N, int K, int group, uint8_t* q, uint8_t* zp, uint16_t* s) {
  const int G = K / group;
  for (int r = 0; r < K / 8; ++r)
    for (int n = 0; n < N; ++n) {
      const uint32_t w = qweight[(size_t)r * N + n];
      for (int i = 0; i < 8; ++i) q[(size_t)n * K + 8 * r + kAwqOrder[i]] = (uint8_t)((w >> (4 * i)) & 0xF);
    }
  untranspose_scales(scales, N, G, s);
  unpack_zeros_awq(zeros, N, G, zp);
}

void or_pack_awq_n(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                   int group, uint32_t* qweight, uint16_t* scales, uint32_t* zeros) {
  const int G = K / group;
  for (int k = 0; k < K; ++k)
    for (int c = 0; c < N / 8; ++c) {
      uint32_t w = 0;
      for (int i = 0; i < 8; ++i) w |= (uint32_t)(q[(size_t)(8 * c + kAwqOrder[i]) * K + k] & 0xF) << (4 * i);
      qweight[(size_t)k * (N / 8) + c] = w;
    }
  transpose_scales(s, N, G, scales);
  pack_zeros_awq(zp, N, G, zeros);
}

void or_unpack_awq_n(const uint32_t* qweight, const uint16_t* scales, const uint32_t* zeros,
                     int N, int K, int group, uint8_t* q, uint8_t* zp, uint16_t* s) {
  const int G = K / group;
  for (int k = 0; k < K; ++k)
    for (int c = 0; c < N / 8; ++c) {
      const uint32_t w = qweight[(size_t)k * (N / 8) + c];
      for (int i = 0; i < 8; ++i) q[(size_t)(8 * c + kAwqOrder[i]) * K + k] = (uint8_t)((w >> (4 * i)) & 0xF);
    }
  untranspose_scales(scales, N, G, s);
  unpack_zeros_awq(zeros, N, G, zp);
}

/* ---------------------------------------------------------------- dequant */
/* gemm_w4a16.cu:26-36 (and tests/gate_dequant.cpp:73-76): fp32 (q - z) * s. */
void or_dequant_f32(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                    int group, int row0, int nrows, float* w) {
  const int G = K / group;
  (void)N;
  for (int r = 0; r < nrows; ++r) {
    const int n = row0 + r;
    for (int k = 0; k < K; ++k) {
      const int g = k / group;
      const float sc = or_bf16_to_f32(s[(size_t)n * G + g]);
      const float d = (float)((int)q[(size_t)n * K + k] - (int)zp[(size_t)n * G + g]);
      w[(size_t)r * K + k] = d * sc;
    }
  }
}

void or_dequant_bf16(const uint8_t* q, const uint8_t* zp, const uint16_t* s, int N, int K,
                     int group, int row0, int nrows, uint16_t* w) {
  const int G = K / group;
  (void)N;
  for (int r = 0; r < nrows; ++r) {
    const int n = row0 + r;
    for (int k = 0; k < K; ++k) {
      const int g = k / group;
      const float sc = or_bf16_to_f32(s[(size_t)n * G + g]);
      const float d = (float)((int)q[(size_t)n * K + k] - (int)zp[(size_t)n * G + g]);
      w[(size_t)r * K + k] = or_f32_to_bf16(d * sc);
    }
  }
}

/* ---------------------------------------------------------- thread helper */
typedef struct {
  void (*fn)(void*, int, int);
  void* ctx;
  int lo, hi;
} span_t;

static void* span_main(void* p) {
  span_t* s = (span_t*)p;
  s->fn(s->ctx, s->lo, s->hi);
  return NULL;
}

static int parallel_for(int n, int nthreads, void (*fn)(void*, int, int), void* ctx) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > n) nthreads = n > 0 ? n : 1;
  if (nthreads > 256) nthreads = 256;
  if (nthreads == 1) {
    fn(ctx, 0, n);
    return 1;
  }
  pthread_t th[256];
  span_t sp[256];
  for (int t = 0; t < nthreads; ++t) {
    sp[t].fn = fn;
    sp[t].ctx = ctx;
    sp[t].lo = (int)((long long)n * t / nthreads);
    sp[t].hi = (int)((long long)n * (t + 1) / nthreads);
    pthread_create(&th[t], NULL, span_main, &sp[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  return nthreads;
}

/* ----------------------------------------------------------- fp64 matmul */
typedef struct {
  const uint16_t* x;
  int M;
  const uint8_t *q, *zp;
  const uint16_t* s;
  int N, K, group, round_w;
  double* y;
} mm_ctx;

/* tests/gate_gemv.cu:96-115 / tests/gate_gemm.cu:73-90: acc += (q - zp) * s * x in fp64,
 * here for every (m, n). With round_w the weight is first rounded to bf16. */
static void mm_rows(void* p, int lo, int hi) {
  const mm_ctx* c = (const mm_ctx*)p;
  const int G = c->K / c->group;
  double* wrow = (double*)malloc(sizeof(double) * (size_t)c->K);
  for (int n = lo; n < hi; ++n) {
    for (int k = 0; k < c->K; ++k) {
      const int g = k / c->group;
      const float sc = or_bf16_to_f32(c->s[(size_t)n * G + g]);
      const float d = (float)((int)c->q[(size_t)n * c->K + k] - (int)c->zp[(size_t)n * G + g]);
      wrow[k] = c->round_w ? (double)or_bf16_to_f32(or_f32_to_bf16(d * sc)) : (double)d * (double)sc;
    }
    for (int m = 0; m < c->M; ++m) {
      const uint16_t* xr = c->x + (size_t)m * c->K;
      double acc = 0.0;
      for (int k = 0; k < c->K; ++k) acc += wrow[k] * (double)or_bf16_to_f32(xr[k]);
      c->y[(size_t)m * c->N + n] = acc;
    }
  }
  free(wrow);
}

void or_matmul_f64(const uint16_t* x, int M, const uint8_t* q, const uint8_t* zp,
                   const uint16_t* s, int N, int K, int group, double* y, int nthreads) {
  mm_ctx c = {x, M, q, zp, s, N, K, group, 0, y};
  parallel_for(N, nthreads, mm_rows, &c);
}

void or_matmul_bf16w_f64(const uint16_t* x, int M, const uint8_t* q, const uint8_t* zp,
                         const uint16_t* s, int N, int K, int group, double* y,
                         int nthreads) {
  mm_ctx c = {x, M, q, zp, s, N, K, group, 1, y};
  parallel_for(N, nthreads, mm_rows, &c);
}

/* ------------------------------------------------------------------ W8A16 */
/* src/kernels/gemv_w4a16.cu:478-495 (k_quant_w8). */
void or_w8_quantize(const uint16_t* w, int N, int K, int group, int8_t* q, uint16_t* s) {
  const int G = K / group;
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < G; ++g) {
      const uint16_t* src = w + (size_t)n * K + (size_t)g * group;
      float mx = 0.f;
      for (int i = 0; i < group; ++i) mx = fmaxf(mx, fabsf(or_bf16_to_f32(src[i])));
      const float sc = mx / 127.0f;
      const float inv = mx > 0.f ? 127.0f / mx : 0.f;
      s[(size_t)n * G + g] = or_f32_to_bf16(sc);
      for (int i = 0; i < group; ++i) {
        const float prod = or_bf16_to_f32(src[i]) * inv;
        int v = (int)rintf(prod);
        v = v < -127 ? -127 : (v > 127 ? 127 : v);
        q[(size_t)n * K + (size_t)g * group + i] = (int8_t)v;
      }
    }
}

/* The reference's INT4 g128 lm_head quantizer, k_quant_i4
 * (src/model/model.cu:140-172), over a bf16 [N][K] matrix, writing the
 * compressed-tensors (A0) tensors awq_repack takes (model.cu:176-183):
 * packed [N][K/8] (element e of a word at bits 4e), bf16 scale [N][G],
 * zero points [N/8][G] (row r at bits 4 (r % 8) of word (r / 8, g)), all
 * nibbles 0..15 (w = (q - z) s). fp32 arithmetic as the reference's CUDA:
 * IEEE division, rintf (round half even) for __float2int_rn. */
void or_quant_i4(const uint16_t* w, int N, int K, int group, uint32_t* packed, uint16_t* scale,
                 uint32_t* zp) {
  const int G = K / group;
  memset(zp, 0, (size_t)(N / 8) * G * 4);
  for (int r = 0; r < N; ++r)
    for (int g = 0; g < G; ++g) {
      const uint16_t* src = w + (size_t)r * K + (size_t)g * group;
      float lo = 1e30f, hi = -1e30f;
      for (int i = 0; i < group; ++i) {
        const float v = or_bf16_to_f32(src[i]);
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      }
      float s = (hi - lo) / 15.0f;
      if (!(s > 0.f)) s = 1e-8f;
      int z = (int)rintf(-lo / s);
      z = z < 0 ? 0 : (z > 15 ? 15 : z);
      scale[(size_t)r * G + g] = or_f32_to_bf16(s);
      zp[(size_t)(r >> 3) * G + g] |= (uint32_t)z << ((r & 7) * 4);
      const float inv = 1.0f / s;
      for (int i = 0; i < group; i += 8) {
        uint32_t word = 0;
        for (int k = 0; k < 8; ++k) {
          int q = (int)rintf(or_bf16_to_f32(src[i + k]) * inv) + z;
          q = q < 0 ? 0 : (q > 15 ? 15 : q);
          word |= (uint32_t)q << (4 * k);
        }
        packed[(size_t)r * (K / 8) + ((size_t)g * group + i) / 8] = word;
      }
    }
}

typedef struct {
  const uint16_t* x;
  int M;
  const int8_t* q;
  const uint16_t* s;
  int N, K, group;
  double* y;
} mm8_ctx;

static void mm8_rows(void* p, int lo, int hi) {
  const mm8_ctx* c = (const mm8_ctx*)p;
  const int G = c->K / c->group;
  for (int n = lo; n < hi; ++n)
    for (int m = 0; m < c->M; ++m) {
      const uint16_t* xr = c->x + (size_t)m * c->K;
      double acc = 0.0;
      for (int k = 0; k < c->K; ++k)
        acc += (double)c->q[(size_t)n * c->K + k] *
               (double)or_bf16_to_f32(c->s[(size_t)n * G + k / c->group]) *
               (double)or_bf16_to_f32(xr[k]);
      c->y[(size_t)m * c->N + n] = acc;
    }
}

void or_w8_matmul_f64(const uint16_t* x, int M, const int8_t* q, const uint16_t* s, int N,
                      int K, int group, double* y, int nthreads) {
  mm8_ctx c = {x, M, q, s, N, K, group, y};
  parallel_for(N, nthreads, mm8_rows, &c);
}

/* ------------------------------------------------------------ CPU baseline */
typedef struct {
  const uint16_t* x;
  int M;
  const uint32_t* packed;
  const uint16_t* scale;
  const uint32_t* zpw;
  int N, K, group;
  uint16_t* y;
  const float* xf;
} cpu_ctx;

/* gate_gemm.cu:73-90 restated with fp32 accumulation and all rows: per output row,
 * unpack each nibble from the A0 words (w4a16_unpack.h:25-42), dequantize in fp32
 * and accumulate against the bf16 activation rows. */
static void cpu_rows(void* p, int lo, int hi) {
  const cpu_ctx* c = (const cpu_ctx*)p;
  const int G = c->K / c->group, W = c->K / 8;
  float* wrow = (float*)malloc(sizeof(float) * (size_t)c->K);
  for (int n = lo; n < hi; ++n) {
    const uint32_t* pr = c->packed + (size_t)n * W;
    for (int g = 0; g < G; ++g) {
      const float sc = or_bf16_to_f32(c->scale[(size_t)n * G + g]);
      const int z = or_ct_zp(c->zpw, G, n, g);
      for (int k = g * c->group; k < (g + 1) * c->group; ++k) {
        const int qv = (int)((pr[k >> 3] >> ((k & 7) * 4)) & 0xFu) - 8;
        wrow[k] = (float)(qv - z) * sc;
      }
    }
    for (int m = 0; m < c->M; ++m) {
      const float* xr = c->xf + (size_t)m * c->K;
      float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
      for (int k = 0; k < c->K; k += 4) {
        a0 += wrow[k] * xr[k];
        a1 += wrow[k + 1] * xr[k + 1];
        a2 += wrow[k + 2] * xr[k + 2];
        a3 += wrow[k + 3] * xr[k + 3];
      }
      c->y[(size_t)m * c->N + n] = or_f32_to_bf16((a0 + a1) + (a2 + a3));
    }
  }
  free(wrow);
}

int or_cpu_w4a16_matmul(const uint16_t* x, int M, const uint32_t* packed,
                        const uint16_t* scale, const uint32_t* zpw, int N, int K,
                        int group, uint16_t* y, int nthreads) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
  for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = or_bf16_to_f32(x[i]);
  cpu_ctx c = {x, M, packed, scale, zpw, N, K, group, y, xf};
  const int used = parallel_for(N, nthreads, cpu_rows, &c);
  free(xf);
  return used;
}

/* ---------------------------------------------------------------- argmax */
/* elementwise.cu:103-104: strict '>' keeps the lowest index on ties. */
void or_argmax_rows_f64(const double* v, int rows, int n, int32_t* idx, double* margin) {
  for (int r = 0; r < rows; ++r) {
    const double* p = v + (size_t)r * n;
    int bi = 0;
    double best = p[0];
    for (int i = 1; i < n; ++i)
      if (p[i] > best) { best = p[i]; bi = i; }
    double second = -INFINITY;
    for (int i = 0; i < n; ++i)
      if (i != bi && p[i] > second) second = p[i];
    idx[r] = bi;
    if (margin) margin[r] = best - second;
  }
}

void or_argmax_rows_f32(const float* v, int rows, int n, int32_t* idx) {
  for (int r = 0; r < rows; ++r) {
    const float* p = v + (size_t)r * n;
    int bi = 0;
    float best = p[0];
    for (int i = 1; i < n; ++i)
      if (p[i] > best) { best = p[i]; bi = i; }
    idx[r] = bi;
  }
}

void or_argmax_rows_bf16(const uint16_t* v, int rows, int n, int32_t* idx) {
  for (int r = 0; r < rows; ++r) {
    const uint16_t* p = v + (size_t)r * n;
    int bi = 0;
    float best = or_bf16_to_f32(p[0]);
    for (int i = 1; i < n; ++i) {
      const float f = or_bf16_to_f32(p[i]);
      if (f > best) { best = f; bi = i; }
    }
    idx[r] = bi;
  }
}
