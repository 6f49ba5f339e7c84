// Shared definitions of the gfx950 W4A16 library: the repacked weight layout,
// vector types and the nibble -> bf16 conversion every kernel uses.
//
// Repacked layout (one "tile" = 64 output rows, one "group" = 128 inputs):
//
//   qweight u32 [N/64][G][4 j][64 p][4 w]          (4 KiB per (tile, group))
//       position p of a tile holds row  n = 4*(p % 16) + p / 16,
//       word w of chunk j covers k = 128*g + 32*j + 8*w + e, e = 0..7,
//       element e sits in nibble slot (e % 2) * 4 + e / 2.
//   scale   u16  [N/64][G][80]        per (tile, group) one 160-byte record: the
//                                     64 bf16 scales in natural row order, then
//                                     a copy of the block's 16 zero-point words
//   zeros   u16  [N/64][G][16]        u16 c holds rows 4c..4c+3, row 4c+t at bits 4t
//
// Why this shape:
//   * nibble slot order: ((w >> 4p) & 0x000F000F) | 0x43004300 is the bf16 pair
//     (128 + q[2p], 128 + q[2p+1]) -- exact, since bf16 has ulp 1 on [128, 256) --
//     so four AND-OR operations (three after shifts) turn one word into the 8
//     consecutive-k bf16 operand of an MFMA, with no activation permutation.
//   * position order: a wave loading 16-byte chunk j of positions 16*st + c
//     (c = lane % 16) reads 256 contiguous bytes and gets rows 4c + st, so after
//     the four st loads each lane owns four consecutive rows: its scales are one
//     8-byte load, its zero points one u16, its outputs one 8-byte store.
//   * the (tile, group) block is 4 KiB contiguous: the decode kernels stream
//     it with 16-byte loads and the prefill GEMM stages it into LDS unchanged.
//   * scales and zero points of a block sit in one 160-byte record, so the
//     decode GEMV fetches both with one load per item (the zero points are
//     also kept on their own for the other kernels).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qwen_w4a16.h"

namespace qw4 {

constexpr int kTileN = 64;          // output rows per tile
constexpr int kGroup = 128;         // inputs per quantization group
constexpr int kWordsPerBlock = 1024;  // u32 words per (tile, group)
constexpr int kMetaU16 = 80;        // u16 per (tile, group) in the 4-bit scale array
constexpr int kMetaBytes = 2 * kMetaU16;
static_assert(kTileN == QW4_TILE_ROWS && kMetaBytes == QW4_META_BYTES,
              "the public layout sizes in qwen_w4a16.h");

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Row n of a tile <-> storage position p.
__host__ __device__ inline int tile_pos_of_row(int r) { return 16 * (r & 3) + (r >> 2); }
__host__ __device__ inline int tile_row_of_pos(int p) { return 4 * (p & 15) + (p >> 4); }
// Element e of a word <-> nibble slot.
__host__ __device__ inline int slot_of_elem(int e) { return (e & 1) * 4 + (e >> 1); }

// Nibble-unpack constants held in VGPRs. gfx9-family VOP3 encodings take at
// most one scalar/literal operand, so with both constants as literals the
// compiler emits v_and + v_or per pair; with the constants in opaque VGPRs
// (materialized once, hoisted out of loops) it selects one v_and_or_b32.
// Only the materialization is asm; the arithmetic stays visible to the
// compiler, which inserts the VALU -> MFMA wait states itself.
struct NibConst {
  uint32_t mask, magic;
};
__device__ __forceinline__ NibConst nib_const() {
  NibConst c;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(c.mask));
  asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(c.magic));
  return c;
}

// One packed word -> 8 bf16 values 128 + q, elements 0..7 in order.
__device__ __forceinline__ u32x4 nib8_bits(uint32_t w, NibConst k) {
  u32x4 r;
  r[0] = (w & k.mask) | k.magic;
  r[1] = ((w >> 4) & k.mask) | k.magic;
  r[2] = ((w >> 8) & k.mask) | k.magic;
  r[3] = ((w >> 12) & k.mask) | k.magic;
  return r;
}

__device__ __forceinline__ bf16x8 nib8(uint32_t w, NibConst k) {
  return __builtin_bit_cast(bf16x8, nib8_bits(w, k));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Round-to-nearest-even fp32 -> bf16 for a pair (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint16_t to_bf16(float f) {
  return (uint16_t)(pack_bf16x2(f, 0.f) & 0xffffu);
}

// bf16(silu(g) * u) for bf16 g, u: silu(g) = g / (1 + exp(-g)) in fp32, the
// reference's k_swiglu (src/kernels/elementwise.cu:40-49).
__device__ __forceinline__ uint16_t swiglu_bf16_bits(uint32_t g, uint32_t u) {
  const float gf = bf16_bits_to_f32(g & 0xffffu), uf = bf16_bits_to_f32(u & 0xffffu);
  return to_bf16((gf / (1.f + expf(-gf))) * uf);
}

// rmsnorm's sum of squares (src/kernels/elementwise.cu:8-31 sums x^2 in
// fp32). Every rmsnorm form here -- stand-alone and fused into the GEMVs --
// uses this one order, so that they agree bit for bit, and it spreads over a
// whole workgroup: 1024 virtual threads; virtual thread v adds the 16-byte
// chunks v, v + 1024, ... of the row in order (each chunk's words in order,
// each word as s + (lo*lo + hi*hi), every operation rounded once); each run of
// 64 virtual threads (a virtual wave) reduces with a butterfly (xor 32, 16, 8,
// 4, 2, 1); the 16 virtual-wave sums are added in order.
constexpr int kNormVThreads = 1024;
constexpr int kNormVWaves = kNormVThreads / 64;

__device__ __forceinline__ float norm_sumsq(float s, const u32x4& v) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __uint_as_float(v[e] << 16), hi = __uint_as_float(v[e] & 0xffff0000u);
    s = __fadd_rn(s, __fadd_rn(__fmul_rn(lo, lo), __fmul_rn(hi, hi)));
  }
  return s;
}

__device__ __forceinline__ float norm_wave_sum(float s) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s = __fadd_rn(s, __shfl_xor(s, off, 64));
  return s;
}

// 1 / rms from the 16 virtual-wave sums (in LDS or registers, in order).
__device__ __forceinline__ float norm_inv(const float* vwave, int dim, float eps) {
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kNormVWaves; ++i) t = __fadd_rn(t, vwave[i]);
  return rsqrtf(t / (float)dim + eps);
}

// bf16(x * inv * (1 + w)) for bf16 x, w: the rmsnorm output rounding of the
// reference's k_rmsnorm (src/kernels/elementwise.cu:29-30).
__device__ __forceinline__ float rmsnorm_f32(uint32_t x, uint32_t w, float inv) {
  return bf16_bits_to_f32(x & 0xffffu) * inv * (1.0f + bf16_bits_to_f32(w & 0xffffu));
}

}  // namespace qw4

// Host-side helpers shared by the C-ABI translation units.
namespace qw4 {
void set_hip_error(int e);
}
#define QW4_LAUNCH_CHECK()                                   \
  do {                                                       \
    hipError_t e_ = hipGetLastError();                       \
    if (e_ != hipSuccess) {                                  \
      qw4::set_hip_error((int)e_);                           \
      return QW4_ERR_HIP;                                    \
    }                                                        \
  } while (0)
