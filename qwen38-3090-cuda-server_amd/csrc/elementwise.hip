// The elementwise steps either side of the W4A16 projections in the
// reference's layer (src/kernels/elementwise.cuh:8-22, .cu:8-49): rmsnorm
// before qkv / gate|up, swiglu after gate|up, residual_add after o / down.
// The decode kernels can fuse each of them (qw4_gemv_rmsnorm / _swiglu /
// _residual); these stand-alone forms serve larger M and callers that keep
// the steps apart. Data are bf16 [rows][dim]; 16-byte chunks of 8 elements.
//
// rmsnorm sums the squares of a row in the order every form shares
// (norm_sumsq: 1024 virtual threads, butterflies per virtual wave, the wave
// sums in order), so it agrees with the fused qw4_gemv_rmsnorm bit for bit.
#include <hip/hip_runtime.h>

#include "../../include/qwen_w4a16.h"
#include "w4a16_common.h"

namespace qw4 {
namespace {

constexpr int kEwThreads = 256;

__global__ __launch_bounds__(kEwThreads) void k_rmsnorm(uint16_t* __restrict__ out,
                                                        const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w,
                                                        int dim, float eps) {
  // thread t stands for the virtual threads t + 256 k of the shared order
  // (norm_sumsq): virtual wave wave + 4 k
  constexpr int kPer = kNormVThreads / kEwThreads;
  const int row = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kc = dim / 8;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (size_t)row * dim);
  __shared__ float vsum[kNormVWaves];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    float ss = 0.f;
    for (int i = threadIdx.x + kEwThreads * k; i < kc; i += kNormVThreads) ss = norm_sumsq(ss, xr[i]);
    ss = norm_wave_sum(ss);
    if (lane == 0) vsum[wave + (kEwThreads / 64) * k] = ss;
  }
  __syncthreads();
  const float inv = norm_inv(vsum, dim, eps);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  u32x4* orow = reinterpret_cast<u32x4*>(out + (size_t)row * dim);
  for (int i = threadIdx.x; i < kc; i += kEwThreads) {
    const u32x4 v = xr[i], g = wr[i];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(rmsnorm_f32(v[e], g[e], inv), rmsnorm_f32(v[e] >> 16, g[e] >> 16, inv));
    orow[i] = o;
  }
}

// out[i] = bf16(out[i] + x[i])
__global__ __launch_bounds__(kEwThreads) void k_residual_add(uint16_t* __restrict__ out,
                                                             const uint16_t* __restrict__ x,
                                                             size_t n) {
  const size_t n8 = n / 8;
  const size_t stride = (size_t)gridDim.x * kEwThreads;
  for (size_t i = (size_t)blockIdx.x * kEwThreads + threadIdx.x; i < n8; i += stride) {
    u32x4 a = reinterpret_cast<const u32x4*>(out)[i];
    const u32x4 b = reinterpret_cast<const u32x4*>(x)[i];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      a[e] = pack_bf16x2(bf16_bits_to_f32(a[e] & 0xffffu) + bf16_bits_to_f32(b[e] & 0xffffu),
                         bf16_bits_to_f32(a[e] >> 16) + bf16_bits_to_f32(b[e] >> 16));
    reinterpret_cast<u32x4*>(out)[i] = a;
  }
  // tail (n % 8 elements): the first threads of block 0
  const size_t t = n8 * 8 + threadIdx.x;
  if (blockIdx.x == 0 && t < n)
    out[t] = to_bf16(bf16_bits_to_f32(out[t]) + bf16_bits_to_f32(x[t]));
}

// out[r][i] = bf16(silu(fused[r][i]) * fused[r][inter + i])
__global__ __launch_bounds__(kEwThreads) void k_swiglu(uint16_t* __restrict__ out,
                                                       const uint16_t* __restrict__ fused,
                                                       int inter) {
  const int row = blockIdx.y;
  const int kc = inter / 8;
  const u32x4* g = reinterpret_cast<const u32x4*>(fused + (size_t)row * 2 * inter);
  const u32x4* u = g + kc;
  u32x4* o = reinterpret_cast<u32x4*>(out + (size_t)row * inter);
  for (int i = blockIdx.x * kEwThreads + threadIdx.x; i < kc; i += gridDim.x * kEwThreads) {
    const u32x4 a = g[i], b = u[i];
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      r[e] = (uint32_t)swiglu_bf16_bits(a[e], b[e]) |
             ((uint32_t)swiglu_bf16_bits(a[e] >> 16, b[e] >> 16) << 16);
    o[i] = r;
  }
}

}  // namespace
}  // namespace qw4

using namespace qw4;

extern "C" {

int qw4_rmsnorm(uint16_t* out, const uint16_t* x, const uint16_t* w, int rows, int dim,
                float eps, void* stream) {
  if (!out || !x || !w) return QW4_ERR_NULL;
  if (rows < 0 || dim <= 0 || dim % 8) return QW4_ERR_SHAPE;
  if (((uintptr_t)out | (uintptr_t)x | (uintptr_t)w) & 15) return QW4_ERR_ALIGN;
  if (rows == 0) return QW4_OK;
  k_rmsnorm<<<rows, kEwThreads, 0, (hipStream_t)stream>>>(out, x, w, dim, eps);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

int qw4_residual_add(uint16_t* out, const uint16_t* x, size_t n, void* stream) {
  if (!out || !x) return QW4_ERR_NULL;
  if (((uintptr_t)out | (uintptr_t)x) & 15) return QW4_ERR_ALIGN;
  if (n == 0) return QW4_OK;
  const size_t blocks = std::max<size_t>(1, std::min<size_t>((n / 8 + kEwThreads - 1) / kEwThreads, 4096));
  k_residual_add<<<(unsigned)blocks, kEwThreads, 0, (hipStream_t)stream>>>(out, x, n);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

int qw4_swiglu(uint16_t* out, const uint16_t* fused, int rows, int inter, void* stream) {
  if (!out || !fused) return QW4_ERR_NULL;
  if (rows < 0 || inter <= 0 || inter % 8 || rows > 65535) return QW4_ERR_SHAPE;
  if (((uintptr_t)out | (uintptr_t)fused) & 15) return QW4_ERR_ALIGN;
  if (rows == 0) return QW4_OK;
  const int bx = std::min(64, (inter / 8 + kEwThreads - 1) / kEwThreads);
  k_swiglu<<<dim3(bx, rows), kEwThreads, 0, (hipStream_t)stream>>>(out, fused, inter);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

}  // extern "C"
