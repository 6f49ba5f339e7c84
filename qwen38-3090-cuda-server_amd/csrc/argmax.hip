// Row argmax over bf16 logits, lowest index on ties -- the call-compatible
// counterparts of argmax / argmax_rows (src/kernels/elementwise.cu:96-158,
// :184-194). The lm_head path itself uses the fused fp32 argmax of the skinny
// kernel; these serve callers that already hold bf16 logits.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "../../include/qwen_w4a16.h"
#include "w4a16_common.h"

namespace qw4 {
namespace {

__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

// Block-wide (256 threads) reduction of (value, index) pairs.
__device__ __forceinline__ void block_best(float& v, int& i) {
  __shared__ float sv[4];
  __shared__ int si[4];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) better(v, i, __shfl_xor(v, off, 64), __shfl_xor(i, off, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sv[wave] = v; si[wave] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) better(v, i, sv[w], si[w]);
  }
}

__device__ __forceinline__ float ldbf(const uint16_t* p) { return bf16_bits_to_f32(*p); }

// Same semantics as the reference's kernels: each thread starts from
// (-FLT_MAX, 0) and takes a value only if strictly greater, so the lowest index
// wins ties and values never above -FLT_MAX (or NaN) leave index 0.
__global__ __launch_bounds__(256) void k_argmax_rows(int32_t* out, const uint16_t* x, int n) {
  const uint16_t* row = x + (size_t)blockIdx.x * n;
  float v = -FLT_MAX;
  int i = 0;
  for (int k = threadIdx.x; k < n; k += 256) {
    const float f = ldbf(row + k);
    if (f > v) { v = f; i = k; }
  }
  block_best(v, i);
  if (threadIdx.x == 0) out[blockIdx.x] = i;
}

__global__ __launch_bounds__(256) void k_argmax_partial(int32_t* idx, float* val,
                                                        const uint16_t* x, int n) {
  float v = -FLT_MAX;
  int i = 0;
  for (int k = blockIdx.x * 256 + threadIdx.x; k < n; k += gridDim.x * 256) {
    const float f = ldbf(x + k);
    if (f > v) { v = f; i = k; }
  }
  block_best(v, i);
  if (threadIdx.x == 0) { idx[blockIdx.x] = i; val[blockIdx.x] = v; }
}

__global__ __launch_bounds__(256) void k_argmax_final(int32_t* out, const int32_t* idx,
                                                      const float* val, int chunks) {
  float v = -FLT_MAX;
  int i = 0;
  for (int k = threadIdx.x; k < chunks; k += 256) better(v, i, val[k], idx[k]);
  block_best(v, i);
  if (threadIdx.x == 0) out[0] = i;
}

}  // namespace
}  // namespace qw4

using namespace qw4;

extern "C" {

int qw4_argmax(int32_t* out, const uint16_t* x, int n, int32_t* scratch, void* stream) {
  if (!out || !x || !scratch) return QW4_ERR_NULL;
  if (n <= 0) return QW4_ERR_SHAPE;
  const int chunks = 256;
  int32_t* idx = scratch;
  float* val = reinterpret_cast<float*>(scratch + chunks);
  hipStream_t hs = (hipStream_t)stream;
  k_argmax_partial<<<chunks, 256, 0, hs>>>(idx, val, x, n);
  k_argmax_final<<<1, 256, 0, hs>>>(out, idx, val, chunks);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

int qw4_argmax_rows(int32_t* out, const uint16_t* x, int rows, int n, void* stream) {
  if (!out || !x) return QW4_ERR_NULL;
  if (rows < 0 || n <= 0) return QW4_ERR_SHAPE;
  if (rows == 0) return QW4_OK;
  k_argmax_rows<<<rows, 256, 0, (hipStream_t)stream>>>(out, x, n);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

}  // extern "C"
