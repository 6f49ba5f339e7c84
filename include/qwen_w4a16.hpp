// qwen_w4a16.hpp -- call-compatible C++ layer over the C-ABI (qwen_w4a16.h).
//
// The declarations keep the names, argument order and meaning of the
// reference's namespace qwen entry points so its callers drop in with the type
// substitutions __nv_bfloat16 -> __hip_bfloat16 (bit-identical) and
// cudaStream_t -> hipStream_t:
//   src/kernels/gemv_w4a16.cuh:50-135, :187-188   (W4A16 GEMV / skinny / MMA)
//   src/kernels/gemv_w4a16.cuh:147-166             (W8A16 lm_head)
//   src/kernels/gemm_w4a16.cuh:30-48              (prefill GEMM, dequant rows)
//   src/kernels/elementwise.cuh:39-43              (argmax, argmax_rows)
// Like the reference, these print a message and abort() on invalid input; the
// C-ABI underneath returns status codes instead.
//
// Differences callers may observe (none changes a documented result):
//   * W4A16Weights' device layout is private and differs (tile-major, 4-bit
//     zero points); qweight / scale / zp are still three separate hipMalloc
//     allocations, each freeable with hipFree.
//   * GemvScratch holds split-K state instead of widened activations; its
//     public fields max_m and partial_elems keep their meaning.
//   * GemmWorkspace holds no BLAS handle and no dequantized weights: the prefill
//     GEMM is one fused kernel; a workspace of >= 2 x CUs x 256 KiB lets it
//     split tiles across workgroups (their fp32 partials live there).
//   * group_size must be 128; out_f % 64 == 0 and in_f % 128 == 0.
#pragma once
#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qwen_w4a16.h"

namespace qwen {

struct W4A16Weights {
  uint32_t* qweight = nullptr;
  __hip_bfloat16* scale = nullptr;
  uint8_t* zp = nullptr;   // 4-bit zero points, 4 rows per 16-bit word
  int out_f = 0, in_f = 0, group_size = 0, num_groups = 0;

  size_t qweight_bytes() const { return size_t(out_f) * in_f / 2; }
  // per (64-row tile, group) one record: 64 bf16 scales + 16 zero-point words
  size_t scale_bytes() const {
    return size_t(out_f) / QW4_TILE_ROWS * num_groups * QW4_META_BYTES;
  }
  size_t zp_bytes() const { return size_t(out_f) * num_groups / 2; }
  size_t total_bytes() const { return qweight_bytes() + scale_bytes() + zp_bytes(); }
};

// awq_repack (gemv_w4a16.cuh:70-75): compressed-tensors source tensors.
void awq_repack(W4A16Weights& dst, const uint32_t* src_packed, const __hip_bfloat16* src_scale,
                const uint32_t* src_zp, int out_f, int in_f, int group_size,
                hipStream_t stream = 0);
void awq_alloc_fused(W4A16Weights& dst, int total_out_f, int in_f, int group_size,
                     hipStream_t stream = 0);
void awq_repack_into(W4A16Weights& dst, int dst_row_offset, const uint32_t* src_packed,
                     const __hip_bfloat16* src_scale, const uint32_t* src_zp, int out_f,
                     hipStream_t stream = 0);
// AWQ-order sources (layout QW4_LAYOUT_AWQ_K or QW4_LAYOUT_AWQ_N); no reference
// counterpart.
void awq_repack_awq_into(W4A16Weights& dst, int dst_row_offset, const uint32_t* qweight,
                         const __hip_bfloat16* scales, const uint32_t* zeros, int out_f,
                         int layout, hipStream_t stream = 0);
void awq_free(W4A16Weights& w);

struct GemvScratch {
  float* partial = nullptr;   // split-K accumulation area (partial_elems floats)
  size_t partial_elems = 0;
  int max_in = 0, max_out = 0, max_m = 1;
  qw4_scratch impl{};         // the C-ABI scratch these fields mirror
};

void gemv_scratch_alloc(GemvScratch& s, int max_in, int max_out, int min_group, int max_m = 1);
void gemv_scratch_free(GemvScratch& s);
void gemv_partial_check(const GemvScratch& s, int splits, int out_f, int M);
size_t gemv_scratch_bytes_for_m(const GemvScratch& s, int max_m);

void gemm_small_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                      GemvScratch& s, hipStream_t stream = 0);
void gemv_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x,
                GemvScratch& s, hipStream_t stream = 0);
void gemv_w4a16_f32(float* y, const W4A16Weights& w, const __hip_bfloat16* x, GemvScratch& s,
                    hipStream_t stream = 0);
int gemv_choose_splits(int out_f, int num_groups);
void gemm_mma_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                    GemvScratch& s, hipStream_t stream = 0);
// lm_head GEMV + fused fp32 row-argmax (head() + argmax, model.cu:796-815).
void gemv_argmax_w4a16(int32_t* idx, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                       GemvScratch& s, hipStream_t stream = 0);

// W8A16Weights (gemv_w4a16.cuh:147-154): 8-bit lm_head weights. The device
// layout is private (64-row tiles, q + 128 bytes); qweight and scale are two
// separate hipMalloc allocations; total_bytes() keeps the reference's formula.
struct W8A16Weights {
  int8_t* qweight = nullptr;
  __hip_bfloat16* scale = nullptr;
  int out_f = 0, in_f = 0, group_size = 0, num_groups = 0;
  size_t total_bytes() const {
    return size_t(out_f) * in_f + size_t(out_f) * num_groups * 2;
  }
};

void quantize_w8a16(W8A16Weights& dst, const __hip_bfloat16* src, int out_f, int in_f,
                    int group_size, hipStream_t stream = 0);
// quantize_w4a16_raw (src/model/model.cu:174-186): the INT4 g128 lm_head
// quantizer, straight into the repacked layout (no host sync).
void quantize_w4a16_raw(W4A16Weights& dst, const __hip_bfloat16* src, int rows, int cols,
                        int group, hipStream_t stream = 0);
void gemv_w8a16(__hip_bfloat16* y, const W8A16Weights& w, const __hip_bfloat16* x,
                GemvScratch& s, hipStream_t stream = 0);
void gemm_small_w8a16(__hip_bfloat16* y, const W8A16Weights& w, const __hip_bfloat16* x,
                      int M, GemvScratch& s, hipStream_t stream = 0);
void w8a16_free(W8A16Weights& w);
// 8-bit lm_head + fused fp32 row-argmax (head() with lm_head_bits 8,
// model.cu:796-815); no reference counterpart as one call.
void gemv_argmax_w8a16(int32_t* idx, const W8A16Weights& w, const __hip_bfloat16* x, int M,
                       GemvScratch& s, hipStream_t stream = 0);
void w8a16_dequant_rows(__hip_bfloat16* dst, const W8A16Weights& w, int row0, int nrows,
                        hipStream_t stream = 0);

struct GemmWorkspace {
  __hip_bfloat16* wbuf = nullptr;
  size_t bytes = 0;
  int max_rows = 0;
};

void gemm_workspace_alloc(GemmWorkspace& ws, size_t bytes);
void gemm_workspace_free(GemmWorkspace& ws);
void gemm_w4a16(__hip_bfloat16* C, const W4A16Weights& w, const __hip_bfloat16* A, int M,
                GemmWorkspace& ws, hipStream_t stream = 0);
void w4a16_dequant_rows(__hip_bfloat16* dst, const W4A16Weights& w, int row0, int nrows,
                        hipStream_t stream = 0);

void argmax(int32_t* out, const __hip_bfloat16* x, int n, int32_t* scratch,
            hipStream_t stream = 0);
void argmax_rows(int32_t* out, const __hip_bfloat16* x, int rows, int n, hipStream_t stream = 0);

// The layer steps either side of the projections (src/kernels/elementwise.cuh:8-22).
void rmsnorm(__hip_bfloat16* out, const __hip_bfloat16* x, const __hip_bfloat16* w, int rows,
             int dim, float eps, hipStream_t stream = 0);
void residual_add(__hip_bfloat16* out, const __hip_bfloat16* x, int n, hipStream_t stream = 0);
void swiglu(__hip_bfloat16* out, const __hip_bfloat16* fused, int rows, int inter,
            hipStream_t stream = 0);

// The same steps fused into the decode / verify GEMV, 1 <= M <= 16 (no
// reference counterparts: the reference runs them as separate kernels around
// linear(), src/model/model.cu:697-700, :772-785).
//   h = bf16(h + bf16(x @ W^T))                         (linear + residual_add)
void gemv_w4a16_residual(__hip_bfloat16* h, const W4A16Weights& w, const __hip_bfloat16* x,
                         int M, GemvScratch& s, hipStream_t stream = 0);
//   y = swiglu(x @ [gate | up]^T), y [M][out_f / 2]; tmp [M][out_f] (or
//   nullptr) carries the projection for M > 2     (linear + swiglu)
void gemv_w4a16_swiglu(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                       __hip_bfloat16* tmp, GemvScratch& s, hipStream_t stream = 0);
//   y = rmsnorm(h) @ W^T; tmp [M][in_f] is used when the rows do not fit the
//   kernel's staging (may be nullptr otherwise)       (rmsnorm + linear)
void gemv_w4a16_rmsnorm(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* h,
                        const __hip_bfloat16* norm_w, float eps, int M, __hip_bfloat16* tmp,
                        GemvScratch& s, hipStream_t stream = 0);

// linear() with lin_path() (src/model/model.cu:522-565, :643-658) over T rows.
void linear_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int T,
                  GemvScratch& s, GemmWorkspace& ws, hipStream_t stream = 0);

}  // namespace qwen
