// namespace qwen: the reference's C++ entry points (include/qwen_w4a16.hpp) as a
// thin layer over the C-ABI. A non-zero status prints a message and aborts, the
// reference's behaviour on bad input (src/kernels/gemv_w4a16.cu:359-366, :392,
// :429; src/kernels/gemm_w4a16.cu:9-10, :68).
#include <cstdio>
#include <cstdlib>

#include "../../include/qwen_w4a16.hpp"

namespace qwen {
namespace {

void check(int st, const char* where) {
  if (st == QW4_OK) return;
  std::fprintf(stderr, "qwen::%s: %s (status %d", where, qw4_status_string(st), st);
  if (st == QW4_ERR_HIP) std::fprintf(stderr, ", hipError %d", qw4_last_hip_error());
  std::fprintf(stderr, ")\n");
  std::abort();
}

qw4_weights view(const W4A16Weights& w) {
  qw4_weights v;
  v.qweight = w.qweight;
  v.scale = reinterpret_cast<uint16_t*>(w.scale);
  v.zeros = reinterpret_cast<uint16_t*>(w.zp);
  v.out_f = w.out_f;
  v.in_f = w.in_f;
  v.group_size = w.group_size;
  v.num_groups = w.num_groups;
  return v;
}

void adopt(W4A16Weights& w, const qw4_weights& v) {
  w.qweight = v.qweight;
  w.scale = reinterpret_cast<__hip_bfloat16*>(v.scale);
  w.zp = reinterpret_cast<uint8_t*>(v.zeros);
  w.out_f = v.out_f;
  w.in_f = v.in_f;
  w.group_size = v.group_size;
  w.num_groups = v.num_groups;
}

void mirror(GemvScratch& s) {
  s.partial = s.impl.partial;
  s.partial_elems = s.impl.partial_elems;
  s.max_in = s.impl.max_in;
  s.max_out = s.impl.max_out;
  s.max_m = s.impl.max_m;
}

qw4_w8_weights view8(const W8A16Weights& w) {
  qw4_w8_weights v;
  v.qweight = reinterpret_cast<uint8_t*>(w.qweight);
  v.scale = reinterpret_cast<uint16_t*>(w.scale);
  v.out_f = w.out_f;
  v.in_f = w.in_f;
  v.group_size = w.group_size;
  v.num_groups = w.num_groups;
  return v;
}

const uint16_t* u16(const __hip_bfloat16* p) { return reinterpret_cast<const uint16_t*>(p); }
uint16_t* u16(__hip_bfloat16* p) { return reinterpret_cast<uint16_t*>(p); }

}  // namespace

void awq_alloc_fused(W4A16Weights& dst, int total_out_f, int in_f, int group_size,
                     hipStream_t stream) {
  qw4_weights v{};
  check(qw4_weights_alloc(&v, total_out_f, in_f, group_size, stream), "awq_alloc_fused");
  adopt(dst, v);
}

void awq_repack_into(W4A16Weights& dst, int dst_row_offset, const uint32_t* src_packed,
                     const __hip_bfloat16* src_scale, const uint32_t* src_zp, int out_f,
                     hipStream_t stream) {
  qw4_weights v = view(dst);
  check(qw4_repack_ct_into(&v, dst_row_offset, src_packed, u16(src_scale), src_zp, out_f,
                           stream),
        "awq_repack_into");
}

void awq_repack(W4A16Weights& dst, const uint32_t* src_packed, const __hip_bfloat16* src_scale,
                const uint32_t* src_zp, int out_f, int in_f, int group_size,
                hipStream_t stream) {
  qw4_weights v{};
  check(qw4_repack_ct(&v, src_packed, u16(src_scale), src_zp, out_f, in_f, group_size, stream),
        "awq_repack");
  adopt(dst, v);
}

void awq_repack_awq_into(W4A16Weights& dst, int dst_row_offset, const uint32_t* qweight,
                         const __hip_bfloat16* scales, const uint32_t* zeros, int out_f,
                         int layout, hipStream_t stream) {
  qw4_weights v = view(dst);
  check(qw4_repack_awq_into(&v, dst_row_offset, qweight, u16(scales), zeros, out_f, layout,
                            stream),
        "awq_repack_awq_into");
}

void awq_free(W4A16Weights& w) {
  qw4_weights v = view(w);
  check(qw4_weights_free(&v), "awq_free");
  w = W4A16Weights{};
}

void gemv_scratch_alloc(GemvScratch& s, int max_in, int max_out, int min_group, int max_m) {
  check(qw4_scratch_alloc(&s.impl, max_in, max_out, min_group, max_m), "gemv_scratch_alloc");
  mirror(s);
}

void gemv_scratch_free(GemvScratch& s) {
  check(qw4_scratch_free(&s.impl), "gemv_scratch_free");
  s = GemvScratch{};
}

void gemv_partial_check(const GemvScratch& s, int splits, int out_f, int M) {
  check(qw4_partial_check(&s.impl, splits, out_f, M), "gemv_partial_check");
}

// Declared but never defined by the reference (gemv_w4a16.cuh:126): the device
// bytes a scratch of this shape holds for max_m rows.
size_t gemv_scratch_bytes_for_m(const GemvScratch& s, int max_m) {
  (void)max_m;
  return s.impl.partial_elems * sizeof(float);
}

void gemm_small_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                      GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemm_small(u16(y), &v, u16(x), M, &s.impl, stream), "gemm_small_w4a16");
}

void gemv_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x,
                GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemv(u16(y), &v, u16(x), &s.impl, stream), "gemv_w4a16");
}

void gemv_w4a16_f32(float* y, const W4A16Weights& w, const __hip_bfloat16* x, GemvScratch& s,
                    hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemv_f32(y, &v, u16(x), &s.impl, stream), "gemv_w4a16_f32");
}

int gemv_choose_splits(int out_f, int num_groups) { return qw4_choose_splits(out_f, num_groups); }

void gemm_mma_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                    GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemm_mma(u16(y), &v, u16(x), M, &s.impl, stream), "gemm_mma_w4a16");
}

void gemv_argmax_w4a16(int32_t* idx, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                       GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemv_argmax(idx, &v, u16(x), M, &s.impl, stream), "gemv_argmax_w4a16");
}

void quantize_w4a16_raw(W4A16Weights& dst, const __hip_bfloat16* src, int rows, int cols,
                        int group, hipStream_t stream) {
  qw4_weights v{};
  check(qw4_quantize_w4a16(&v, u16(src), rows, cols, group, stream), "quantize_w4a16_raw");
  adopt(dst, v);
}

void quantize_w8a16(W8A16Weights& dst, const __hip_bfloat16* src, int out_f, int in_f,
                    int group_size, hipStream_t stream) {
  qw4_w8_weights v{};
  check(qw4_w8_quantize(&v, u16(src), out_f, in_f, group_size, stream), "quantize_w8a16");
  dst.qweight = reinterpret_cast<int8_t*>(v.qweight);
  dst.scale = reinterpret_cast<__hip_bfloat16*>(v.scale);
  dst.out_f = v.out_f;
  dst.in_f = v.in_f;
  dst.group_size = v.group_size;
  dst.num_groups = v.num_groups;
}

void gemv_w8a16(__hip_bfloat16* y, const W8A16Weights& w, const __hip_bfloat16* x,
                GemvScratch& s, hipStream_t stream) {
  const qw4_w8_weights v = view8(w);
  check(qw4_w8_gemv(u16(y), &v, u16(x), &s.impl, stream), "gemv_w8a16");
}

void gemm_small_w8a16(__hip_bfloat16* y, const W8A16Weights& w, const __hip_bfloat16* x,
                      int M, GemvScratch& s, hipStream_t stream) {
  const qw4_w8_weights v = view8(w);
  check(qw4_w8_gemm_small(u16(y), &v, u16(x), M, &s.impl, stream), "gemm_small_w8a16");
}

void gemv_argmax_w8a16(int32_t* idx, const W8A16Weights& w, const __hip_bfloat16* x, int M,
                       GemvScratch& s, hipStream_t stream) {
  const qw4_w8_weights v = view8(w);
  check(qw4_w8_gemv_argmax(idx, &v, u16(x), M, &s.impl, stream), "gemv_argmax_w8a16");
}

void w8a16_dequant_rows(__hip_bfloat16* dst, const W8A16Weights& w, int row0, int nrows,
                        hipStream_t stream) {
  const qw4_w8_weights v = view8(w);
  check(qw4_w8_dequant_rows(u16(dst), &v, row0, nrows, stream), "w8a16_dequant_rows");
}

void w8a16_free(W8A16Weights& w) {
  qw4_w8_weights v = view8(w);
  check(qw4_w8_free(&v), "w8a16_free");
  w = W8A16Weights{};
}

void gemm_workspace_alloc(GemmWorkspace& ws, size_t bytes) {
  qw4_workspace q{};
  check(qw4_workspace_alloc(&q, bytes), "gemm_workspace_alloc");
  ws.wbuf = static_cast<__hip_bfloat16*>(q.buf);
  ws.bytes = q.bytes;
  ws.max_rows = 0;
}

void gemm_workspace_free(GemmWorkspace& ws) {
  qw4_workspace q{ws.wbuf, ws.bytes};
  check(qw4_workspace_free(&q), "gemm_workspace_free");
  ws = GemmWorkspace{};
}

void gemm_w4a16(__hip_bfloat16* C, const W4A16Weights& w, const __hip_bfloat16* A, int M,
                GemmWorkspace& ws, hipStream_t stream) {
  const qw4_weights v = view(w);
  qw4_workspace q{ws.wbuf, ws.bytes};
  check(qw4_gemm(u16(C), &v, u16(A), M, &q, stream), "gemm_w4a16");
}

void w4a16_dequant_rows(__hip_bfloat16* dst, const W4A16Weights& w, int row0, int nrows,
                        hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_dequant_rows(u16(dst), &v, row0, nrows, stream), "w4a16_dequant_rows");
}

void argmax(int32_t* out, const __hip_bfloat16* x, int n, int32_t* scratch, hipStream_t stream) {
  check(qw4_argmax(out, u16(x), n, scratch, stream), "argmax");
}

void argmax_rows(int32_t* out, const __hip_bfloat16* x, int rows, int n, hipStream_t stream) {
  check(qw4_argmax_rows(out, u16(x), rows, n, stream), "argmax_rows");
}

void rmsnorm(__hip_bfloat16* out, const __hip_bfloat16* x, const __hip_bfloat16* w, int rows,
             int dim, float eps, hipStream_t stream) {
  check(qw4_rmsnorm(u16(out), u16(x), u16(w), rows, dim, eps, stream), "rmsnorm");
}

void residual_add(__hip_bfloat16* out, const __hip_bfloat16* x, int n, hipStream_t stream) {
  check(n < 0 ? QW4_ERR_SHAPE : qw4_residual_add(u16(out), u16(x), (size_t)n, stream),
        "residual_add");
}

void swiglu(__hip_bfloat16* out, const __hip_bfloat16* fused, int rows, int inter,
            hipStream_t stream) {
  check(qw4_swiglu(u16(out), u16(fused), rows, inter, stream), "swiglu");
}

void gemv_w4a16_residual(__hip_bfloat16* h, const W4A16Weights& w, const __hip_bfloat16* x,
                         int M, GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemv_residual(u16(h), &v, u16(x), M, &s.impl, stream), "gemv_w4a16_residual");
}

void gemv_w4a16_swiglu(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int M,
                       __hip_bfloat16* tmp, GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemv_swiglu(u16(y), &v, u16(x), M, u16(tmp), &s.impl, stream), "gemv_w4a16_swiglu");
}

void gemv_w4a16_rmsnorm(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* h,
                        const __hip_bfloat16* norm_w, float eps, int M, __hip_bfloat16* tmp,
                        GemvScratch& s, hipStream_t stream) {
  const qw4_weights v = view(w);
  check(qw4_gemv_rmsnorm(u16(y), &v, u16(h), u16(norm_w), eps, M, u16(tmp), &s.impl, stream),
        "gemv_w4a16_rmsnorm");
}

void linear_w4a16(__hip_bfloat16* y, const W4A16Weights& w, const __hip_bfloat16* x, int T,
                  GemvScratch& s, GemmWorkspace& ws, hipStream_t stream) {
  const qw4_weights v = view(w);
  qw4_workspace q{ws.wbuf, ws.bytes};
  check(qw4_linear(u16(y), &v, u16(x), T, &s.impl, &q, stream), "linear_w4a16");
}

}  // namespace qwen
