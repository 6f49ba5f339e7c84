// Gate for the call-compatible namespace qwen layer, written the way the
// reference's gates are (tests/gate_gemv.cu, tests/gate_gemm.cu): build weights
// from compressed-tensors tensors with qwen::awq_repack, run the entry points a
// caller uses, and check them against the CPU oracle (fp64). Exit 0 = pass.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/qwen_w4a16.hpp"
#include "../../oracle/oracle.h"

#define CK(x)                                                                   \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      std::fprintf(stderr, "HIP %s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      return 2;                                                                 \
    }                                                                           \
  } while (0)

template <class T>
static T* upload(const std::vector<T>& h) {
  T* d = nullptr;
  if (hipMalloc(&d, h.size() * sizeof(T)) != hipSuccess) return nullptr;
  if (hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
  return d;
}

static double rel_err(const std::vector<double>& ref, const std::vector<float>& got) {
  double me = 0, mm = 0;
  for (size_t i = 0; i < ref.size(); ++i) {
    me = std::max(me, std::fabs(ref[i] - got[i]));
    mm = std::max(mm, std::fabs(ref[i]));
  }
  return mm > 0 ? me / mm : 0;
}

int main() {
  const int N = 512, K = 1024, G = K / 128;
  std::mt19937 rng(1234);
  // compressed-tensors pack-quantized tensors (src/loader/w4a16_unpack.h:1-18)
  std::vector<uint8_t> q((size_t)N * K), zp((size_t)N * G);
  std::vector<uint16_t> s((size_t)N * G);
  for (auto& v : q) v = rng() & 15;
  for (auto& v : zp) v = rng() & 15;
  std::normal_distribution<float> nd(0.f, 1.f);
  for (auto& v : s) v = or_f32_to_bf16(std::fabs(nd(rng) * 0.02f) + 1e-4f);
  std::vector<uint32_t> packed((size_t)N * K / 8), zpw((size_t)N / 8 * G);
  std::vector<uint16_t> scale((size_t)N * G);
  or_pack_ct(q.data(), zp.data(), s.data(), N, K, 128, packed.data(), scale.data(), zpw.data());

  uint32_t* d_packed = upload(packed);
  uint16_t* d_scale = upload(scale);
  uint32_t* d_zp = upload(zpw);
  if (!d_packed || !d_scale || !d_zp) return 2;

  qwen::W4A16Weights W;
  qwen::awq_repack(W, d_packed, reinterpret_cast<__hip_bfloat16*>(d_scale), d_zp, N, K, 128);
  CK(hipDeviceSynchronize());
  {   // the C++ size helpers agree with the library's allocation
    qw4_weights cw{W.qweight, reinterpret_cast<uint16_t*>(W.scale),
                   reinterpret_cast<uint16_t*>(W.zp), W.out_f, W.in_f, W.group_size,
                   W.num_groups};
    if (W.total_bytes() != qw4_weights_bytes(&cw)) {
      std::printf("FAIL total_bytes %zu vs qw4_weights_bytes %zu\n", W.total_bytes(),
                  qw4_weights_bytes(&cw));
      return 1;
    }
  }
  // the reference frees its sources right after the repack (model.cu:124-125)
  CK(hipFree(d_packed));
  CK(hipFree(d_scale));
  CK(hipFree(d_zp));

  qwen::GemvScratch S;
  qwen::gemv_scratch_alloc(S, K, N, 128, 16);
  int fails = 0;

  // decode GEMV, fp32 output: rel < 1e-5 (tests/gate_gemv.cu:130)
  const int M = 9;
  std::vector<uint16_t> x((size_t)M * K);
  for (auto& v : x) v = or_f32_to_bf16(nd(rng) * 0.05f);
  std::vector<double> ref((size_t)M * N);
  or_matmul_f64(x.data(), M, q.data(), zp.data(), s.data(), N, K, 128, ref.data(), 4);
  uint16_t* d_x = upload(x);
  float* d_yf = nullptr;
  uint16_t* d_y = nullptr;
  CK(hipMalloc(&d_yf, (size_t)N * 4));
  CK(hipMalloc(&d_y, (size_t)M * N * 2));
  qwen::gemv_w4a16_f32(d_yf, W, reinterpret_cast<__hip_bfloat16*>(d_x), S);
  std::vector<float> yf(N);
  CK(hipMemcpy(yf.data(), d_yf, (size_t)N * 4, hipMemcpyDeviceToHost));
  const double r1 = rel_err(std::vector<double>(ref.begin(), ref.begin() + N), yf);
  std::printf("gemv_w4a16_f32   rel %.3e %s\n", r1, r1 < 1e-5 ? "ok" : "FAIL");
  fails += !(r1 < 1e-5);

  // verify block (M = 9), bf16 output: rel < 2e-2 (bench/bench_verify.cu:55-75)
  qwen::gemm_mma_w4a16(reinterpret_cast<__hip_bfloat16*>(d_y), W,
                       reinterpret_cast<__hip_bfloat16*>(d_x), M, S);
  std::vector<uint16_t> y((size_t)M * N);
  CK(hipMemcpy(y.data(), d_y, y.size() * 2, hipMemcpyDeviceToHost));
  std::vector<float> yv(y.size());
  for (size_t i = 0; i < y.size(); ++i) yv[i] = or_bf16_to_f32(y[i]);
  const double r2 = rel_err(ref, yv);
  std::printf("gemm_mma_w4a16   rel %.3e %s\n", r2, r2 < 1e-2 ? "ok" : "FAIL");
  fails += !(r2 < 1e-2);

  // prefill GEMM: bf16 dequantized weights, rel < 2e-2 (tests/gate_gemm.cu:105)
  const int Mp = 77;
  std::vector<uint16_t> A((size_t)Mp * K);
  for (auto& v : A) v = or_f32_to_bf16(nd(rng) * 0.05f);
  std::vector<double> refp((size_t)Mp * N);
  or_matmul_bf16w_f64(A.data(), Mp, q.data(), zp.data(), s.data(), N, K, 128, refp.data(), 4);
  uint16_t* d_A = upload(A);
  uint16_t* d_C = nullptr;
  CK(hipMalloc(&d_C, (size_t)Mp * N * 2));
  qwen::GemmWorkspace ws;
  qwen::gemm_workspace_alloc(ws, 256ull << 20);   // as the reference sizes it (model.cu:440)
  qwen::gemm_w4a16(reinterpret_cast<__hip_bfloat16*>(d_C), W,
                   reinterpret_cast<__hip_bfloat16*>(d_A), Mp, ws);
  std::vector<uint16_t> Cm((size_t)Mp * N);
  CK(hipMemcpy(Cm.data(), d_C, Cm.size() * 2, hipMemcpyDeviceToHost));
  std::vector<float> cv(Cm.size());
  for (size_t i = 0; i < Cm.size(); ++i) cv[i] = or_bf16_to_f32(Cm[i]);
  const double r3 = rel_err(refp, cv);
  std::printf("gemm_w4a16       rel %.3e %s\n", r3, r3 < 2e-2 ? "ok" : "FAIL");
  fails += !(r3 < 2e-2);

  // dequant rows: bit-exact (tests/gate_dequant.cpp:87)
  uint16_t* d_deq = nullptr;
  CK(hipMalloc(&d_deq, (size_t)N * K * 2));
  qwen::w4a16_dequant_rows(reinterpret_cast<__hip_bfloat16*>(d_deq), W, 0, N);
  std::vector<uint16_t> deq((size_t)N * K), want((size_t)N * K);
  CK(hipMemcpy(deq.data(), d_deq, deq.size() * 2, hipMemcpyDeviceToHost));
  or_dequant_bf16(q.data(), zp.data(), s.data(), N, K, 128, 0, N, want.data());
  const bool exact = std::memcmp(deq.data(), want.data(), deq.size() * 2) == 0;
  std::printf("w4a16_dequant_rows %s\n", exact ? "bit-exact" : "FAIL");
  fails += !exact;

  // argmax_rows over the bf16 verify logits (elementwise.cuh:41-43)
  int32_t* d_idx = nullptr;
  CK(hipMalloc(&d_idx, M * 4));
  qwen::argmax_rows(d_idx, reinterpret_cast<__hip_bfloat16*>(d_y), M, N);
  std::vector<int32_t> idx(M), widx(M);
  CK(hipMemcpy(idx.data(), d_idx, M * 4, hipMemcpyDeviceToHost));
  or_argmax_rows_bf16(y.data(), M, N, widx.data());
  const bool am = idx == widx;
  std::printf("argmax_rows      %s\n", am ? "ok" : "FAIL");
  fails += !am;

  // layer steps around the projections (src/model/model.cu:772-785): each
  // fused entry point equals the unfused steps bit for bit, and linear()
  // equals the path it dispatches to
  {
    auto bf = [](uint16_t* p) { return reinterpret_cast<__hip_bfloat16*>(p); };
    const size_t yb = (size_t)M * N * 2;
    std::vector<uint16_t> h0((size_t)M * N), nwh(K);
    for (auto& v : h0) v = or_f32_to_bf16(nd(rng));
    for (auto& v : nwh) v = or_f32_to_bf16(nd(rng) * 0.1f);
    uint16_t *d_h = upload(h0), *d_h2 = upload(h0), *d_nw = upload(nwh);
    uint16_t *d_a = nullptr, *d_b = nullptr, *d_t = nullptr;
    CK(hipMalloc(&d_a, yb));
    CK(hipMalloc(&d_b, yb));
    CK(hipMalloc(&d_t, (size_t)M * K * 2));
    std::vector<uint16_t> ua((size_t)M * N), ub((size_t)M * N);
    auto same = [&](const char* what, uint16_t* p, uint16_t* q, size_t n) {
      std::vector<uint16_t> a(n), b(n);
      if (hipMemcpy(a.data(), p, n * 2, hipMemcpyDeviceToHost) != hipSuccess ||
          hipMemcpy(b.data(), q, n * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return false;
      const bool ok = std::memcmp(a.data(), b.data(), n * 2) == 0;
      std::printf("%-16s %s\n", what, ok ? "bit-exact" : "FAIL");
      return ok;
    };
    // linear + residual_add
    qwen::gemv_w4a16_residual(bf(d_h), W, bf(d_x), M, S);
    qwen::gemm_small_w4a16(bf(d_a), W, bf(d_x), M, S);
    qwen::residual_add(bf(d_h2), bf(d_a), M * N);
    fails += !same("gemv_residual", d_h, d_h2, (size_t)M * N);
    // linear + swiglu over [gate | up] (out_f = 2 x 256)
    qwen::gemv_w4a16_swiglu(bf(d_a), W, bf(d_x), M, nullptr, S);
    qwen::gemm_small_w4a16(bf(d_b), W, bf(d_x), M, S);
    qwen::swiglu(bf(d_t), bf(d_b), M, N / 2);
    fails += !same("gemv_swiglu", d_a, d_t, (size_t)M * N / 2);
    // rmsnorm + linear (M = 1: staged in LDS)
    qwen::gemv_w4a16_rmsnorm(bf(d_a), W, bf(d_x), bf(d_nw), 1e-6f, 1, d_t ? bf(d_t) : nullptr, S);
    qwen::rmsnorm(bf(d_t), bf(d_x), bf(d_nw), 1, K, 1e-6f);
    qwen::gemv_w4a16(bf(d_b), W, bf(d_t), S);
    fails += !same("gemv_rmsnorm", d_a, d_b, (size_t)N);
    // linear(): T = M -> 16-row skinny pass, T = Mp -> (by size) skinny or GEMM
    qwen::linear_w4a16(bf(d_a), W, bf(d_x), M, S, ws);
    qwen::gemm_small_w4a16(bf(d_b), W, bf(d_x), M, S);
    fails += !same("linear T=9", d_a, d_b, (size_t)M * N);
    CK(hipFree(d_h));
    CK(hipFree(d_h2));
    CK(hipFree(d_nw));
    CK(hipFree(d_a));
    CK(hipFree(d_b));
    CK(hipFree(d_t));
  }

  qwen::gemm_workspace_free(ws);
  qwen::gemv_scratch_free(S);
  qwen::awq_free(W);
  std::printf("gate_w4a16: %s\n", fails ? "FAIL" : "PASS");
  return fails ? 1 : 0;
}
