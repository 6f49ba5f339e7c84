// The reference's linear() path choice (src/model/model.cu:522-565,
// :643-658) over this library's kernels: the GEMV for one row, the skinny
// kernel in chunks of up to 16 rows while it reads the weights fewer times
// than the prefill GEMM would cost, the prefill GEMM beyond. Host code only.
#include <atomic>

#include "../../include/qwen_w4a16.h"

namespace {

std::atomic<int> g_lin_max_t{0};   // qw4_tune_linear override (0: the rule below)

// Rows up to which 16-row skinny passes beat the prefill GEMM. Measured on
// MI355X over the model's projections (T = 16 .. 256): a skinny pass costs
// about 0.245 us per MB of weights + 5.8 us, the prefill GEMM about 60 us +
// 0.4 us per MB at these row counts, so the crossover is 16 whole passes
// under their ratio -- 48 rows for gate|up (93 MB; measured ~55), 64 for down
// (46 MB; ~60), 96 for qkv (19 MB; ~107), 112 for o_proj (11 MB; ~127).
int lin_max_t(const qw4_weights* w) {
  const int v = g_lin_max_t.load(std::memory_order_relaxed);
  if (v > 0) return v;
  const double mb = (double)w->out_f * w->in_f * (0.5 + 2.5 / 128) / 1e6;
  const int chunks = (int)((60.0 + 0.4 * mb) / (0.245 * mb + 5.8));
  return 16 * (chunks < 1 ? 1 : chunks);
}

}  // namespace

extern "C" {

int qw4_tune_linear(int max_t) {
  if (max_t < 0) return QW4_ERR_SHAPE;
  g_lin_max_t.store(max_t, std::memory_order_relaxed);
  return 0;
}

int qw4_linear_max_t(const qw4_weights* w) {
  if (!w || w->out_f <= 0 || w->in_f <= 0) return QW4_ERR_NULL;
  return lin_max_t(w);
}

int qw4_linear(uint16_t* y, const qw4_weights* w, const uint16_t* x, int T, qw4_scratch* s,
               qw4_workspace* ws, void* stream) {
  if (!y || !w || !x) return QW4_ERR_NULL;
  if (T < 1) return QW4_ERR_M;
  if (T == 1) return qw4_gemv(y, w, x, s, stream);
  if (T <= lin_max_t(w) && s) {
    const int chunk = s->max_m < 16 ? s->max_m : 16;
    if (chunk < 1) return QW4_ERR_SCRATCH;
    for (int i = 0; i < T; i += chunk) {
      const int n = T - i < chunk ? T - i : chunk;
      const int st = qw4_gemm_small(y + (size_t)i * w->out_f, w, x + (size_t)i * w->in_f, n, s,
                                    stream);
      if (st) return st;
    }
    return QW4_OK;
  }
  return qw4_gemm(y, w, x, T, ws, stream);
}

}  // extern "C"
