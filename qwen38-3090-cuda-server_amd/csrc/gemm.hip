// Prefill W4A16 GEMM: C [M][N] = A [M][K] @ W^T, bf16 in/out, fp32 accumulate.
//
// The reference dequantizes whole weight tiles to a bf16 workspace and calls
// cublasGemmEx (src/kernels/gemm_w4a16.cu:63-88). Here the dequant is fused:
// each K step stages the packed 4 KiB (tile, group) blocks straight from the
// repacked layout, converts them to bf16 in registers -- exactly RNE((q-z)*s),
// the reference's k_dequant_rows arithmetic (gemm_w4a16.cu:26-36) -- and
// writes them into LDS next to the activation tile; bf16 MFMA
// (v_mfma_f32_16x16x32_bf16) consumes both.
//
// Workgroup tile BM x BN = 128 x 128, 4 waves (2 x 2), each wave 64 x 64 =
// 4 x 4 MFMA blocks; BK = 128 = one quantization group. Global loads for
// step k+1 are issued before the MFMAs of step k (register double buffer).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "../../include/qwen_w4a16.h"
#include "w4a16_common.h"

namespace qw4 {
int check_weights_public(const qw4_weights* w);

namespace {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LDA = BK + 8;   // bf16 elements per LDS row (272 B: conflict-free b128 reads)

struct GemmArgs {
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* zr;
  const uint16_t* A;
  uint16_t* C;
  int M, N, K, G;
};

struct Stage {
  u32x4 a[8];     // 8 x 16 B of activations
  u32x4 w[2];     // 2 x 16 B of packed weights
  uint32_t s[2];  // scale bits of the two rows
  uint32_t z[2];  // zero point of the two rows
};

__device__ __forceinline__ void load_stage(Stage& st, const GemmArgs& a, int m0, int n0, int g,
                                           int tid) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = tid + 256 * i;
    const int r = id >> 4, ch = id & 15;
    const int m = m0 + r;
    st.a[i] = m < a.M ? *reinterpret_cast<const u32x4*>(a.A + (size_t)m * a.K + g * BK + ch * 8)
                      : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int id = tid + 256 * i;
    const int tile = (n0 >> 6) + (id >> 8);
    const int within = id & 255;              // 16-byte chunk in the 4 KiB block
    const int p = within & 63;
    const int row = tile_row_of_pos(p);
    if (tile * kTileN < a.N) {
      const size_t blk = (size_t)tile * a.G + g;
      st.w[i] = *reinterpret_cast<const u32x4*>(a.qw + blk * kWordsPerBlock + within * 4);
      st.s[i] = a.sc[blk * 64 + row];
      st.z[i] = (a.zr[blk * 16 + (row >> 2)] >> (4 * (row & 3))) & 0xFu;
    } else {
      st.w[i] = u32x4{0, 0, 0, 0};
      st.s[i] = 0;
      st.z[i] = 0;
    }
  }
}

// bf16 pair (128+q_lo, 128+q_hi) -> RNE((q - z) * s) pair, exact before rounding:
// (128 + z) * s has at most 16 significant bits, so the fma is exact.
__device__ __forceinline__ uint32_t deq_pair(uint32_t magic, float s, float c) {
  const float lo = __uint_as_float(magic << 16);
  const float hi = __uint_as_float(magic & 0xffff0000u);
  return pack_bf16x2(__builtin_fmaf(lo, s, c), __builtin_fmaf(hi, s, c));
}

__device__ __forceinline__ void store_stage(const Stage& st, uint16_t* sA, uint16_t* sB,
                                            int tid, NibConst kc) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = tid + 256 * i;
    const int r = id >> 4, ch = id & 15;
    *reinterpret_cast<u32x4*>(sA + r * LDA + ch * 8) = st.a[i];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int id = tid + 256 * i;
    const int within = id & 255;
    const int j = within >> 6, p = within & 63;
    const int row = (id >> 8) * kTileN + tile_row_of_pos(p);
    const float s = bf16_bits_to_f32(st.s[i]);
    const float c = -(128.0f + (float)st.z[i]) * s;
    uint16_t* dst = sB + row * LDA + 32 * j;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32x4 m = nib8_bits(st.w[i][w], kc);
      *reinterpret_cast<u32x4*>(dst + 8 * w) =
          u32x4{deq_pair(m[0], s, c), deq_pair(m[1], s, c), deq_pair(m[2], s, c),
                deq_pair(m[3], s, c)};
    }
  }
}

__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t sB[BN * LDA];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int ntn = (a.N + BN - 1) / BN;
  const int m0 = (blockIdx.x / ntn) * BM, n0 = (blockIdx.x % ntn) * BN;
  const int l16 = lane & 15, lq = lane >> 4;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const NibConst kc = nib_const();
  Stage st;
  load_stage(st, a, m0, n0, 0, tid);
  for (int g = 0; g < a.G; ++g) {
    store_stage(st, sA, sB, tid, kc);
    __syncthreads();
    if (g + 1 < a.G) load_stage(st, a, m0, n0, g + 1, tid);
#pragma unroll
    for (int t = 0; t < BK / 32; ++t) {
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = *reinterpret_cast<const bf16x8*>(sA + (wm * 64 + 16 * i + l16) * LDA + 32 * t + 8 * lq);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[j] = *reinterpret_cast<const bf16x8*>(sB + (wn * 64 + 16 * j + l16) * LDA + 32 * t + 8 * lq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // D layout: lane holds rows 4*lq + r of block i, column l16 of block j.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + 16 * j + l16;
      if (n >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + 16 * i + 4 * lq + r;
        if (m < a.M) a.C[(size_t)m * a.N + n] = to_bf16(acc[i][j][r]);
      }
    }
}

}  // namespace
}  // namespace qw4

using namespace qw4;

extern "C" {

int qw4_workspace_alloc(qw4_workspace* ws, size_t bytes) {
  if (!ws) return QW4_ERR_NULL;
  std::memset(ws, 0, sizeof(*ws));
  if (bytes == 0) return QW4_OK;
  hipError_t e = hipMalloc(&ws->buf, bytes);
  if (e != hipSuccess) {
    set_hip_error((int)e);
    (void)hipGetLastError();
    ws->buf = nullptr;
    return QW4_ERR_NOMEM;
  }
  ws->bytes = bytes;
  return QW4_OK;
}

int qw4_workspace_free(qw4_workspace* ws) {
  if (!ws) return QW4_ERR_NULL;
  if (ws->buf) (void)hipFree(ws->buf);
  std::memset(ws, 0, sizeof(*ws));
  return QW4_OK;
}

int qw4_gemm(uint16_t* C, const qw4_weights* w, const uint16_t* A, int M, qw4_workspace* ws,
             void* stream) {
  (void)ws;
  int st = check_weights_public(w);
  if (st) return st;
  if (!C || !A) return QW4_ERR_NULL;
  if (M < 1) return QW4_ERR_M;
  if (((uintptr_t)A & 15) || ((uintptr_t)C & 1)) return QW4_ERR_ALIGN;
  GemmArgs a{w->qweight, w->scale, w->zeros, A, C, M, w->out_f, w->in_f, w->num_groups};
  const int grid = ((M + BM - 1) / BM) * ((w->out_f + BN - 1) / BN);
  k_gemm<<<grid, 256, 0, (hipStream_t)stream>>>(a);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

}  // extern "C"
