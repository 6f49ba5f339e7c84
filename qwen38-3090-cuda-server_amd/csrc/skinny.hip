// Decode GEMV (M = 1), speculative-verify skinny GEMM (M = 2..16) and the
// lm_head GEMV with a fused fp32 row-argmax, all on one gfx950 kernel.
//
// Work decomposition
//   * A workgroup is 4 waves and owns one 64-row tile of W and a contiguous
//     range of quantization groups (split s of S). Its 4 waves split that range
//     again and are summed through LDS in wave order.
//   * Per group a wave streams the tile's 4 KiB block with four 16-byte loads
//     per lane (lane c + 16q reads chunk q of positions 16*st + c, i.e. rows
//     4c + st), and feeds bf16 MFMA v_mfma_f32_16x16x32_bf16:
//        A = activations, 16 rows (rows >= M are zero), 32 k per instruction
//        B = the packed word turned into 8 bf16 values (128 + q) by AND-OR
//     Four instructions per row-quad st cover the group; a fifth B operand of
//     ones gives S_m = sum_k x[m][k] in the same output layout, so the
//     zero-point / +128 correction is
//        acc[m][n] += s[n] * (C[m][n] - (128 + zp[n]) * S_m)
//     (the reference's identity, src/kernels/gemv_w4a16.cuh:25-37, with the
//     group sum computed by the matrix core instead of a prologue kernel).
//   * Split-K partials go to scratch; the last workgroup of a tile to arrive
//     (per-tile counter) sums them in split order 0..S-1, so results are
//     bitwise deterministic (the property of gemv_w4a16.cu:262-279), and resets
//     the counter so the next call -- or a graph replay -- starts from zero.
//   * Cross-workgroup exchange never flushes or invalidates an L2: each XCD has
//     its own L2, and a device-scope fence (buffer_wbl2 + buffer_inv) per
//     workgroup costs more than the whole weight stream. Only the exchanged
//     words are made coherent: partials are written through to memory
//     (system-scope relaxed stores, sc0 sc1), the writer waits for their
//     completion (s_waitcnt) before its memory-side counter increment (sc1), and
//     the last workgroup reads them back with memory-coherent loads.
//
// Output layout per lane after the loop: acc[st][jj] is row m = 4q + jj,
// column n = 64*tile + 4c + st.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "../../include/qwen_w4a16.h"
#include "w4a16_common.h"

namespace qw4 {
int check_weights_public(const qw4_weights* w);

namespace {

enum { OUT_BF16 = 0, OUT_F32 = 1, OUT_ARGMAX = 2 };

struct SkinnyArgs {
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* zr;
  const uint16_t* x;
  void* y;
  float* partial;
  uint32_t* counters;   // one counter per 128-byte line (kCounterStride words):
                        //   [0, tiles)            split arrival, per tile
                        //   [max_tiles, +64)      argmax arrival, per key group
                        //   [max_tiles + 64]      argmax arrival, of key groups
  uint64_t* keys;       // argmax keys [64 groups][16 rows], one line per group
  int M, N, K, G, S, tiles, max_tiles;
};

// Memory-side atomics on one cache line serialize; each counter gets its own line.
constexpr int kCounterStride = 32;
constexpr int kKeyGroups = 64;

// Monotonic key: larger value first, then lower index (elementwise.cu:103-104).
__device__ __forceinline__ uint64_t argmax_key(float v, int n) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(~(uint32_t)n);
}

// Coherent scalar exchange between workgroups of one launch (see header).
__device__ __forceinline__ void st_sys(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_sys(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t inc_sys(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

struct GroupData {
  u32x4 w[4];   // row quad st -> 4 words (k chunks t = 0..3)
  u32x4 x[4];   // activation row c, k chunk t: 8 bf16
  u32x2 s;      // scales of rows 4c..4c+3
  uint32_t z;   // zero points of rows 4c..4c+3 (4 bits each)
};

__device__ __forceinline__ void load_group(GroupData& d, const SkinnyArgs& a, int b, int g,
                                           int c, int q, bool xrow) {
  const size_t blk = (size_t)b * a.G + g;
  const uint32_t* wp = a.qw + blk * kWordsPerBlock + q * 256 + c * 4;
#pragma unroll
  for (int st = 0; st < 4; ++st) d.w[st] = *reinterpret_cast<const u32x4*>(wp + st * 64);
  const uint16_t* xp = a.x + (size_t)c * a.K + (size_t)g * kGroup + 32 * q;
#pragma unroll
  for (int t = 0; t < 4; ++t)
    d.x[t] = xrow ? *reinterpret_cast<const u32x4*>(xp + 8 * t) : u32x4{0, 0, 0, 0};
  d.s = *reinterpret_cast<const u32x2*>(a.sc + blk * 64 + 4 * c);
  d.z = a.zr[blk * 16 + c];
}

__device__ __forceinline__ void mma_group(f32x4 (&acc)[4], const GroupData& d, NibConst k) {
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u,
                                                       0x3F803F80u, 0x3F803F80u});
  f32x4 C[4], Cs;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const bf16x8 A = __builtin_bit_cast(bf16x8, d.x[t]);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bf16x8 B = nib8(d.w[st][t], k);
      C[st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          A, B, t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : C[st], 0, 0, 0);
    }
    Cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, ones,
                                                 t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : Cs,
                                                 0, 0, 0);
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const uint32_t sbits = (st & 1) ? (d.s[st >> 1] >> 16) : (d.s[st >> 1] & 0xffffu);
    const float sf = bf16_bits_to_f32(sbits);
    const float zf = 128.0f + (float)((d.z >> (4 * st)) & 0xFu);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[st][jj] += sf * (C[st][jj] - zf * Cs[jj]);
  }
}

template <int OUT>
__global__ __launch_bounds__(256) void k_skinny(SkinnyArgs a) {
  __shared__ f32x4 red[3][4][64];
  __shared__ int s_last;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const int b = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const int gb = (int)((long)a.G * s / a.S), ge = (int)((long)a.G * (s + 1) / a.S);
  const int g0 = gb + (ge - gb) * wave / 4, g1 = gb + (ge - gb) * (wave + 1) / 4;
  const bool xrow = c < a.M;

  f32x4 acc[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) acc[st] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (g0 < g1) {
    const NibConst k = nib_const();
    // Ping-pong buffers: the loads of group g+1 are in flight during the MFMAs
    // of group g, with no register copies between iterations.
    GroupData d0, d1;
    load_group(d0, a, b, g0, c, q, xrow);
    int g = g0;
    for (; g + 1 < g1; g += 2) {
      load_group(d1, a, b, g + 1, c, q, xrow);
      mma_group(acc, d0, k);
      if (g + 2 < g1) load_group(d0, a, b, g + 2, c, q, xrow);
      mma_group(acc, d1, k);
    }
    if (g < g1) mma_group(acc, d0, k);
  }

  // Sum the four waves in wave order.
  if (wave) {
#pragma unroll
    for (int st = 0; st < 4; ++st) red[wave - 1][st][lane] = acc[st];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int st = 0; st < 4; ++st) acc[st] += red[w][st][lane];
  }

  if (a.S > 1) {
    // Partial layout: [tile][split][lane][16], element 4*st + jj.
    if (wave == 0) {
      float* mine = a.partial + ((size_t)b * a.S + s) * 1024 + lane * 16;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) st_sys(mine + 4 * st + jj, acc[st][jj]);
      wait_all_mem();
    }
    __syncthreads();
    if (threadIdx.x == 0) s_last = inc_sys(&a.counters[b * kCounterStride]) == (uint32_t)(a.S - 1);
    __syncthreads();
    if (!s_last) return;
    if (wave != 0) return;
    const float* base = a.partial + (size_t)b * a.S * 1024 + lane * 16;
#pragma unroll
    for (int st = 0; st < 4; ++st) acc[st] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < a.S; ++sp) {
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[st][jj] += ld_sys(base + (size_t)sp * 1024 + 4 * st + jj);
    }
    if (lane == 0)
      __hip_atomic_store(&a.counters[b * kCounterStride], 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  if (wave != 0) return;

  const int n0 = b * kTileN + 4 * c;
  if (OUT == OUT_BF16) {
    uint16_t* y = static_cast<uint16_t*>(a.y);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int m = 4 * q + jj;
      if (m < a.M)
        *reinterpret_cast<u32x2*>(y + (size_t)m * a.N + n0) =
            u32x2{pack_bf16x2(acc[0][jj], acc[1][jj]), pack_bf16x2(acc[2][jj], acc[3][jj])};
    }
  } else if (OUT == OUT_F32) {
    float* y = static_cast<float*>(a.y);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int m = 4 * q + jj;
      if (m < a.M)
        *reinterpret_cast<f32x4*>(y + (size_t)m * a.N + n0) =
            f32x4{acc[0][jj], acc[1][jj], acc[2][jj], acc[3][jj]};
    }
  } else {
    // Two-level argmax without hot spots: tile b folds its best (value, index)
    // per row into key group b % 64 (one cache line per group); the last tile
    // of a group to arrive bumps the group counter, and the last group to
    // finish folds the 64 groups, writes the indices and clears the state.
    const int grp = b % kKeyGroups;
    uint64_t* gkeys = a.keys + grp * 16;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float v = acc[0][jj];
      int n = n0;
#pragma unroll
      for (int st = 1; st < 4; ++st)
        if (acc[st][jj] > v) { v = acc[st][jj]; n = n0 + st; }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const float v2 = __shfl_xor(v, off, 64);
        const int n2 = __shfl_xor(n, off, 64);
        if (v2 > v || (v2 == v && n2 < n)) { v = v2; n = n2; }
      }
      const int m = 4 * q + jj;
      if (c == 0 && m < a.M)
        __hip_atomic_fetch_max(&gkeys[m], argmax_key(v, n), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_all_mem();   // this tile's key updates are complete before it is counted
    if (lane == 0) {
      const int ngroups = a.tiles < kKeyGroups ? a.tiles : kKeyGroups;
      const uint32_t in_grp = (uint32_t)((a.tiles - 1 - grp) / kKeyGroups + 1);
      uint32_t* gcnt = a.counters + (size_t)(a.max_tiles + grp) * kCounterStride;
      uint32_t* done = a.counters + (size_t)(a.max_tiles + kKeyGroups) * kCounterStride;
      if (inc_sys(gcnt) == in_grp - 1 && inc_sys(done) == (uint32_t)(ngroups - 1)) {
        int32_t* idx = static_cast<int32_t*>(a.y);
        for (int m = 0; m < a.M; ++m) {
          uint64_t best = 0;
          for (int g2 = 0; g2 < ngroups; ++g2) {
            const uint64_t k = __hip_atomic_load(&a.keys[g2 * 16 + m], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            best = k > best ? k : best;
          }
          idx[m] = (int32_t)(~(uint32_t)(best & 0xffffffffu));
        }
        for (int g2 = 0; g2 < ngroups; ++g2) {
          for (int m = 0; m < a.M; ++m)
            __hip_atomic_store(&a.keys[g2 * 16 + m], (uint64_t)0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.counters + (size_t)(a.max_tiles + g2) * kCounterStride, 0u,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

int g_target_wgs = 0;
std::once_flag g_once;

int target_wgs() {
  std::call_once(g_once, [] {
    const char* e = std::getenv("QW4_SKINNY_WGS");
    int v = e ? std::atoi(e) : 0;
    g_target_wgs = v > 0 ? v : 1024;
  });
  return g_target_wgs;
}

int choose_splits(int out_f, int G) {
  const int tiles = out_f / kTileN;
  int S = (target_wgs() + tiles - 1) / tiles;
  S = std::max(1, std::min(S, G / 4));
  return S;
}

// Scratch bound: S > 1 only when tiles < target, and then tiles * S < 2 * target.
size_t partial_elems_needed(int out_f, int G, int M) {
  (void)M;
  const int S = choose_splits(out_f, G);
  return S > 1 ? (size_t)(out_f / kTileN) * S * 1024 : 0;
}

template <int OUT>
int run_skinny(void* y, const qw4_weights* w, const uint16_t* x, int M, qw4_scratch* s,
               void* stream) {
  int st = check_weights_public(w);
  if (st) return st;
  if (!y || !x || !s || !s->counters) return QW4_ERR_NULL;
  if (M < 1 || M > 16) return QW4_ERR_M;
  if (((uintptr_t)x & 15) || ((uintptr_t)y & (OUT == OUT_F32 ? 15 : (OUT == OUT_BF16 ? 7 : 3))))
    return QW4_ERR_ALIGN;
  const int tiles = w->out_f / kTileN;
  if (tiles > s->max_tiles || M > s->max_m) return QW4_ERR_SCRATCH;
  const int S = choose_splits(w->out_f, w->num_groups);
  if (S > 1 && (size_t)tiles * S * 1024 > s->partial_elems) return QW4_ERR_SCRATCH;
  SkinnyArgs a;
  a.qw = w->qweight;
  a.sc = w->scale;
  a.zr = w->zeros;
  a.x = x;
  a.y = y;
  a.partial = s->partial;
  a.counters = s->counters;
  a.keys = s->keys;
  a.M = M;
  a.N = w->out_f;
  a.K = w->in_f;
  a.G = w->num_groups;
  a.S = S;
  a.tiles = tiles;
  a.max_tiles = s->max_tiles;
  k_skinny<OUT><<<tiles * S, 256, 0, (hipStream_t)stream>>>(a);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

}  // namespace
}  // namespace qw4

using namespace qw4;

extern "C" {

int qw4_choose_splits(int out_f, int num_groups) {
  if (out_f <= 0 || num_groups <= 0) return 1;
  return choose_splits(out_f, num_groups);
}

int qw4_scratch_alloc(qw4_scratch* s, int max_in, int max_out, int min_group, int max_m) {
  if (!s) return QW4_ERR_NULL;
  if (min_group != kGroup) return QW4_ERR_GROUP;
  if (max_in <= 0 || max_out <= 0) return QW4_ERR_SHAPE;
  if (max_m < 1 || max_m > 16) return QW4_ERR_M;
  std::memset(s, 0, sizeof(*s));
  s->max_in = max_in;
  s->max_out = max_out;
  s->max_m = max_m;
  s->max_tiles = (max_out + kTileN - 1) / kTileN;
  // Any out_f <= max_out: S > 1 implies tiles * S < 2 * target.
  s->partial_elems = (size_t)2 * target_wgs() * 1024;
  const size_t cnt_bytes = (size_t)(s->max_tiles + kKeyGroups + 1) * kCounterStride * 4;
  const size_t key_bytes = (size_t)kKeyGroups * 16 * 8;
  hipError_t e = hipMalloc((void**)&s->partial, s->partial_elems * 4);
  if (e == hipSuccess) e = hipMalloc((void**)&s->counters, cnt_bytes);
  if (e == hipSuccess) e = hipMalloc((void**)&s->keys, key_bytes);
  if (e == hipSuccess) e = hipMemset(s->counters, 0, cnt_bytes);
  if (e == hipSuccess) e = hipMemset(s->keys, 0, key_bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    set_hip_error((int)e);
    (void)hipGetLastError();
    qw4_scratch_free(s);
    return QW4_ERR_NOMEM;
  }
  return QW4_OK;
}

int qw4_scratch_free(qw4_scratch* s) {
  if (!s) return QW4_ERR_NULL;
  if (s->partial) (void)hipFree(s->partial);
  if (s->counters) (void)hipFree(s->counters);
  if (s->keys) (void)hipFree(s->keys);
  std::memset(s, 0, sizeof(*s));
  return QW4_OK;
}

int qw4_partial_check(const qw4_scratch* s, int splits, int out_f, int M) {
  if (!s) return QW4_ERR_NULL;
  if (M > s->max_m || (out_f + kTileN - 1) / kTileN > s->max_tiles) return QW4_ERR_SCRATCH;
  const size_t need = splits > 1 ? (size_t)((out_f + kTileN - 1) / kTileN) * splits * 1024 : 0;
  return need > s->partial_elems ? QW4_ERR_SCRATCH : QW4_OK;
}

int qw4_gemv(uint16_t* y, const qw4_weights* w, const uint16_t* x, qw4_scratch* s,
             void* stream) {
  return run_skinny<OUT_BF16>(y, w, x, 1, s, stream);
}

int qw4_gemv_f32(float* y, const qw4_weights* w, const uint16_t* x, qw4_scratch* s,
                 void* stream) {
  return run_skinny<OUT_F32>(y, w, x, 1, s, stream);
}

int qw4_gemm_small(uint16_t* y, const qw4_weights* w, const uint16_t* x, int M,
                   qw4_scratch* s, void* stream) {
  return run_skinny<OUT_BF16>(y, w, x, M, s, stream);
}

int qw4_gemm_mma(uint16_t* y, const qw4_weights* w, const uint16_t* x, int M,
                 qw4_scratch* s, void* stream) {
  return run_skinny<OUT_BF16>(y, w, x, M, s, stream);
}

int qw4_gemv_argmax(int32_t* idx, const qw4_weights* w, const uint16_t* x, int M,
                    qw4_scratch* s, void* stream) {
  return run_skinny<OUT_ARGMAX>(idx, w, x, M, s, stream);
}

}  // extern "C"
