// Decode GEMV (M = 1), speculative-verify skinny GEMM (M = 2..16) and the
// lm_head GEMV with a fused fp32 row-argmax, all on one gfx950 kernel.
//
// Why stream-K. The path is HBM-bound and the chip streams at most ~10 bytes
// per clock per CU, so the kernel runs at the speed of its most loaded CU.
// Giving each workgroup one 64-row tile leaves CUs unevenly loaded (544 tiles on
// 256 CUs) or idle (80 tiles for a 5120-row projection). Instead the grid is a
// fixed number of workgroups P sized to the chip, and the flattened list of
// U = tiles x groups blocks (one 4 KiB (tile, group) block each) is cut into P
// equal contiguous ranges. A workgroup walks the tiles its range touches; a
// tile it covers completely it finishes itself, a tile cut by a range boundary
// is finished by whichever of its (at most a few) workgroups arrives last.
//
// Per block, a wave streams 4 KiB with four 16-byte loads per lane (lane
// c + 16q reads chunk q of positions 16*st + c, i.e. rows 4c + st) and feeds
// bf16 MFMA v_mfma_f32_16x16x32_bf16:
//    A = activations, 16 rows (rows >= M are zero), 32 k per instruction
//    B = the packed word turned into 8 bf16 values (128 + q) by AND-OR
// Four instructions per row quad st cover the group; a fifth B operand of ones
// gives S_m = sum_k x[m][k] in the same output layout, so the zero-point and
// +128 correction is
//    acc[m][n] += s[n] * (C[m][n] - (128 + zp[n]) * S_m)
// (the reference's identity, src/kernels/gemv_w4a16.cuh:25-37, with the group
// sum computed by the matrix core instead of a prologue kernel). The 4 waves of
// a workgroup take interleaved blocks of each tile and are summed through LDS.
//
// Determinism: a tile's sum is always formed in the same order (waves 0..3 in
// LDS; partial workgroups in workgroup order), so repeated calls are bitwise
// identical (the property of gemv_w4a16.cu:262-279).
//
// Cross-workgroup exchange never flushes or invalidates an L2 (each XCD has its
// own, and a device-scope fence per workgroup costs more than the weight
// stream). Only the exchanged data is made coherent: partials are written
// through with 16-byte device-coherent (sc1) buffer stores, the writer waits
// for completion (s_waitcnt) before its device-scope counter increment, and the
// last workgroup reads them back with sc1 loads. Counters sit one per 128-byte
// line and reset themselves, so the next call -- or a graph replay -- starts
// from zero.
//
// Output layout per lane: acc[st][jj] is row m = 4q + jj, column
// n = 64*tile + 4c + st.
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

// Memory-side atomics on one cache line serialize; each counter gets its own line.
constexpr int kCounterStride = 32;
constexpr int kKeyGroups = 64;
// The most workgroups per CU a scratch buffer is sized for.
constexpr int kMaxWgsPerCu = 8;

struct SkinnyArgs {
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* zr;
  const uint16_t* x;
  void* y;
  float* partial;       // [P][2 slots][4 st][64 lanes] f32x4
  uint32_t* counters;   // one counter per 128-byte line (kCounterStride words):
                        //   [0, tiles)            partial-tile arrival, per tile
                        //   [max_tiles, +64)      argmax arrival, per key group
                        //   [max_tiles + 64]      argmax arrival, of key groups
  uint64_t* keys;       // argmax keys [64 groups][16 rows], one line per group
  const uint16_t* zero_row;   // >= K bf16 zeros: the activation row of lanes m >= M
  int M, N, K, G, tiles, max_tiles, P, U;
  uint32_t partial_bytes;
};

// Monotonic key: larger value first, then lower index (elementwise.cu:103-104).
__device__ __forceinline__ uint64_t argmax_key(float v, int n) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(~(uint32_t)n);
}

__device__ __forceinline__ uint32_t inc_dev(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void clear_dev(uint32_t* p) {
  __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

// 16-byte device-coherent (sc1) accesses to the partial buffer.
constexpr int kCpolSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(const SkinnyArgs& a) {
  return __builtin_amdgcn_make_buffer_rsrc(a.partial, 0, (int)a.partial_bytes, 0x00020000);
}
__device__ __forceinline__ void st_partial(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kCpolSc1);
}
__device__ __forceinline__ f32x4 ld_partial(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1));
}

// Stream-K range arithmetic: workgroup p owns blocks [start(p), start(p+1)).
__device__ __forceinline__ int range_start(const SkinnyArgs& a, int p) {
  return (int)((long long)p * a.U / a.P);
}
// Largest p with range_start(p) <= u.
__device__ __forceinline__ int owner_of(const SkinnyArgs& a, int u) {
  return (int)(((long long)(u + 1) * a.P - 1) / a.U);
}

struct GroupData {
  u32x4 w[4];   // row quad st -> 4 words (k chunks t = 0..3)
  u32x4 x[4];   // activation row c, k chunk t: 8 bf16
  u32x2 s;      // scales of rows 4c..4c+3
  uint32_t z;   // zero points of rows 4c..4c+3 (4 bits each)
};

// xrow: this lane's activation row (row c of x, or the zero row for c >= M),
// offset by its k chunk -- a pointer select instead of masking 16 registers.
__device__ __forceinline__ void load_group(GroupData& d, const SkinnyArgs& a, int b, int g,
                                           int c, int q, const uint16_t* xrow) {
  const size_t blk = (size_t)b * a.G + g;
  const uint32_t* wp = a.qw + blk * kWordsPerBlock + q * 256 + c * 4;
#pragma unroll
  for (int st = 0; st < 4; ++st) d.w[st] = *reinterpret_cast<const u32x4*>(wp + st * 64);
  const uint16_t* xp = xrow + (size_t)g * kGroup;
#pragma unroll
  for (int t = 0; t < 4; ++t) d.x[t] = *reinterpret_cast<const u32x4*>(xp + 8 * t);
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

// Running argmax of one workgroup: per lane, the best (value, column) of rows
// m = 4q + jj over the tiles this workgroup finished.
struct Best {
  float v[4];
  int n[4];
};

__device__ __forceinline__ void best_init(Best& bs) {
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    bs.v[jj] = -__builtin_inff();
    bs.n[jj] = 0x7fffffff;
  }
}

// Final values of tile b (wave 0 of the finishing workgroup): store them, or
// fold them into the workgroup's running argmax (lowest column on ties).
template <int OUT>
__device__ __forceinline__ void emit_tile(const SkinnyArgs& a, int b, const f32x4 (&acc)[4],
                                          int lane, Best& bs) {
  const int c = lane & 15, q = lane >> 4;
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
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const float v = acc[st][jj];
        const int n = n0 + st;
        if (v > bs.v[jj] || (v == bs.v[jj] && n < bs.n[jj])) {
          bs.v[jj] = v;
          bs.n[jj] = n;
        }
      }
  }
}

// Wave 0 at the end of an argmax workgroup: fold the workgroup's best per row
// into key group p % 64 (one cache line per group); the last workgroup of a
// group bumps the group counter, and the last group to finish folds the 64
// groups, writes the indices and clears the state for the next call.
__device__ __forceinline__ void argmax_arrive(const SkinnyArgs& a, int p, Best& bs, int lane) {
  const int c = lane & 15, q = lane >> 4;
  const int grp = p % kKeyGroups;
  uint64_t* gkeys = a.keys + grp * 16;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    float v = bs.v[jj];
    int n = bs.n[jj];
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
  wait_all_mem();   // key updates complete before this workgroup is counted
  if (lane == 0) {
    const int ngroups = a.P < kKeyGroups ? a.P : kKeyGroups;
    const uint32_t in_grp = (uint32_t)((a.P - 1 - grp) / kKeyGroups + 1);
    uint32_t* gcnt = a.counters + (size_t)(a.max_tiles + grp) * kCounterStride;
    uint32_t* done = a.counters + (size_t)(a.max_tiles + kKeyGroups) * kCounterStride;
    if (inc_dev(gcnt) == in_grp - 1 && inc_dev(done) == (uint32_t)(ngroups - 1)) {
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
        clear_dev(a.counters + (size_t)(a.max_tiles + g2) * kCounterStride);
      }
      clear_dev(done);
    }
  }
}

// Wave 0: the summed segment [lo, hi) of tile b is complete for this
// workgroup. A whole tile is emitted at once; a partial one is only written
// through to this workgroup's slot (0: its first tile, 1: its last) -- the
// completion wait and the arrival count happen once, in arrive_partial, after
// the workgroup's last segment, so no wave stalls on them mid-stream.
template <int OUT>
__device__ __forceinline__ bool store_segment(const SkinnyArgs& a, int p, int b, int lo, int hi,
                                              bool first_tile, const f32x4 (&acc)[4], int lane,
                                              Best& bs) {
  if (lo == 0 && hi == a.G) {
    emit_tile<OUT>(a, b, acc, lane, bs);
    return false;
  }
  const int q = lane >> 4;
  if (4 * q < a.M) {   // lanes holding rows m < M
    const __amdgpu_buffer_rsrc_t pr = partial_rsrc(a);
    const uint32_t mine = (uint32_t)((p * 2 + (first_tile ? 0 : 1)) * 4096 + lane * 16);
#pragma unroll
    for (int st = 0; st < 4; ++st) st_partial(pr, mine + st * 1024, acc[st]);
  }
  return true;
}

// Wave 0, after all partial slots of this workgroup are written and complete:
// count this workgroup in for tile b; the last contributor sums the partials in
// workgroup order p0..p1 and emits the tile.
template <int OUT>
__device__ __forceinline__ void arrive_partial(const SkinnyArgs& a, int b, int lane, Best& bs) {
  const int p0 = owner_of(a, b * a.G), p1 = owner_of(a, b * a.G + a.G - 1);
  uint32_t old = 0;
  if (lane == 0) old = inc_dev(&a.counters[b * kCounterStride]);
  old = __shfl(old, 0, 64);
  if (old != (uint32_t)(p1 - p0)) return;
  const int q = lane >> 4;
  const __amdgpu_buffer_rsrc_t pr = partial_rsrc(a);
  f32x4 acc[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) acc[st] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (4 * q < a.M) {
    for (int pp = p0; pp <= p1; ++pp) {
      const int slot = (pp == p0 && range_start(a, pp) / a.G != b) ? 1 : 0;
      const uint32_t off = (uint32_t)((pp * 2 + slot) * 4096 + lane * 16);
#pragma unroll
      for (int st = 0; st < 4; ++st) acc[st] += ld_partial(pr, off + st * 1024);
    }
  }
  if (lane == 0) clear_dev(&a.counters[b * kCounterStride]);
  emit_tile<OUT>(a, b, acc, lane, bs);
}

// W waves per workgroup. Inside a tile segment each wave takes groups
// lo + wave, lo + wave + W, ... in batches of two blocks: both loads issued,
// then both computed. Latency is hidden by occupancy (about 128 VGPRs, 4 waves
// per SIMD) rather than by a deep per-wave ring. W = 4: LDS sums double-buffered
// per segment; W = 8: one buffer and a second barrier.
template <int OUT, int W>
__global__ __launch_bounds__(64 * W) void k_skinny(SkinnyArgs a) {
  constexpr int kNbuf = W == 4 ? 2 : 1;
  __shared__ f32x4 red[kNbuf][W - 1][4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const uint16_t* xrow = (c < a.M ? a.x + (size_t)c * a.K : a.zero_row) + 32 * q;
  const int p = blockIdx.x;
  const int u0 = range_start(a, p), u1 = range_start(a, p + 1);
  if (u0 >= u1) return;   // whole workgroup: no work
  const int bfirst = u0 / a.G, blast = (u1 - 1) / a.G;
  const int lo_first = u0 - bfirst * a.G;
  const int hi_last = u1 - blast * a.G;
  const NibConst k = nib_const();

  int par = 0;
  bool part_first = false, part_last = false;   // partial slots written (wave 0)
  Best bs;
  best_init(bs);
  for (int sb = bfirst; sb <= blast; ++sb) {
    const int lo = sb == bfirst ? lo_first : 0;
    const int hi = sb == blast ? hi_last : a.G;
    f32x4 acc[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) acc[st] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g = lo + wave; g < hi; g += 2 * W) {
      GroupData d0, d1;
      const bool two = g + W < hi;
      load_group(d0, a, sb, g, c, q, xrow);
      if (two) load_group(d1, a, sb, g + W, c, q, xrow);
      mma_group(acc, d0, k);
      if (two) mma_group(acc, d1, k);
    }
    // Sum the segment over the W waves in wave order.
    if (wave) {
#pragma unroll
      for (int st = 0; st < 4; ++st) red[par][wave - 1][st][lane] = acc[st];
    }
    __syncthreads();
    if (wave == 0) {
      for (int w = 0; w < W - 1; ++w)
#pragma unroll
        for (int st = 0; st < 4; ++st) acc[st] += red[par][w][st][lane];
      const bool part = store_segment<OUT>(a, p, sb, lo, hi, sb == bfirst, acc, lane, bs);
      if (sb == bfirst) part_first = part;
      else part_last = part;
    }
    if (kNbuf == 2)
      par ^= 1;
    else
      __syncthreads();   // red is reused by the next segment
  }
  if (wave == 0 && (part_first || part_last)) {
    wait_all_mem();   // partial slots complete before they are counted
    if (part_first) arrive_partial<OUT>(a, bfirst, lane, bs);
    if (part_last) arrive_partial<OUT>(a, blast, lane, bs);
  }
  if (OUT == OUT_ARGMAX && wave == 0) argmax_arrive(a, p, bs, lane);
}

// ------------------------------------------------------------- host side
// Workgroups per CU: the kernel's occupancy (all workgroups resident in one
// round, equal work each), or QW4_SKINNY_WGS_PER_CU (tuning only).
int g_env_wgs = 0;
std::once_flag g_env_once;
int g_cus[64] = {0};
int g_occ[64][3][2] = {{{0}}};
int g_env_w = 0;   // QW4_SKINNY_W=4|8 (tuning)

int g_env_tiles_per_wg = 0;   // QW4_SKINNY_WG_TILES=n: n/4 tiles per workgroup (tuning)

int env_wgs_per_cu() {
  std::call_once(g_env_once, [] {
    const char* e = std::getenv("QW4_SKINNY_WGS_PER_CU");
    const int v = e ? std::atoi(e) : 0;
    g_env_wgs = (v >= 1 && v <= kMaxWgsPerCu) ? v : 0;
    const char* t = std::getenv("QW4_SKINNY_WG_TILES");
    g_env_tiles_per_wg = t ? std::atoi(t) : 0;
    const char* w = std::getenv("QW4_SKINNY_W");
    g_env_w = w ? std::atoi(w) : 0;
  });
  return g_env_wgs;
}

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  return dev;
}

int device_cus() {
  const int dev = current_device();
  if (!g_cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

template <int OUT, int W>
int wgs_per_cu() {
  if (env_wgs_per_cu()) return env_wgs_per_cu();
  const int dev = current_device();
  int& slot = g_occ[dev][OUT][W == 4 ? 0 : 1];
  if (!slot) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_skinny<OUT, W>, 64 * W, 0) !=
            hipSuccess ||
        n <= 0)
      n = 1;
    slot = std::min(n, kMaxWgsPerCu);
  }
  return slot;
}

struct Launch {
  int W, P;
};

// W = 8 with one workgroup per tile when the tiles alone cannot give every CU
// a workgroup and K is short enough for few blocks per wave; otherwise W = 4
// stream-K over every resident slot.
template <int OUT>
Launch launch_for(int out_f, int G) {
  env_wgs_per_cu();
  const int tiles = out_f / kTileN;
  const long long U = (long long)tiles * G;
  Launch l;
  l.W = (tiles < device_cus() && G <= 48) ? 8 : 4;
  if (g_env_w == 4 || g_env_w == 8) l.W = g_env_w;
  long long cap = (long long)device_cus() * (l.W == 4 ? wgs_per_cu<OUT, 4>() : wgs_per_cu<OUT, 8>());
  if (l.W == 8) cap = tiles;
  if (g_env_tiles_per_wg > 0) cap = std::max<long long>(1, (long long)tiles * 4 / g_env_tiles_per_wg);
  l.P = (int)std::max<long long>(1, std::min(cap, (U + l.W - 1) / l.W));
  return l;
}

template <int OUT>
int run_skinny(void* y, const qw4_weights* w, const uint16_t* x, int M, qw4_scratch* s,
               void* stream) {
  int st = check_weights_public(w);
  if (st) return st;
  if (!y || !x || !s || !s->counters || !s->partial) return QW4_ERR_NULL;
  if (M < 1 || M > 16) return QW4_ERR_M;
  if (((uintptr_t)x & 15) || ((uintptr_t)y & (OUT == OUT_F32 ? 15 : (OUT == OUT_BF16 ? 7 : 3))))
    return QW4_ERR_ALIGN;
  const int tiles = w->out_f / kTileN;
  if (tiles > s->max_tiles || M > s->max_m) return QW4_ERR_SCRATCH;
  const Launch l = launch_for<OUT>(w->out_f, w->num_groups);
  const int P = l.P;
  if ((size_t)P * 2 * 1024 > s->partial_elems) return QW4_ERR_SCRATCH;
  SkinnyArgs a;
  a.qw = w->qweight;
  a.sc = w->scale;
  a.zr = w->zeros;
  a.x = x;
  a.y = y;
  a.partial = s->partial;
  a.counters = s->counters;
  a.keys = s->keys;
  a.zero_row = reinterpret_cast<const uint16_t*>(s->keys + kKeyGroups * 16);
  a.M = M;
  a.N = w->out_f;
  a.K = w->in_f;
  a.G = w->num_groups;
  a.tiles = tiles;
  a.max_tiles = s->max_tiles;
  a.P = P;
  a.U = tiles * w->num_groups;
  a.partial_bytes = (uint32_t)(s->partial_elems * 4);
  if (l.W == 8)
    k_skinny<OUT, 8><<<P, 512, 0, (hipStream_t)stream>>>(a);
  else
    k_skinny<OUT, 4><<<P, 256, 0, (hipStream_t)stream>>>(a);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

}  // namespace
}  // namespace qw4

using namespace qw4;

extern "C" {

int qw4_choose_splits(int out_f, int num_groups) {
  if (out_f < kTileN || num_groups <= 0) return 1;
  const long long U = (long long)(out_f / kTileN) * num_groups;
  const long long P = launch_for<OUT_BF16>(out_f, num_groups).P;
  // workgroups sharing one tile, at most: ceil(G / blocks-per-workgroup) + 1
  const long long per = std::max<long long>(1, U / P);
  return (int)std::min<long long>(P, (num_groups + per - 1) / per + (U % P ? 1 : 0));
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
  // two 4 KiB partial slots per stream-K workgroup, for the largest grid
  s->partial_elems = (size_t)device_cus() * kMaxWgsPerCu * 2 * 1024;
  const size_t cnt_bytes = (size_t)(s->max_tiles + kKeyGroups + 1) * kCounterStride * 4;
  // argmax keys, then a zero activation row of max_in bf16 (never written)
  const size_t key_bytes = (size_t)kKeyGroups * 16 * 8 + (size_t)max_in * 2 + 256;
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
  (void)splits;
  if (M > s->max_m || (out_f + kTileN - 1) / kTileN > s->max_tiles) return QW4_ERR_SCRATCH;
  const size_t need = (size_t)launch_for<OUT_BF16>(out_f, s->max_in / kGroup).P * 2 * 1024;
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
