// Decode GEMV (M = 1), speculative-verify skinny GEMM (M = 2..16) and the
// lm_head GEMV with a fused fp32 row-argmax: two gfx950 kernels.
//
// k_dec (M = 1, 4-bit weights, every epilogue): integer MFMA. Each 128-group
// of x becomes exact 3-byte fixed point (int8 rows of the A operand of
// v_mfma_i32_16x16x64_i8), the packed nibbles are masked into int8 B operands
// (3 VALU per word), and the zero point and scale are applied per row and
// group in int32 / fp32. Items (one group of a 32-row unit: 2 KiB of weights
// plus a 160-byte scale/zero-point record) stream into per-wave LDS slots.
//
// k_rows (M > 1, the 8-bit head, and M = 1 shapes k_dec does not take): bf16
// MFMA. A 64-row tile of packed weights is split into 4 KiB (tile, group)
// blocks (8 KiB for 8-bit weights). Lane c + 16q of a wave reads chunk q of
// positions 16 st + c, i.e. rows 4c + st, and feeds v_mfma_f32_16x16x32_bf16:
//    A = activations, 16 rows (rows >= M unused), 32 k per instruction
//    B = the packed word turned into 8 bf16 values (128 + q) by AND-OR
// Four instructions per row quad st cover the group; a fifth B operand of ones
// gives S_m = sum_k x[m][k] in the same output layout, so the zero-point and
// +128 correction is
//    acc[m][n] += s[n] * (C[m][n] - (128 + zp[n]) * S_m)
// (the reference's identity, src/kernels/gemv_w4a16.cuh:25-37, with the group
// sum computed by the matrix core instead of a prologue kernel).
//
// Both are data-parallel: a workgroup owns whole units (S row quads of a tile
// over all of K), its waves split K and are summed in LDS in wave order; no
// workgroup exchanges partials with another, so a launch ends when its loads
// end and every output is bitwise reproducible (the property of
// gemv_w4a16.cu:262-279). Epilogues: bf16 / fp32 output, residual add, swiglu
// of gate|up pairs, rmsnorm of x in LDS before the projection, and the fused
// argmax.
//
// Output layout per lane (k_rows): acc[st][jj] is row m = 4q + jj, column
// n = 64*tile + 4c + st.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "../../include/qwen_w4a16.h"
#include "w4a16_common.h"

namespace qw4 {
// Cache policy of the decode kernels' weight loads: nontemporal (each byte is
// read once per call; measured 3-6% faster than the default policy).
constexpr int kWeightAux = 2;
int check_weights_public(const qw4_weights* w);

namespace {

// Epilogues of the skinny kernels:
//   OUT_BF16   y = bf16(acc)
//   OUT_F32    y = acc
//   OUT_ARGMAX the row argmax of acc (no logits written)
//   OUT_RES    y = bf16(res + bf16(acc)): linear then residual_add
//              (src/model/model.cu:781-783; y may be res)
//   OUT_SWIGLU y = bf16(silu(bf16(acc_gate)) * bf16(acc_up)) over a fused
//              [gate | up] weight: linear then swiglu (model.cu:776-778)
//   OUT_NORM   bf16 y of rmsnorm(x): rmsnorm then linear (model.cu:773-777)
enum { OUT_BF16 = 0, OUT_F32 = 1, OUT_ARGMAX = 2, OUT_RES = 3, OUT_SWIGLU = 4, OUT_NORM = 5 };

// Memory-side atomics on one cache line serialize; each counter gets its own line.
constexpr int kCounterStride = 32;
constexpr int kKeyGroups = 64;

struct SkinnyArgs {
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* zr;
  const uint16_t* x;
  void* y;
  uint32_t* counters;   // argmax arrival counters, one per 128-byte line
                        // (kCounterStride words): [0, 64) per key group,
                        // [64] of key groups
  uint64_t* keys;       // argmax keys [64 groups][16 rows], one line per group
  int M, N, K, G, tiles, P, U;
  uint32_t weight_bytes;   // packed weights (4- or 8-bit blocks)
  const uint16_t* res;     // OUT_RES: residual [M][N] (may be y)
  const uint16_t* nw;      // OUT_NORM: rmsnorm weight [K] (applied as 1 + w)
  float eps;               // OUT_NORM: rmsnorm epsilon
  int ld;                  // row stride of y (N; the intermediate size for OUT_SWIGLU)
};

// Monotonic key: larger value first, then lower index (elementwise.cu:103-104).
__device__ __forceinline__ uint64_t argmax_key(float v, int n) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(~(uint32_t)n);
}

// Arrival: release this workgroup's key updates, and acquire those of the
// workgroups counted before it (the last arriver then reads every key).
__device__ __forceinline__ uint32_t arrive_dev(uint32_t* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void clear_dev(uint32_t* p) {
  __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

// Workgroup p owns units [start(p), start(p + 1)).
__device__ __forceinline__ int range_start(const SkinnyArgs& a, int p) {
  return (int)((long long)p * a.U / a.P);
}

// Buffer-resource loads: a loop-invariant per-lane offset plus a wave-uniform
// scalar offset per block. Activation rows past M lie outside the x resource
// (M rows of K) and read as zeros without touching memory: for M = 1, 60 of
// the 64 lanes issue no activation traffic.
struct SkinnyRsrc {
  __amdgpu_buffer_rsrc_t qw, sc, zr, x;
};

__device__ __forceinline__ SkinnyRsrc skinny_rsrc(const SkinnyArgs& a) {
  SkinnyRsrc r;
  r.qw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.qw), 0, (int)a.weight_bytes,
                                           0x00020000);
  // 4-bit: 160-byte (scale, zero-point) records per block; 8-bit: 128 bytes of scales
  r.sc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.sc), 0,
      (int)((uint32_t)a.N / kTileN * (uint32_t)a.G * (a.zr ? (uint32_t)kMetaBytes : 128u)),
      0x00020000);
  r.zr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.zr), 0,
                                           a.zr ? (int)((uint32_t)a.N * (uint32_t)a.G / 2u) : 0,
                                           0x00020000);
  r.x = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.x), 0,
                                          (int)((uint32_t)a.M * (uint32_t)a.K * 2u), 0x00020000);
  return r;
}

// ------------------------------------------------------- 8-bit weights
// W8A16 (the reference's lm_head format, gemv_w4a16.cuh:141-166): per (row,
// 128-group) a bf16 scale and int8 q in [-127, 127], stored as the byte
// u = q + 128. Block = (64-row tile, group), 8 KiB: [4 j][64 p][32 B], position
// p holding row 4 (p % 16) + p / 16 as in the 4-bit layout, chunk j covering
// k = 128 g + 32 j + [0, 32) in natural byte order. A byte is an exact bf16
// (u <= 255 needs 8 significant bits); the offset is removed like the 4-bit
// zero point: acc += s (C - 128 S_m), with S_m from the ones operand.
// Eight bytes -> eight bf16 values (exact).
__device__ __forceinline__ bf16x8 bytes8_bf16(uint32_t lo, uint32_t hi) {
  u32x4 o;
  o[0] = pack_bf16x2((float)(lo & 0xffu), (float)((lo >> 8) & 0xffu));
  o[1] = pack_bf16x2((float)((lo >> 16) & 0xffu), (float)(lo >> 24));
  o[2] = pack_bf16x2((float)(hi & 0xffu), (float)((hi >> 8) & 0xffu));
  o[3] = pack_bf16x2((float)((hi >> 16) & 0xffu), (float)(hi >> 24));
  return __builtin_bit_cast(bf16x8, o);
}

// Lane offset of its 16-byte chunk inside a block, per weight format: chunk
// q of position c (4-bit: 1 KiB per chunk; 8-bit: 2 KiB, two 16-byte halves).
template <int FMT>
struct Fmt {
  __device__ static uint32_t woff(int q, int c) {
    return FMT == 8 ? (uint32_t)(q * 2048 + c * 32) : (uint32_t)(q * 1024 + c * 16);
  }
};

// ------------------------------------------------------------- epilogues
// Running argmax of one workgroup: per lane, the best (value, column) of rows
// m = 4q + jj over the elements this workgroup finished.
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

__device__ __forceinline__ void best_fold(Best& bs, int jj, float v, int n) {
  if (v > bs.v[jj] || (v == bs.v[jj] && n < bs.n[jj])) {
    bs.v[jj] = v;
    bs.n[jj] = n;
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
    uint32_t* gcnt = a.counters + (size_t)grp * kCounterStride;
    uint32_t* done = a.counters + (size_t)kKeyGroups * kCounterStride;
    // memory order: each workgroup's key updates happen before its release
    // increment of its group counter; the group's last arriver acquires them
    // and releases them on `done`, whose last arriver acquires all of them
    if (arrive_dev(gcnt) == in_grp - 1 && arrive_dev(done) == (uint32_t)(ngroups - 1)) {
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
        clear_dev(a.counters + (size_t)g2 * kCounterStride);
      }
      clear_dev(done);
    }
  }
}

// ------------------------------------------------------ data-parallel rows
// k_rows: workgroup p owns whole units [start(p), start(p + 1)); a unit is S
// row quads st0 .. st0 + S - 1 of one tile (16 S rows: 4c + st for lanes c)
// over all of K, split among the workgroup's W waves only and summed in LDS.
// No workgroup exchanges partial sums with another, so nothing is waited on
// at the end but the stores. Small units (S = 1: 16 rows) balance a launch
// over the CUs where whole 64-row tiles cannot.
// k_rows with activations in LDS: at most this many 16-byte chunks per thread
// (M K 2 <= kRowsXChunks * 16 * 64 W bytes); twice as many with LDS-DMA items
// (no item registers).
constexpr int kRowsXChunks = 4;
constexpr int rows_xchunks(bool dma) { return dma ? 2 * kRowsXChunks : kRowsXChunks; }
// k_rows with LDS-DMA items and M > 1 rows staged (XM, 8 waves): at most this
// many 16-byte chunks per thread
constexpr int kRowsXmChunks = 16;
constexpr int kLdsBytes = 160 * 1024;   // LDS per CU on gfx950


template <int FMT, int S, bool XL>
struct RowsData {
  u32x4 w[S][FMT == 8 ? 2 : 1];
  u32x4 x[XL ? 1 : 4];       // activations (registers) unless they sit in LDS
  uint32_t s[(S + 1) / 2];   // bf16 scales of rows 4c + st0 + i, two per word
  uint32_t z;                // zero points of rows 4c .. 4c + 3 (4-bit)
};

template <int FMT, int S, bool XL>
__device__ __forceinline__ void rows_load(RowsData<FMT, S, XL>& d, const SkinnyRsrc& r, uint32_t blk,
                                          int g, uint32_t woff, uint32_t soff, uint32_t zoff,
                                          uint32_t xoff) {
  constexpr uint32_t kBlk = FMT == 8 ? 8192u : 4096u;
  constexpr uint32_t kQuad = FMT == 8 ? 512u : 256u;   // bytes of one row quad in a chunk
  constexpr uint32_t kScB = FMT == 8 ? 128u : (uint32_t)kMetaBytes;   // scale bytes per block
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int h = 0; h < (FMT == 8 ? 2 : 1); ++h)
      d.w[i][h] = __builtin_amdgcn_raw_buffer_load_b128(r.qw, woff + i * kQuad + h * 16,
                                                        blk * kBlk, kWeightAux);
  if (!XL) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      d.x[t & (XL ? 0 : 3)] =
          __builtin_amdgcn_raw_buffer_load_b128(r.x, xoff + t * 16, (uint32_t)g * 256u, 0);
  }
  if (S == 4) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r.sc, soff, blk * kScB, 0);
    d.s[0] = v[0];
    d.s[(S + 1) / 2 - 1] = v[1];
  } else if (S == 2) {
    d.s[0] = __builtin_amdgcn_raw_buffer_load_b32(r.sc, soff, blk * kScB, 0);
  } else {
    // the aligned word holding this row's scale (half st0 & 1)
    d.s[0] = __builtin_amdgcn_raw_buffer_load_b32(r.sc, soff & ~3u, blk * kScB, 0);
  }
  // 32-bit loads only: a 16-bit load result gets masked right after the load,
  // which makes the compiler wait for it there (zoff: the aligned word holding
  // this lane's 16 bits)
  if (FMT == 4) d.z = __builtin_amdgcn_raw_buffer_load_b32(r.zr, zoff, blk * 32u, 0);
}

// ---- LDS-DMA items (k_rows with DMA): the weight, scale and zero-point
// loads of an item go straight into an LDS slot of the wave (buffer_load ...
// lds, lane i's bytes at slot + i * size), so the number of items in flight is
// bounded by LDS, not by registers. The compiler does not order LDS reads
// after these loads: each item waits with an explicit vmcnt (the loads issued
// after it, which complete after it) before reading its slot.
// Slot layout (16-byte units): NQ x 64 weight chunks, then a 256-byte area
// for the block's metadata, one 4-byte load per lane: 4-bit, the 160-byte
// (scale, zero-point) record (lane l < 40: word l; the others repeat word 0);
// 8-bit, the 128 bytes of scales (lane l: word l & 31). One metadata load per
// item instead of a scale and a zero-point load: every LDS-DMA instruction
// holds the CU's address unit ~16 cycles whatever its size.
template <int FMT, int S>
struct DmaSlot {
  static constexpr int kH = FMT == 8 ? 2 : 1;          // 16-byte chunks per row quad
  static constexpr int kNQ = S * kH;                     // weight loads per item
  static constexpr int kLoads = kNQ + 1;                 // loads per item
  static constexpr int kUnits = kNQ * 64 + 16;
};

// k_rows item slot with LDS-DMA items (16-byte units): DmaSlot's weights and
// metadata, then -- when the activations are not staged for the whole
// workgroup (!XL: M > 1 rows of a long K) -- the item's group of all 16
// activation rows (rows past M read as zeros), 16 chunks per row, chunk j of
// row r at unit 16 r + (j ^ r): the 16 lanes reading one k-chunk of rows
// 0..15 hit 16 different 16-byte bank groups.
template <int FMT, int S, bool XL>
constexpr int rows_slot_units() {
  return DmaSlot<FMT, S>::kUnits + (XL ? 0 : 256);
}

// 16 bytes per lane, nontemporal (weights); 4 bytes per lane (metadata)
__device__ __forceinline__ void dma_load16(__amdgpu_buffer_rsrc_t r, u32x4* dst, uint32_t voff,
                                           uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, soff, 0, kWeightAux);
}
// 16 bytes per lane, default cache policy (activations: every workgroup
// reads them, mostly from L2)
__device__ __forceinline__ void dma_load16c(__amdgpu_buffer_rsrc_t r, u32x4* dst, uint32_t voff,
                                            uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, soff, 0, 0);
}
__device__ __forceinline__ void dma_load4(__amdgpu_buffer_rsrc_t r, u32x4* dst, uint32_t voff,
                                          uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4,
                                           voff, soff, 0, 0);
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for LDS data written by ds_write. With LDS-DMA loads in
// flight __syncthreads() would also wait for all of them (its fence counts
// them as LDS writes); the unit sums only need this wave's LDS writes done.
template <bool DMA>
__device__ __forceinline__ void lds_barrier() {
  if constexpr (DMA)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else
    __syncthreads();
}

template <int J, int D, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (J < D) {
    f(std::integral_constant<int, J>{});
    static_for<J + 1, D>(f);
  }
}

// Wait until at most n items' loads (kL each) of this wave are outstanding,
// n in [0, D) known only at run time (the immediate needs a switch).
template <int kL, int D>
__device__ __forceinline__ void wait_items(int n) {
  static_for<0, D>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if (n == i) wait_vm<i * kL>();
  });
}


template <int FMT, int S>
__device__ __forceinline__ void dma_issue(u32x4* slot, const SkinnyRsrc& r, uint32_t blk,
                                          uint32_t woff, int lane) {
  using L = DmaSlot<FMT, S>;
  constexpr uint32_t kBlk = FMT == 8 ? 8192u : 4096u;
  constexpr uint32_t kQuad = FMT == 8 ? 512u : 256u;
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int h = 0; h < L::kH; ++h)
      dma_load16(r.qw, slot + (i * L::kH + h) * 64, woff + i * kQuad + h * 16, blk * kBlk);
  if (FMT == 4)
    dma_load4(r.sc, slot + L::kNQ * 64, lane < 40 ? (uint32_t)lane * 4u : 0u,
              blk * (uint32_t)kMetaBytes);
  else
    dma_load4(r.sc, slot + L::kNQ * 64, (uint32_t)(lane & 31) * 4u, blk * 128u);
}

template <int FMT, int S, bool XL>
__device__ __forceinline__ void dma_read(RowsData<FMT, S, XL>& d, const u32x4* slot, int lane,
                                         int st0) {
  using L = DmaSlot<FMT, S>;
  const int c = lane & 15;
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int h = 0; h < L::kH; ++h) d.w[i][h] = slot[(i * L::kH + h) * 64 + lane];
  const uint32_t* sm = reinterpret_cast<const uint32_t*>(slot + L::kNQ * 64);
  if (S == 4) {
    d.s[0] = sm[2 * c];
    d.s[(S + 1) / 2 - 1] = sm[2 * c + 1];
  } else {
    d.s[0] = sm[(4 * c + st0) >> 1];
  }
  if (FMT == 4) d.z = sm[32 + (c >> 1)];   // the record's copy of the zero-point words
}

// XL: activations come from LDS (xl: this lane's row, k chunk q, group g);
// otherwise from the registers rows_load filled. JJ: the output rows
// m = 4q + jj, jj < JJ, that are accumulated (M = 1: only jj = 0 is read).
template <int FMT, int S, bool XL, int JJ = 4>
__device__ __forceinline__ void rows_mma(f32x4 (&acc)[S], const RowsData<FMT, S, XL>& d, NibConst k,
                                         int st0, int zsh, const u32x4* xl) {
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u,
                                                       0x3F803F80u, 0x3F803F80u});
  f32x4 C[S], Cs;
  u32x4 xr[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) xr[t] = XL ? xl[t] : d.x[t & (XL ? 0 : 3)];
  // Scale and zero point first, pinned here: the loaded words must be dead
  // before the caller reloads this buffer, or the compiler keeps both copies
  // and moves them at the loop's back edge (waiting for the newest loads).
  float sf[S], zf[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const uint32_t sbits = (d.s[i >> 1] >> (16 * (S == 1 ? (st0 & 1) : (i & 1)))) & 0xffffu;
    sf[i] = bf16_bits_to_f32(sbits);
    zf[i] = FMT == 4 ? 128.0f + (float)((d.z >> (zsh + 4 * (st0 + i))) & 0xFu) : 128.0f;
    // staged activations (M = 1): pinned here, so the loaded words are dead
    // before the caller reloads the buffer (measured 1% faster; with
    // activations in registers the extra live values would spill)
    if (XL) asm volatile("" : "+v"(sf[i]), "+v"(zf[i])::"memory");
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const bf16x8 A = __builtin_bit_cast(bf16x8, xr[t]);
#pragma unroll
    for (int i = 0; i < S; ++i) {
      bf16x8 B;
      if (FMT == 4) {
        B = nib8(d.w[i][0][t], k);
      } else {
        const u32x4 v = d.w[i][(t >> 1) & (FMT == 8 ? 1 : 0)];
        B = bytes8_bf16(v[(t & 1) * 2], v[(t & 1) * 2 + 1]);
      }
      C[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          A, B, t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : C[i], 0, 0, 0);
    }
    Cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, ones,
                                                 t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : Cs,
                                                 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj) acc[i][jj] += sf[i] * (C[i][jj] - zf[i] * Cs[jj]);
}

// Final values of one unit (wave 0): rows m = 4q + jj, columns b*64 + 4c + st0 + i.
template <int OUT, int S>
__device__ __forceinline__ void emit_rows(const SkinnyArgs& a, int b, int st0,
                                          const f32x4 (&acc)[S], int lane, Best& bs) {
  const int c = lane & 15, q = lane >> 4;
  const int n0 = b * kTileN + 4 * c + st0;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int m = 4 * q + jj;
    if (OUT == OUT_ARGMAX) {
#pragma unroll
      for (int i = 0; i < S; ++i) best_fold(bs, jj, acc[i][jj], n0 + i);
      continue;
    }
    if (m >= a.M) continue;
    if (OUT == OUT_RES) {
      // bf16(res + bf16(acc)), the reference's linear then residual_add
      uint16_t* y = static_cast<uint16_t*>(a.y) + (size_t)m * a.ld + n0;
      const uint16_t* r = a.res + (size_t)m * a.ld + n0;
#pragma unroll
      for (int i = 0; i < S; ++i)
        y[i] = to_bf16(bf16_bits_to_f32(r[i]) + bf16_bits_to_f32(to_bf16(acc[i][jj])));
    } else if (OUT == OUT_BF16 || OUT == OUT_NORM) {
      uint16_t* y = static_cast<uint16_t*>(a.y) + (size_t)m * a.ld + n0;
      if (S == 4)
        *reinterpret_cast<u32x2*>(y) = u32x2{pack_bf16x2(acc[0][jj], acc[1 % S][jj]),
                                             pack_bf16x2(acc[2 % S][jj], acc[3 % S][jj])};
      else if (S == 2)
        *reinterpret_cast<uint32_t*>(y) = pack_bf16x2(acc[0][jj], acc[1 % S][jj]);
      else
        *y = to_bf16(acc[0][jj]);
    } else {
      float* y = static_cast<float*>(a.y) + (size_t)m * a.ld + n0;
#pragma unroll
      for (int i = 0; i < S; ++i) y[i] = acc[i][jj];
    }
  }
}


// OUT_SWIGLU (wave 0): gate rows of tile b (the intermediate index), their up
// rows' sums in u.
template <int S>
__device__ __forceinline__ void emit_swiglu(const SkinnyArgs& a, int b, int st0,
                                            const f32x4 (&g)[S], const f32x4 (&u)[S], int lane) {
  const int c = lane & 15, q = lane >> 4;
  const int n0 = b * kTileN + 4 * c + st0;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int m = 4 * q + jj;
    if (m >= a.M) continue;
    uint16_t* y = static_cast<uint16_t*>(a.y) + (size_t)m * a.ld + n0;
#pragma unroll
    for (int i = 0; i < S; ++i) y[i] = swiglu_bf16_bits(to_bf16(g[i][jj]), to_bf16(u[i][jj]));
  }
}

// k_rows: workgroup p owns the whole units [start(p), start(p + 1)). Each
// wave walks its items (unit u, group g), g = wave, wave + W, ... < G, over
// those units in order, D items ahead of the math (the next loads are issued
// across unit boundaries too). Buffer j holds items j, j + D, ...: the loop is
// unrolled by D, so no buffer is ever copied (a register copy would have to
// wait for its load and drain the pipeline every item), and every item issues
// the same loads -- past the end they are out of range and return zeros with
// no traffic -- so the wait counts are static. Every wave closes every unit:
// it writes its partial (zero if it had no item) to one of two LDS buffers
// and passes one barrier, so the waves stay in step for any G; wave 0 then
// sums the W partials in wave order and emits the unit. No workgroup depends
// on another.
// DMA: items' weights and metadata are loaded into LDS slots (DmaSlot)
// instead of registers, D per wave after the staged activations (if any).
// With XL (M = 1) the one output row sits in lanes 0..15 (element jj = 0), so
// only those lanes take part in the unit sums and only that element is
// accumulated; without (M > 1) each item's activations still go to registers,
// loaded with the item.
template <int OUT, int FMT, int S, int W, bool XL, int D, bool DMA = false, bool XM = false>
__global__ __launch_bounds__(64 * W) void k_rows(SkinnyArgs a) {
  // LDS-DMA items with staged activations: M = 1, or (XM) M > 1 with each
  // activation row padded by one 16-byte chunk, so that the 16 lanes reading
  // one k-chunk of 16 different rows hit different banks
  static_assert(!XM || (DMA && XL && OUT != OUT_NORM), "XM: staged rows, LDS-DMA items");
  constexpr bool kM1 = DMA && XL && !XM;
  constexpr uint32_t kPer = 4 / S;   // units per tile (unit indices are never negative)
  constexpr uint32_t kQuad = FMT == 8 ? 512u : 256u;
  constexpr int kRedLanes = kM1 ? 16 : 64;
  // XM, and 8-bit items with their activations in the slots: one buffer (LDS),
  // a second barrier per unit
  constexpr int kRedBufs = (XM || (DMA && !XL && FMT == 8)) ? 1 : 2;
  constexpr int kXC = XM ? kRowsXmChunks : rows_xchunks(DMA);
  __shared__ f32x4 red[kRedBufs][W][S][kRedLanes];
  extern __shared__ u32x4 xlds[];
  // wave-uniform (scalar) so the item cursors live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const SkinnyRsrc rs = skinny_rsrc(a);
  const uint32_t xoff = (uint32_t)(c * a.K + 32 * q) * 2u;
  const uint32_t zoff = (uint32_t)(c & ~1) * 2u;   // word with this lane's zero points
  const int zsh = 16 * (c & 1);
  const uint32_t wbase = Fmt<FMT>::woff(q, c);
  const int p = blockIdx.x;
  // OUT_SWIGLU: units come in pairs (gate unit v, its up unit v + U / 2),
  // numbered 2v and 2v + 1 and never split between workgroups
  const int u0 = OUT == OUT_SWIGLU ? 2 * (int)((long long)p * (a.U / 2) / a.P) : range_start(a, p);
  const int u1 =
      OUT == OUT_SWIGLU ? 2 * (int)((long long)(p + 1) * (a.U / 2) / a.P) : range_start(a, p + 1);
  auto real_unit = [&](int v) {
    return OUT == OUT_SWIGLU ? ((v & 1) ? (v >> 1) + (int)((uint32_t)a.U / 2u) : (v >> 1)) : v;
  };
  const NibConst k = nib_const();
  Best bs;
  best_init(bs);

  const int nw = wave < a.G ? (a.G - 1 - wave) / W + 1 : 0;   // items per unit
  const int T = nw * (u1 - u0);
  const uint32_t oob_blk = (uint32_t)a.tiles * (uint32_t)a.G;
  int lu = u0, lg = wave;   // load cursor (wave-uniform)
  auto load_next = [&](RowsData<FMT, S, XL>& d) {
    const bool in = lu < u1;
    const int ru = real_unit(lu);
    const int b = in ? (int)((uint32_t)ru / kPer) : 0;
    const int st0 = in ? (int)((uint32_t)ru % kPer) * S : 0;
    const int g = in ? lg : 0;
    rows_load<FMT, S, XL>(d, rs, in ? (uint32_t)b * (uint32_t)a.G + (uint32_t)g : oob_blk, g,
                          wbase + (uint32_t)st0 * kQuad, (uint32_t)(4 * c + st0) * 2u, zoff,
                          xoff);
    lg += W;
    if (lg >= a.G) {
      lg = wave;
      ++lu;
    }
  };

  RowsData<FMT, S, XL> buf[kM1 ? 1 : D];
  const int xs16 = a.K / 8 + (XM ? 1 : 0);   // staged row stride, 16-byte chunks
  constexpr int kSlotU = rows_slot_units<FMT, S, XL>();
  u32x4* const ring = xlds + (XL ? a.M * xs16 : 0) + wave * D * kSlotU;
  // !XL: lane l of activation load t fetches row 4 t + l / 16, chunk
  // (l % 16) ^ row, into slot unit 64 t + l (see rows_slot_units)
  const int xr_ = lane >> 4, xj_ = lane & 15;
  uint32_t xdoff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    xdoff[t] = (uint32_t)(4 * t + xr_) * (uint32_t)a.K * 2u +
               (uint32_t)((xj_ ^ (4 * t + xr_)) & 15) * 16u;
  auto load_slot = [&](int j) __attribute__((always_inline)) {
    const bool in = lu < u1;
    const int ru = real_unit(lu);
    const int b = in ? (int)((uint32_t)ru / kPer) : 0;
    const int st0 = in ? (int)((uint32_t)ru % kPer) * S : 0;
    const int g = in ? lg : 0;
    dma_issue<FMT, S>(ring + j * kSlotU, rs,
                      in ? (uint32_t)b * (uint32_t)a.G + (uint32_t)g : oob_blk,
                      wbase + (uint32_t)st0 * kQuad, lane);
    if (!XL) {
      u32x4* const xs = ring + j * kSlotU + DmaSlot<FMT, S>::kUnits;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        dma_load16c(rs.x, xs + 64 * t, xdoff[t], (uint32_t)g * 256u);
    }
    lg += W;
    if (lg >= a.G) {
      lg = wave;
      ++lu;
    }
  };
  const u32x4* xrow = xlds + (c < a.M ? c : a.M - 1) * xs16 + 4 * q;
  auto prime = [&]() {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      if constexpr (DMA)
        load_slot(j);
      else
        load_next(buf[j & (DMA ? 0 : 0xff)]);
    }
  };
  if (XL) {
    // x loads first, then the first weight items: waiting for x leaves the
    // weights in flight (loads complete in order). A wave issues a round of
    // loads only if it has chunks in range (a 16-byte load of a wave holds
    // the CU's address unit for ~16 cycles whatever its addresses); its lanes
    // past the last chunk load that chunk again. Only in-range chunks are
    // stored (a wave storing one address from every lane serializes on one
    // LDS bank).
    const int n16 = a.M * a.K / 8;
    u32x4 xv[kXC], nv[OUT == OUT_NORM ? kXC : 1];
    int xi[kXC];
    const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.nw), 0, OUT == OUT_NORM ? a.K * 2 : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < kXC; ++j) {
      xi[j] = min((int)threadIdx.x + j * 64 * W, n16 - 1);
      xv[j] = u32x4{0u, 0u, 0u, 0u};
      nv[j & (OUT == OUT_NORM ? 0xff : 0)] = u32x4{0u, 0u, 0u, 0u};
      if (64 * wave + j * 64 * W < n16) {   // wave-uniform: this wave has chunks in range
        xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rs.x, (uint32_t)xi[j] * 16u, 0, 0);
        if (OUT == OUT_NORM)
          nv[j & (OUT == OUT_NORM ? 0xff : 0)] = __builtin_amdgcn_raw_buffer_load_b128(
              rn, (uint32_t)(xi[j] % (a.K / 8)) * 16u, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    prime();
#pragma unroll
    for (int j = 0; j < kXC; ++j)
      if ((int)threadIdx.x + j * 64 * W < n16) xlds[XM ? xi[j] + xi[j] / (a.K / 8) : xi[j]] = xv[j];
    lds_barrier<DMA>();
    if (OUT == OUT_NORM) {
      // rmsnorm of each row in place (src/kernels/elementwise.cu:8-31):
      // x * rsqrt(mean(x^2) + eps) * (1 + w), fp32, rounded to bf16 once; the
      // sum of squares of row m in the shared order (norm_sumsq), thread t
      // standing for virtual threads t + 64 W k and reading the staged row
      constexpr int kP = kNormVThreads / (64 * W);
      static_assert(kNormVThreads % (64 * W) == 0, "workgroup of 1024 / kP threads");
      __shared__ float vsum[16][kNormVWaves];
      const int kc = a.K / 8;
      for (int m = 0; m < a.M; ++m) {
#pragma unroll
        for (int k = 0; k < kP; ++k) {
          float ss = 0.f;
          for (int i = (int)threadIdx.x + 64 * W * k; i < kc; i += kNormVThreads)
            ss = norm_sumsq(ss, xlds[m * kc + i]);
          ss = norm_wave_sum(ss);
          if (lane == 0) vsum[m][wave + W * k] = ss;
        }
      }
      lds_barrier<DMA>();
#pragma unroll
      for (int j = 0; j < kXC; ++j) {
        if ((int)threadIdx.x + j * 64 * W >= n16) continue;
        const float inv = norm_inv(vsum[xi[j] / kc], a.K, a.eps);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t xw = xv[j][e], ww = nv[j & (OUT == OUT_NORM ? 0xff : 0)][e];
          o[e] = pack_bf16x2(rmsnorm_f32(xw, ww, inv), rmsnorm_f32(xw >> 16, ww >> 16, inv));
        }
        xlds[xi[j]] = o;
      }
      lds_barrier<DMA>();
    }
  } else {
    prime();
  }

  f32x4 acc[S];
#pragma unroll
  for (int i = 0; i < S; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  int par = 0, closed = u0;
  f32x4 gate[OUT == OUT_SWIGLU ? S : 1];   // OUT_SWIGLU: the gate unit's sums (wave 0)
  auto close_unit = [&]() {
    if (!kM1 || lane < kRedLanes) {
#pragma unroll
      for (int i = 0; i < S; ++i) red[par % kRedBufs][wave][i][lane % kRedLanes] = acc[i];
    }
    lds_barrier<DMA>();
    if (wave == 0) {
      const int rl = lane % kRedLanes;
      f32x4 t[S];
#pragma unroll
      for (int i = 0; i < S; ++i) t[i] = red[par % kRedBufs][0][i][rl];
      for (int w = 1; w < W; ++w)
#pragma unroll
        for (int i = 0; i < S; ++i) t[i] += red[par % kRedBufs][w][i][rl];
      if (OUT == OUT_SWIGLU) {
        const int gu = closed >> 1;   // the gate unit (= the output unit)
        if ((closed & 1) == 0) {
#pragma unroll
          for (int i = 0; i < S; ++i) gate[i & (OUT == OUT_SWIGLU ? 0xff : 0)] = t[i];
        } else {
          f32x4 g[S];
#pragma unroll
          for (int i = 0; i < S; ++i) g[i] = gate[i & (OUT == OUT_SWIGLU ? 0xff : 0)];
          emit_swiglu<S>(a, (int)((uint32_t)gu / kPer), (int)((uint32_t)gu % kPer) * S, g, t,
                         lane);
        }
      } else {
        emit_rows<OUT, S>(a, (int)((uint32_t)closed / kPer), (int)((uint32_t)closed % kPer) * S, t,
                          lane, bs);
      }
    }
    if (kRedBufs == 1) lds_barrier<DMA>();   // wave 0 has read the buffer
    par ^= 1;
    ++closed;
#pragma unroll
    for (int i = 0; i < S; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  int cg = wave;   // compute cursor: unit `closed`, group cg
  auto step = [&](RowsData<FMT, S, XL>& d, bool reload) {
    rows_mma<FMT, S, XL>(acc, d, k, (int)((uint32_t)real_unit(closed) % kPer) * S, zsh,
                         xrow + cg * 16);
    if (reload) load_next(d);
    cg += W;
    if (cg >= a.G) {
      cg = wave;
      close_unit();
    }
  };
  // whole rounds of D items with no conditional loads (a conditional load
  // would make the compiler's wait counts assume the shortest path), then
  // the last < D items, already loaded
  int t0 = 0;
  if constexpr (DMA) {
    // item t waits for its slot; the loads of the items after it (all D - 1
    // of them in the main loop, fewer in the tail) may still be in flight
    constexpr int kL = DmaSlot<FMT, S>::kLoads + (XL ? 0 : 4);
    auto step_dma = [&](auto jc, auto nc, bool reload, int nwait = 0) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      if constexpr (decltype(nc)::value >= 0)
        wait_vm<decltype(nc)::value>();
      else
        wait_items<kL, D>(nwait);
      const int st0 = (int)((uint32_t)real_unit(closed) % kPer) * S;
      RowsData<FMT, S, XL> d;
      dma_read<FMT, S, XL>(d, ring + j * kSlotU, lane, st0);
      if constexpr (!XL) {
        // row c, k-chunk 4 q + t (the k order of the register form, xoff)
        const u32x4* xs = ring + j * kSlotU + DmaSlot<FMT, S>::kUnits + 16 * c;
#pragma unroll
        for (int t = 0; t < 4; ++t) d.x[t & (XL ? 0 : 3)] = xs[(4 * q + t) ^ c];
      }
      rows_mma<FMT, S, XL, kM1 ? 1 : 4>(acc, d, k, st0, zsh, xrow + cg * 16);
      if (reload) {
        // the slot's LDS reads have returned before it is loaded again
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        load_slot(j);
      }
      cg += W;
      if (cg >= a.G) {
        cg = wave;
        close_unit();
      }
    };
    // whole batches whose reloads are all real items, then the last r < 2 D
    // items: item j reloads only a real item (j + D < r) and waits for the
    // min(D - 1, r - 1 - j) items loaded after it (no load is issued past
    // the last item: an out-of-range LDS-DMA load costs as much as a real one)
    for (; t0 + 2 * D <= T; t0 += D)
      static_for<0, D>([&](auto jc) {
        step_dma(jc, std::integral_constant<int, (D - 1) * kL>{}, true);
      });
    const int r = T - t0;
    static_for<0, 2 * D - 1>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if (j < r)
        step_dma(std::integral_constant<int, j % D>{}, std::integral_constant<int, -1>{},
                 j + D < r, min(D - 1, r - 1 - j));
    });
  } else {
    for (; t0 + D <= T; t0 += D) {
#pragma unroll
      for (int j = 0; j < D; ++j) step(buf[j & (DMA ? 0 : 0xff)], true);
    }
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
      if (t0 + j < T) step(buf[j & (DMA ? 0 : 0xff)], false);
  }
  while (closed < u1) close_unit();   // waves with no items (wave >= G)
  if (OUT == OUT_ARGMAX && wave == 0) argmax_arrive(a, p, bs, lane);
  // loads issued past the last item land in LDS: done before the workgroup
  // releases it
  if constexpr (DMA) wait_vm<0>();
}

// ------------------------------------- verify, several units per workgroup
// k_rows_gm: M > 1, 4-bit weights, 32-row units, 8 waves, for shapes where
// every workgroup owns n units, kGmMinU <= n <= kGmMaxU (gate|up: 4 or 5).
// k_rows loads an item's group of the 16 activation rows with every item, so
// a workgroup fetches each activation group n times; here the items run
// group-major -- wave w takes groups g = w + W gi and, for each, first loads
// the group's activation rows once into one of two activation slots (four
// 1 KiB LDS-DMA loads), then the n weight items (u0 + ui, g) into a ring of
// kGmD weight slots -- so the activations are fetched once per workgroup and
// group. Each wave keeps the n units' sums and the units are summed over the
// waves at the end. Math per item and the unit sums' order are k_rows's, so
// the results are bitwise equal to k_rows with LDS-DMA items.
// Slot reuse: the activation slot of group gi + 2 is loaded with the first
// item of that group, kGmD items before it is consumed, when every item of
// group gi (n >= kGmD of them) has been consumed.
constexpr int kGmD = 3;      // weight items in flight per wave
constexpr int kGmMinU = 3;   // = kGmD: the activation slots' reuse rule
constexpr int kGmMaxU = 6;   // unit sums kept per wave

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 15].
__device__ __forceinline__ void wait_vm_rt(int n) {
  static_for<0, 16>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if (n == i) wait_vm<i>();
  });
}

__host__ __device__ constexpr int gm_wave_units() {
  return kGmD * DmaSlot<4, 2>::kUnits + 2 * 256;
}

template <int OUT>
__global__ __launch_bounds__(512) void k_rows_gm(SkinnyArgs a) {
  constexpr int FMT = 4, S = 2, W = 8, D = kGmD;
  constexpr uint32_t kPer = 4 / S;
  constexpr uint32_t kQuad = 256u;
  constexpr int kWU = DmaSlot<FMT, S>::kUnits;
  constexpr int kLw = DmaSlot<FMT, S>::kLoads;   // loads of a weight item
  constexpr int kLx = 4;                         // loads of an activation group
  static_assert(kLw + kLx + kLw <= 15, "wait range");
  __shared__ f32x4 red[2][W][S][64];
  extern __shared__ u32x4 gm_lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const SkinnyRsrc rs = skinny_rsrc(a);
  const int zsh = 16 * (c & 1);
  const uint32_t wbase = Fmt<FMT>::woff(q, c);
  const int p = blockIdx.x;
  const int u0 = range_start(a, p), n = range_start(a, p + 1) - u0;   // kGmMinU..kGmMaxU
  const NibConst k = nib_const();
  Best bs;
  best_init(bs);
  u32x4* const wring = gm_lds + wave * gm_wave_units();
  u32x4* const xring = wring + D * kWU;
  const int xr_ = lane >> 4, xj_ = lane & 15;
  uint32_t xdoff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    xdoff[t] = (uint32_t)(4 * t + xr_) * (uint32_t)a.K * 2u +
               (uint32_t)((xj_ ^ (4 * t + xr_)) & 15) * 16u;

  const int ng = wave < a.G ? (a.G - 1 - wave) / W + 1 : 0;   // groups of this wave
  const int T = ng * n;                                        // items of this wave
  // load cursor (wave-uniform): group index lgi, unit index lui
  int lgi = 0, lui = 0;
  // issue the next item into weight slot j; returns its load count
  auto issue = [&](int j) __attribute__((always_inline)) -> int {
    const int g = wave + W * lgi;
    int nl = kLw;
    if (lui == 0) {   // the group's first item: its activation rows first
      u32x4* const xs = xring + (lgi & 1) * 256;
#pragma unroll
      for (int t = 0; t < 4; ++t) dma_load16c(rs.x, xs + 64 * t, xdoff[t], (uint32_t)g * 256u);
      nl += kLx;
    }
    const int u = u0 + lui;
    const int st0 = (int)((uint32_t)u % kPer) * S;
    dma_issue<FMT, S>(wring + j * kWU, rs, (uint32_t)((uint32_t)u / kPer) * (uint32_t)a.G + (uint32_t)g,
                      wbase + (uint32_t)st0 * kQuad, lane);
    if (++lui == n) {
      lui = 0;
      ++lgi;
    }
    return nl;
  };
  // load counts of the items in flight after the one being consumed (FIFO)
  int f1 = 0, f2 = 0;
  static_assert(D == 3, "FIFO of two");
  int li = 0;   // items issued
  const int np = T < D ? T : D;
  int f0 = 0;
  if (np > 0) f0 = issue(0);
  if (np > 1) f1 = issue(1);
  if (np > 2) f2 = issue(2);
  li = np;

  f32x4 acc[kGmMaxU][S];
#pragma unroll
  for (int ui = 0; ui < kGmMaxU; ++ui)
#pragma unroll
    for (int i = 0; i < S; ++i) acc[ui][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  int j = 0;   // weight slot of the item being consumed
  for (int gi = 0; gi < ng; ++gi) {
    const u32x4* const xs = xring + (gi & 1) * 256 + 16 * c;
    static_for<0, kGmMaxU>([&](auto uc) {
      constexpr int ui = decltype(uc)::value;
      if (ui < n) {
        wait_vm_rt(f1 + f2);   // this item's loads (and its group's rows) have landed
        const int u = u0 + ui;
        const int st0 = (int)((uint32_t)u % kPer) * S;
        RowsData<FMT, S, false> d;
        dma_read<FMT, S, false>(d, wring + j * kWU, lane, st0);
#pragma unroll
        for (int t = 0; t < 4; ++t) d.x[t] = xs[(4 * q + t) ^ c];
        rows_mma<FMT, S, false>(acc[ui], d, k, st0, zsh, nullptr);
        // the slot's LDS reads have returned before it is loaded again
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        int fn = 0;
        if (li < T) {
          fn = issue(j);
          ++li;
        }
        f0 = f1;
        f1 = f2;
        f2 = fn;
        j = j + 1 == D ? 0 : j + 1;
      }
    });
  }
  (void)f0;
  // unit sums over the waves, in wave order (k_rows's close_unit)
  static_for<0, kGmMaxU>([&](auto uc) {
    constexpr int ui = decltype(uc)::value;
    if (ui < n) {
#pragma unroll
      for (int i = 0; i < S; ++i) red[ui & 1][wave][i][lane] = acc[ui][i];
      lds_barrier<true>();
      if (wave == 0) {
        f32x4 t[S];
#pragma unroll
        for (int i = 0; i < S; ++i) t[i] = red[ui & 1][0][i][lane];
        for (int w = 1; w < W; ++w)
#pragma unroll
          for (int i = 0; i < S; ++i) t[i] += red[ui & 1][w][i][lane];
        const int u = u0 + ui;
        emit_rows<OUT, S>(a, (int)((uint32_t)u / kPer), (int)((uint32_t)u % kPer) * S, t, lane, bs);
      }
    }
  });
  wait_vm<0>();   // no load lands in LDS after the workgroup released it
}

// ------------------------------------------------- decode with integer MFMA
// k_dec: M = 1, 4-bit weights. The work split and epilogues are k_rows's
// (whole units per workgroup, waves split K, unit sums in LDS in wave order);
// items are loaded into registers, D per wave (or into LDS slots, DMA); the
// math per item is integer:
//  * activations: each 128-group of x (bf16) is written as the integers
//    X = rne(x * 2^e_g), e_g chosen so that max |X| lies in [2^20, 2^21) --
//    exact for every element within 13 binades of the group's largest, and
//    within 2^-22 of it for the rest -- and split into bytes,
//    X = 65536 a + 256 b + c with a in [-32, 32], b, c in [-128, 127]: rows 0,
//    1, 2 of the int8 A operand of v_mfma_i32_16x16x64_i8 (rows 3..15 repeat
//    row 2; their outputs are not used). Per group the LDS also holds 2^-e_g,
//    -sum(256 a + b) and -sum c.
//  * weights: the low nibbles of a lane's four packed words (w & 0x0F0F0F0F)
//    and the high ones ((w >> 4) & 0x0F0F0F0F) are two int8 B operands of 16 k
//    each (the activation layout follows the nibble order): 3 VALU per word,
//    and 2 MFMAs per row quad and group give all three byte rows.
//  * per row and group, exact in int32 (|V1| <= 15 * 2^13 * 128):
//    V1 = 256 D[0] + D[1] - zp * sum(256 a + b),  V2 = D[2] - zp * sum c,
//    acc += (256 V1 + V2) * (s * 2^-e_g) in fp32.
// The activation rounding is the only departure from the exact dot product
// (relative 2^-21 per element at most); the rest is fp32 accumulation.
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kDecPrepIters = 8;   // per-wave prep rounds of 4 groups: G <= 32 W
constexpr int kDecQ = 24;          // 16-byte operand chunks per group in LDS

// Row-of-16 reductions (DPP): xor 1, xor 2, half-row mirror, row mirror.
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}
__device__ __forceinline__ int row16_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  return v;
}
__device__ __forceinline__ int sum4_i8(uint32_t w, int acc) {
  return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}

// Activation operands of one group in LDS (384 bytes): parts
// [L_a | L_b | L_c | H_a | H_b | H_c] x [k chunk q][word r][byte b], where
// L / H are the k held in the low / high nibbles of a weight byte:
// k = 128 g + 32 q + 8 r + {0, 4, 1, 5}[b] (L) or {2, 6, 3, 7}[b] (H).
// The lane that prepares chunk c16 = 4 q + r of group g (8 bf16 in v) writes
// word c16 of each part and, for c16 = 0, the group's constants.
__device__ __forceinline__ void dec_prep_chunk(uint32_t* xw, u32x4* cst, int g, int c16,
                                               const u32x4& v, bool valid) {
  float f[8];
  uint32_t m = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(v[e] << 16);
    f[2 * e + 1] = __uint_as_float(v[e] & 0xffff0000u);
    m = max(m, max(v[e] << 17 >> 1, v[e] & 0x7fff0000u));
  }
  m = row16_max(m);   // |x| bits of the group's largest element
  // 2^sh scales it into [2^20, 2^21): 1.5 * 2^23 + 0x8080 + X stays in
  // [2^23, 2^24), where the fp32 ulp is 1
  // A group holding Inf or NaN (exponent 255) gets a NaN constant, so every
  // output is NaN, as the reference's fp32 group sum gives (Inf - Inf). A group
  // whose largest |x| is an fp32 subnormal (below 2^-126) keeps the cap 2^126:
  // its terms then round to ~0, an absolute error below 2^-100 per output.
  const int sh = min(20 - ((int)(m >> 23) - 127), 126);
  const float p2 = __uint_as_float((uint32_t)(sh + 127) << 23);
  const float inv = (m >> 23) >= 255u ? __uint_as_float(0x7fc00000u)
                                      : __uint_as_float((uint32_t)(127 - sh) << 23);
  // T = X + 0x8080: byte 0 = c + 128, byte 1 = b + 128, byte 2 = a
  uint32_t t[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    t[j] = __float_as_uint(__builtin_fmaf(f[j], p2, 12615808.0f)) - 0x4B400000u;
  uint32_t o[6];
#pragma unroll
  for (int h = 0; h < 2; ++h) {   // L: elements 0, 4, 1, 5; H: 2, 6, 3, 7
    const uint32_t e0 = t[2 * h], e4 = t[2 * h + 4], e1 = t[2 * h + 1], e5 = t[2 * h + 5];
    const uint32_t pa = __builtin_amdgcn_perm(e4, e0, 0x05010400u);   // e0.b0 e4.b0 e0.b1 e4.b1
    const uint32_t pb = __builtin_amdgcn_perm(e5, e1, 0x05010400u);
    const uint32_t pc = __builtin_amdgcn_perm(e4, e0, 0x0C0C0602u);   // e0.b2 e4.b2
    const uint32_t pd = __builtin_amdgcn_perm(e5, e1, 0x0C0C0602u);
    o[3 * h] = __builtin_amdgcn_perm(pd, pc, 0x05040100u);
    o[3 * h + 1] = __builtin_amdgcn_perm(pb, pa, 0x07060302u) ^ 0x80808080u;
    o[3 * h + 2] = __builtin_amdgcn_perm(pb, pa, 0x05040100u) ^ 0x80808080u;
  }
  int sy = (sum4_i8(o[0], sum4_i8(o[3], 0)) << 8) + sum4_i8(o[1], sum4_i8(o[4], 0));
  int sc = sum4_i8(o[2], sum4_i8(o[5], 0));
  sy = row16_sum(sy);
  sc = row16_sum(sc);
  if (valid) {
#pragma unroll
    for (int k = 0; k < 6; ++k) xw[g * (kDecQ * 4) + k * 16 + c16] = o[k];
    if (c16 == 0)
      cst[g] = u32x4{__float_as_uint(inv), (uint32_t)(-sy), (uint32_t)(-sc), 0u};
  }
}

template <int S>
__device__ __forceinline__ void dec_mma(float (&acc)[S], const RowsData<4, S, true>& d,
                                        const u32x4* xg, u32x4 cs, int aoff, int st0, int zsh) {
  const i32x4 AL = __builtin_bit_cast(i32x4, xg[aoff]);
  const i32x4 AH = __builtin_bit_cast(i32x4, xg[12 + aoff]);
  const float inv = __uint_as_float(cs[0]);
  const int ny = (int)cs[1], nc = (int)cs[2];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    i32x4 BL, BH;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      BL[r] = (int)(d.w[i][0][r] & 0x0F0F0F0Fu);
      BH[r] = (int)((d.w[i][0][r] >> 4) & 0x0F0F0F0Fu);
    }
    i32x4 Dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(AL, BL, i32x4{0, 0, 0, 0}, 0, 0, 0);
    Dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(AH, BH, Dm, 0, 0, 0);
    const int zp = (int)((d.z >> (zsh + 4 * (st0 + i))) & 0xFu);
    const int v1 = (Dm[0] << 8) + Dm[1] + __mul24(zp, ny);
    const int v2 = Dm[2] + __mul24(zp, nc);
    const float val = __builtin_fmaf((float)v1, 256.0f, (float)v2);
    const uint32_t sbits = (d.s[i >> 1] >> (16 * (S == 1 ? (st0 & 1) : (i & 1)))) & 0xffffu;
    acc[i] = __builtin_fmaf(val, bf16_bits_to_f32(sbits) * inv, acc[i]);
  }
}

// k_dec item slot (16-byte units): S x 64 weight chunks (lane l's 16 bytes
// of row quad i at 64 i + l), then the block's 160-byte (scale, zero-point)
// record in a 256-byte area (lane l's 4 bytes at 4 l; lanes >= 40 repeat
// word 0).
template <int S>
constexpr int kDecSlot = S * 64 + 16;

template <int S>
__device__ __forceinline__ void dec_issue(u32x4* slot, const SkinnyRsrc& r, uint32_t blk,
                                          uint32_t woff, int lane) {
#pragma unroll
  for (int i = 0; i < S; ++i) dma_load16(r.qw, slot + i * 64, woff + i * 256, blk * 4096u);
  dma_load4(r.sc, slot + S * 64, lane < 40 ? (uint32_t)lane * 4u : 0u, blk * (uint32_t)kMetaBytes);
}

template <int S>
__device__ __forceinline__ void dec_read(RowsData<4, S, true>& d, const u32x4* slot, int lane,
                                         int st0) {
  const int c = lane & 15;
#pragma unroll
  for (int i = 0; i < S; ++i) d.w[i][0] = slot[i * 64 + lane];
  const uint32_t* sm = reinterpret_cast<const uint32_t*>(slot + S * 64);
  if (S == 4) {
    d.s[0] = sm[2 * c];
    d.s[(S + 1) / 2 - 1] = sm[2 * c + 1];
  } else {
    d.s[0] = sm[(4 * c + st0) >> 1];
  }
  d.z = sm[32 + (c >> 1)];
}

// LDS of k_dec (16-byte units): operands 24 G | constants G | OUT_NORM: the
// staged x (K / 8) | the waves' item slots.
__host__ __device__ constexpr int dec_lds_units(int K, int G, bool norm, int S, int W, int D) {
  return kDecQ * G + G + (norm ? K / 8 : 0) + W * D * (S * 64 + 16);
}

// k_dec: workgroup p owns the whole units [p U / P, (p + 1) U / P) (unit =
// S row quads of a 64-row tile over all of K; OUT_SWIGLU: (gate, up) unit
// pairs). Its waves split each unit's groups (wave w takes g = w, w + W, ...,
// the groups whose activation operands it prepared), keep D items in flight in
// LDS slots (buffer_load ... lds) across unit boundaries, and at each unit's
// end sum their partials in LDS in wave order; wave 0 emits. No workgroup
// exchanges partials with another (measured on MI355X: both a fixed-point
// atomic exchange of cut units and a flagged pair exchange cost more at the
// tail than the imbalance of whole units).
template <int OUT, int S, int W, int D>
__global__ __launch_bounds__(64 * W) void k_dec(SkinnyArgs a) {
  constexpr uint32_t kPer = 4 / S;
  constexpr uint32_t kQuad = 256u;
  constexpr int kXC = rows_xchunks(true);
  __shared__ float red[2][W][S][16];
  extern __shared__ u32x4 xlds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4, c16 = c;
  const int aoff = (c < 2 ? c : 2) * 4 + q;
  const SkinnyRsrc rs = skinny_rsrc(a);
  const uint32_t zsh = 16 * (c & 1);
  const uint32_t wbase = Fmt<4>::woff(q, c);
  const int p = blockIdx.x;
  const int G = a.G;
  // OUT_SWIGLU: units 2v (gate v) and 2v + 1 (its up unit), never split
  const int u0 = OUT == OUT_SWIGLU ? 2 * (int)((long long)p * (a.U / 2) / a.P) : range_start(a, p);
  const int u1 =
      OUT == OUT_SWIGLU ? 2 * (int)((long long)(p + 1) * (a.U / 2) / a.P) : range_start(a, p + 1);
  auto real_unit = [&](int v) {
    return OUT == OUT_SWIGLU ? ((v & 1) ? (v >> 1) + (int)((uint32_t)a.U / 2u) : (v >> 1)) : v;
  };
  Best bs;
  best_init(bs);
  const int n16 = a.K / 8;
  u32x4* const xq = xlds;
  u32x4* const cst = xlds + kDecQ * G;
  u32x4* const raw = cst + G;   // OUT_NORM
  u32x4* const ring = raw + (OUT == OUT_NORM ? n16 : 0) + wave * D * kDecSlot<S>;

  const int nw = wave < G ? (G - 1 - wave) / W + 1 : 0;   // items per unit
  const int T = nw * (u1 - u0);
  const uint32_t oob_blk = (uint32_t)a.tiles * (uint32_t)G;
  int lu = u0, lg = wave;   // load cursor (wave-uniform)
  auto load_item = [&](int j) __attribute__((always_inline)) {
    const bool in = lu < u1;
    const int ru = real_unit(lu);
    const int st0 = in ? (int)((uint32_t)ru % kPer) * S : 0;
    const uint32_t blk = in ? (uint32_t)((uint32_t)ru / kPer) * (uint32_t)G + (uint32_t)lg : oob_blk;
    dec_issue<S>(ring + j * kDecSlot<S>, rs, blk, wbase + (uint32_t)st0 * kQuad, lane);
    lg += W;
    if (lg >= G) {
      lg = wave;
      ++lu;
    }
  };
  uint32_t* const xw = reinterpret_cast<uint32_t*>(xq);
  if constexpr (OUT != OUT_NORM) {
    // x loads of this wave's groups first (g = wave + W (4 it + lane / 16),
    // chunk lane % 16), then the first weight items; out-of-range chunks
    // read zeros without traffic. Rounds with no group of this wave issue
    // nothing: every 16-byte load of a wave holds the CU's address unit for
    // ~16 cycles whatever its addresses, and 8 waves share one.
    u32x4 xv[kDecPrepIters];
#pragma unroll
    for (int it = 0; it < kDecPrepIters; ++it) {
      const int g = wave + W * (4 * it + (lane >> 4));
      xv[it] = u32x4{0u, 0u, 0u, 0u};
      if (wave + W * 4 * it < G)   // wave-uniform
        xv[it] = __builtin_amdgcn_raw_buffer_load_b128(
            rs.x, g < G ? (uint32_t)(g * 16 + c16) * 16u : 0x7ffffff0u, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < D; ++j) load_item(j);
#pragma unroll
    for (int it = 0; it < kDecPrepIters; ++it) {
      if (wave + W * 4 * it >= G) break;   // wave-uniform
      const int g = wave + W * (4 * it + (lane >> 4));
      dec_prep_chunk(xw, cst, g, c16, xv[it], g < G);
    }
  } else {
    // rmsnorm of x (src/kernels/elementwise.cu:8-31) with the sum of squares
    // in the order every rmsnorm form here shares (norm_sumsq): this thread's
    // chunk j, t + 64 W j, belongs to virtual thread t + 64 W (j mod kP);
    // x * rsqrt(mean(x^2) + eps) * (1 + w) rounded to bf16 once, staged in
    // LDS, then each wave prepares its groups from there
    constexpr int kP = kNormVThreads / (64 * W);
    static_assert(kNormVThreads % (64 * W) == 0, "workgroup of 1024 / kP threads");
    u32x4 xv[kXC], nv[kXC];
    int xi[kXC];
    const __amdgpu_buffer_rsrc_t rn =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.nw), 0, a.K * 2, 0x00020000);
#pragma unroll
    for (int j = 0; j < kXC; ++j) {
      xi[j] = min((int)threadIdx.x + j * 64 * W, n16 - 1);
      xv[j] = nv[j] = u32x4{0u, 0u, 0u, 0u};
      if (64 * wave + j * 64 * W < n16) {   // wave-uniform (see the loads above)
        xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rs.x, (uint32_t)xi[j] * 16u, 0, 0);
        nv[j] = __builtin_amdgcn_raw_buffer_load_b128(rn, (uint32_t)xi[j] * 16u, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < D; ++j) load_item(j);
    __shared__ float vsum[kNormVWaves];
    float part[kP];
#pragma unroll
    for (int k = 0; k < kP; ++k) part[k] = 0.f;
#pragma unroll
    for (int j = 0; j < kXC; ++j)
      if ((int)threadIdx.x + j * 64 * W < n16) part[j % kP] = norm_sumsq(part[j % kP], xv[j]);
#pragma unroll
    for (int k = 0; k < kP; ++k) {
      const float sk = norm_wave_sum(part[k]);
      if (lane == 0) vsum[wave + W * k] = sk;
    }
    lds_barrier<true>();
    const float inv = norm_inv(vsum, a.K, a.eps);
#pragma unroll
    for (int j = 0; j < kXC; ++j) {   // in-range chunks only (see k_rows's staging)
      if ((int)threadIdx.x + j * 64 * W >= n16) continue;
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t xw2 = xv[j][e], ww = nv[j][e];
        o[e] = pack_bf16x2(rmsnorm_f32(xw2, ww, inv), rmsnorm_f32(xw2 >> 16, ww >> 16, inv));
      }
      raw[xi[j]] = o;
    }
    lds_barrier<true>();
#pragma unroll
    for (int it = 0; it < kDecPrepIters; ++it) {
      if (wave + W * 4 * it >= G) break;
      const int g = wave + W * (4 * it + (lane >> 4));
      const bool valid = g < G;
      dec_prep_chunk(xw, cst, g, c16, raw[(valid ? g : 0) * 16 + c16], valid);
    }
  }

  float acc[S];
#pragma unroll
  for (int i = 0; i < S; ++i) acc[i] = 0.f;
  int par = 0;
  float gate[OUT == OUT_SWIGLU ? S : 1];   // OUT_SWIGLU: the gate unit's sums (wave 0)
  // Close unit u: every wave passes here once per unit of the range, in order.
  auto close_unit = [&](int u) {
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < S; ++i) red[par][wave][i][lane] = acc[i];
    }
    lds_barrier<true>();
    if (wave == 0) {
      float t[S];
#pragma unroll
      for (int i = 0; i < S; ++i) {
        float v = red[par][0][i][c];
        for (int w = 1; w < W; ++w) v += red[par][w][i][c];
        t[i] = v;
      }
      const int ru = real_unit(u);
      const int b = (int)((uint32_t)ru / kPer), st0 = (int)((uint32_t)ru % kPer) * S;
      if (OUT == OUT_SWIGLU) {
        if ((u & 1) == 0) {
#pragma unroll
          for (int i = 0; i < S; ++i) gate[i & (OUT == OUT_SWIGLU ? 0xff : 0)] = t[i];
        } else {
          f32x4 gg[S], uu[S];
#pragma unroll
          for (int i = 0; i < S; ++i) {
            gg[i] = f32x4{gate[i & (OUT == OUT_SWIGLU ? 0xff : 0)], 0.f, 0.f, 0.f};
            uu[i] = f32x4{t[i], 0.f, 0.f, 0.f};
          }
          emit_swiglu<S>(a, (int)((uint32_t)(u >> 1) / kPer), (int)((uint32_t)(u >> 1) % kPer) * S,
                         gg, uu, lane);
        }
      } else {
        f32x4 tv[S];
#pragma unroll
        for (int i = 0; i < S; ++i) tv[i] = f32x4{t[i], 0.f, 0.f, 0.f};
        emit_rows<OUT, S>(a, b, st0, tv, lane, bs);
      }
    }
    par ^= 1;
#pragma unroll
    for (int i = 0; i < S; ++i) acc[i] = 0.f;
  };

  int cu = u0, cg = wave;   // compute cursor (wave-uniform)
  int t0 = 0;
  constexpr int kL = S + 1;   // loads per item
  // item j waits for its slot (the loads of the D - 1 items after it may
  // still be in flight)
  auto step = [&](auto jc, auto nc, bool reload, int nwait = 0) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
    const int st0 = (int)((uint32_t)real_unit(cu) % kPer) * S;
    if constexpr (decltype(nc)::value >= 0)
      wait_vm<decltype(nc)::value>();
    else
      wait_items<kL, D>(nwait);
    RowsData<4, S, true> d;
    dec_read<S>(d, ring + j * kDecSlot<S>, lane, st0);
    dec_mma<S>(acc, d, xq + cg * kDecQ, cst[cg], aoff, st0, zsh);
    if (reload) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      load_item(j);
    }
    cg += W;
    if (cg >= G) {
      cg = wave;
      close_unit(cu);
      ++cu;
    }
  };
  // whole batches, then the last r < 2 D items with no load past the end (as k_rows)
  for (; t0 + 2 * D <= T; t0 += D)
    static_for<0, D>([&](auto jc) { step(jc, std::integral_constant<int, (D - 1) * kL>{}, true); });
  const int r = T - t0;
  static_for<0, 2 * D - 1>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j < r)
      step(std::integral_constant<int, j % D>{}, std::integral_constant<int, -1>{}, j + D < r,
           min(D - 1, r - 1 - j));
  });
  while (cu < u1) {   // waves with no items (wave >= G)
    close_unit(cu);
    ++cu;
  }
  wait_vm<0>();   // no load lands in LDS after the workgroup released it
  if (OUT == OUT_ARGMAX && wave == 0) argmax_arrive(a, p, bs, lane);
}

// ------------------------------------------------------------- host side
// Per-device caches are filled once per device under std::call_once, or are
// atomics whose racing writers store the same value; no launch reads the
// environment.
constexpr int kMaxDevices = 64;

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  return dev;
}

int device_cus() {
  static std::once_flag once[kMaxDevices];
  static int cus[kMaxDevices];
  const int dev = current_device();
  std::call_once(once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  });
  return cus[dev];
}

// Tuning and test override of the skinny launch (qw4_tune_decode); all zero =
// the measured policy.
struct DecTune {
  // 0 policy; 1 k_rows for M = 1 too (S forces the unit size, D the LDS-DMA
  // depth 2..4); 2 k_rows with register items (S / W force unit size, waves);
  // 3 k_dec of the given S / W / D (OUT_BF16); 4 the policy, but M > 1 rows
  // never staged in LDS (activations loaded with each item)
  std::atomic<int> mode{0};
  std::atomic<int> S{0}, W{0}, D{0}, P{0};
};
DecTune g_dec_tune;

struct Launch {
  int W, P;
  int S;         // units of S row quads
  bool XL;       // activations staged in LDS
  int DMA = 0;   // items in LDS slots, this many per wave (0: registers)
  bool XM = false;   // DMA with M > 1 rows staged (padded rows)
  bool GM = false;   // k_rows_gm: group-major items, several units per workgroup
};

// Items each k_rows wave keeps in flight (the one being computed included),
// by output, weight format, unit size, activation source and waves: as deep
// as fits the registers without spilling (16 waves: 128 VGPRs; 8 waves: 256).
// The argmax runs with 8 waves only.
template <int OUT, int FMT, int S, bool XL, int W>
constexpr int rows_depth() {
  if (FMT == 8) {
    if (OUT == OUT_ARGMAX) return XL ? (S == 1 ? 4 : (S == 2 ? 2 : 1)) : 1;
    if (W == 16) return XL ? (S == 1 ? 3 : 1) : 1;
    return XL ? (S == 1 ? 4 : (S == 2 ? 3 : 2)) : (S == 4 ? 1 : 2);
  }
  if (OUT == OUT_ARGMAX) {
    if (W == 16) return 1;
    return XL ? (S == 1 ? 5 : (S == 2 ? 3 : 2)) : (S == 4 ? 1 : 2);
  }
  if (W == 16) return XL ? (S == 1 ? 4 : (S == 2 ? (OUT == OUT_SWIGLU ? 2 : 3) : 1)) : 1;
  return XL ? (S == 1 ? 4 : (S == 2 ? 3 : 2)) : (S == 4 ? 2 : 3);
}

// Workgroups per CU of k_rows without dynamic LDS (registers, waves and static
// LDS), per device; the caller applies the staged activations' LDS.
template <int OUT, int FMT, int S, int W>
int rows_wgs_per_cu(bool xl) {
  static std::atomic<int> slot[kMaxDevices][2];
  std::atomic<int>& v = slot[current_device()][xl ? 1 : 0];
  int n = v.load(std::memory_order_relaxed);
  if (!n) {
    hipError_t e = xl ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                            &n, k_rows<OUT, FMT, S, W, true, rows_depth<OUT, FMT, S, true, W>()>, 64 * W, 0)
                      : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                            &n, k_rows<OUT, FMT, S, W, false, rows_depth<OUT, FMT, S, false, W>()>, 64 * W, 0);
    if (e != hipSuccess || n <= 0) n = 1;
    n = std::min(n, 8);
    v.store(n, std::memory_order_relaxed);
  }
  return n;
}

// Static LDS of the staged-activation kernel (hipFuncGetAttributes).
template <int OUT, int FMT, int S, int W>
int rows_static_lds_s() {
  static std::atomic<int> slot[kMaxDevices];
  std::atomic<int>& v = slot[current_device()];
  int n = v.load(std::memory_order_relaxed);
  if (!n) {
    hipFuncAttributes at{};
    n = hipFuncGetAttributes(&at, reinterpret_cast<const void*>(
                                      k_rows<OUT, FMT, S, W, true, rows_depth<OUT, FMT, S, true, W>()>)) ==
                hipSuccess
            ? (int)at.sharedSizeBytes + 1
            : kLdsBytes + 1;   // unknown: never stage
    v.store(n, std::memory_order_relaxed);
  }
  return n - 1;
}

template <int OUT, int FMT, int W>
int rows_static_lds(int S) {
  return S == 4   ? rows_static_lds_s<OUT, FMT, 4, W>()
         : S == 2 ? rows_static_lds_s<OUT, FMT, 2, W>()
                  : rows_static_lds_s<OUT, FMT, 1, W>();
}

template <int OUT, int FMT, int W>
int rows_occ(int S, bool xl) {
  return S == 4   ? rows_wgs_per_cu<OUT, FMT, 4, W>(xl)
         : S == 2 ? rows_wgs_per_cu<OUT, FMT, 2, W>(xl)
                  : rows_wgs_per_cu<OUT, FMT, 1, W>(xl);
}

// k_rows policy (measured on MI355X over the model's projections, their 8-way
// shards and the heads): S = 1 (16-row units) when the output has fewer
// 64-row tiles than CUs / 4 (a 896-row shard: 4.7 vs 5.6 us), S = 2 when it
// has fewer tiles than CUs (OUT_SWIGLU pairs a gate unit with its up unit in
// one workgroup: 32-row units keep as many workgroups as the plain GEMV's
// 64-row units), else S = 4; M = 1: 16 waves for K >= 64 groups, else 8;
// M > 1 and the argmax: 8 waves. Items in LDS slots (LDS-DMA):
//  * M = 1 (the 8-bit head and the shapes k_dec does not take): 32-row
//    units and 8 waves, 4 items per wave when the output has at least 1.5
//    64-row tiles per CU, 3 for long K (>= 64 groups), else 2; the fused
//    rmsnorm and the 8-bit head run faster with register items.
//  * M > 1 (verify, heads): weight items in slots, 2 items per wave;
//    activations staged in LDS (padded rows, 32-row units) when they fit and
//    the workgroups own several units each, else loaded with each item in
//    units of the register policy's size (3% / 5% per layer at M = 9 / 16
//    over register items; deeper was slower).
// Tuning override (qw4_tune_decode): mode 2 keeps register items everywhere
// (S / W force unit size and waves), mode 1 forces the LDS-DMA depth.
template <int OUT, int FMT>
Launch launch_for(int out_f, int G, int M) {
  const int tiles = out_f / kTileN;
  const int cus = device_cus();
  const int mode = g_dec_tune.mode.load(std::memory_order_relaxed);
  const int tS = g_dec_tune.S.load(std::memory_order_relaxed);
  const int tW = g_dec_tune.W.load(std::memory_order_relaxed);
  const int tD = g_dec_tune.D.load(std::memory_order_relaxed);
  const bool regs = mode == 2;
  Launch l;
  l.S = (OUT != OUT_SWIGLU && 4 * tiles < cus) ? 1 : (OUT == OUT_SWIGLU || tiles < cus) ? 2 : 4;
  l.W = OUT == OUT_ARGMAX ? 8 : (M == 1 && G >= 64) ? 16 : 8;
  if ((mode == 1 || mode == 2) && (tS == 1 || tS == 2 || tS == 4) && (OUT != OUT_SWIGLU || tS != 1))
    l.S = tS;
  if (regs && OUT != OUT_ARGMAX && (tW == 8 || tW == 16)) l.W = tW;
  const int xbytes = M * G * kGroup * 2;
  // the kernel's static LDS + the activations within the CU's LDS
  int static_lds = 0;
  if constexpr (OUT == OUT_ARGMAX)
    static_lds = rows_static_lds<OUT, FMT, 8>(l.S);
  else
    static_lds = l.W == 8 ? rows_static_lds<OUT, FMT, 8>(l.S) : rows_static_lds<OUT, FMT, 16>(l.S);
  l.XL = xbytes <= kRowsXChunks * 16 * 64 * l.W && static_lds + xbytes <= kLdsBytes;
  const long long units = (long long)tiles * 4 / l.S;
  int occ = 1;
  if constexpr (OUT == OUT_ARGMAX)
    occ = rows_occ<OUT, FMT, 8>(l.S, l.XL);
  else
    occ = l.W == 8 ? rows_occ<OUT, FMT, 8>(l.S, l.XL) : rows_occ<OUT, FMT, 16>(l.S, l.XL);
  if (l.XL) occ = std::max(1, std::min(occ, kLdsBytes / (static_lds + xbytes)));
  // OUT_SWIGLU: whole (gate, up) unit pairs per workgroup
  l.P = (int)std::max<long long>(1, std::min(OUT == OUT_SWIGLU ? units / 2 : units,
                                             (long long)cus * occ));
  if (regs) return l;
  if (M == 1 && l.S != 1) {
    const int dd = (mode == 1 && tD >= 2 && tD <= 4) ? tD
                   : (OUT == OUT_NORM || FMT == 8)    ? 0
                                                      : (2 * tiles >= 3 * cus ? 4 : (G >= 64 ? 3 : 2));
    const int slot = (FMT == 8 ? 4 : 2) * 1024 + 256;
    const int need = xbytes + 8 * dd * slot + 2 * 8 * 2 * 16 * 16 + (OUT == OUT_NORM ? 64 : 0);
    if (dd >= 2 && xbytes <= rows_xchunks(true) * 16 * 64 * 8 && need <= kLdsBytes) {
      l.DMA = dd;
      l.S = 2;
      l.W = 8;
      l.XL = true;
      const long long u2 = (long long)tiles * 2;
      const long long pc2 = (long long)cus * (kLdsBytes / need);
      l.P = (int)std::max<long long>(1, std::min(OUT == OUT_SWIGLU ? u2 / 2 : u2, pc2));
    }
  } else if (M > 1 && OUT != OUT_NORM && l.S != 1) {
    // All M rows staged in LDS once (padded rows, 32-row units, 2 items per
    // wave, one reduction buffer) when they fit and the workgroups own more
    // than one unit on average: the per-item loads re-read x once per unit.
    // Measured on MI355X, both forms in one process: gate|up at M = 9 (4.25
    // units per workgroup) 22.3 against 24.1 us; with one unit per workgroup
    // (qkv, o_proj) within +-5% either way, so those keep the per-item loads.
    const int xm_need = M * (G * kGroup * 2 + 16) +
                        8 * 2 * ((FMT == 8 ? 4 : 2) * 1024 + 256) +
                        8 * 2 * 64 * 16 + 512;
    if (mode != 1 && mode != 4 && 2LL * tiles > cus && M * G * kGroup / 8 <= kRowsXmChunks * 64 * 8 &&
        xm_need <= kLdsBytes) {
      l.DMA = 2;
      l.S = 2;
      l.W = 8;
      l.XL = true;
      l.XM = true;
      const long long u2 = (long long)tiles * 2;
      l.P = (int)std::max<long long>(1, std::min(OUT == OUT_SWIGLU ? u2 / 2 : u2, (long long)cus));
      return l;
    }
    if constexpr (FMT == 4 && (OUT == OUT_BF16 || OUT == OUT_F32 || OUT == OUT_RES)) {
      // Otherwise, several units per workgroup: group-major items, each
      // activation group fetched once per workgroup (k_rows_gm). Measured on
      // MI355X, gate|up at M = 16: 24.2 against 28.1 us for the per-item
      // loads; at M = 9 the staged rows above stay faster (23.7 against 24.1).
      const long long u2 = (long long)tiles * 2;
      const long long pg = std::min<long long>(u2, cus);
      if (mode != 1 && mode != 2 && mode != 4 && mode != 5 && u2 / pg >= kGmMinU &&
          (u2 + pg - 1) / pg <= kGmMaxU) {
        l.GM = true;
        l.S = 2;
        l.W = 8;
        l.DMA = kGmD;
        l.XL = false;
        l.P = (int)pg;
        return l;
      }
    }
    int S = l.S;
    const int dd = (mode == 1 && tD >= 2 && tD <= 4 && !(OUT == OUT_ARGMAX && S == 4)) ? tD : 2;
    // weights, metadata and the item's 16 activation rows (rows_slot_units)
    auto need_for = [&](int s_) {
      const int slot = (FMT == 8 ? 2 * s_ : s_) * 1024 + 256 + 4096;
      return 8 * dd * slot + (FMT == 8 ? 1 : 2) * 8 * s_ * 64 * 16;
    };
    // 64-row units whose slots do not fit: 32-row units with the activations
    // in the slots (measured on MI355X: gate|up at M = 16, 28.1 us against 29.6
    // for 64-row units with the activations loaded into registers)
    // (4-bit only: the 8-bit head at M = 9 keeps its 64-row register form,
    // 352 against 368 us for 32-row units with the activations in the slots)
    if (FMT == 4 && S == 4 && need_for(4) > kLdsBytes && !(mode == 1 && tS == 4)) S = 2;
    const int need = need_for(S);
    if (need <= kLdsBytes) {
      l.S = S;
      l.DMA = dd;
      l.W = 8;
      l.XL = false;
      const long long us = (long long)tiles * 4 / S;
      const long long pc2 = (long long)cus * (kLdsBytes / need);
      l.P = (int)std::max<long long>(1, std::min(OUT == OUT_SWIGLU ? us / 2 : us, pc2));
    }
  }
  return l;
}

template <int OUT, int FMT, int W, bool XL>
void launch_rows_x(const SkinnyArgs& a, int S, hipStream_t st) {
  const size_t lds = XL ? (size_t)a.M * a.K * 2 : 0;
  if (S == 4)
    k_rows<OUT, FMT, 4, W, XL, rows_depth<OUT, FMT, 4, XL, W>()><<<a.P, 64 * W, lds, st>>>(a);
  else if (S == 2)
    k_rows<OUT, FMT, 2, W, XL, rows_depth<OUT, FMT, 2, XL, W>()><<<a.P, 64 * W, lds, st>>>(a);
  else
    k_rows<OUT, FMT, 1, W, XL, rows_depth<OUT, FMT, 1, XL, W>()><<<a.P, 64 * W, lds, st>>>(a);
}

// Dynamic LDS above the default limit is allowed per kernel, once per device:
// qw4_scratch_alloc raises every LDS-DMA kernel to its maximum, so no launch --
// captured into a graph or not -- has to. A launch that needs more than a
// kernel was raised to (no scratch allocated on this device yet) raises it
// under a lock.
std::mutex g_lds_mutex;

template <auto Kern>
void allow_lds(int bytes) {
  static std::atomic<int> set[kMaxDevices];
  std::atomic<int>& v = set[current_device()];
  if (bytes <= v.load(std::memory_order_acquire)) return;
  std::lock_guard<std::mutex> lock(g_lds_mutex);
  if (bytes <= v.load(std::memory_order_relaxed)) return;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(Kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess)
    v.store(bytes, std::memory_order_release);
  else
    (void)hipGetLastError();   // not sticky: the launch reports what matters
}

// ---- k_dec launch (M = 1, 4-bit)
struct DecCfg {
  int S, W, D, P;
  int lds;   // dynamic LDS bytes
};

// red + rinv, rounded up (the launch checks the total against the CU's LDS)
int dec_static_lds(int S, int W) { return 2 * W * S * 16 * 4 + 256; }

// The k_dec instantiations: the first kDecPolicy are the policy's (built for
// every output mode), the rest tuning alternatives (OUT_BF16 only).
struct DecVariant {
  int S, W, D;
};
constexpr DecVariant kDecAll[] = {{2, 8, 3}, {2, 8, 2}, {2, 16, 2}, {2, 8, 4},
                                  {1, 8, 3}, {1, 16, 3}, {2, 4, 4}, {4, 8, 2}};
constexpr int kDecPolicy = 3;
constexpr int kDecCount = (int)(sizeof(kDecAll) / sizeof(kDecAll[0]));

// Returns false when the shape does not fit k_dec (activations beyond the
// per-wave prep, LDS beyond the CU's). Policy, measured on MI355X over the
// config-2 projections with every variant forced in one process (32-row
// units throughout; 16-row units and deeper items were slower): when the
// output has fewer tiles than CUs, 2 items per wave, 16 waves for long K
// (down: 10.9 us against 11.3 for 8 x 3), 8 for short (qkv: 5.7 against
// 6.0; o_proj 4.9 against 5.0); else 2 items per wave for short K (32
// groups) and 8 waves of 3 items otherwise (gate|up).
bool dec_config(int out_f, int G, int OUTmode, DecCfg& c) {
  const int tiles = out_f / kTileN;
  const int K = G * kGroup;
  DecVariant v = tiles < device_cus() ? (G >= 64 ? kDecAll[2] : kDecAll[1])
                 : G <= 32            ? kDecAll[1]
                                      : kDecAll[0];
  if (OUTmode == OUT_BF16 && g_dec_tune.mode.load(std::memory_order_relaxed) == 3) {
    const int tS = g_dec_tune.S.load(std::memory_order_relaxed);
    const int tW = g_dec_tune.W.load(std::memory_order_relaxed);
    const int tD = g_dec_tune.D.load(std::memory_order_relaxed);
    bool found = false;
    for (const DecVariant& x : kDecAll)
      if ((!tS || x.S == tS) && (!tW || x.W == tW) && (!tD || x.D == tD)) {
        v = x;
        found = true;
        break;
      }
    if (!found) return false;
  }
  c.S = v.S;
  c.W = v.W;
  c.D = v.D;
  if (G > kDecPrepIters * 4 * c.W) return false;
  if (OUTmode == OUT_NORM && K / 8 > rows_xchunks(true) * 64 * c.W) return false;
  c.lds = dec_lds_units(K, G, OUTmode == OUT_NORM, c.S, c.W, c.D) * 16;
  const int per_wg = c.lds + dec_static_lds(c.S, c.W);
  if (per_wg > kLdsBytes) return false;
  const long long units = (long long)tiles * 4 / c.S;
  // one workgroup per CU (gate|up: 256 workgroups 17.6 us, two per CU 19.1 us)
  const long long cap = OUTmode == OUT_SWIGLU ? units / 2 : units;
  const int tP = g_dec_tune.P.load(std::memory_order_relaxed);
  c.P = (int)std::max<long long>(1, std::min(cap, tP > 0 ? (long long)tP : (long long)device_cus()));
  return true;
}

template <int OUT, int I>
void launch_dec_i(const SkinnyArgs& a, const DecCfg& c, hipStream_t st) {
  constexpr DecVariant v = kDecAll[I];
  constexpr auto kern = &k_dec<OUT, v.S, v.W, v.D>;
  if (c.S == v.S && c.W == v.W && c.D == v.D) {
    allow_lds<kern>(c.lds);
    kern<<<a.P, 64 * v.W, c.lds, st>>>(a);
    return;
  }
  if constexpr (I + 1 < (OUT == OUT_BF16 ? kDecCount : kDecPolicy)) launch_dec_i<OUT, I + 1>(a, c, st);
}

template <int OUT>
void launch_dec(const SkinnyArgs& a, const DecCfg& c, hipStream_t st) {
  launch_dec_i<OUT, 0>(a, c, st);
}

template <int OUT, int I>
void prepare_dec_i() {
  constexpr DecVariant v = kDecAll[I];
  allow_lds<&k_dec<OUT, v.S, v.W, v.D>>(kLdsBytes - dec_static_lds(v.S, v.W));
  if constexpr (I + 1 < (OUT == OUT_BF16 ? kDecCount : kDecPolicy)) prepare_dec_i<OUT, I + 1>();
}

template <int OUT>
void prepare_dec() {
  prepare_dec_i<OUT, 0>();
}

template <int OUT, int FMT, int S, int W, int D, bool XL, bool XM = false>
void launch_rows_dma_d(const SkinnyArgs& a, hipStream_t st) {
  const int lds = (XL ? a.M * (a.K * 2 + (XM ? 16 : 0)) : 0) + W * D * rows_slot_units<FMT, S, XL>() * 16;
  constexpr auto kern = &k_rows<OUT, FMT, S, W, XL, D, true, XM>;
  allow_lds<kern>(lds);
  kern<<<a.P, 64 * W, lds, st>>>(a);
}

template <int OUT, int FMT, int S, bool XL, int D, bool XM = false>
void prepare_dma_one() {
  constexpr auto kern = &k_rows<OUT, FMT, S, 8, XL, D, true, XM>;
  hipFuncAttributes at{};
  if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(kern)) == hipSuccess)
    allow_lds<kern>(kLdsBytes - (int)at.sharedSizeBytes);
}

template <int OUT>
void prepare_gm() {
  constexpr auto kern = &k_rows_gm<OUT>;
  hipFuncAttributes at{};
  if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(kern)) == hipSuccess)
    allow_lds<kern>(kLdsBytes - (int)at.sharedSizeBytes);
}

// Every LDS-DMA kernel the launch code can pick (launch_rows_dma).
template <int OUT, int FMT>
void prepare_dma_out() {
  prepare_dma_one<OUT, FMT, 2, true, 2>();
  prepare_dma_one<OUT, FMT, 2, true, 3>();
  prepare_dma_one<OUT, FMT, 2, true, 4>();
  if constexpr (OUT != OUT_NORM) {
    prepare_dma_one<OUT, FMT, 2, true, 2, true>();
    prepare_dma_one<OUT, FMT, 2, false, 2>();
    prepare_dma_one<OUT, FMT, 2, false, 3>();
    prepare_dma_one<OUT, FMT, 2, false, 4>();
    prepare_dma_one<OUT, FMT, 4, false, 2>();
    if constexpr (OUT != OUT_ARGMAX) {
      prepare_dma_one<OUT, FMT, 4, false, 3>();
      prepare_dma_one<OUT, FMT, 4, false, 4>();
    }
  }
}

void prepare_dma_lds() {
  static std::once_flag once[kMaxDevices];
  std::call_once(once[current_device()], [] {
    prepare_dec<OUT_BF16>();
    prepare_dec<OUT_F32>();
    prepare_dec<OUT_ARGMAX>();
    prepare_dec<OUT_RES>();
    prepare_dec<OUT_SWIGLU>();
    prepare_dec<OUT_NORM>();
    prepare_gm<OUT_BF16>();
    prepare_gm<OUT_F32>();
    prepare_gm<OUT_RES>();
    prepare_dma_out<OUT_BF16, 4>();
    prepare_dma_out<OUT_F32, 4>();
    prepare_dma_out<OUT_ARGMAX, 4>();
    prepare_dma_out<OUT_RES, 4>();
    prepare_dma_out<OUT_SWIGLU, 4>();
    prepare_dma_out<OUT_NORM, 4>();
    prepare_dma_out<OUT_BF16, 8>();
    prepare_dma_out<OUT_ARGMAX, 8>();
  });
}

// LDS-DMA items: units of S row quads, 8 waves, D items per wave; staged
// activations (M = 1, S = 2) or activations loaded with each item (M > 1)
template <int OUT, int FMT, int S, bool XL>
void launch_rows_dma(const SkinnyArgs& a, int D, hipStream_t st) {
  if constexpr (OUT == OUT_ARGMAX && S == 4) {   // deeper would spill (launch_for caps D)
    launch_rows_dma_d<OUT, FMT, S, 8, 2, XL>(a, st);
  } else {
    if (D == 2)
      launch_rows_dma_d<OUT, FMT, S, 8, 2, XL>(a, st);
    else if (D == 3)
      launch_rows_dma_d<OUT, FMT, S, 8, 3, XL>(a, st);
    else
      launch_rows_dma_d<OUT, FMT, S, 8, 4, XL>(a, st);
  }
}

template <int OUT>
void launch_rows_gm(const SkinnyArgs& a, hipStream_t st) {
  const int lds = 8 * gm_wave_units() * 16;
  constexpr auto kern = &k_rows_gm<OUT>;
  allow_lds<kern>(lds);
  kern<<<a.P, 512, lds, st>>>(a);
}

template <int OUT, int FMT>
void launch_rows(const SkinnyArgs& a, const Launch& l, hipStream_t st) {
  if constexpr (FMT == 4 && (OUT == OUT_BF16 || OUT == OUT_F32 || OUT == OUT_RES)) {
    if (l.GM) {
      launch_rows_gm<OUT>(a, st);
      return;
    }
  }
  if (l.DMA) {
    if constexpr (OUT != OUT_NORM) {
      if (l.XM) {   // M > 1 rows staged: 2 items per wave (launch_for)
        launch_rows_dma_d<OUT, FMT, 2, 8, 2, true, true>(a, st);
        return;
      }
    }
    if (l.XL)
      launch_rows_dma<OUT, FMT, 2, true>(a, l.DMA, st);
    else if constexpr (OUT != OUT_NORM) {
      if (l.S == 4)
        launch_rows_dma<OUT, FMT, 4, false>(a, l.DMA, st);
      else
        launch_rows_dma<OUT, FMT, 2, false>(a, l.DMA, st);
    }
    return;
  }
  if (OUT == OUT_ARGMAX || l.W == 8)
    l.XL ? launch_rows_x<OUT, FMT, 8, true>(a, l.S, st) : launch_rows_x<OUT, FMT, 8, false>(a, l.S, st);
  else
    if constexpr (OUT != OUT_ARGMAX)
      l.XL ? launch_rows_x<OUT, FMT, 16, true>(a, l.S, st)
           : launch_rows_x<OUT, FMT, 16, false>(a, l.S, st);
}

// The packed weights of either format, as the kernel sees them.
struct WeightView {
  const void* qw;
  const uint16_t* sc;
  const uint16_t* zr;   // 4-bit zero points; null for 8-bit
  int out_f, in_f, G;
  size_t weight_bytes;
};

// Epilogue inputs (see the OUT_* modes).
struct Epi {
  const uint16_t* res = nullptr;
  const uint16_t* nw = nullptr;
  float eps = 0.f;
  bool tmp_ok = false;   // OUT_NORM: the caller can run rmsnorm into a buffer first
};

// run_skinny's internal status (never returned through the C-ABI): an rmsnorm
// projection to run as rmsnorm into the caller's buffer, then the plain
// projection -- rows beyond the LDS staging, or an M = 1 row the decode kernel
// cannot stage (where that path is the faster one).
constexpr int kStatusNeedTmp = -100;

template <int OUT, int FMT>
int run_skinny(void* y, const WeightView& w, const uint16_t* x, int M, qw4_scratch* s,
               void* stream, const Epi& e = Epi()) {
  if (!y || !x || !s || !s->counters || !s->keys) return QW4_ERR_NULL;
  if (M < 1 || M > 16) return QW4_ERR_M;
  if (((uintptr_t)x & 15) || ((uintptr_t)y & (OUT == OUT_F32 ? 15 : (OUT == OUT_BF16 ? 7 : 3))))
    return QW4_ERR_ALIGN;
  const int tiles = w.out_f / kTileN;
  if (tiles > s->max_tiles || M > s->max_m || w.in_f > s->max_in) return QW4_ERR_SCRATCH;
  // loads address weights and x through 32-bit buffer offsets
  if (w.weight_bytes >= (1ull << 32)) return QW4_ERR_SHAPE;
  if (OUT == OUT_SWIGLU && (w.out_f % (2 * kTileN))) return QW4_ERR_SHAPE;
  if (OUT == OUT_RES && !e.res) return QW4_ERR_NULL;
  if (OUT == OUT_NORM && !e.nw) return QW4_ERR_NULL;
  SkinnyArgs a{};
  a.qw = static_cast<const uint32_t*>(w.qw);
  a.sc = w.sc;
  a.zr = w.zr;
  a.x = x;
  a.y = y;
  a.counters = s->counters;
  a.keys = s->keys;
  a.M = M;
  a.N = w.out_f;
  a.K = w.in_f;
  a.G = w.G;
  a.tiles = tiles;
  a.weight_bytes = (uint32_t)w.weight_bytes;
  a.res = e.res;
  a.nw = e.nw;
  a.eps = e.eps;
  a.ld = OUT == OUT_SWIGLU ? w.out_f / 2 : w.out_f;
  const int mode = g_dec_tune.mode.load(std::memory_order_relaxed);
  if constexpr (FMT == 4) {
    DecCfg dc{};
    // M = 1 rmsnorm that the decode kernel cannot stage (its LDS): the caller's
    // tmp path (rmsnorm, then the decode kernel) beats the bf16 skinny kernel
    // and equals the unfused steps
    if (OUT == OUT_NORM && M == 1 && e.tmp_ok && mode != 1 && mode != 2 &&
        !dec_config(w.out_f, w.G, OUT, dc) && dec_config(w.out_f, w.G, OUT_BF16, dc))
      return kStatusNeedTmp;
    if (M == 1 && mode != 1 && mode != 2 && dec_config(w.out_f, w.G, OUT, dc)) {
      a.U = tiles * 4 / dc.S;
      a.P = dc.P;
      launch_dec<OUT>(a, dc, (hipStream_t)stream);
      QW4_LAUNCH_CHECK();
      return QW4_OK;
    }
  }
  const Launch l = launch_for<OUT, FMT>(w.out_f, w.G, M);
  // x must fit the LDS staging; beyond it, the caller's tmp path or an error
  if (OUT == OUT_NORM && !l.XL) return e.tmp_ok ? kStatusNeedTmp : QW4_ERR_SHAPE;
  a.P = l.P;
  a.U = tiles * 4 / l.S;
  launch_rows<OUT, FMT>(a, l, (hipStream_t)stream);
  QW4_LAUNCH_CHECK();
  return QW4_OK;
}

template <int OUT>
int run_skinny(void* y, const qw4_weights* w, const uint16_t* x, int M, qw4_scratch* s,
               void* stream, const Epi& e = Epi()) {
  const int st = check_weights_public(w);
  if (st) return st;
  const WeightView v{w->qweight, w->scale, w->zeros, w->out_f, w->in_f, w->num_groups,
                     (size_t)w->out_f * w->in_f / 2};
  return run_skinny<OUT, 4>(y, v, x, M, s, stream, e);
}

int check_w8(const qw4_w8_weights* w) {
  if (!w || !w->qweight || !w->scale) return QW4_ERR_NULL;
  if (w->group_size != kGroup) return QW4_ERR_GROUP;
  if (w->out_f <= 0 || w->out_f % kTileN || w->in_f <= 0 || w->in_f % kGroup ||
      w->num_groups != w->in_f / kGroup)
    return QW4_ERR_SHAPE;
  return QW4_OK;
}

template <int OUT>
int run_skinny8(void* y, const qw4_w8_weights* w, const uint16_t* x, int M, qw4_scratch* s,
                void* stream) {
  const int st = check_w8(w);
  if (st) return st;
  const WeightView v{w->qweight, w->scale, nullptr, w->out_f, w->in_f, w->num_groups,
                     (size_t)w->out_f * w->in_f};
  return run_skinny<OUT, 8>(y, v, x, M, s, stream);
}

// ---- the argmax head without allocation (qw4_gemv_argmax_noalloc)
// Its scratch: 64 key lines (16 rows of u64 keys each), then 65 arrival-counter
// lines of 128 bytes, in the file-scope array `scratch` (16.5 KiB, one copy
// per GPU, held until the process ends). Host code uses the array's device
// address from hipGetSymbolAddress, never its name.
constexpr int kNoAllocKeyWords = kKeyGroups * 16;
constexpr int kNoAllocWords = kNoAllocKeyWords + (kKeyGroups + 1) * kCounterStride / 2;

}  // namespace
}  // namespace qw4

static __device__ __align__(256) uint64_t scratch[qw4::kNoAllocWords];

namespace qw4 {
namespace {

// Per-device address of `scratch`, looked up once with that device current.
// The array is zero when the code object loads and every call's last
// workgroup clears what it used, so no set-up kernel runs (a first call under
// graph capture records nothing extra). A failed look-up is not cached: the
// next call tries again.
struct NoAllocState {
  std::mutex mu;
  std::atomic<uint64_t*> ptr{nullptr};
};
NoAllocState g_noalloc[kMaxDevices];

int noalloc_scratch(uint64_t*& ptr) {
  NoAllocState& st = g_noalloc[current_device()];
  ptr = st.ptr.load(std::memory_order_acquire);
  if (ptr) return QW4_OK;
  std::lock_guard<std::mutex> lock(st.mu);
  ptr = st.ptr.load(std::memory_order_relaxed);
  if (ptr) return QW4_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    set_hip_error((int)e);
    (void)hipGetLastError();
    return QW4_ERR_HIP;
  }
  prepare_dma_lds();
  ptr = static_cast<uint64_t*>(p);
  st.ptr.store(ptr, std::memory_order_release);
  return QW4_OK;
}

}  // namespace
}  // namespace qw4

using namespace qw4;

extern "C" {

int qw4_tune_decode(int mode, int S, int W, int D, int P) {
  g_dec_tune.mode.store(mode, std::memory_order_relaxed);
  g_dec_tune.S.store(S, std::memory_order_relaxed);
  g_dec_tune.W.store(W, std::memory_order_relaxed);
  g_dec_tune.D.store(D, std::memory_order_relaxed);
  g_dec_tune.P.store(P, std::memory_order_relaxed);
  return QW4_OK;
}

int qw4_choose_splits(int out_f, int num_groups) {
  // Every skinny launch gives each workgroup whole units over all of K: no
  // output is split across workgroups (measured on MI355X: each exchange of
  // partials tried cost more at the tail than the imbalance it removed).
  (void)out_f;
  (void)num_groups;
  return 1;
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
  // the reference's split-K capacity at splits = 1 (M rows of the widest
  // output); no kernel here writes partials, the field is kept for callers
  s->partial_elems = (size_t)max_m * s->max_tiles * kTileN;
  const size_t cnt_bytes = (size_t)(kKeyGroups + 1) * kCounterStride * 4;
  // argmax keys: one 128-byte line per key group
  const size_t key_bytes = (size_t)kKeyGroups * 16 * 8;
  hipError_t e = hipMalloc((void**)&s->partial, s->partial_elems * 4);
  if (e == hipSuccess) e = hipMemset(s->partial, 0, s->partial_elems * 4);
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
  prepare_dma_lds();
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
  if (splits < 1 || M < 1 || out_f < 1) return QW4_ERR_SHAPE;
  if (M > s->max_m || (out_f + kTileN - 1) / kTileN > s->max_tiles) return QW4_ERR_SCRATCH;
  return (size_t)splits * M * out_f > s->partial_elems ? QW4_ERR_SCRATCH : QW4_OK;
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

int qw4_gemv_argmax_noalloc(int32_t* idx, const qw4_weights* w, const uint16_t* x, int M,
                            void* stream) {
  if (M < 1 || M > 16) return QW4_ERR_M;   // the keys hold 16 rows
  uint64_t* p = nullptr;
  const int st = noalloc_scratch(p);
  if (st) return st;
  qw4_scratch s{};
  s.keys = p;
  s.counters = reinterpret_cast<uint32_t*>(p + kNoAllocKeyWords);
  s.max_m = 16;
  s.max_in = INT32_MAX;
  s.max_out = INT32_MAX;
  s.max_tiles = INT32_MAX;
  return run_skinny<OUT_ARGMAX>(idx, w, x, M, &s, stream);
}

int qw4_gemv_residual(uint16_t* h, const qw4_weights* w, const uint16_t* x, int M,
                      qw4_scratch* s, void* stream) {
  if (!h) return QW4_ERR_NULL;
  Epi e;
  e.res = h;
  return run_skinny<OUT_RES>(h, w, x, M, s, stream, e);
}

int qw4_gemv_swiglu(uint16_t* y, const qw4_weights* w, const uint16_t* x, int M, uint16_t* tmp,
                    qw4_scratch* s, void* stream) {
  // Fused for M <= 2; beyond, the pairing of gate and up rows in one
  // workgroup is slower than the projection plus a separate swiglu (measured
  // on MI355X), which runs through tmp when one is given.
  if (M <= 2 || !tmp) return run_skinny<OUT_SWIGLU>(y, w, x, M, s, stream);
  if (!w) return QW4_ERR_NULL;
  if (w->out_f % (2 * kTileN)) return QW4_ERR_SHAPE;
  const int st = run_skinny<OUT_BF16>(tmp, w, x, M, s, stream);
  if (st) return st;
  return qw4_swiglu(y, tmp, M, w->out_f / 2, stream);
}

int qw4_gemv_rmsnorm(uint16_t* y, const qw4_weights* w, const uint16_t* h,
                     const uint16_t* norm_w, float eps, int M, uint16_t* tmp, qw4_scratch* s,
                     void* stream) {
  if (!norm_w) return QW4_ERR_NULL;
  Epi e;
  e.nw = norm_w;
  e.eps = eps;
  e.tmp_ok = tmp != nullptr;
  const int st = run_skinny<OUT_NORM>(y, w, h, M, s, stream, e);
  if (st != kStatusNeedTmp) return st;
  // M = 1 activations the decode kernel cannot stage: rmsnorm into tmp, then
  // the decode kernel (without tmp the call runs the bf16 skinny kernel, which
  // stages them)
  const int st2 = qw4_rmsnorm(tmp, h, norm_w, M, w->in_f, eps, stream);
  if (st2) return st2;
  return run_skinny<OUT_BF16>(y, w, tmp, M, s, stream);
}

int qw4_w8_gemv(uint16_t* y, const qw4_w8_weights* w, const uint16_t* x, qw4_scratch* s,
                void* stream) {
  return run_skinny8<OUT_BF16>(y, w, x, 1, s, stream);
}

int qw4_w8_gemm_small(uint16_t* y, const qw4_w8_weights* w, const uint16_t* x, int M,
                      qw4_scratch* s, void* stream) {
  return run_skinny8<OUT_BF16>(y, w, x, M, s, stream);
}

int qw4_w8_gemv_argmax(int32_t* idx, const qw4_w8_weights* w, const uint16_t* x, int M,
                       qw4_scratch* s, void* stream) {
  return run_skinny8<OUT_ARGMAX>(idx, w, x, M, s, stream);
}

}  // extern "C"
