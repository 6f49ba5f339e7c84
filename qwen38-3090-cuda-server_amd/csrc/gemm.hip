// Prefill W4A16 GEMM: C [M][N] = A [M][K] @ W^T, bf16 in/out, fp32 accumulate.
//
// The reference dequantizes whole weight tiles to a bf16 workspace and calls
// cublasGemmEx (src/kernels/gemm_w4a16.cu:63-88). Here the dequant is fused
// into one gfx950 kernel: each wave converts its packed weight rows in
// registers to exactly RNE((q - z) * s) -- the reference's k_dequant_rows
// arithmetic (gemm_w4a16.cu:26-36) -- and feeds them to bf16 MFMA against
// activation tiles staged in LDS. Tiles that would leave CUs idle in a last
// partial round are instead split across workgroups (stream-K, hybrid or
// split-K) when a workspace is given; the workspace then holds fp32 partial
// tiles, summed in a fixed order by a second kernel.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "../../include/qwen_w4a16.h"
#include "w4a16_common.h"

namespace qw4 {
int check_weights_public(const qw4_weights* w);

namespace {

// ---------------------------------------------------------------------------
// k_gemm: 256 (M) x 256 (N) workgroup tile, v_mfma_f32_32x32x16_bf16 (the
// full-rate bf16 shape on gfx950). The default: 4 waves, one per SIMD, each a
// whole 64-row weight tile against all 256 activation rows (its 256
// accumulator registers in AGPRs); G2Split below lists the 8-wave forms.
//
//  * Weights are the MFMA A operand (rows = output columns n). Each wave loads
//    its packed rows straight into registers -- 32 B per lane per group, one
//    group ahead -- and dequantizes them in registers to exactly
//    RNE((q - z) * s): every weight element is converted once per workgroup
//    and never touches LDS.
//  * Activations are the B operand. A group's 256 x 128 activation tile goes
//    global -> LDS directly (global_load_lds_dwordx4), double-buffered, one
//    instruction per 4 full rows (1 KiB, fully coalesced). LDS row m holds
//    16-byte chunk c of the row at slot c ^ (m % 16): lane i of a load
//    instruction writes slot i % 16 and so fetches chunk (i % 16) ^ (m % 16)
//    (the XOR keeps each 4-lane group inside one 64-byte sector). The MFMA
//    operand reads (32 rows x 16 B per half-wave) then hit distinct banks.
//  * k permutation: lane l (row r = l % 32, half h = l / 32) of k-step (s, t)
//    holds k = 64 s + 32 h + 8 t + e -- word t of chunk 2 s + h of its weight
//    row -- and reads the activation chunk 8 s + 4 h + t, the same k.
//  * Row permutation: MFMA row r of tile half b reads tile position
//    p = 16 (r % 4) + 8 b + 2 (r / 8) + (r / 4) % 2, so the four D rows a lane
//    holds for each r / 8 are four consecutive output columns (an 8-byte
//    piece of a staged row, see g2_store_staged).
constexpr int G2_BM = 256, G2_BN = 256;
constexpr int G2_ROWBLOCKS = G2_BM / 4;  // 1 KiB (4-row) activation loads per group

typedef float f32x16v __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* zr;
  const uint16_t* A;
  uint16_t* C;
  float* slots;         // stream-K: [P][2] fp32 partial tiles
  int M, N, K, G, tiles_n, tiles_m, map;
  int P;                // workgroups
  // map: 0 blockIdx order; 1 XCD-contiguous runs of workgroups; 2 split-K:
  // XCD-contiguous runs over (k-slice, tile row-major), P / tiles slices
  int full;             // tiles [0, full) are done whole, P at a time
  int U;                // (tile, group) units of tiles [full, tiles), split over P
};

// Work split of a workgroup's 4 weight tiles x 8 m-blocks over its NW waves:
//  * NH = 1, NW = 8: a wave owns one 32-row tile half against all 8 m-blocks;
//  * NH = 2, NW = 8: a wave owns a whole 64-row tile against 4 m-blocks (half
//    the LDS reads per MFMA, every weight dequantized by two waves);
//  * NH = 2, NW = 4: one wave per SIMD owns a whole tile against all 8
//    m-blocks (half the LDS reads, every weight dequantized once; its 256
//    accumulator registers take the AGPR half of the register file).
template <int NH, int NW>
struct G2Split {
  static constexpr int MBW = 64 / (NW * NH);         // m-blocks per wave
  static constexpr int UNITS = NH * MBW;             // (half, m-block) pairs per wave
  static constexpr int ACT = G2_ROWBLOCKS / NW;      // activation loads per wave and group
  static constexpr int FIXP = 32 / NW;               // fixup blocks per wave region
  // k-step schedule (measured on MI355X at the config-4 shapes): VALU slots
  // after each MFMA, LDS operand reads after each of the first MFMAs, and the
  // k-steps that carry the next group's activation loads.
  static constexpr int VALU = NW == 8 ? 4 * NH : 2;
  static constexpr int DS = 2;
  static constexpr int ACTSTEPS = NW == 8 ? 4 : 8;
  static_assert(MBW * NH * NW == 64 && ACT % 4 == 0, "unsupported split");
  __device__ static void coords(int wave, int& wt, int& b0, int& mw) {
    wt = NH == 1 ? (wave >> 1) : (wave & 3);   // tile of the 4 this wave owns
    b0 = NH == 1 ? (wave & 1) : 0;             // first tile half
    mw = NH == 1 ? 0 : (wave >> 2) * MBW;      // first m-block
  }
};

template <int NH>
struct WeightGroup {
  u32x4 q[NH][2];    // [half][s]: chunk 2 s + h of this lane's weight row
  uint32_t s[NH];    // scale bits
  uint32_t z[NH];    // zero-point word (4 rows, 4 bits each)
};

// Buffer-resource addressing: a 32-bit per-lane offset (loop-invariant) plus
// a scalar offset, instead of a 64-bit address per lane and load. Loads are
// unconditional (an out-of-range wave reads the last tile and stores nothing),
// and the zero-point word is kept raw: arithmetic on a loaded value here
// would make the compiler wait for every earlier load, including the
// activation loads just issued.
struct G2Rsrc {
  __amdgpu_buffer_rsrc_t qw, sc, zr;
};

// part j < NH: the packed words of tile half j; part NH: the scales and zero
// points; part -1: everything.
template <int NH>
__device__ __forceinline__ void g2_load_weights(WeightGroup<NH>& wg, const G2Rsrc& rs, int G,
                                                int tile, int b0, int g, int lane, int part = -1) {
  const int r = lane & 31, h = lane >> 5;
  const uint32_t blk = (uint32_t)tile * (uint32_t)G + (uint32_t)g;   // < 2^26
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    const int a16 = 8 * (b0 + j) + 2 * (r >> 3) + ((r >> 2) & 1);   // position % 16
    const int p = 16 * (r & 3) + a16;
    if (part < 0 || part == j) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
        wg.q[j][s] = __builtin_amdgcn_raw_buffer_load_b128(rs.qw, ((2 * s + h) * 64 + p) * 16,
                                                           blk * 4096u, 0);
    }
    if (part < 0 || part == NH) {
      wg.s[j] = __builtin_amdgcn_raw_buffer_load_b16(rs.sc, (4 * a16 + (r & 3)) * 2, blk * (uint32_t)kMetaBytes, 0);
      wg.z[j] = __builtin_amdgcn_raw_buffer_load_b16(rs.zr, a16 * 2, blk * 32u, 0);
    }
  }
}

// Issue load i (of G2_ROWBLOCKS / NW) of this wave's share of the activation
// rows of group g into buf. `act` covers rows [m0, M); rows past M lie outside
// it and read as zeros. voff[i % 4] is the lane's byte offset of load i
// relative to its first row (the swizzle repeats every 4 loads).
template <int NW>
__device__ __forceinline__ void g2_load_act1(__amdgpu_buffer_rsrc_t act, const uint32_t (&voff)[4],
                                             uint32_t row_bytes, u32x4* buf, int g, int wave,
                                             int i) {
  const int rb = wave * (G2_ROWBLOCKS / NW) + i;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(act, buf + rb * 64, 16,
                                           voff[i & 3] + (uint32_t)(4 * rb) * row_bytes,
                                           (uint32_t)g * (kGroup * 2), 0, 0);
}
template <int NW>
__device__ __forceinline__ void g2_load_act(__amdgpu_buffer_rsrc_t act, const uint32_t (&voff)[4],
                                            uint32_t row_bytes, u32x4* buf, int g, int wave) {
#pragma unroll
  for (int i = 0; i < G2_ROWBLOCKS / NW; ++i) g2_load_act1<NW>(act, voff, row_bytes, buf, g, wave, i);
}

// One packed word -> 8 bf16 weights RNE((q - z) s), c = -z s, in the order
// of nib8_bits (register i: elements i and i + 4). The even nibbles are the
// low nibbles of the bytes of w & 0x0F0F0F0F, the odd ones of (w >> 4): each
// converts to fp32 in one v_cvt_f32_ubyteN, and fma(q, s, -z s) is exact
// (both products have at most 12 significant bits) -- 23 VALU per word.
__device__ __forceinline__ bf16x8 g2_deq(uint32_t w, float s, float c) {
  const uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;
  float q[8];   // q[2 b] = byte b of ev, q[2 b + 1] = byte b of od
  asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(q[0]) : "v"(ev));
  asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(q[2]) : "v"(ev));
  asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(q[4]) : "v"(ev));
  asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(q[6]) : "v"(ev));
  asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(q[1]) : "v"(od));
  asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(q[3]) : "v"(od));
  asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(q[5]) : "v"(od));
  asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(q[7]) : "v"(od));
  auto f = [&](int e) { return __builtin_fmaf(q[e], s, c); };
  u32x4 o;
  o[0] = pack_bf16x2(f(0), f(4));   // elements 0, 4 (bytes 0 and 2 of ev)
  o[1] = pack_bf16x2(f(1), f(5));   // 1, 5
  o[2] = pack_bf16x2(f(2), f(6));   // 2, 6
  o[3] = pack_bf16x2(f(3), f(7));   // 3, 7
  return __builtin_bit_cast(bf16x8, o);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void g2_wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Linear tile index -> (tn, tm), in bands of 4 M-tiles: consecutive tiles
// share an activation tile (and, 4 apart, a weight tile), so the ~32
// workgroups an XCD runs at once touch ~4 activation and ~8 weight tiles.
__device__ __forceinline__ void g2_tile_coords(const GemmArgs& a, int t, int& tn, int& tm) {
  if (a.map == 2) {   // split-K: row-major, so an XCD's run shares the rows of A
    tm = t / a.tiles_n;
    tn = t - tm * a.tiles_n;
    return;
  }
  const int band = 4 * a.tiles_n;
  const int b = t / band, w = t % band;
  const int rows = min(4, a.tiles_m - 4 * b);
  tm = 4 * b + w % rows;
  tn = w / rows;
}

// Workgroups are dealt round-robin to the 8 XCDs (each with its own L2): XCD x
// runs blocks x, x + 8, ... Renumber so that each XCD owns a contiguous run of
// work. Needs count % 8 == 0 (then it is a bijection).
__device__ __forceinline__ int g2_xcd_order(int blk, int count) {
  return (blk & 7) * (count >> 3) + (blk >> 3);
}

// One wave's share of one (tile, group range) segment: acc = sum over groups
// [g0, g1) of this wave's weight rows x the tile's activation rows.
template <int NH, int NW>
__device__ __forceinline__ void g2_segment(const GemmArgs& a, const G2Rsrc& rs,
                                           u32x4 (*lds)[G2_BM * 16],
                                           f32x16v (&acc)[NH][G2Split<NH, NW>::MBW], int m0,
                                           int ltile, int b0, int mw, int g0, int g1, int wave,
                                           int lane) {
  using Sp = G2Split<NH, NW>;
  constexpr int MBW = Sp::MBW;
  const int r = lane & 31, h = lane >> 5;
  const int zsh = 4 * (r & 3);
#pragma unroll
  for (int j = 0; j < NH; ++j)
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) acc[j][mb] = f32x16v{};
  WeightGroup<NH> cur, nxt;
  // Activation rows [m0, M): the buffer's end turns rows past M into zeros.
  const uint32_t row_bytes = (uint32_t)a.K * 2u;
  const __amdgpu_buffer_rsrc_t act = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.A) + (size_t)m0 * a.K, 0, (int)((uint32_t)(a.M - m0) * row_bytes),
      0x00020000);
  const __amdgpu_buffer_rsrc_t act_none =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.A), 0, 0, 0x00020000);
  const G2Rsrc rs_none = {
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.qw), 0, 0, 0x00020000),
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.sc), 0, 0, 0x00020000),
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.zr), 0, 0, 0x00020000)};
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * i + (lane >> 4);                 // row within the 16-row swizzle period
    const int c = (lane & 15) ^ (row & 15);
    voff[i] = (uint32_t)(lane >> 4) * row_bytes + (uint32_t)c * 16u;
  }
  __syncthreads();   // the previous segment's last LDS reads are done
  g2_load_act<NW>(act, voff, row_bytes, lds[0], g0, wave);
  g2_load_weights(cur, rs, a.G, ltile, b0, g0, lane);
  for (int g = g0; g < g1; ++g) {
    g2_wait_vm0();
    __syncthreads();
    const int sb = (g - g0) & 1;
    const u32x4* buf = lds[sb] + (32 * mw + r) * 16;
    // Group g + 1's activation rows spread evenly over the first Sp::ACTSTEPS
    // k-steps below, so that the 64 KiB the workgroup writes into LDS per
    // group do not arrive in one burst on top of the first steps' operand
    // reads (8 waves: steps 0-3, 4% faster than one burst and 1.5% than one
    // load per step; 4 waves: all 8 steps, equal to steps 0-3); its weights
    // in k-steps kWStep.. kWStep + NH (0.5-0.8% faster than all at the
    // group's start, where they delay its first MFMA).
    // Past the segment's last group the loads go through zero-length
    // resources: they fetch nothing (out-of-range buffer loads return zeros)
    // and need no branch, which would split the k-step schedule below.
    const bool more = g + 1 < g1;
    const __amdgpu_buffer_rsrc_t actn = more ? act : act_none;
    const G2Rsrc rsn = more ? rs : rs_none;
    float sf[NH], cf[NH];
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      sf[j] = bf16_bits_to_f32(cur.s[j]);
      cf[j] = -(float)((cur.z[j] >> zsh) & 0xFu) * sf[j];
    }
    // Software pipeline over the group's 8 k-steps: the activation operands
    // and the dequantized weight operands of step u + 1 are produced while
    // step u's MFMAs run.
    u32x4 xo[2][MBW];
    bf16x8 wd[2][NH];
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) xo[0][mb] = buf[mb * 512 + ((4 * h) ^ (r & 15))];
#pragma unroll
    for (int j = 0; j < NH; ++j) wd[0][j] = g2_deq(cur.q[j][0][0], sf[j], cf[j]);
    // Fence: the prologue's reads must not fill the DS slots of the pattern below.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cu = u & 1, nu = cu ^ 1;
      constexpr int kWStep = 4;
      if (u >= kWStep && u <= kWStep + NH)
        g2_load_weights(nxt, rsn, a.G, ltile, b0, g + 1, lane, u - kWStep);
      if (u < Sp::ACTSTEPS) {
#pragma unroll
        for (int i = 0; i < Sp::ACT / Sp::ACTSTEPS; ++i)
          g2_load_act1<NW>(actn, voff, row_bytes, lds[sb ^ 1], g + 1, wave,
                           Sp::ACT / Sp::ACTSTEPS * u + i);
      }
      if (u + 1 < 8) {
        const int s1 = (u + 1) >> 2, t1 = (u + 1) & 3;
        const int slot = (8 * s1 + 4 * h + t1) ^ (r & 15);
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) xo[nu][mb] = buf[mb * 512 + slot];
#pragma unroll
        for (int j = 0; j < NH; ++j) wd[nu][j] = g2_deq(cur.q[j][s1][t1], sf[j], cf[j]);
      }
#pragma unroll
      for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
        for (int j = 0; j < NH; ++j)
          acc[j][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              wd[cu][j], __builtin_bit_cast(bf16x8, xo[cu][mb]), acc[j][mb], 0, 0, 0);
      if (u + 1 < 8) {
#pragma unroll
        for (int i = 0; i < MBW * NH; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (i < MBW / Sp::DS) __builtin_amdgcn_sched_group_barrier(0x100, Sp::DS, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x002, Sp::VALU, 0);  // VALU
        }
      }
      // NW = 4: one scheduling region per k-step, so that the next step's
      // operand reads stay under this step's MFMAs instead of sinking to their
      // first use (with one wave per SIMD nothing else hides their latency).
      if (NW == 4) __builtin_amdgcn_sched_barrier(0);
    }
    cur = nxt;
  }
}

// Tile store. Accumulator layout: lane holds column m = 32 mb + r and rows
// 8 jq + 4 h + i, i.e. output columns n = 64 tile + 4 (8 b + 2 jq + h) + i.
// Stored from that layout directly, a store instruction writes 8 bytes per
// lane to 32 rows (16-byte pieces of 32 lines), and the partial-line requests
// bound the store of a tile (gate M = 4096: ~10% of the kernel's time). So the
// tile goes through LDS and every store instruction writes whole 128-byte row
// segments of C: each wave stages its own region of the 128 KiB activation
// buffers (its rows x NH * 64 bytes, 16-byte chunk c of row m at c ^ (m %
// CPR)) -- after a wait and a barrier, so that all waves are done with the
// segment's operand reads and their loads have landed -- and reads it back
// row by row. Measured: gate M = 4096 0.617 -> 0.601 ms.
template <int NH, int NW>
__device__ __forceinline__ void g2_store_staged(const GemmArgs& a,
                                                const f32x16v (&acc)[NH][G2Split<NH, NW>::MBW],
                                                u32x4* lds, int m0, int tile, int b0, int mw,
                                                bool valid, int wave, int lane) {
  constexpr int MBW = G2Split<NH, NW>::MBW;
  constexpr int CPR = NH * 4;                      // 16-byte chunks per staged row
  constexpr int ROWS = MBW * 32;
  constexpr int RPI = 64 / CPR;                    // rows per read-back instruction
  const int r = lane & 31, h = lane >> 5;
  g2_wait_vm0();
  __syncthreads();
  u32x4* reg = lds + wave * (ROWS * CPR);
  uint32_t* reg32 = reinterpret_cast<uint32_t*>(reg);
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb) {
    const int row = 32 * mb + r;
#pragma unroll
    for (int j = 0; j < NH; ++j)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const int c = (4 * j + jq) ^ (row % CPR);
        const u32x2 o = {pack_bf16x2(acc[j][mb][4 * jq], acc[j][mb][4 * jq + 1]),
                         pack_bf16x2(acc[j][mb][4 * jq + 2], acc[j][mb][4 * jq + 3])};
        *reinterpret_cast<u32x2*>(reg32 + (row * CPR + c) * 4 + 2 * h) = o;
      }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  if (!valid) return;
  const int cl = lane % CPR;
#pragma unroll
  for (int t = 0; t < ROWS / RPI; ++t) {
    const int row = RPI * t + lane / CPR;
    const u32x4 v = reg[row * CPR + (cl ^ (row % CPR))];
    const int m = m0 + 32 * mw + row;
    if (m < a.M)
      *reinterpret_cast<u32x4*>(a.C + (size_t)m * a.N + tile * kTileN + 32 * b0 + 8 * cl) = v;
  }
}

// Stream-K partial tiles. Each workgroup has two fp32 slots (for its first
// and its last tile), laid out [wave][pair][i][lane]: 16-byte piece i of a
// lane's 64 bytes at 1024 i + 16 lane, so that every store (and the fixup's
// every load) covers 1 KiB contiguously; lane-major 64-byte runs made each
// instruction write 16-byte pieces of 32 lines (down M = 512: 0.111 -> 0.098
// ms). A workgroup whose range cuts a tile writes its partial there; a second
// kernel (k_gemm_fixup, stream-ordered after this one) sums each cut tile's
// slots in workgroup order -- a fixed order, so results are bitwise
// reproducible -- and stores the tile.
constexpr uint32_t kSlotBytes = (uint32_t)G2_BM * G2_BN * 4;   // 256 KiB

// idx: the wave's (half, m-block) pair j * MBW + mb, of `units` per wave.
__device__ __forceinline__ uint32_t g2_slot_off(int vp, int which, int wave, int units, int idx,
                                                int lane) {
  return (uint32_t)(vp * 2 + which) * kSlotBytes + (uint32_t)((wave * units + idx) * 4096 + lane * 16);
}

template <int NH, int NW>
__device__ __forceinline__ void g2_slot_store(__amdgpu_buffer_rsrc_t rs,
                                              const f32x16v (&acc)[NH][G2Split<NH, NW>::MBW],
                                              int vp, int which, int wave, int lane) {
  constexpr int MBW = G2Split<NH, NW>::MBW;
#pragma unroll
  for (int j = 0; j < NH; ++j)
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) {
      const uint32_t off = g2_slot_off(vp, which, wave, NH * MBW, j * MBW + mb, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = {__float_as_uint(acc[j][mb][4 * i]), __float_as_uint(acc[j][mb][4 * i + 1]),
                         __float_as_uint(acc[j][mb][4 * i + 2]),
                         __float_as_uint(acc[j][mb][4 * i + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, off + 1024 * i, 0, 0);
      }
    }
}

// Ranges over the split tiles' units (unit u: tile full + u / G).
__device__ __forceinline__ int g2_range_start(const GemmArgs& a, int vp) {
  return (int)((long long)vp * a.U / a.P);
}
// Largest vp with g2_range_start(vp) <= u.
__device__ __forceinline__ int g2_owner_of(const GemmArgs& a, int u) {
  return (int)(((long long)(u + 1) * a.P - 1) / a.U);
}

// The cut tiles' fp32 partials are summed by many small blocks: block
// (tile ts, main-kernel wave w, part) owns the pairs [part * 2, part * 2 + 2)
// of wave w's region (the slot layout [wave][pair][i][lane] keeps them
// contiguous), so a cut tile is read by 32 blocks at once instead of one
// workgroup (one workgroup summing its tile inside k_gemm measured slower). A block loads kFixAhead pieces before it adds them, in piece
// order, so that the loads of a tile split many ways overlap instead of
// paying one memory latency per piece. Tiles a single workgroup covered were
// stored by the main kernel.
constexpr int kFixBlocksPerTile = 32;
constexpr int kFixAhead = 4;

template <int NH, int NW>
__global__ __launch_bounds__(64) void k_gemm_fixup(GemmArgs a) {
  using Sp = G2Split<NH, NW>;
  constexpr int MBW = Sp::MBW;
  constexpr int kPer = Sp::UNITS / Sp::FIXP;   // (half, m-block) pairs per block
  static_assert(NW * Sp::FIXP == kFixBlocksPerTile && kPer == 2, "fixup split");
  const int ts = blockIdx.x / kFixBlocksPerTile;   // split tile full + ts
  const int wave = (blockIdx.x / Sp::FIXP) % NW;
  const int part = blockIdx.x % Sp::FIXP;
  const int t = a.full + ts;
  const int p0 = g2_owner_of(a, ts * a.G), p1 = g2_owner_of(a, ts * a.G + a.G - 1);
  if (p0 == p1) return;
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  int wt, b0, mw;
  Sp::coords(wave, wt, b0, mw);
  int tn, tm;
  g2_tile_coords(a, t, tn, tm);
  const int tile = tn * 4 + wt;
  if (tile * kTileN >= a.N) return;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(a.slots, 0, (int)(2u * a.P * kSlotBytes), 0x00020000);
  f32x16v acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) acc[e] = f32x16v{};
  for (int pp = p0; pp <= p1; pp += kFixAhead) {
    u32x4 v[kFixAhead][kPer][4];
#pragma unroll
    for (int k = 0; k < kFixAhead; ++k) {
      // pieces past p1 read out of range (zeros, no memory access) and are
      // never added: adding +0 would turn a -0 sum into +0
      const int q = pp + k;
      const bool live = q <= p1;
      const int which = (live && g2_range_start(a, q) / a.G == ts) ? 0 : 1;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const uint32_t off =
            live ? g2_slot_off(q, which, wave, Sp::UNITS, part * kPer + e, lane) : 0x80000000u;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[k][e][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 1024 * i, 0, 0);
      }
    }
#pragma unroll
    for (int k = 0; k < kFixAhead; ++k) {
      if (pp + k > p1) break;
#pragma unroll
      for (int e = 0; e < kPer; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[e][4 * i + c] += __uint_as_float(v[k][e][i][c]);
    }
  }
  // pair index j * MBW + mb (g2_slot_store's order)
  const int m0 = tm * G2_BM;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int idx = part * kPer + e, j = idx / MBW, mb = idx % MBW;
    const int m = m0 + 32 * (mw + mb) + r;
    if (m >= a.M) continue;
    uint16_t* crow = a.C + (size_t)m * a.N + tile * kTileN;
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const u32x2 o = {pack_bf16x2(acc[e][4 * jq], acc[e][4 * jq + 1]),
                       pack_bf16x2(acc[e][4 * jq + 2], acc[e][4 * jq + 3])};
      *reinterpret_cast<u32x2*>(crow + 4 * (8 * (b0 + j) + 2 * jq + h)) = o;
    }
  }
}

template <int NH, int NW>
__global__ __launch_bounds__(64 * NW, 1) void k_gemm(GemmArgs a) {
  using Sp = G2Split<NH, NW>;
  constexpr int MBW = Sp::MBW;              // m-blocks per wave
  __shared__ u32x4 lds[2][G2_BM * 16];      // 2 x 64 KiB: [row][16 swizzled chunks]
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
  const int lane = threadIdx.x & 63;
  int wt, b0, mw;
  Sp::coords(wave, wt, b0, mw);
  f32x16v acc[NH][MBW];

  // Virtual workgroup vp (XCD x owns a contiguous run of vp) first does the
  // whole tiles vp, vp + P, ... < full, then the units [start(vp),
  // start(vp + 1)) of the U = (tiles - full) x G units of the remaining
  // tiles: ranges that cut a tile (stream-K) are combined through slots.
  // P = tiles, full = tiles: one whole tile per workgroup.
  int vp = a.map ? g2_xcd_order(blockIdx.x, a.P) : (int)blockIdx.x;
  if (a.map == 2) {
    // Split-K: the P = tiles x S ranges are the S k-slices of each tile (vp =
    // tile S + slice). The XCD runs go over slices, then tiles row-major, so
    // the ~30 workgroups of an XCD work on the same k-slice of one or two
    // rows of tiles: they share A's rows in their L2, at the same k.
    const int nt = a.tiles_n * a.tiles_m, S = a.P / nt;
    const int sl = vp / nt, ts = vp - sl * nt;
    vp = ts * S + sl;
  }
  const int u0 = g2_range_start(a, vp), u1 = g2_range_start(a, vp + 1);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(a.slots, 0, (int)(2u * a.P * kSlotBytes), 0x00020000);
  G2Rsrc wr;
  wr.qw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.qw), 0,
                                            (int)((uint32_t)a.N * (uint32_t)a.K / 2u), 0x00020000);
  wr.sc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.sc), 0,
      (int)((uint32_t)a.N / kTileN * (uint32_t)a.G * (uint32_t)kMetaBytes), 0x00020000);
  wr.zr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.zr), 0,
                                            (int)((uint32_t)a.N * (uint32_t)a.G / 2u), 0x00020000);
  for (int t = vp; t < a.full; t += a.P) {
    int tn, tm;
    g2_tile_coords(a, t, tn, tm);
    const int tile = tn * 4 + wt;
    const bool valid = tile * kTileN < a.N;
    const int ltile = valid ? tile : (a.N / kTileN - 1);
    g2_segment<NH, NW>(a, wr, lds, acc, tm * G2_BM, ltile, b0, mw, 0, a.G, wave, lane);
    g2_store_staged<NH, NW>(a, acc, &lds[0][0], tm * G2_BM, tile, b0, mw, valid, wave, lane);
  }
  for (int u = u0; u < u1;) {
    const int ts = u / a.G, g0 = u - ts * a.G;
    const int g1 = min(a.G, u1 - ts * a.G);
    int tn, tm;
    g2_tile_coords(a, a.full + ts, tn, tm);
    const int tile = tn * 4 + wt;
    const bool valid = tile * kTileN < a.N;
    const int ltile = valid ? tile : (a.N / kTileN - 1);
    g2_segment<NH, NW>(a, wr, lds, acc, tm * G2_BM, ltile, b0, mw, g0, g1, wave, lane);
    if (g0 == 0 && g1 == a.G) {
      g2_store_staged<NH, NW>(a, acc, &lds[0][0], tm * G2_BM, tile, b0, mw, valid, wave, lane);
    } else {
      g2_slot_store<NH, NW>(rs, acc, vp, u == u0 ? 0 : 1, wave, lane);
    }
    u = ts * a.G + g1;
  }
}

// Workspace bytes that enable stream-K: two fp32 partial tiles per CU.
size_t gemm_workspace_need(int cus) { return 2ull * (size_t)cus * kSlotBytes; }

int device_cus() {
  static std::once_flag once[64];
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::call_once(once[dev], [dev] {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  });
  return cus[dev];
}

// Tuning and test override of the prefill schedule (qw4_tune_gemm): -1 the
// cost model, 0 per tile, 1 stream-K, 2 hybrid, 3 split-K.
std::atomic<int> g_gemm_schedule{-1};
// Kernel variant (qw4_tune_gemm): 0 the default, 4 waves of whole 64-row
// tiles against all 256 activation rows; 1 8 waves of 32-row tile halves; 2 8
// waves of whole tiles against 128 rows. All three sum every output in the
// same order, so their results are bitwise equal.
std::atomic<int> g_gemm_variant{0};

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

int qw4_tune_gemm(int schedule, int variant) {
  if (schedule < -1 || schedule > 3 || variant < 0 || variant > 2) return QW4_ERR_SHAPE;
  g_gemm_schedule.store(schedule, std::memory_order_relaxed);
  g_gemm_variant.store(variant, std::memory_order_relaxed);
  return QW4_OK;
}

int qw4_gemm(uint16_t* C, const qw4_weights* w, const uint16_t* A, int M, qw4_workspace* ws,
             void* stream) {
  int st = check_weights_public(w);
  if (st) return st;
  if (!C || !A) return QW4_ERR_NULL;
  if (M < 1) return QW4_ERR_M;
  if (((uintptr_t)A & 15) || ((uintptr_t)C & 7)) return QW4_ERR_ALIGN;
  // Loads address A and the weights through 32-bit buffer offsets.
  if ((size_t)M * w->in_f * 2 >= (1ull << 32) || (size_t)w->out_f * w->in_f / 2 >= (1ull << 32))
    return QW4_ERR_SHAPE;
  {
    const int tiles_n = (w->out_f + G2_BN - 1) / G2_BN;
    const int tiles_m = (M + G2_BM - 1) / G2_BM;
    const int nt = tiles_n * tiles_m;
    GemmArgs a{w->qweight, w->scale, w->zeros, A, C, nullptr, M, w->out_f, w->in_f,
                w->num_groups, tiles_n, tiles_m, nt % 8 == 0, nt, nt, 0};
    int grid = nt;
    // Three schedules, costed in group-steps per CU (one 256 x 256 x 128
    // tile step; measured on MI355X at the config-4 shapes):
    //  * per tile: one workgroup per tile, ceil(nt / CUs) G;
    //  * stream-K: one workgroup per CU, all nt G (tile, group) units split
    //    evenly, nt G / CUs + 16 (two fp32 partial tiles written per
    //    workgroup) + 0.1 per piece of a cut tile (k_gemm_fixup's blocks read
    //    a tile's pieces one after another);
    //  * hybrid: whole tiles for the floor(nt / CUs) full rounds, then the
    //    other nt % CUs tiles split over the CUs: the same work, one partial
    //    per workgroup (+8), CUs / (nt % CUs) pieces per cut tile;
    //  * split-K (at most CUs / 2 tiles): every tile cut into the same S
    //    k-slices, S = CUs / nt (P = nt S workgroups, a multiple of 8, at
    //    least 2 groups per slice): G / S + 8 + 0.1 S. Against stream-K it
    //    writes one partial per workgroup instead of up to two, and the
    //    workgroups of an XCD share A at the same k (down M = 1024: 0.159
    //    against 0.170-0.180 ms; down M = 512 0.094 against 0.102-0.107).
    // A split schedule runs when it beats per-tile by 5% (qw4_tune_gemm
    // forces one, for tests and tuning): gate M = 512, 136 tiles, costs 37.6
    // against 40 and measured 0.880 against 0.842 PFLOP/s.
    const int sk_env = g_gemm_schedule.load(std::memory_order_relaxed);
    const int cus = device_cus();
    const long long G = w->num_groups;
    const int rem = nt % cus;
    const double t_dp = (double)((nt + cus - 1) / cus) * G;
    const double work = (double)nt * G / cus;
    const double t_sk = work + 16.0 + 0.1 * ((cus + nt - 1) / nt + 1);
    const double t_hy = work + 8.0 + 0.1 * (rem ? (cus + rem - 1) / rem + 1 : 0);
    const bool ws_ok = ws && ws->buf && ws->bytes >= gemm_workspace_need(cus) && cus % 8 == 0 &&
                       rem != 0 && (long long)nt * G < (1LL << 31);
    const bool sk_ok = ws_ok && (long long)nt * G >= 2LL * cus;
    const bool hy_ok = ws_ok && nt > cus && (long long)rem * G >= (long long)cus;
    int S = 2 * nt <= cus ? (int)std::min<long long>(cus / nt, G / 2) : 0;
    while (S >= 2 && (nt * S) % 8) --S;
    const bool kk_ok = ws_ok && S >= 2;
    const double t_kk = (double)G / (S > 0 ? S : 1) + 8.0 + 0.1 * S;
    int pick = 0;   // 0 per tile, 1 stream-K, 2 hybrid, 3 split-K
    if (sk_env == 1 && sk_ok) pick = 1;
    else if (sk_env == 2 && hy_ok) pick = 2;
    else if (sk_env == 3 && kk_ok) pick = 3;
    else if (sk_env == -1) {
      double best = 0.95 * t_dp;
      if (sk_ok && t_sk < best) { pick = 1; best = t_sk; }
      if (hy_ok && t_hy < best) { pick = 2; best = t_hy; }
      if (kk_ok && t_kk < best) pick = 3;
    }
    if (pick == 3) {
      a.slots = static_cast<float*>(ws->buf);
      a.P = nt * S;
      a.full = 0;
      a.U = (int)(nt * G);
      a.map = 2;
      grid = a.P;
    } else if (pick) {
      a.slots = static_cast<float*>(ws->buf);
      a.P = cus;
      a.full = pick == 2 ? nt - rem : 0;
      a.U = (int)((nt - a.full) * G);
      a.map = 1;
      grid = cus;
    }
    hipStream_t s = (hipStream_t)stream;
    const int variant = g_gemm_variant.load(std::memory_order_relaxed);
    if (variant == 1)
      k_gemm<1, 8><<<grid, 512, 0, s>>>(a);
    else if (variant == 2)
      k_gemm<2, 8><<<grid, 512, 0, s>>>(a);
    else
      k_gemm<2, 4><<<grid, 256, 0, s>>>(a);
    QW4_LAUNCH_CHECK();
    if (a.full != nt) {   // the split tiles
      const int fb = (nt - a.full) * kFixBlocksPerTile;
      if (variant == 1)
        k_gemm_fixup<1, 8><<<fb, 64, 0, s>>>(a);
      else if (variant == 2)
        k_gemm_fixup<2, 8><<<fb, 64, 0, s>>>(a);
      else
        k_gemm_fixup<2, 4><<<fb, 64, 0, s>>>(a);
    }
    QW4_LAUNCH_CHECK();
    return QW4_OK;
  }
}

}  // extern "C"
