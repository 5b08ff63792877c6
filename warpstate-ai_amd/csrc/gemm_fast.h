// Fast-path BF16 GEMM for gfx950: direct-to-LDS operand loads, 16x16x32 MFMA.
//
// C[m, n] = sum_k A[m, k] B[k, n] with FP32 accumulation and the same epilogues as
// gemm.h, for operands whose reduction dim or row dim is contiguous (every layout the
// training step produces: X and W^T are K-contiguous; dY^T, X in weight gradients and W
// in input gradients are M/N-contiguous).
//
// Workgroup: 256 x 256 output tile, BK = 64, 8 waves on a 4 x 2 grid (wave tile 64 x 128),
// two LDS stages of 64 KiB (A 32 KiB + B 32 KiB).
//  * Loads: `buffer_load_dword x4 ... lds` writes 16 bytes per lane straight into LDS at
//    M0 + 16 * lane; the choice of global address per lane implements the LDS swizzle.
//    Out-of-range rows, columns and k take an offset beyond the buffer's range and land
//    as zeros.
//  * K-contiguous operand tile: [rows][64 k], 128-byte rows of eight 16-byte chunks,
//    chunk c of row r at slot c ^ swz(r) (gemm.h). Fragments are one ds_read_b128.
//  * M/N-contiguous operand tile: four blocks of 64 operand rows, each [64 k][128 B]
//    (8 KiB): chunk c (operand rows 8c .. 8c + 7 of the block) of k-row kk at slot
//    c ^ mnsw(kk), mnsw(kk) = 2 ((kk >> 1 & 1) | (kk >> 3 & 1) << 1). A load instruction
//    then covers 8 k-rows x 128 bytes, one cache line each (a [64 k][512 B] layout, with
//    2 k-rows x 512 bytes per instruction, ran the weight gradients 7-10 % slower).
//    Fragments are two ds_read_b64_tr_b16: within each 16-lane group the transposing read
//    hands element q of the 8 bytes addressed by lane L to lane 4 (L & 3) + q, slot L >> 2,
//    so lane L addressing k-row k0 + (L >> 2), rows 4 (L & 3) .. + 3 leaves each lane four
//    consecutive k of one row. Per read the 16 k-rows x 32 bytes fall on 16 distinct
//    16-byte bank slots twice each (two passes of 256 bytes, no conflicts).
//  * MFMA v_mfma_f32_16x16x32_bf16 with the B fragment as the instruction's A operand:
//    lane l then holds output row m = m0 + 16 i + (l & 15), columns n0 + 16 j + 4 (l >> 4)
//    + e, e = 0..3, which the epilogues store as 8-byte (BF16) or 16-byte (FP32) vectors.
//  * Pipeline per k-tile, both operands K-contiguous: A has two LDS stages and B three
//    (160 KiB). Wait for this wave's loads of the tile (leaving the 4 loads of B two tiles
//    ahead in flight), s_barrier (no memory fence: the explicit vmcnt wait is the only
//    ordering needed), issue A of the next tile, then the two k32 steps with the second
//    step's fragment reads interleaved between the first step's MFMAs, and between the two
//    steps the loads of B two tiles ahead. Those land while the second step runs without
//    LDS reads, and only half a tile's loads leave in a burst after the barrier (the
//    forward GEMMs 3-7 % faster than with both operands' next tile loaded there).
//  * Both operands M/N-contiguous (the weight gradients): two stages of 64 KiB; after the
//    barrier the next tile's loads for both operands, then the transposing fragment reads.
//    The reads are inline assembly with explicit lgkmcnt waits: the compiler orders the
//    transposing-read builtin after every pending direct-to-LDS load (it cannot rule out
//    an alias), which would otherwise hold those loads back until after the tile's last
//    read and leave them half a k-tile of lead (the weight gradients 9 % slower).
//  * One operand of each kind: both in two stages, the next tile's loads between the two
//    steps (after the tile's last transposing read).
//  * Tiles follow the grouped raster of ops/matmul_kernels.py:72-78 after an XCD remap.
#pragma once

#include <type_traits>

#include "gemm.h"

namespace ws {

constexpr int kFBM = 256, kFBN = 256, kFBK = 64, kFWM = 4, kFWN = 2;
constexpr int kFNT = kFWM * kFWN * kWave;               // 512 threads
constexpr int kFTileBytes = 256 * kFBK * 2;             // one operand tile, 32 KiB
constexpr int kFStageBytes = 2 * kFTileBytes;
constexpr int kFLdsBytes = 2 * kFStageBytes;            // 128 KiB
// Epilogue staging: each wave's 64 x 128 BF16 tile, rows padded to 272 bytes so that both
// the fragment-order writes and the row-order 16-byte reads are bank-conflict free.
constexpr int kFStageRow = 272;
constexpr int kFStageWave = 64 * kFStageRow;
constexpr int kFLdsAlloc = 8 * kFStageWave > kFLdsBytes ? 8 * kFStageWave : kFLdsBytes;
// Both operands K-contiguous: A in two stages, B in three (the whole 160 KiB of a CU).
constexpr int kFLdsAllocKK = 5 * kFTileBytes;
static_assert(kFLdsAllocKK >= 8 * kFStageWave, "the epilogue staging fits the K-contiguous layout");
template <int AM, int BM>
constexpr int fast_lds_bytes() { return AM == kKContig && BM == kKContig ? kFLdsAllocKK : kFLdsAlloc; }
constexpr int kFIns = kFTileBytes / (kFNT * 16);         // 4 loads per thread per operand
// Cache policy of the epilogues' outputs and auxiliary inputs: non-temporal. Each is
// touched once, in bursts when all CUs reach their epilogues together, and it should not
// displace the operand tiles that other workgroups are still reading from L2 (dAct 4-5 %
// faster). The FP32 accumulation keeps the default: its gradient and split-K partial
// blocks are read again soon.
constexpr int kEpiNT = 2;

typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int mnsw(int kk) { return 2 * (((kk >> 1) & 1) | (((kk >> 3) & 1) << 1)); }

// waitcnt immediate for "vmcnt <= n" leaving the other counters unconstrained (gfx9).
constexpr int wait_vmcnt(int n) { return (n & 0xF) | (7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

#define WS_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Direct-to-LDS loader of one 256-row operand tile. `off[i]` is the byte offset of this
// lane's 16-byte chunk for load i relative to the tile's global base at k0, or kOOB.
template <int MODE, bool PAIRED>
struct DmaTile {
  unsigned off[kFIns];

  // k offset within the tile of load i's chunk: 8 c (K-contiguous) or the k-row kk.
  __device__ __forceinline__ static int k_of(int i, int wave, int lane) {
    const int byte = (i * (kFNT / kWave) + wave) * 1024 + lane * 16;
    if constexpr (MODE == kKContig) return 8 * (((byte >> 4) & 7) ^ swz(byte >> 7));
    else return ((byte >> 10) & 7) * 8 + (lane >> 3);
  }
  __device__ __forceinline__ void init(const OperandDesc& d, int row0, int rows_valid, int half,
                                       int wave, int lane) {
#pragma unroll
    for (int i = 0; i < kFIns; ++i) {
      const int byte = (i * (kFNT / kWave) + wave) * 1024 + lane * 16;
      if constexpr (MODE == kKContig) {
        const int r = byte >> 7, c = ((byte >> 4) & 7) ^ swz(r);
        const int logical = row0 + (PAIRED && r >= 128 ? r - 128 : r);
        const int phys = PAIRED && r >= 128 ? half + logical : logical;
        off[i] = logical < rows_valid ? (unsigned)((long)(phys - row0) * d.s_row * 2 + 16 * c) : kOOB;
      } else {
        const int q = byte >> 10, kk = (q & 7) * 8 + (lane >> 3);
        const int c = (lane & 7) ^ mnsw(kk);
        const int r = (q >> 3) * 64 + 8 * c;  // first operand row of the chunk
        const int logical = row0 + (PAIRED && r >= 128 ? r - 128 : r);
        const int phys = PAIRED && r >= 128 ? half + logical : logical;
        off[i] = logical < rows_valid ? (unsigned)((phys - row0) * 2 + (long)kk * d.s_k * 2) : kOOB;
      }
    }
  }
  // Load i alone of the tile at k0, branch-free so that it can be scheduled among MFMAs:
  // a chunk at k >= K, or every chunk when `live` is false, takes the out-of-range offset
  // and lands as zeros without a memory read.
  __device__ __forceinline__ void issue_one(const OperandDesc& d, int row0, int k0, int K,
                                            unsigned char* lds_tile, int wave, int lane, int i,
                                            bool live) const {
    const unsigned short* base =
        MODE == kKContig ? d.ptr + (long)row0 * d.s_row + k0 : d.ptr + row0 + (long)k0 * d.s_k;
    __amdgpu_buffer_rsrc_t rs = make_rsrc(base, 0x7fffffff);
    int l = lane;
    asm volatile("" : "+v"(l));
    const bool dead = !live | (k0 + k_of(i, wave, l) >= K);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, WS_LDS(lds_tile + (i * (kFNT / kWave) + wave) * 1024),
                                             16, dead ? kOOB : off[i], 0, 0, 0);
  }
  // Loads of the tile at k0 into `lds_tile`; chunks at k >= K load zeros. The per-lane k
  // test only runs on a ragged last tile.
  __device__ __forceinline__ void issue(const OperandDesc& d, int row0, int k0, int K,
                                        unsigned char* lds_tile, int wave, int lane) const {
    const unsigned short* base =
        MODE == kKContig ? d.ptr + (long)row0 * d.s_row + k0 : d.ptr + row0 + (long)k0 * d.s_k;
    __amdgpu_buffer_rsrc_t rs = make_rsrc(base, 0x7fffffff);
    if (k0 + kFBK <= K) {
#pragma unroll
      for (int i = 0; i < kFIns; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, WS_LDS(lds_tile + (i * (kFNT / kWave) + wave) * 1024),
                                                 16, off[i], 0, 0, 0);
    } else {
      // Ragged last k-tile. The lane index goes through an empty asm so that the per-lane
      // k offsets are computed here and not kept live across the k-loop.
      int l = lane;
      asm volatile("" : "+v"(l));
#pragma unroll
      for (int i = 0; i < kFIns; ++i) {
        const unsigned o = k0 + k_of(i, wave, l) >= K ? kOOB : off[i];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, WS_LDS(lds_tile + (i * (kFNT / kWave) + wave) * 1024),
                                                 16, o, 0, 0, 0);
      }
    }
  }
};

// Fragment reads for 16-row block at tile row `rb` (multiple of 16), k32 step s.
template <int MODE>
__device__ __forceinline__ bf16x8_t read_frag(const unsigned char* tile, int rb, int s, int lane) {
  if constexpr (MODE == kKContig) {
    const int r = rb + (lane & 15);
    const int c = (4 * s + (lane >> 4)) ^ swz(r);
    return *reinterpret_cast<const bf16x8_t*>(tile + r * 128 + c * 16);
  } else {
    const int L = lane & 15, g = lane >> 4;
    const int m = rb + 4 * (L & 3);
    const int kk0 = 32 * s + 8 * g + (L >> 2);
    const int kk1 = kk0 + 4;
    const int blk = (m >> 6) * 8192, c = (m >> 3) & 7, hb = (m & 4) * 2;  // hb: 0 or 8
    const unsigned char* p0 = tile + blk + kk0 * 128 + ((c ^ mnsw(kk0)) << 4) + hb;
    const unsigned char* p1 = tile + blk + kk1 * 128 + ((c ^ mnsw(kk1)) << 4) + hb;
    i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4_t*)(p0));
    i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4_t*)(p1));
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    i16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
  }
}

// Transposing fragment reads as inline assembly, for the loop with both operands
// M/N-contiguous. The compiler does not see them as LDS accesses, so the direct-to-LDS
// loads of the next tile may be issued before them without an added vmcnt wait; their
// results are made visible by tie_wait, an explicit lgkmcnt(0) that redefines the
// fragment registers, so no MFMA reading them can be scheduled ahead of the wait.
template <int OFF>
__device__ __forceinline__ u32x2_t tr_read(unsigned addr) {
  u32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
// Fragment of k32 step S at LDS byte address `addr` (tr_base plus the stage offset): the
// two reads of read_frag<kMNContig>, k-rows kk0 and kk0 + 4 (the same swizzle, 512 bytes
// apart); step 1 is 32 k-rows (4096 bytes) further with the same swizzle.
template <int S>
__device__ __forceinline__ bf16x8_t tr_frag(unsigned addr) {
  const u32x2_t lo = tr_read<S * 4096>(addr), hi = tr_read<S * 4096 + 512>(addr);
  const u32x4_t v = {lo[0], lo[1], hi[0], hi[1]};
  return __builtin_bit_cast(bf16x8_t, v);
}
// Byte offset, within an M/N-contiguous operand tile, of lane's first read of the
// fragment of the 16-row block at tile row rb, k32 step 0 (read_frag<kMNContig>).
__device__ __forceinline__ unsigned tr_base(int rb, int lane) {
  const int L = lane & 15, g = lane >> 4;
  const int m = rb + 4 * (L & 3);
  const int kk0 = 8 * g + (L >> 2);
  const int blk = (m >> 6) * 8192, c = (m >> 3) & 7, hb = (m & 4) * 2;
  return (unsigned)(blk + kk0 * 128 + ((c ^ mnsw(kk0)) << 4) + hb);
}
__device__ __forceinline__ void tie_wait(bf16x8_t (&f)[12]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                 "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11])
               :: "memory");
}

template <int FA, int FB>
struct Acc16 {
  f32x4_v v[FA][FB];
};

// The lane index through an empty asm: per-lane address math that depends on it stays in
// the epilogue instead of being hoisted out of the tile loop and kept live (spilled)
// across the main loop.
__device__ __forceinline__ void opaque_lane(int& lane) { asm volatile("" : "+v"(lane)); }

// --------------------------------------------------------------------------------------
// Epilogues on the 16x16 accumulator layout. Lane l holds, for block (i, j), row
//   m = m_base + 16 i + (l & 15) and columns n = n_base + 16 j + 4 (l >> 4) + e.
// They store whole 4-column vectors only (GemmParams::vec_out); the host sends shapes
// without vector outputs to the generic kernel of gemm.h.

// Plain BF16 store with optional column-range sigmoid and BF16 residual add
// (same numerics as EpiStore). The wave's 64 x 128 tile goes through its LDS staging rows
// so that the global writes (and residual reads) are 16-byte pieces covering 256 bytes
// of each row, instead of 8-byte pieces scattered over 16 rows per instruction.
template <bool SIGMOID, bool RESIDUAL>
struct FEpiStore {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    static_assert(FA * 16 == 64 && FB * 16 == 128, "staging holds a 64 x 128 wave tile");
    opaque_lane(lane);
    // Fragment order -> staging rows, sigmoid applied, every value rounded to BF16. The
    // gate test is made once per wave for its 128 columns (n_base is wave-uniform): with a
    // per-element test the compiler evaluates the sigmoid of every element and selects,
    // which cost the 9216-wide projection 7 % for its 2048 gate columns.
    enum { kNone, kAll, kSome };
    const int gate = !SIGMOID || n_base >= p.gate_hi || n_base + FB * 16 <= p.gate_lo ? kNone
                     : n_base >= p.gate_lo && n_base + FB * 16 <= p.gate_hi        ? kAll
                                                                                   : kSome;
    auto stage_frags = [&](auto f) {
#pragma unroll
      for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          const int r = 16 * i + (lane & 15), c = 16 * j + 4 * (lane >> 4);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = f(acc.v[i][j][e], n_base + c + e);
          u32x2_t w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          *reinterpret_cast<u32x2_t*>(stage + r * kFStageRow + c * 2) = w;
        }
    };
    if (gate == kNone) {
      stage_frags([](float x, int) { return x; });
    } else if (gate == kAll) {
      stage_frags([](float x, int) { return sigmoid(rbf16(x)); });
    } else {
      stage_frags([&](float x, int n) {
        x = rbf16(x);
        return n >= p.gate_lo && n < p.gate_hi ? sigmoid(x) : x;
      });
    }
    // The accumulators are dead from here; the loads below must not be hoisted above.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes landed
    // Row order: lane (16 per row) owns 8 columns; 4 rows per instruction.
    const int c8 = 8 * (lane & 15);
    const int n = n_base + c8;
    const bool full = n + 7 < p.N, half = n + 3 < p.N;  // N % 4 == 0 (vec_out)
    __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c + (long)m_base * p.ldc + n_base, 0x7fffffff);
    u32x4_t rv[16];
    if (RESIDUAL) {
      __amdgpu_buffer_rsrc_t rr = make_rsrc(p.aux + (long)m_base * p.ldaux + n_base, 0x7fffffff);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = 4 * q + (lane >> 4);
        const bool ok = m_base + r < p.M;
        const long off = (long)r * p.ldaux + c8;
        if (full) {
          rv[q] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rr, store_off(ok, off, 2), 0, kEpiNT));
        } else {
          const u32x2_t h = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
              rr, store_off(ok && half, off, 2), 0, kEpiNT));
          rv[q] = u32x4_t{h[0], h[1], 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = 4 * q + (lane >> 4);
      const bool ok = m_base + r < p.M;
      u32x4_t vd = *reinterpret_cast<const u32x4_t*>(stage + r * kFStageRow + c8 * 2);
      if (RESIDUAL) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          vd[d] = pack_bf16x2(lo_bf16(vd[d]) + lo_bf16(rv[q][d]), hi_bf16(vd[d]) + hi_bf16(rv[q][d]));
      }
      const long off = (long)r * p.ldc + c8;
      if (full) {
        __builtin_amdgcn_raw_buffer_store_b128(vd, rc, store_off(ok, off, 2), 0, kEpiNT);
      } else {
        const u32x2_t h = {vd[0], vd[1]};
        __builtin_amdgcn_raw_buffer_store_b64(h, rc, store_off(ok && half, off, 2), 0, kEpiNT);
      }
    }
  }
};

// Paired SwiGLU forward (EpiSwiglu numerics): blocks j < FB/2 are up columns, j + FB/2
// the gate columns of the same output columns. The rounded up | gate tile goes through the
// wave's LDS staging rows (64 rows x 64 up + 64 gate columns); then each lane takes 8
// columns of one row, computes their activations and writes up, gate and activation as
// 16-byte pieces (8 lanes per 128-byte row piece, 8 rows per instruction).
struct FEpiSwiglu {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    static_assert(FA * 16 == 64 && FB * 16 == 128, "staging holds a 64 x 128 wave tile");
    opaque_lane(lane);
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int r = 16 * i + (lane & 15), c = 16 * j + 4 * (lane >> 4);
        u32x2_t w = {pack_bf16x2(acc.v[i][j][0], acc.v[i][j][1]),
                     pack_bf16x2(acc.v[i][j][2], acc.v[i][j][3])};
        *reinterpret_cast<u32x2_t*>(stage + r * kFStageRow + c * 2) = w;
      }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes landed
    const int c8 = 8 * (lane & 7);
    const int n = n_base + c8;  // column in [0, H)
    const bool full = n + 7 < p.H, half = n + 3 < p.H;  // H % 4 == 0 (vec_out)
    __amdgpu_buffer_rsrc_t rp = make_rsrc(p.c + (long)m_base * p.ldc + n_base, 0x7fffffff);
    __amdgpu_buffer_rsrc_t ra = make_rsrc(p.c2 + (long)m_base * p.ldc2 + n_base, 0x7fffffff);
    const long hoff = p.H;
    const bool eager = p.eager;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int r = 8 * q + (lane >> 3);
      const bool ok = m_base + r < p.M;
      const u32x4_t vu = *reinterpret_cast<const u32x4_t*>(stage + r * kFStageRow + c8 * 2);
      const u32x4_t vg = *reinterpret_cast<const u32x4_t*>(stage + r * kFStageRow + (64 + c8) * 2);
      u32x4_t va;
      // The rounding mode is tested once per row group, not per element (the compiler
      // otherwise computes both and selects).
      if (eager) {
        // The pair's two SiLU values rounded by one packed conversion.
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          unsigned ws = pack_bf16x2(silu(lo_bf16(vg[d])), silu(hi_bf16(vg[d])));
          asm volatile("" : "+v"(ws));  // keeps the conversion packed
          va[d] = pack_bf16x2(lo_bf16(ws) * lo_bf16(vu[d]), hi_bf16(ws) * hi_bf16(vu[d]));
        }
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          va[d] = pack_bf16x2(silu(lo_bf16(vg[d])) * lo_bf16(vu[d]), silu(hi_bf16(vg[d])) * hi_bf16(vu[d]));
      }
      const long po = (long)r * p.ldc + c8, ao = (long)r * p.ldc2 + c8;
      if (full) {
        __builtin_amdgcn_raw_buffer_store_b128(vu, rp, store_off(ok, po, 2), 0, kEpiNT);
        __builtin_amdgcn_raw_buffer_store_b128(vg, rp, store_off(ok, po + hoff, 2), 0, kEpiNT);
        __builtin_amdgcn_raw_buffer_store_b128(va, ra, store_off(ok, ao, 2), 0, kEpiNT);
      } else {
        const bool okh = ok && half;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{vu[0], vu[1]}, rp, store_off(okh, po, 2), 0, kEpiNT);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{vg[0], vg[1]}, rp, store_off(okh, po + hoff, 2), 0, kEpiNT);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{va[0], va[1]}, ra, store_off(okh, ao, 2), 0, kEpiNT);
      }
    }
  }
};

// SwiGLU backward on the dAct GEMM (EpiSwigluBwd numerics). With vector outputs the
// rounded dAct tile goes through this wave's LDS staging region so that the saved packed
// projection is read, and dPacked written, as 16-byte row-contiguous pieces (8 columns
// per lane, 16 lanes per 128-column row, 4 rows per instruction, 16 rows in flight).
struct FEpiSwigluBwd {
  // Two elements, the low and high BF16 halves of the dAct, up and gate words, to the
  // packed dUp and dGate words. Under eager rounding the pair's s and dsilu each go
  // through one packed conversion (the same round-to-nearest-even as one at a time).
  template <bool EAGER>
  __device__ __forceinline__ static void math2(unsigned wd, unsigned wu, unsigned wg,
                                               unsigned& du, unsigned& dg) {
    const float dy0 = lo_bf16(wd), dy1 = hi_bf16(wd);
    const float g0 = lo_bf16(wg), g1 = hi_bf16(wg);
    const float sg0 = sigmoid(g0), sg1 = sigmoid(g1);
    float s0 = g0 * sg0, s1 = g1 * sg1;
    float ds0 = dy0 * lo_bf16(wu), ds1 = dy1 * hi_bf16(wu);
    if (EAGER) {
      unsigned ws = pack_bf16x2(s0, s1), wds = pack_bf16x2(ds0, ds1);
      // Opaque to the compiler, which would otherwise convert each half on its own.
      asm volatile("" : "+v"(ws), "+v"(wds));
      s0 = lo_bf16(ws);
      s1 = hi_bf16(ws);
      ds0 = lo_bf16(wds);
      ds1 = hi_bf16(wds);
    }
    du = pack_bf16x2(dy0 * s0, dy1 * s1);
    dg = pack_bf16x2((ds0 * sg0) * (1.0f + g0 * (1.0f - sg0)),
                     (ds1 * sg1) * (1.0f + g1 * (1.0f - sg1)));
  }
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    opaque_lane(lane);
    const long hoff = p.H;
    {
      // Fragment order -> staging rows (64 x 128 BF16, 272-byte rows).
#pragma unroll
      for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          const int r = 16 * i + (lane & 15), c = 16 * j + 4 * (lane >> 4);
          u32x2_t v = {pack_bf16x2(acc.v[i][j][0], acc.v[i][j][1]),
                       pack_bf16x2(acc.v[i][j][2], acc.v[i][j][3])};
          *reinterpret_cast<u32x2_t*>(stage + r * kFStageRow + c * 2) = v;
        }
      // Keep the scheduler from hoisting the loads below above the staging writes (the
      // accumulators must be dead before the loaded rows take their registers).
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes landed
      const int c8 = 8 * (lane & 15);       // this lane's 8 columns
      const int n = n_base + c8;
      // Buffer bases at this wave's tile origin keep the byte offsets small.
      __amdgpu_buffer_rsrc_t rp = make_rsrc(p.aux + (long)m_base * p.ldaux + n_base, 0x7fffffff);
      __amdgpu_buffer_rsrc_t rd = make_rsrc(p.c + (long)m_base * p.ldc + n_base, 0x7fffffff);
      // All 16 rows' saved up/gate values are requested first (128 VGPRs; the
      // accumulators are dead once staged), so the four row groups below wait for one
      // memory latency instead of four.
      u32x4_t vu[4][4], vg[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int r = 16 * q + 4 * h + (lane >> 4);
          const int m = m_base + r;
          const bool ok = m < p.M && n + 7 < p.N;
          const long off = (long)r * p.ldaux + c8;
          vu[q][h] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rp, store_off(ok, off, 2), 0, kEpiNT));
          vg[q][h] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rp, store_off(ok, off + hoff, 2), 0, kEpiNT));
        }
      // The rounding mode is tested once here, not per element (the compiler otherwise
      // computes both and selects).
      auto finish = [&](auto eager) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const int r = 16 * q + 4 * h + (lane >> 4);
            const int m = m_base + r;
            const bool ok = m < p.M && n + 7 < p.N;
            const u32x4_t vd = *reinterpret_cast<const u32x4_t*>(stage + r * kFStageRow + c8 * 2);
            u32x4_t od, og;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              unsigned wu, wg;
              math2<decltype(eager)::value>(vd[d], vu[q][h][d], vg[q][h][d], wu, wg);
              od[d] = wu;
              og[d] = wg;
            }
            const long off = (long)r * p.ldc + c8;
            __builtin_amdgcn_raw_buffer_store_b128(od, rd, store_off(ok, off, 2), 0, kEpiNT);
            __builtin_amdgcn_raw_buffer_store_b128(og, rd, store_off(ok, off + hoff, 2), 0, kEpiNT);
          }
        }
      };
      if (p.eager) finish(std::true_type{});
      else finish(std::false_type{});
    }
  }
};

// FP32 accumulation (EpiAccF32 numerics); raw FP32 split-K partials when SPLIT. With
// kAccStore in round_acc the tile is stored instead (G = f32(r(A B)), G not read).
template <bool SPLIT>
struct FEpiAccF32 {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    add(p.g + (SPLIT ? (long)blockIdx.y * p.split_stride : 0), p.ldg, p.M, p.N, p.round_acc, acc,
        m_base, n_base, lane, tm, tn);
  }
  // The tile's accumulators into the [M, N] output g (row stride ldg).
  template <int FA, int FB>
  __device__ __forceinline__ static void add(float* g, long ldg, int M, int N, int round_acc,
                                             Acc16<FA, FB>& acc, int m_base, int n_base, int lane,
                                             int tm, int tn) {
    opaque_lane(lane);
    const int m0 = tm * kFBM, n0 = tn * kFBN;
    __amdgpu_buffer_rsrc_t rg = make_rsrc(g + (long)m0 * ldg + n0, 0x7fffffff);
#pragma unroll
    for (int i = 0; i < FA; ++i) {
      const int m = m_base + 16 * i + (lane & 15);
      const bool mok = m < M;
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int n = n_base + 16 * j + 4 * (lane >> 4);
        {
          const bool ok = mok && (n + 3 < N);
          const unsigned off = store_off(ok, (long)(m - m0) * ldg + (n - n0), 4);
          f32x4_t add;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = acc.v[i][j][e];
            add[e] = (!SPLIT && (round_acc & kAccRound)) ? rbf16(x) : x;
          }
          if (!SPLIT && !(round_acc & kAccStore)) {
            f32x4_t old = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0));
            add = old + add;
          }
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, add), rg, off, 0, 0);
        }
      }
    }
  }
};

// Raw FP32 partial sums of one stream-K piece into a 256 x 256 block (row-major, 256
// floats per row) at `block`; (r0, c0) is this wave's offset inside the tile.
struct FEpiPartial {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(Acc16<FA, FB>& acc, int r0, int c0, int lane,
                                             float* block) {
    opaque_lane(lane);
#pragma unroll
    for (int i = 0; i < FA; ++i) {
      const int r = r0 + 16 * i + (lane & 15);
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int c = c0 + 16 * j + 4 * (lane >> 4);
        *reinterpret_cast<f32x4_v*>(block + r * kFBN + c) = acc.v[i][j];
      }
    }
  }
};

// LM-head pass 1 (EpiCEStats numerics): per row, over this wave's 128 columns of BF16
// logits, the max and the sum of exp(l - max), one partial per (row, wave column block),
// and the target's logit. The four lanes l, l^16, l^32, l^48 share a row.
struct FEpiCEStats {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    opaque_lane(lane);
    const int part = tn * kFWN + wn;
    const int c0 = 4 * (lane >> 4);  // this lane's first column of each 16-column block
    const int ncols = p.N - n_base;  // columns of this wave inside the vocabulary
    // Columns past the vocabulary (only in a ragged last column tile: a wave-uniform test)
    // become -inf, so the max and the sum below need no per-element column test: such a
    // column adds exp(-inf) = 0. A wave with no column inside takes 0 as the sum's
    // reference point instead of its max of -inf, and writes max -inf and sum 0.
    if (ncols < FB * 16) {
#pragma unroll
      for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (16 * j + c0 + e >= ncols) acc.v[i][j][e] = -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < FA; ++i) {
      const int m = m_base + 16 * i + (lane & 15);
      const bool mok = m < p.M;
      // The row's target as a column of this wave's 128 (-1 if outside).
      const long trel = (mok ? p.targets[m] : -1) - n_base;
      const int t = trel >= 0 && trel < FB * 16 && trel < ncols ? (int)trel : -1;
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < FB; ++j)
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          // Two neighbouring logits rounded by one packed conversion (opaque to the
          // compiler, which would otherwise convert each on its own).
          unsigned w = pack_bf16x2(acc.v[i][j][e], acc.v[i][j][e + 1]);
          asm volatile("" : "+v"(w));
          acc.v[i][j][e] = lo_bf16(w);
          acc.v[i][j][e + 1] = hi_bf16(w);
          mx = fmaxf(fmaxf(mx, acc.v[i][j][e]), acc.v[i][j][e + 1]);
        }
      // The target logit: a 32-bit compare and select per element, only in the waves where
      // some row's target falls in these columns (1 in 16 for a 32768 vocabulary), and one
      // store per row.
      if (__builtin_amdgcn_ballot_w64(t >= 0) != 0) {
        float tv = 0.0f;
#pragma unroll
        for (int j = 0; j < FB; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) tv = 16 * j + c0 + e == t ? acc.v[i][j][e] : tv;
        if (t >= c0 && t < c0 + 16 * FB && ((t - c0) & 12) == 0) p.tgt_logit[m] = tv;
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float ref = ncols > 0 ? mx : 0.0f;
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < FB; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += exp_e(acc.v[i][j][e] - ref);
      sum += __shfl_xor(sum, 16, kWave);
      sum += __shfl_xor(sum, 32, kWave);
      if (mok && lane < 16) {
        p.part_max[(long)m * p.parts_per_row + part] = mx;
        p.part_sum[(long)m * p.parts_per_row + part] = sum;
      }
    }
  }
};

// LM-head pass 2 (EpiCEGrad numerics): r(scale * (softmax - onehot)), 0 for ignored rows.
// The rounded logits go through the wave's LDS staging rows; each lane then takes 8
// columns of one row (16 lanes per 256-byte row piece, 4 rows per instruction) and writes
// 16-byte pieces.
struct FEpiCEGrad {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    static_assert(FA * 16 == 64 && FB * 16 == 128, "staging holds a 64 x 128 wave tile");
    opaque_lane(lane);
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int r = 16 * i + (lane & 15), c = 16 * j + 4 * (lane >> 4);
        u32x2_t w = {pack_bf16x2(acc.v[i][j][0], acc.v[i][j][1]),
                     pack_bf16x2(acc.v[i][j][2], acc.v[i][j][3])};
        *reinterpret_cast<u32x2_t*>(stage + r * kFStageRow + c * 2) = w;
      }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes landed
    const int c8 = 8 * (lane & 15);
    const int n = n_base + c8;
    const bool full = n + 7 < p.N, half = n + 3 < p.N;  // N % 4 == 0 (vec_out)
    __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c + (long)m_base * p.ldc + n_base, 0x7fffffff);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = 4 * q + (lane >> 4);
      const int m = m_base + r;
      const bool ok = m < p.M;
      const long tgt = ok ? p.targets[m] : -100;
      const float lse = ok ? p.lse[m] : 0.0f;
      const float scale = (tgt == -100) ? 0.0f : *p.grad_scale;
      const u32x4_t vl = *reinterpret_cast<const u32x4_t*>(stage + r * kFStageRow + c8 * 2);
      u32x4_t o;
      // The one-hot term only where some lane of the wave holds its row's target among
      // its 8 columns (for 4 rows x 128 columns of a 32768 vocabulary, 1 in 64); elsewhere
      // the term is 0 and x - 0 = x.
      if (__builtin_amdgcn_ballot_w64(tgt >= n && tgt < n + 8) != 0) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const long e = n + 2 * d;
          const float v0 = scale * exp_e(lo_bf16(vl[d]) - lse) - (e == tgt ? scale : 0.0f);
          const float v1 = scale * exp_e(hi_bf16(vl[d]) - lse) - (e + 1 == tgt ? scale : 0.0f);
          o[d] = pack_bf16x2(v0, v1);
        }
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          o[d] = pack_bf16x2(scale * exp_e(lo_bf16(vl[d]) - lse), scale * exp_e(hi_bf16(vl[d]) - lse));
      }
      const long off = (long)r * p.ldc + c8;
      if (full) {
        __builtin_amdgcn_raw_buffer_store_b128(o, rc, store_off(ok, off, 2), 0, kEpiNT);
      } else {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{o[0], o[1]}, rc, store_off(ok && half, off, 2), 0, kEpiNT);
      }
    }
  }
};

// LM-head pass 1 that also keeps the logits: the statistics of FEpiCEStats, then the
// rounded BF16 logits through the wave's LDS staging rows into c [M, N] (row stride ldc,
// N % 4 == 0) as 16-byte row pieces, so that the backward reads them instead of
// recomputing the GEMM.
struct FEpiCEStatsLogits {
  template <int FA, int FB>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc16<FA, FB>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             unsigned char* stage) {
    static_assert(FA * 16 == 64 && FB * 16 == 128, "staging holds a 64 x 128 wave tile");
    FEpiCEStats::run(p, acc, m_base, n_base, lane, tm, tn, wn, stage);  // acc now rounded
    opaque_lane(lane);
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int r = 16 * i + (lane & 15), c = 16 * j + 4 * (lane >> 4);
        u32x2_t w = {pack_bf16x2(acc.v[i][j][0], acc.v[i][j][1]),
                     pack_bf16x2(acc.v[i][j][2], acc.v[i][j][3])};
        *reinterpret_cast<u32x2_t*>(stage + r * kFStageRow + c * 2) = w;
      }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes landed
    const int c8 = 8 * (lane & 15);
    const int n = n_base + c8;
    const bool full = n + 7 < p.N, half = n + 3 < p.N;
    __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c + (long)m_base * p.ldc + n_base, 0x7fffffff);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = 4 * q + (lane >> 4);
      const bool ok = m_base + r < p.M;
      const u32x4_t vl = *reinterpret_cast<const u32x4_t*>(stage + r * kFStageRow + c8 * 2);
      const long off = (long)r * p.ldc + c8;
      if (full) {
        __builtin_amdgcn_raw_buffer_store_b128(vl, rc, store_off(ok, off, 2), 0, kEpiNT);
      } else {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{vl[0], vl[1]}, rc, store_off(ok && half, off, 2), 0, kEpiNT);
      }
    }
  }
};

// --------------------------------------------------------------------------------------
// The kernel.

template <int AMODE, int BMODE, bool PAIRED, class Epi>
__global__ void __launch_bounds__(kFNT) gemm_fast_kernel(const GemmParams p) {
  static_assert(AMODE != kGeneric && BMODE != kGeneric, "fast path needs vector operands");
  constexpr int TM = kFBM / kFWM, TN = kFBN / kFWN;  // 64 x 128
  constexpr int FA = TM / 16, FB = TN / 16;          // 4 x 8
  constexpr int RA = AMODE == kKContig ? 1 : 2, RB = BMODE == kKContig ? 1 : 2;
  constexpr int NR = FA * RA + FB * RB;              // DS read instructions per k32 step
  constexpr int NM = FA * FB;                        // MFMAs per k32 step
  // With an M/N-contiguous operand the next k-tile's loads are issued in the middle of
  // the k-tile, after the last fragment read: their LDS writes then fall in the
  // read-free second half instead of competing with the transposing reads (12-16 %
  // faster). With both operands K-contiguous, A keeps the full k-tile of lead time
  // (issuing it mid-tile costs 10 % there) and B, with a third stage, two k-tiles.
  constexpr bool kMidIssue = AMODE == kMNContig || BMODE == kMNContig;
  // Both operands M/N-contiguous (and not paired): the loop with assembly fragment reads.
  constexpr bool kBothMN = AMODE == kMNContig && BMODE == kMNContig && !PAIRED;

  extern __shared__ __attribute__((aligned(1024))) unsigned char fsmem[];
  if (p.skip_if != nullptr && *p.skip_if != 0) return;  // uniform: the whole grid exits

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / kFWN, wn = wave % kFWN;
  const int bn_cols = PAIRED ? kFBN / 2 : kFBN;
  const int k_tiles_total = cdiv(p.K, kFBK);
  const int kt_begin = blockIdx.y * p.k_tiles_per_split;
  const int kt_end = min(k_tiles_total, kt_begin + p.k_tiles_per_split);

  DmaTile<AMODE, false> la;
  DmaTile<BMODE, PAIRED> lb;

  // Tile rows of this wave's fragments (B rows for paired tiles: up blocks then gate).
  int b_rb[FB];
#pragma unroll
  for (int j = 0; j < FB; ++j) {
    if (PAIRED) b_rb[j] = (j < FB / 2) ? wn * (TN / 2) + 16 * j : 128 + wn * (TN / 2) + 16 * (j - FB / 2);
    else b_rb[j] = wn * TN + 16 * j;
  }

  // One output tile (raster index t of GEMM q) over k-tiles [kb, ke), then `epi(acc,
  // m_base, n_base, tm, tn)` and a barrier (the next tile's loads reuse the epilogue's
  // staging space).
  auto run_tile = [&](const GemmMember& q, int t, int kb, int ke, auto&& epi) {
    int tm, tn;
    tile_position(t, q.tiles_m, q.tiles_n, tm, tn);
    const int row0_a = tm * kFBM;
    const int row0_b = tn * bn_cols;
    la.init(q.a, row0_a, q.M, 0, wave, lane);
    lb.init(q.b, row0_b, PAIRED ? p.H : q.N, PAIRED ? p.H : 0, wave, lane);

    Acc16<FA, FB> acc;
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) acc.v[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};

    if (kb < ke && !kMidIssue) {
      unsigned char* const sA = fsmem;                    // A stage c at sA + c * 32 KiB
      unsigned char* const sB = fsmem + 2 * kFTileBytes;  // B stage c at sB + c * 32 KiB
      la.issue(q.a, row0_a, kb * kFBK, p.K, sA, wave, lane);
      lb.issue(q.b, row0_b, kb * kFBK, p.K, sB, wave, lane);
      // B of the second k-tile, or zero-filling loads of the same count, so that every wait
      // below leaves exactly the last kFIns loads (B two tiles ahead) in flight.
#pragma unroll
      for (int i = 0; i < kFIns; ++i)
        lb.issue_one(q.b, row0_b, (kb + 1) * kFBK, p.K, sB + kFTileBytes, wave, lane, i, kb + 1 < ke);
      int bst = 0;  // B stage of k-tile kt: (kt - kb) % 3
      for (int kt = kb; kt < ke; ++kt) {
        // A(kt) and B(kt) have landed; B(kt + 1), issued after A(kt), may be in flight.
        __builtin_amdgcn_s_waitcnt(wait_vmcnt(kFIns));
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < ke)
          la.issue(q.a, row0_a, (kt + 1) * kFBK, p.K, sA + ((kt - kb + 1) & 1) * kFTileBytes, wave, lane);
        const unsigned char* sa = sA + ((kt - kb) & 1) * kFTileBytes;
        const unsigned char* sb = sB + bst * kFTileBytes;
        // B(kt + 2) goes to the stage B(kt - 1) used, which every wave has read (barrier).
        unsigned char* const nb = sB + (bst == 0 ? 2 : bst - 1) * kFTileBytes;
        bf16x8_t af[2][FA], bfr[2][FB];
#pragma unroll
        for (int i = 0; i < FA; ++i) af[0][i] = read_frag<AMODE>(sa, wm * TM + 16 * i, 0, lane);
#pragma unroll
        for (int j = 0; j < FB; ++j) bfr[0][j] = read_frag<BMODE>(sb, b_rb[j], 0, lane);
#pragma unroll
        for (int i = 0; i < FA; ++i) af[1][i] = read_frag<AMODE>(sa, wm * TM + 16 * i, 1, lane);
#pragma unroll
        for (int j = 0; j < FB; ++j) bfr[1][j] = read_frag<BMODE>(sb, b_rb[j], 1, lane);
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
          for (int j = 0; j < FB; ++j)
            acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[0][j], af[0][i], acc.v[i][j], 0, 0, 0);
        // Step-0 reads first, then step 1's reads spread over step 0's MFMAs.
        __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, NM / NR > 0 ? NM / NR : 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NM - (NM / NR > 0 ? NM / NR : 1) * NR, 0);
        __builtin_amdgcn_sched_barrier(0);
        // B two tiles ahead, between the steps: it lands while step 1 reads nothing.
#pragma unroll
        for (int i = 0; i < kFIns; ++i)
          lb.issue_one(q.b, row0_b, (kt + 2) * kFBK, p.K, nb, wave, lane, i, kt + 2 < ke);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
          for (int j = 0; j < FB; ++j)
            acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[1][j], af[1][i], acc.v[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
        bst = bst == 2 ? 0 : bst + 1;
      }
      // The zero-filling loads of the last two k-tiles land, and every wave is done reading,
      // before the epilogue's staging writes and the next tile's first loads.
      __builtin_amdgcn_s_waitcnt(wait_vmcnt(0));
      __builtin_amdgcn_s_barrier();
    } else if (kb < ke && kBothMN) {
      static_assert(FA + FB == 12, "tie_wait binds 12 fragments");
      const unsigned lds0 =
          (unsigned)(unsigned long)(__attribute__((address_space(3))) unsigned char*)fsmem;
      unsigned abase[FA], bbase[FB];
#pragma unroll
      for (int i = 0; i < FA; ++i) abase[i] = lds0 + tr_base(wm * TM + 16 * i, lane);
#pragma unroll
      for (int j = 0; j < FB; ++j) bbase[j] = lds0 + kFTileBytes + tr_base(b_rb[j], lane);
      la.issue(q.a, row0_a, kb * kFBK, p.K, fsmem, wave, lane);
      lb.issue(q.b, row0_b, kb * kFBK, p.K, fsmem + kFTileBytes, wave, lane);
      for (int kt = kb; kt < ke; ++kt) {
        const int cur = (kt - kb) & 1;
        __builtin_amdgcn_s_waitcnt(wait_vmcnt(0));
        __builtin_amdgcn_s_barrier();
        // The next tile's loads first: a full k-tile of lead.
        if (kt + 1 < ke) {
          unsigned char* nxt = fsmem + (cur ^ 1) * kFStageBytes;
          la.issue(q.a, row0_a, (kt + 1) * kFBK, p.K, nxt, wave, lane);
          lb.issue(q.b, row0_b, (kt + 1) * kFBK, p.K, nxt + kFTileBytes, wave, lane);
        }
        const unsigned st = (unsigned)(cur * kFStageBytes);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8_t f0[FA + FB], f1[FA + FB];  // steps 0 and 1: A blocks, then B blocks
#pragma unroll
        for (int i = 0; i < FA; ++i) f0[i] = tr_frag<0>(abase[i] + st);
#pragma unroll
        for (int j = 0; j < FB; ++j) f0[FA + j] = tr_frag<0>(bbase[j] + st);
        tie_wait(f0);
        __builtin_amdgcn_sched_barrier(0);
        // Step 0's MFMAs, step 1's fragment r read after MFMA ceil(r NM / 12).
#pragma unroll
        for (int n = 0; n < NM; ++n) {
          const int i = n / FB, j = n % FB;
          acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f0[FA + j], f0[i], acc.v[i][j], 0, 0, 0);
          if ((n * (FA + FB)) % NM < FA + FB) {
            const int r = n * (FA + FB) / NM;
            f1[r] = r < FA ? tr_frag<1>(abase[r] + st) : tr_frag<1>(bbase[r - FA] + st);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        tie_wait(f1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
          for (int j = 0; j < FB; ++j)
            acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f1[FA + j], f1[i], acc.v[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      // All waves are done reading both stages before the next tile's first load.
      __builtin_amdgcn_s_barrier();
    } else if (kb < ke) {
      la.issue(q.a, row0_a, kb * kFBK, p.K, fsmem, wave, lane);
      lb.issue(q.b, row0_b, kb * kFBK, p.K, fsmem + kFTileBytes, wave, lane);
      for (int kt = kb; kt < ke; ++kt) {
        const int cur = (kt - kb) & 1;
        __builtin_amdgcn_s_waitcnt(wait_vmcnt(0));
        __builtin_amdgcn_s_barrier();
        const unsigned char* sa = fsmem + cur * kFStageBytes;
        const unsigned char* sb = sa + kFTileBytes;
        bf16x8_t af[2][FA], bfr[2][FB];
#pragma unroll
        for (int i = 0; i < FA; ++i) af[0][i] = read_frag<AMODE>(sa, wm * TM + 16 * i, 0, lane);
#pragma unroll
        for (int j = 0; j < FB; ++j) bfr[0][j] = read_frag<BMODE>(sb, b_rb[j], 0, lane);
#pragma unroll
        for (int s = 0; s < kFBK / 32; ++s) {
          if (s == 1) {
            // Step-0 reads first, then step 1's reads spread over step 0's MFMAs; then the
            // next k-tile's loads, after this wave's last fragment read of the tile.
            __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
            for (int r = 0; r < NR; ++r) {
              __builtin_amdgcn_sched_group_barrier(0x008, NM / NR > 0 ? NM / NR : 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - (NM / NR > 0 ? NM / NR : 1) * NR, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (kt + 1 < ke) {
              unsigned char* nxt = fsmem + (cur ^ 1) * kFStageBytes;
              la.issue(q.a, row0_a, (kt + 1) * kFBK, p.K, nxt, wave, lane);
              lb.issue(q.b, row0_b, (kt + 1) * kFBK, p.K, nxt + kFTileBytes, wave, lane);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          if (s + 1 < kFBK / 32) {
#pragma unroll
            for (int i = 0; i < FA; ++i) af[(s + 1) & 1][i] = read_frag<AMODE>(sa, wm * TM + 16 * i, s + 1, lane);
#pragma unroll
            for (int j = 0; j < FB; ++j) bfr[(s + 1) & 1][j] = read_frag<BMODE>(sb, b_rb[j], s + 1, lane);
          }
#pragma unroll
          for (int i = 0; i < FA; ++i)
#pragma unroll
            for (int j = 0; j < FB; ++j)
              acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[s & 1][j], af[s & 1][i],
                                                                     acc.v[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
      }
      // All waves are done reading both stages before the next tile's first load.
      __builtin_amdgcn_s_barrier();
    }
    const int m_base = row0_a + wm * TM;
    const int n_base = row0_b + (PAIRED ? wn * (TN / 2) : wn * TN);
    epi(acc, m_base, n_base, tm, tn);
    __builtin_amdgcn_s_barrier();
  };
  const GemmMember self{p.a, p.b, p.M, p.N, p.tiles_m, p.tiles_n, 0, p.g, p.ldg};
  if constexpr (std::is_same<Epi, FEpiAccF32<false>>::value) {
    // Balanced accumulation (the other instantiations use the plain tile loop below).
    if (p.balanced) {
      // The GEMM that launch raster index t belongs to (uniform selects over the member
      // table of a grouped launch).
      auto member = [&](int t) {
        if (p.group_count == 0) return self;
        GemmMember q = p.grp[0];
#pragma unroll
        for (int i = 1; i < kMaxGroup; ++i)
          if (i < p.group_count && t >= p.grp[i].tile_base) q = p.grp[i];
        return q;
      };
      // Whole tiles, accumulated straight into G.
      for (int w = blockIdx.x; w < p.dp_tiles; w += gridDim.x) {
        const int t = xcd_remap(w, p.dp_tiles, gridDim.x);
        const GemmMember q = member(t);
        run_tile(q, t - q.tile_base, 0, p.k_tiles,
                 [&](auto& acc, int m_base, int n_base, int tm, int tn) {
                   // Selected again here, so that only t stays live across the k-loop.
                   const GemmMember o = member(t);
                   Epi::add(o.g, o.ldg, o.M, o.N, p.round_acc, acc, m_base, n_base, lane, tm, tn);
                 });
      }
      // This workgroup's stream-K share of the remaining tiles' k-tiles. Worker indices
      // run XCD-contiguous (the dispatcher deals workgroups round-robin to the XCDs) so
      // that the pieces running together on one XCD belong to neighbouring tiles. With
      // fewer units than workgroups only the first sk_units workers take a share, so that
      // no share is empty and a tile's pieces are numbered without gaps.
      const long G = gridDim.x, b = blockIdx.x;
      const long v = G % kXcds == 0 ? (b % kXcds) * (G / kXcds) + b / kXcds : b;
      const long W = min(G, p.sk_units);
      long x = v < W ? sk_begin(v, p.sk_units, W) : 0;
      const long end = v < W ? sk_begin(v + 1, p.sk_units, W) : 0;
      while (x < end) {
        const long ti = x / p.k_tiles;
        const int kb = (int)(x - ti * p.k_tiles);
        const int ke = (int)min((long)p.k_tiles, kb + (end - x));
        const long piece = v - sk_worker(ti * p.k_tiles, p.sk_units, W);
        float* block = p.sk_ws + (ti * p.sk_pieces + piece) * (long)(kFBM * kFBN);
        const GemmMember q = member(p.dp_tiles + (int)ti);
        run_tile(q, p.dp_tiles + (int)ti - q.tile_base, kb, ke,
                 [&](auto& acc, int m_base, int n_base, int tm, int tn) {
                   FEpiPartial::run(acc, m_base - tm * kFBM, n_base - tn * kFBN, lane, block);
                 });
        x += ke - kb;
      }
      return;
    }
  }
  for (int w = blockIdx.x; w < p.total_tiles; w += gridDim.x)
    run_tile(self, xcd_remap(w, p.total_tiles, gridDim.x), kt_begin, kt_end,
             [&](auto& acc, int m_base, int n_base, int tm, int tn) {
               Epi::run(p, acc, m_base, n_base, lane, tm, tn, wn, fsmem + wave * kFStageWave);
             });
}

}  // namespace ws
