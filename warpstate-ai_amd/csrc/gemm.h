// BF16 GEMM for gfx950 with fused prologues and epilogues.
//
// C[m, n] = sum_k A[m, k] * B[k, n], BF16 operands, FP32 accumulation in MFMA
// (v_mfma_f32_32x32x16_bf16), epilogue applied in registers before one HBM write.
// Replaces the Triton kernels `_matmul_kernel` (ops/matmul_kernels.py:81-108),
// `_persistent_tma_kernel` (ops/matmul_kernels.py:111-132) and
// `_paired_swiglu_mm_kernel` (ops/matmul_epilogue.py:30-83), and adds the fused
// epilogues of the pieces the reference composes from separate ops (gate sigmoid,
// residual add, SwiGLU backward, FP32 gradient accumulation, cross-entropy).
//
// Layout of one workgroup (BM x BN macro-tile, BK = 64):
//  * LDS holds two stages of the A tile [BM rows][64 k] and the B tile [BN rows][64 k]
//    (B is stored n-major, i.e. as B^T), k contiguous. Each 128-byte row is split into
//    eight 16-byte chunks; chunk c of row r lives at chunk slot c ^ swz(r) with
//    swz(r) = (r >> 1) ^ ((r & 1) << 2) (mod 8). The LDS serves a 16-byte read for 16
//    lanes per clock across its 64 banks; a fragment read has those 16 lanes on 16
//    consecutive rows of one chunk, and swz makes (r & 1, slot) distinct over any 16
//    consecutive rows (and the slot alone distinct over any 8), so fragment reads and
//    tile writes are bank-conflict free.
//  * Operands whose reduction dim is contiguous (row-major X, or W^T of an nn.Linear
//    weight) are copied with 16-byte buffer loads straight into that layout. Operands
//    whose reduction dim is strided (dY^T and X in weight gradients, W in input
//    gradients) are read as 16-byte rows of 8 consecutive m/n, transposed 4x8 in
//    registers with v_perm_b32, and written as 8-byte k-runs. Any other stride pattern
//    uses element loads.
//  * Each wave owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks. The MFMA
//    "A" operand is the B fragment and the MFMA "B" operand is the A fragment, so the
//    accumulator of a lane holds one output row m and runs of four consecutive n, which
//    the epilogues write as 8-byte (BF16) or 16-byte (FP32) vectors.
//  * Out-of-range rows, columns and k are handled by the buffer unit: such loads use an
//    offset past num_records and return zero; such stores are dropped.
//  * Tiles are visited in the grouped order of `_tile_position`
//    (ops/matmul_kernels.py:72-78, GROUP_M = 8), after a remap that gives each of the 8
//    XCDs (each with its own L2) a contiguous run of tiles.
#pragma once

#include "common.h"

namespace ws {

constexpr int kBK = 64;
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

enum LoadMode { kKContig = 0, kMNContig = 1, kGeneric = 2 };

struct OperandDesc {
  const unsigned short* ptr;  // element (row r, k) at ptr + r * s_row + k * s_k
  long s_row;                 // stride between rows (m for A, n for B), elements
  long s_k;                   // stride along the reduction dim, elements
};

// One GEMM of a grouped FP32 accumulation: G[M, N] += A[M, K] B[K, N], its tiles at
// raster indices [tile_base, tile_base + tiles_m * tiles_n) of the launch.
struct GemmMember {
  OperandDesc a, b;
  int M, N, tiles_m, tiles_n, tile_base;
  float* g; long ldg;
};
constexpr int kMaxGroup = 4;

struct GemmParams {
  OperandDesc a, b;
  int M, N, K;       // logical sizes; for the paired SwiGLU GEMM N is the packed width 2H
  int H;             // half width: paired SwiGLU forward / SwiGLU backward
  int tiles_m, tiles_n, total_tiles;
  int k_tiles_per_split;  // split-K: k-tiles per blockIdx.y slice
  int vec_out;            // 1 if 4-element vector stores are legal for the output columns
  // epilogue operands
  unsigned short* c;  long ldc;
  unsigned short* c2; long ldc2;
  const unsigned short* aux; long ldaux;
  float* g; long ldg; long split_stride;
  int gate_lo, gate_hi;
  int eager;
  int round_acc;  // AccMode bits (common.h)
  const long* targets;
  const float* lse;
  float* part_max; float* part_sum; float* tgt_logit; int parts_per_row;
  const float* grad_scale;  // device scalar: d(mean) / max(1, count)
  int row_offset;
  // Device flag (nullable): when set, every workgroup exits at once. Lets a path whose need
  // is decided on the device (the LM head's exact-scaling check) be launched unconditionally.
  const int* skip_if;
  // Balanced FP32 accumulation (fast kernel): tiles [0, dp_tiles) of the raster run whole
  // and accumulate into g; the k-tiles of the other sk_tiles tiles (sk_units = sk_tiles x
  // k_tiles in all) are shared evenly by the gridDim.x workgroups, each piece writing a
  // 256 x 256 FP32 block (tile, piece) of sk_ws with at most sk_pieces pieces per tile.
  int balanced;
  int dp_tiles, sk_tiles, k_tiles, sk_pieces;
  long sk_units;
  float* sk_ws;
  // Grouped balanced accumulation: group_count > 0 GEMMs sharing K, the operand layouts
  // and round_acc, their rasters concatenated in member order (a, b, M, N, g, ldg and the
  // tile counts above are then unused).
  int group_count;
  GemmMember grp[kMaxGroup];
};

// --------------------------------------------------------------------------------------
// Tile scheduling

// Spread a dispatch-order index so that the workgroups that run on one XCD at the same
// time (the hardware deals workgroups round-robin to the 8 XCDs) get consecutive tiles.
__device__ __forceinline__ int xcd_remap(int w, int total, int window) {
  int base = (w / window) * window;
  int size = min(window, total - base);
  if (size % kXcds != 0) return w;
  int within = w - base;
  return base + (within % kXcds) * (size / kXcds) + within / kXcds;
}

// Stream-K shares: worker v of W owns units [sk_begin(v), sk_begin(v + 1)) of U.
__host__ __device__ inline long sk_begin(long v, long U, long W) { return v * U / W; }
// The worker whose share holds unit x (the largest v with sk_begin(v) <= x).
__host__ __device__ inline long sk_worker(long x, long U, long W) { return ((x + 1) * W - 1) / U; }
// Number of workers sharing stream-K tile ti (KT units per tile).
__host__ __device__ inline int sk_pieces_of(long ti, long KT, long U, long W) {
  return (int)(sk_worker((ti + 1) * KT - 1, U, W) - sk_worker(ti * KT, U, W) + 1);
}

// Grouped raster order of ops/matmul_kernels.py:72-78.
__device__ __forceinline__ void tile_position(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  int group = kGroupM * tiles_n;
  int first_m = (t / group) * kGroupM;
  int actual = min(tiles_m - first_m, kGroupM);
  int within = t % group;
  tm = first_m + within % actual;
  tn = within / actual;
}

// Chunk-slot swizzle of LDS tile row r (see the header comment).
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

// --------------------------------------------------------------------------------------
// Global -> LDS tile loaders. `R` tile rows, `NT` threads. `rows_valid` bounds the rows;
// with `PAIRED`, tile rows [0, R/2) map to rows row0 + r and rows [R/2, R) map to
// rows half + row0 + (r - R/2), both bounded by rows_valid (the SwiGLU up/gate panels).

template <int R, int NT, int MODE, bool PAIRED>
struct TileLoader;

// Reduction dim contiguous: 16-byte chunk loads, stored directly.
template <int R, int NT, bool PAIRED>
struct TileLoader<R, NT, kKContig, PAIRED> {
  static constexpr int kPer = R * 8 / NT;
  static_assert(kPer >= 1 && R * 8 % NT == 0, "tile/thread mismatch");
  unsigned row_off[kPer];
  int c;
  u32x4_t regs[kPer];

  __device__ __forceinline__ int row_of(int r, int row0, int half) const {
    if (PAIRED) return r < R / 2 ? row0 + r : half + row0 + (r - R / 2);
    return row0 + r;
  }
  __device__ __forceinline__ void init(const OperandDesc& d, int row0, int rows_valid, int half,
                                       int tid) {
    c = tid & 7;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int r = (tid >> 3) + i * (NT / 8);
      int lr = PAIRED ? (r < R / 2 ? row0 + r : row0 + r - R / 2) : row0 + r;
      bool ok = lr < rows_valid;
      long rel = (long)(row_of(r, row0, half) - row0) * d.s_row * 2;
      row_off[i] = ok ? (unsigned)rel : kOOB;
    }
  }
  __device__ __forceinline__ void load(const OperandDesc& d, int row0, int k0, int K) {
    const unsigned short* base = d.ptr + (long)row0 * d.s_row + k0;
    __amdgpu_buffer_rsrc_t rs = make_rsrc(base, 0x7fffffff);
    bool kok = k0 + 8 * c < K;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      unsigned off = (kok && row_off[i] != kOOB) ? row_off[i] + 16u * c : kOOB;
      regs[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
  }
  __device__ __forceinline__ void store(unsigned short* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int r = (tid >> 3) + i * (NT / 8);
      *reinterpret_cast<u32x4_t*>(lds + r * kBK + ((c ^ swz(r)) << 3)) = regs[i];
    }
  }
};

// 8 rows x 4 k -> 8 k-runs of 4 values, as pairs of dwords.
__device__ __forceinline__ void transpose4x8(const u32x4_t (&v)[4], u32x2_t (&w)[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // v[j][p] holds rows (2p, 2p+1) of k-row j.
    unsigned a0 = v[0][p], a1 = v[1][p], a2 = v[2][p], a3 = v[3][p];
    w[2 * p][0] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
    w[2 * p][1] = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
    w[2 * p + 1][0] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
    w[2 * p + 1][1] = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
  }
}

// Writes 8 rows (8rc .. 8rc+7) x 4 k (4kq .. 4kq+3) into the swizzled tile.
__device__ __forceinline__ void store_units(unsigned short* lds, int rc, int kq,
                                            const u32x2_t (&w)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    int r = 8 * rc + e;
    *reinterpret_cast<u32x2_t*>(lds + r * kBK + ((((kq >> 1) ^ swz(r))) << 3) + ((kq & 1) << 2)) = w[e];
  }
}

// Rows contiguous (reduction dim strided): 16-byte loads of 8 rows for 4 k, transposed.
template <int R, int NT, bool PAIRED>
struct TileLoader<R, NT, kMNContig, PAIRED> {
  static constexpr int kPer = 2 * R / NT;
  static_assert(kPer >= 1 && 2 * R % NT == 0, "tile/thread mismatch");
  unsigned row_off[kPer];
  int kq, rc0;
  u32x4_t regs[kPer][4];

  __device__ __forceinline__ void init(const OperandDesc& d, int row0, int rows_valid, int half,
                                       int tid) {
    kq = tid & 15;
    rc0 = tid >> 4;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int r = 8 * (rc0 + i * (NT / 16));
      int lr = PAIRED ? (r < R / 2 ? row0 + r : row0 + r - R / 2) : row0 + r;
      int phys = PAIRED ? (r < R / 2 ? row0 + r : half + row0 + r - R / 2) : row0 + r;
      row_off[i] = lr < rows_valid ? (unsigned)((phys - row0) * 2) : kOOB;
    }
  }
  __device__ __forceinline__ void load(const OperandDesc& d, int row0, int k0, int K) {
    const unsigned short* base = d.ptr + (long)row0 + (long)k0 * d.s_k;
    __amdgpu_buffer_rsrc_t rs = make_rsrc(base, 0x7fffffff);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int kk = 4 * kq + j;
      bool kok = k0 + kk < K;
      unsigned koff = (unsigned)(kk * d.s_k * 2);
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        unsigned off = (kok && row_off[i] != kOOB) ? row_off[i] + koff : kOOB;
        regs[i][j] = __builtin_bit_cast(u32x4_t,
                                        __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      }
    }
  }
  __device__ __forceinline__ void store(unsigned short* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      u32x2_t w[8];
      transpose4x8(regs[i], w);
      store_units(lds, rc0 + i * (NT / 16), kq, w);
    }
  }
};

// Any positive strides: element loads, same unit shape and LDS writes as kMNContig.
template <int R, int NT, bool PAIRED>
struct TileLoader<R, NT, kGeneric, PAIRED> {
  static constexpr int kPer = 2 * R / NT;
  int kq, rc0;
  int lrow[kPer];  // logical first row of each 8-row unit (bounded by rows_valid)
  int prow[kPer];  // physical first row (the gate half of a paired panel is `half` further)
  int lvalid;
  u32x4_t regs[kPer][4];

  __device__ __forceinline__ void init(const OperandDesc& d, int row0, int rows_valid, int half,
                                       int tid) {
    kq = tid & 15;
    rc0 = tid >> 4;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int r = 8 * (rc0 + i * (NT / 16));
      bool upper = PAIRED && r >= R / 2;
      lrow[i] = upper ? row0 + r - R / 2 : row0 + r;
      prow[i] = upper ? half + row0 + r - R / 2 : row0 + r;
    }
    lvalid = rows_valid;
  }
  __device__ __forceinline__ void load(const OperandDesc& d, int row0, int k0, int K) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + 4 * kq + j;
        unsigned e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const bool ok = (k < K) && (lrow[i] + q < lvalid);
          e[q] = ok ? d.ptr[(long)(prow[i] + q) * d.s_row + (long)k * d.s_k] : 0u;
        }
        u32x4_t v;
        v[0] = e[0] | (e[1] << 16);
        v[1] = e[2] | (e[3] << 16);
        v[2] = e[4] | (e[5] << 16);
        v[3] = e[6] | (e[7] << 16);
        regs[i][j] = v;
      }
    }
  }
  __device__ __forceinline__ void store(unsigned short* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      u32x2_t w[8];
      transpose4x8(regs[i], w);
      store_units(lds, rc0 + i * (NT / 16), kq, w);
    }
  }
};

// --------------------------------------------------------------------------------------
// Epilogues. Each receives the accumulators of one wave and the coordinates of its
// sub-tile. Lane l holds, for block (i, j) and register 4g+e, the output element
//   m = m_base + 32 i + (l & 31),   n = n_base + 32 j + 8 g + 4 (l >> 5) + e.

template <int FM, int FN>
struct Acc {
  f32x16_t v[FM][FN];
};

__device__ __forceinline__ unsigned store_off(bool ok, long elem, int bytes) {
  return ok ? (unsigned)(elem * bytes) : kOOB;
}

// Plain BF16 store (launch_mm), optional sigmoid over an output column range
// (in_proj gate slice, warpstate/model.py:174), optional residual add
// x + r(H @ W^T) in BF16 (warpstate/model.py:177-178, ops/residual_experiment.py:25-58).
template <bool SIGMOID, bool RESIDUAL>
struct EpiStore {
  template <int FM, int FN>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc<FM, FN>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             int bm_tile, int bn_tile) {
    int m0 = tm * bm_tile, n0 = tn * bn_tile;
    unsigned short* cbase = p.c + (long)m0 * p.ldc + n0;
    __amdgpu_buffer_rsrc_t rc = make_rsrc(cbase, 0x7fffffff);
    const unsigned short* rbase = RESIDUAL ? p.aux + (long)m0 * p.ldaux + n0 : nullptr;
    __amdgpu_buffer_rsrc_t rr = make_rsrc(RESIDUAL ? rbase : cbase, 0x7fffffff);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int m = m_base + 32 * i + (lane & 31);
      bool mok = m < p.M;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int n = n_base + 32 * j + 8 * g + 4 * (lane >> 5);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = acc.v[i][j][4 * g + e];
            if (SIGMOID) {
              x = rbf16(x);
              int col = n + e;
              if (col >= p.gate_lo && col < p.gate_hi) x = sigmoid(x);
            }
            v[e] = x;
          }
          if (p.vec_out) {
            bool ok = mok && (n + 3 < p.N);
            if (RESIDUAL) {
              u32x2_t rv = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                  rr, store_off(ok, (long)(m - m0) * p.ldaux + (n - n0), 2), 0, 0));
              v[0] = rbf16(v[0]) + lo_bf16(rv[0]);
              v[1] = rbf16(v[1]) + hi_bf16(rv[0]);
              v[2] = rbf16(v[2]) + lo_bf16(rv[1]);
              v[3] = rbf16(v[3]) + hi_bf16(rv[1]);
            }
            u32x2_t out = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            __builtin_amdgcn_raw_buffer_store_b64(
                __builtin_bit_cast(u32x2_t, out), rc,
                store_off(ok, (long)(m - m0) * p.ldc + (n - n0), 2), 0, 0);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              bool ok = mok && (n + e < p.N);
              float x = v[e];
              if (RESIDUAL && ok) x = rbf16(x) + bf16_bits_to_f32(rbase[(long)(m - m0) * p.ldaux + (n + e - n0)]);
              if (ok) cbase[(long)(m - m0) * p.ldc + (n + e - n0)] = to_bf16_bits(x);
            }
          }
        }
      }
    }
  }
};

// Paired SwiGLU forward (ops/matmul_epilogue.py:69-83): up = r(acc_up), gate = r(acc_gate),
// both stored into packed [M, 2H]; s = g / (1 + e^-g) on the rounded gate, r(s) when
// eager rounding is requested; act = r(s * up) stored into [M, H].
struct EpiSwiglu {
  template <int FM, int FN>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc<FM, FN>& acc, int m_base,
                                             int nh_base, int lane, int tm, int tn, int wn,
                                             int bm_tile, int bnh_tile) {
    constexpr int FH = FN / 2;
    int m0 = tm * bm_tile, n0 = tn * bnh_tile;
    unsigned short* pbase = p.c + (long)m0 * p.ldc + n0;
    unsigned short* abase = p.c2 + (long)m0 * p.ldc2 + n0;
    __amdgpu_buffer_rsrc_t rp = make_rsrc(pbase, 0x7fffffff);
    __amdgpu_buffer_rsrc_t ra = make_rsrc(abase, 0x7fffffff);
    const long hoff = p.H;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int m = m_base + 32 * i + (lane & 31);
      bool mok = m < p.M;
#pragma unroll
      for (int j = 0; j < FH; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int n = nh_base + 32 * j + 8 * g + 4 * (lane >> 5);
          float up[4], gate[4], act[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            up[e] = rbf16(acc.v[i][j][4 * g + e]);
            gate[e] = rbf16(acc.v[i][j + FH][4 * g + e]);
            float s = silu(gate[e]);
            if (p.eager) s = rbf16(s);
            act[e] = s * up[e];
          }
          if (p.vec_out) {
            bool ok = mok && (n + 3 < p.H);
            long rowp = (long)(m - m0) * p.ldc + (n - n0);
            u32x2_t vu = {pack_bf16x2(up[0], up[1]), pack_bf16x2(up[2], up[3])};
            u32x2_t vg = {pack_bf16x2(gate[0], gate[1]), pack_bf16x2(gate[2], gate[3])};
            u32x2_t va = {pack_bf16x2(act[0], act[1]), pack_bf16x2(act[2], act[3])};
            __builtin_amdgcn_raw_buffer_store_b64(vu, rp, store_off(ok, rowp, 2), 0, 0);
            __builtin_amdgcn_raw_buffer_store_b64(vg, rp, store_off(ok, rowp + hoff, 2), 0, 0);
            __builtin_amdgcn_raw_buffer_store_b64(
                va, ra, store_off(ok, (long)(m - m0) * p.ldc2 + (n - n0), 2), 0, 0);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (mok && n + e < p.H) {
                long rowp = (long)(m - m0) * p.ldc + (n + e - n0);
                pbase[rowp] = to_bf16_bits(up[e]);
                pbase[rowp + hoff] = to_bf16_bits(gate[e]);
                abase[(long)(m - m0) * p.ldc2 + (n + e - n0)] = to_bf16_bits(act[e]);
              }
            }
          }
        }
      }
    }
  }
};

// SwiGLU backward fused on the dAct GEMM (dY @ W_down): dact = r(acc); with up, gate from
// the saved packed projection, dUp = r(dact * s), dGate = r(r?(dact * up) * sig * (1 + g(1-sig)))
// (ops/activation_execution.py:36-55). Writes dPacked [M, 2H] (up half, then gate half).
struct EpiSwigluBwd {
  template <int FM, int FN>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc<FM, FN>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             int bm_tile, int bn_tile) {
    int m0 = tm * bm_tile, n0 = tn * bn_tile;
    unsigned short* dbase = p.c + (long)m0 * p.ldc + n0;
    const unsigned short* pbase = p.aux + (long)m0 * p.ldaux + n0;
    __amdgpu_buffer_rsrc_t rd = make_rsrc(dbase, 0x7fffffff);
    __amdgpu_buffer_rsrc_t rp = make_rsrc(pbase, 0x7fffffff);
    const long hoff = p.H;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int m = m_base + 32 * i + (lane & 31);
      bool mok = m < p.M;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int n = n_base + 32 * j + 8 * g + 4 * (lane >> 5);
          float up[4], gate[4];
          bool ok4 = mok && (n + 3 < p.N);
          if (p.vec_out) {
            long rowp = (long)(m - m0) * p.ldaux + (n - n0);
            u32x2_t vu = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                rp, store_off(ok4, rowp, 2), 0, 0));
            u32x2_t vg = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                rp, store_off(ok4, rowp + hoff, 2), 0, 0));
            up[0] = lo_bf16(vu[0]); up[1] = hi_bf16(vu[0]); up[2] = lo_bf16(vu[1]); up[3] = hi_bf16(vu[1]);
            gate[0] = lo_bf16(vg[0]); gate[1] = hi_bf16(vg[0]); gate[2] = lo_bf16(vg[1]); gate[3] = hi_bf16(vg[1]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              bool ok = mok && (n + e < p.N);
              long rowp = (long)(m - m0) * p.ldaux + (n + e - n0);
              up[e] = ok ? bf16_bits_to_f32(pbase[rowp]) : 0.0f;
              gate[e] = ok ? bf16_bits_to_f32(pbase[rowp + hoff]) : 0.0f;
            }
          }
          float du[4], dg[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float dy = rbf16(acc.v[i][j][4 * g + e]);
            float sg = sigmoid(gate[e]);
            float s = silu(gate[e]);
            if (p.eager) s = rbf16(s);
            float dsilu = dy * up[e];
            if (p.eager) dsilu = rbf16(dsilu);
            du[e] = dy * s;
            dg[e] = (dsilu * sg) * (1.0f + gate[e] * (1.0f - sg));
          }
          if (p.vec_out) {
            long rowd = (long)(m - m0) * p.ldc + (n - n0);
            u32x2_t vu = {pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3])};
            u32x2_t vg = {pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3])};
            __builtin_amdgcn_raw_buffer_store_b64(vu, rd, store_off(ok4, rowd, 2), 0, 0);
            __builtin_amdgcn_raw_buffer_store_b64(vg, rd, store_off(ok4, rowd + hoff, 2), 0, 0);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (mok && n + e < p.N) {
                long rowd = (long)(m - m0) * p.ldc + (n + e - n0);
                dbase[rowd] = to_bf16_bits(du[e]);
                dbase[rowd + hoff] = to_bf16_bits(dg[e]);
              }
            }
          }
        }
      }
    }
  }
};

// FP32 accumulation G[m, n] += f32(r(acc)) (test_gradient_execution.py:243-246), or
// G += acc without the BF16 rounding when round_acc == 0. With split-K (gridDim.y > 1)
// the raw FP32 partial of slice z is stored to g + z * split_stride instead.
template <bool SPLIT>
struct EpiAccF32 {
  template <int FM, int FN>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc<FM, FN>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             int bm_tile, int bn_tile) {
    int m0 = tm * bm_tile, n0 = tn * bn_tile;
    float* gbase = p.g + (SPLIT ? (long)blockIdx.y * p.split_stride : 0) + (long)m0 * p.ldg + n0;
    __amdgpu_buffer_rsrc_t rg = make_rsrc(gbase, 0x7fffffff);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int m = m_base + 32 * i + (lane & 31);
      bool mok = m < p.M;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int n = n_base + 32 * j + 8 * g + 4 * (lane >> 5);
          if (p.vec_out) {
            bool ok = mok && (n + 3 < p.N);
            unsigned off = store_off(ok, (long)(m - m0) * p.ldg + (n - n0), 4);
            f32x4_t add;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float x = acc.v[i][j][4 * g + e];
              add[e] = (!SPLIT && (p.round_acc & kAccRound)) ? rbf16(x) : x;
            }
            if (!SPLIT && !(p.round_acc & kAccStore)) {
              f32x4_t old = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0));
              add = old + add;
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, add), rg, off, 0, 0);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (mok && n + e < p.N) {
                float x = acc.v[i][j][4 * g + e];
                float* dst = gbase + (long)(m - m0) * p.ldg + (n + e - n0);
                if (SPLIT) *dst = x;
                else {
                  const float v = (p.round_acc & kAccRound) ? rbf16(x) : x;
                  *dst = (p.round_acc & kAccStore) ? v : *dst + v;
                }
              }
            }
          }
        }
      }
    }
  }
};

// LM-head pass 1: per row, over this wave's columns of the logits tile l = f32(r(acc))
// (the BF16 logits of F.linear, warpstate/model.py:321-322), the running max and
// sum exp(l - max), stored as one partial per (row, wave column block); the logit of the
// target column, stored by the lane that holds it. Logits never leave registers.
struct EpiCEStats {
  template <int FM, int FN>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc<FM, FN>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             int bm_tile, int bn_tile) {
    int part = tn * (p.parts_per_row / p.tiles_n) + wn;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int m = m_base + 32 * i + (lane & 31);
      bool mok = m < p.M;
      long tgt = mok ? p.targets[m] : -1;
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          int n = n_base + 32 * j + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          float x = rbf16(acc.v[i][j][r]);
          acc.v[i][j][r] = x;
          if (n < p.N) mx = fmaxf(mx, x);
          if ((long)n == tgt && n < p.N) p.tgt_logit[m] = x;
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          int n = n_base + 32 * j + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (n < p.N) sum += exp_e(acc.v[i][j][r] - mx);
        }
      sum += __shfl_xor(sum, 32, kWave);
      if (mok && lane < 32) {
        p.part_max[(long)m * p.parts_per_row + part] = mx;
        p.part_sum[(long)m * p.parts_per_row + part] = sum;
      }
    }
  }
};

// LM-head pass 2: gradient of the summed cross-entropy times 1/count with respect to the
// BF16 logits, r(scale * (softmax - onehot)) for rows whose target is not -100, zero
// otherwise; stored as BF16 for the dHidden GEMM of this row chunk.
struct EpiCEGrad {
  template <int FM, int FN>
  __device__ __forceinline__ static void run(const GemmParams& p, Acc<FM, FN>& acc, int m_base,
                                             int n_base, int lane, int tm, int tn, int wn,
                                             int bm_tile, int bn_tile) {
    int m0 = tm * bm_tile, n0 = tn * bn_tile;
    unsigned short* cbase = p.c + (long)m0 * p.ldc + n0;
    __amdgpu_buffer_rsrc_t rc = make_rsrc(cbase, 0x7fffffff);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int m = m_base + 32 * i + (lane & 31);
      bool mok = m < p.M;
      long tgt = mok ? p.targets[m] : -100;
      float lse = mok ? p.lse[m] : 0.0f;
      float scale = (tgt == -100) ? 0.0f : *p.grad_scale;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int n = n_base + 32 * j + 8 * g + 4 * (lane >> 5);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float l = rbf16(acc.v[i][j][4 * g + e]);
            float sm = exp_e(l - lse);
            v[e] = scale * sm - ((long)(n + e) == tgt ? scale : 0.0f);
          }
          if (p.vec_out) {
            bool ok = mok && (n + 3 < p.N);
            u32x2_t out = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            __builtin_amdgcn_raw_buffer_store_b64(
                out, rc, store_off(ok, (long)(m - m0) * p.ldc + (n - n0), 2), 0, 0);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (mok && n + e < p.N) cbase[(long)(m - m0) * p.ldc + (n + e - n0)] = to_bf16_bits(v[e]);
          }
        }
      }
    }
  }
};

// --------------------------------------------------------------------------------------
// The kernel.

template <int BM, int BN, int WM, int WN, int AMODE, int BMODE, bool PAIRED, class Epi>
__global__ void __launch_bounds__(WM * WN * kWave)
gemm_kernel(const GemmParams p) {
  constexpr int NT = WM * WN * kWave;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile");
  static_assert(!PAIRED || (FN % 2 == 0), "paired tiles need up/gate block pairs");

  extern __shared__ __attribute__((aligned(16))) unsigned short smem[];
  if (p.skip_if != nullptr && *p.skip_if != 0) return;  // uniform: the whole grid exits
  unsigned short* lds_a = smem;                    // [2][BM * BK]
  unsigned short* lds_b = smem + 2 * BM * kBK;     // [2][BN * BK]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  TileLoader<BM, NT, AMODE, false> la;
  TileLoader<BN, NT, BMODE, PAIRED> lb;

  // Per-lane LDS fragment row offsets (elements).
  int a_row[FM], b_row[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) a_row[i] = (wm * TM + 32 * i + (lane & 31)) * kBK;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    int r;
    if (PAIRED) {
      constexpr int FH = FN / 2;
      r = (j < FH) ? wn * (TN / 2) + 32 * j : BN / 2 + wn * (TN / 2) + 32 * (j - FH);
    } else {
      r = wn * TN + 32 * j;
    }
    b_row[j] = (r + (lane & 31)) * kBK;
  }
  const int hi = lane >> 5, sw = swz(lane & 15);

  const int bn_cols = PAIRED ? BN / 2 : BN;  // output columns per tile
  const int k_tiles_total = cdiv(p.K, kBK);
  const int kt_begin = blockIdx.y * p.k_tiles_per_split;
  const int kt_end = min(k_tiles_total, kt_begin + p.k_tiles_per_split);

  for (int w = blockIdx.x; w < p.total_tiles; w += gridDim.x) {
    int t = xcd_remap(w, p.total_tiles, gridDim.x);
    int tm, tn;
    tile_position(t, p.tiles_m, p.tiles_n, tm, tn);
    const int row0_a = tm * BM;
    const int row0_b = tn * bn_cols;

    la.init(p.a, row0_a, p.M, 0, tid);
    lb.init(p.b, row0_b, PAIRED ? p.H : p.N, PAIRED ? p.H : 0, tid);

    Acc<FM, FN> acc;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc.v[i][j][r] = 0.0f;

    if (kt_begin < kt_end) {
      la.load(p.a, row0_a, kt_begin * kBK, p.K);
      lb.load(p.b, row0_b, kt_begin * kBK, p.K);
      la.store(lds_a, tid);
      lb.store(lds_b, tid);
      __syncthreads();

      for (int kt = kt_begin; kt < kt_end; ++kt) {
        const int cur = (kt - kt_begin) & 1;
        const bool more = kt + 1 < kt_end;
        if (more) {
          la.load(p.a, row0_a, (kt + 1) * kBK, p.K);
          lb.load(p.b, row0_b, (kt + 1) * kBK, p.K);
        }
        const unsigned short* sa = lds_a + cur * BM * kBK;
        const unsigned short* sb = lds_b + cur * BN * kBK;
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
          const int chunk = ((2 * s + hi) ^ sw) << 3;
          bf16x8_t af[FM], bf[FN];
#pragma unroll
          for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const bf16x8_t*>(sa + a_row[i] + chunk);
#pragma unroll
          for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const bf16x8_t*>(sb + b_row[j] + chunk);
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc.v[i][j], 0, 0, 0);
        }
        if (more) {
          la.store(lds_a + (cur ^ 1) * BM * kBK, tid);
          lb.store(lds_b + (cur ^ 1) * BN * kBK, tid);
        }
        __syncthreads();
      }
    }

    const int m_base = row0_a + wm * TM;
    if (PAIRED) {
      Epi::run(p, acc, m_base, row0_b + wn * (TN / 2), lane, tm, tn, wn, BM, bn_cols);
    } else {
      Epi::run(p, acc, m_base, row0_b + wn * TN, lane, tm, tn, wn, BM, bn_cols);
    }
  }
}

template <int BM, int BN>
constexpr int gemm_lds_bytes() {
  return 2 * (BM + BN) * kBK * 2;
}

}  // namespace ws
