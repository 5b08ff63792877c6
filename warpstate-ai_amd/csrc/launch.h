// Host-side launch helpers shared by the C-ABI translation units.
#pragma once

#include <stdarg.h>
#include <stdio.h>

#include "gemm_fast.h"

namespace ws {

// Status codes returned by every entry point.
enum Status { kOk = 0, kInvalid = 1, kHipError = 2 };

int set_error(int code, const char* fmt, ...);  // records the thread's last error, returns code
int device_cus();                               // compute units of the current device
int ensure_lds(const void* kernel, int bytes);  // raises the kernel's dynamic LDS limit on this device to >= bytes

// Whether a pointer is aligned to `bytes`.
inline bool al(const void* p, int bytes) { return reinterpret_cast<unsigned long>(p) % bytes == 0; }

inline int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return set_error(kHipError, "%s: %s", what, hipGetErrorString(e));
  return kOk;
}

// Storage mode of a GEMM operand: `rows` is the operand's M (A) or N (B) extent and
// `K` the reduction length. The vector modes need 16-byte aligned rows and runs whose
// length is a multiple of 8 along the contiguous dimension.
inline int classify(const void* ptr, long s_row, long s_k, long rows, long K) {
  const unsigned long p = reinterpret_cast<unsigned long>(ptr);
  if (s_k == 1 && p % 16 == 0 && s_row % 8 == 0 && K % 8 == 0) return kKContig;
  if (s_row == 1 && p % 16 == 0 && s_k % 8 == 0 && rows % 8 == 0) return kMNContig;
  return kGeneric;
}

// The generic loader computes 64-bit addresses; the vector loaders use 32-bit offsets
// relative to a per-tile base, bounded here.
inline bool offsets_fit(int mode, long s_row, long s_k, int tile_rows) {
  const long lim = 0x7fffffffL;
  if (mode == kKContig) return (long)tile_rows * s_row * 2 + 2 * kBK < lim;
  if (mode == kMNContig) return (long)kBK * s_k * 2 + 2L * tile_rows < lim;
  return true;
}

struct LaunchCfg {
  int persistent;  // grid = resident workgroups instead of one per tile
  int splits;      // split-K slices (blockIdx.y)
  int workers;     // > 0: exactly this many workgroups (balanced accumulation)
};
// The fused entry points' 256 x 256 launches: one workgroup per CU looping over the tiles.
// A workgroup that ends and a new one that starts on the freed CU leave it idle for
// about 3 us per tile; the persistent grid keeps that to about 1 us (the forward
// projections and the LM-head GEMMs 2-4 % faster, results bit-identical).
constexpr LaunchCfg kFusedCfg{1, 1, 0};

template <int BM, int BN, int WM, int WN, int AM, int BMD, bool PAIRED, class Epi>
int run_gemm(GemmParams p, LaunchCfg cfg, hipStream_t stream) {
  constexpr int NT = WM * WN * kWave;
  constexpr int lds = gemm_lds_bytes<BM, BN>();
  const void* kern = reinterpret_cast<const void*>(&gemm_kernel<BM, BN, WM, WN, AM, BMD, PAIRED, Epi>);
  if (int rc = ensure_lds(kern, lds)) return rc;
  const int cols = PAIRED ? p.H : p.N;
  const int bn_cols = PAIRED ? BN / 2 : BN;
  p.tiles_m = cdiv(p.M, BM);
  p.tiles_n = cdiv(cols, bn_cols);
  p.total_tiles = p.tiles_m * p.tiles_n;
  const int k_tiles = cdiv(p.K, kBK);
  const int splits = cfg.splits < 1 ? 1 : cfg.splits;
  p.k_tiles_per_split = cdiv(k_tiles, splits);
  if (p.k_tiles_per_split < 1) p.k_tiles_per_split = 1;
  const int resident = device_cus() * (lds > 80 * 1024 ? 1 : 2);
  dim3 grid(cfg.persistent ? (p.total_tiles < resident ? p.total_tiles : resident) : p.total_tiles,
            splits);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, AM, BMD, PAIRED, Epi>), grid, dim3(NT), lds,
                     stream, p);
  return hip_check(hipGetLastError(), "gemm launch");
}

// Large tile: 256 x 256 with 8 waves (64 x 128 per wave). Small tile: 128 x 128 with
// 4 waves (64 x 64 per wave), two workgroups per CU.
enum TileCfg { kTileLarge = 0, kTileSmall = 1 };

#define WS_TILE_ARGS_LARGE 256, 256, 4, 2
#define WS_TILE_ARGS_SMALL 128, 128, 2, 2

}  // namespace ws

namespace ws {

// Layout-combination bit for (A mode, B mode).
constexpr unsigned ab_bit(int am, int bm) { return 1u << (am * 3 + bm); }
constexpr unsigned kMaskKK = ab_bit(kKContig, kKContig);
constexpr unsigned kMaskGG = ab_bit(kGeneric, kGeneric);
constexpr unsigned kMaskMM = kMaskKK | ab_bit(kKContig, kMNContig) | ab_bit(kMNContig, kKContig) |
                             ab_bit(kMNContig, kMNContig) | kMaskGG;

// Runs the instantiation for (am, bm) if MASK holds it, demoting an operand to the
// generic loader otherwise.
template <unsigned MASK, int BM, int BN, int WM, int WN, bool PAIRED, class Epi>
int dispatch(const GemmParams& p, int am, int bm, LaunchCfg cfg, hipStream_t s) {
  auto has = [](int a, int b) { return (MASK & ab_bit(a, b)) != 0; };
  if (!has(am, bm)) {
    if (has(am, kGeneric)) bm = kGeneric;
    else if (has(kGeneric, bm)) am = kGeneric;
    else { am = kGeneric; bm = kGeneric; }
  }
#define WS_CASE(A_, B_)                                                            \
  case A_ * 3 + B_:                                                                \
    if constexpr ((MASK & ab_bit(A_, B_)) != 0)                                    \
      return run_gemm<BM, BN, WM, WN, A_, B_, PAIRED, Epi>(p, cfg, s);             \
    break;
  switch (am * 3 + bm) {
    WS_CASE(0, 0) WS_CASE(0, 1) WS_CASE(0, 2)
    WS_CASE(1, 0) WS_CASE(1, 1) WS_CASE(1, 2)
    WS_CASE(2, 0) WS_CASE(2, 1) WS_CASE(2, 2)
  }
#undef WS_CASE
  return set_error(kInvalid, "no GEMM instantiation for operand layouts (%d, %d)", am, bm);
}

inline bool fits_i32(long v) { return v >= 0 && v < 0x7fffffffL; }

// Epilogues address an output tile through a buffer resource of at most 2 GiB that starts
// at the tile's first row, so 256 rows of an output (row stride `ld` elements of
// `elem_bytes`) must span less than that; wider outputs are rejected instead of losing
// stores past the limit.
inline int check_out_stride(long ld, int elem_bytes, const char* what) {
  if ((long)kFBM * ld * elem_bytes + (long)kFBN * elem_bytes >= 0x7fffffffL)
    return set_error(kInvalid, "%s row stride %ld is too large: a 256-row tile spans 2 GiB or more",
                     what, ld);
  return kOk;
}

// Fast path (gemm_fast.h): 256 x 256 tiles, direct-to-LDS loads, 16x16x32 MFMA.
template <int AM, int BMD, bool PAIRED, class Epi>
int run_fast(GemmParams p, LaunchCfg cfg, hipStream_t stream) {
  const void* kern = reinterpret_cast<const void*>(&gemm_fast_kernel<AM, BMD, PAIRED, Epi>);
  constexpr int lds_bytes = fast_lds_bytes<AM, BMD>();
  if (int rc = ensure_lds(kern, lds_bytes)) return rc;
  const int cols = PAIRED ? p.H : p.N;
  const int bn_cols = PAIRED ? kFBN / 2 : kFBN;
  p.tiles_m = cdiv(p.M, kFBM);
  p.tiles_n = cdiv(cols, bn_cols);
  p.total_tiles = p.tiles_m * p.tiles_n;
  const int k_tiles = cdiv(p.K, kFBK);
  const int splits = cfg.splits < 1 ? 1 : cfg.splits;
  p.k_tiles_per_split = cdiv(k_tiles, splits);
  if (p.k_tiles_per_split < 1) p.k_tiles_per_split = 1;
  const int resident = device_cus();
  dim3 grid(cfg.persistent ? (p.total_tiles < resident ? p.total_tiles : resident) : p.total_tiles,
            splits);
  if (cfg.workers > 0) grid = dim3(cfg.workers, 1);
  hipLaunchKernelGGL((gemm_fast_kernel<AM, BMD, PAIRED, Epi>), grid, dim3(kFNT), lds_bytes, stream, p);
  return hip_check(hipGetLastError(), "gemm launch");
}

// True when both operand modes can take the fast path for a 256-row tile. The vector
// modes already guarantee 16-byte aligned chunks and whole-chunk edges; the per-tile
// 32-bit offsets are bounded here (paired B tiles reach `half` rows further).
inline bool fast_ok(const GemmParams& p, int am, int bm, bool paired) {
  if (am == kGeneric || bm == kGeneric || !p.vec_out) return false;
  const long lim = 0x7fffffffL;
  const long half = paired ? p.H : 0;
  if (am == kKContig && (256L + 1) * p.a.s_row * 2 >= lim) return false;
  if (am == kMNContig && 2L * 256 + 64L * p.a.s_k * 2 >= lim) return false;
  if (bm == kKContig && (256L + half + 1) * p.b.s_row * 2 >= lim) return false;
  if (bm == kMNContig && 2L * (256 + half) + 64L * p.b.s_k * 2 >= lim) return false;
  return true;
}

template <bool PAIRED, class Epi>
int dispatch_fast(const GemmParams& p, int am, int bm, LaunchCfg cfg, hipStream_t s) {
  switch (am * 2 + bm) {
    case 0: return run_fast<kKContig, kKContig, PAIRED, Epi>(p, cfg, s);
    case 1: return run_fast<kKContig, kMNContig, PAIRED, Epi>(p, cfg, s);
    case 2: return run_fast<kMNContig, kKContig, PAIRED, Epi>(p, cfg, s);
    default: return run_fast<kMNContig, kMNContig, PAIRED, Epi>(p, cfg, s);
  }
}

}  // namespace ws
