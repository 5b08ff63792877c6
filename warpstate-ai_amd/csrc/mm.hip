// C ABI: plain BF16 GEMM (launch_mm) and the paired SwiGLU GEMM (launch_swiglu_mm).
#include "../../include/warpstate_hip.h"
#include "launch.h"

namespace ws {

// Operand descriptors from PyTorch-style (s0, s1) strides of A [m,k] and B [k,n].
inline OperandDesc desc_a(const void* a, long s0, long s1) {
  return OperandDesc{static_cast<const unsigned short*>(a), s0, s1};
}
inline OperandDesc desc_b(const void* b, long s0, long s1) {
  return OperandDesc{static_cast<const unsigned short*>(b), s1, s0};
}

int check_gemm_args(const void* a, long a_s0, long a_s1, const void* b, long b_s0, long b_s1,
                    const void* c, long m, long n, long k) {
  if (!a || !b || !c) return set_error(kInvalid, "null operand pointer");
  if (m < 1 || n < 1 || k < 1 || !fits_i32(m) || !fits_i32(n) || !fits_i32(k))
    return set_error(kInvalid, "matrix sizes must be positive 32-bit integers (m=%ld n=%ld k=%ld)",
                     m, n, k);
  if (a_s0 < 1 || a_s1 < 1 || b_s0 < 1 || b_s1 < 1)
    return set_error(kInvalid, "matrix kernels require positive strides");
  return kOk;
}

int operand_mode(const OperandDesc& d, long rows, long k, int tile_rows) {
  int mode = classify(d.ptr, d.s_row, d.s_k, rows, k);
  if (!offsets_fit(mode, d.s_row, d.s_k, tile_rows)) mode = kGeneric;
  return mode;
}

}  // namespace ws

using namespace ws;

extern "C" int ws_mm(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0,
                     int64_t b_s1, void* c, int64_t m, int64_t n, int64_t k, int algorithm,
                     int tile, void* stream) {
  if (int rc = check_gemm_args(a, a_s0, a_s1, b, b_s0, b_s1, c, m, n, k)) return rc;
  if (algorithm < 0 || algorithm > 2) return set_error(kInvalid, "unknown algorithm %d", algorithm);
  if (tile != kTileLarge && tile != kTileSmall) return set_error(kInvalid, "unknown tile %d", tile);
  if (int rc = check_out_stride(n, 2, "output")) return rc;
  GemmParams p{};
  p.a = desc_a(a, a_s0, a_s1);
  p.b = desc_b(b, b_s0, b_s1);
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.c = static_cast<unsigned short*>(c);
  p.ldc = n;
  p.vec_out = (n % 4 == 0) && (reinterpret_cast<unsigned long>(c) % 8 == 0);
  const int rows = tile == kTileLarge ? 256 : 128;
  const int am = operand_mode(p.a, m, k, rows), bm = operand_mode(p.b, n, k, rows);
  LaunchCfg cfg{algorithm != 0, 1};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tile == kTileLarge && fast_ok(p, am, bm, false))
    return dispatch_fast<false, FEpiStore<false, false>>(p, am, bm, cfg, s);
  if (tile == kTileLarge)
    return dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiStore<false, false>>(p, am, bm, cfg, s);
  return dispatch<kMaskMM, WS_TILE_ARGS_SMALL, false, EpiStore<false, false>>(p, am, bm, cfg, s);
}

extern "C" int ws_swiglu_mm(const void* a, int64_t a_s0, int64_t a_s1, const void* b,
                            int64_t b_s0, int64_t b_s1, void* packed, void* act, int64_t m,
                            int64_t h, int64_t k, int eager_rounding, int algorithm, int tile,
                            void* stream) {
  if (int rc = check_gemm_args(a, a_s0, a_s1, b, b_s0, b_s1, packed, m, 2 * h, k)) return rc;
  if (!act) return set_error(kInvalid, "null activation pointer");
  if (algorithm < 0 || algorithm > 1) return set_error(kInvalid, "unknown SwiGLU algorithm %d", algorithm);
  if (tile != kTileLarge && tile != kTileSmall) return set_error(kInvalid, "unknown tile %d", tile);
  if (int rc = check_out_stride(2 * h, 2, "packed output")) return rc;
  GemmParams p{};
  p.a = desc_a(a, a_s0, a_s1);
  p.b = desc_b(b, b_s0, b_s1);
  p.M = (int)m; p.N = (int)(2 * h); p.K = (int)k; p.H = (int)h;
  p.c = static_cast<unsigned short*>(packed);
  p.ldc = 2 * h;
  p.c2 = static_cast<unsigned short*>(act);
  p.ldc2 = h;
  p.eager = eager_rounding ? 1 : 0;
  p.vec_out = (h % 4 == 0) && (reinterpret_cast<unsigned long>(packed) % 8 == 0) &&
              (reinterpret_cast<unsigned long>(act) % 8 == 0);
  const int rows = tile == kTileLarge ? 256 : 128;
  int am = operand_mode(p.a, m, k, rows);
  // B rows are the paired up/gate columns; vector modes see `h` rows per half and the
  // gate half lives `h` rows further, which the offset bound must also cover.
  int bm = operand_mode(p.b, h, k, rows);
  if (bm == kKContig && !offsets_fit(kKContig, p.b.s_row, 1, (int)(h + rows))) bm = kGeneric;
  if (bm == kMNContig && 2L * (h + rows) >= 0x7fffffffL) bm = kGeneric;
  LaunchCfg cfg{algorithm != 0, 1};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tile == kTileLarge && fast_ok(p, am, bm, true))
    return dispatch_fast<true, FEpiSwiglu>(p, am, bm, cfg, s);
  if (tile == kTileLarge)
    return dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, true, EpiSwiglu>(p, am, bm, cfg, s);
  return dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_SMALL, true, EpiSwiglu>(p, am, bm, cfg, s);
}
