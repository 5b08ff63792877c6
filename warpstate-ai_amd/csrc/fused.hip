// C ABI: fused GEMMs of the forward and backward MLP / attention-input projections.
#include "../../include/warpstate_hip.h"
#include "launch.h"
#include "rowops.h"

namespace ws {
int check_gemm_args(const void* a, long a_s0, long a_s1, const void* b, long b_s0, long b_s1,
                    const void* c, long m, long n, long k);
int operand_mode(const OperandDesc& d, long rows, long k, int tile_rows);
}  // namespace ws

using namespace ws;

static inline OperandDesc desc_a(const void* a, long s0, long s1) {
  return OperandDesc{static_cast<const unsigned short*>(a), s0, s1};
}
static inline OperandDesc desc_b(const void* b, long s0, long s1) {
  return OperandDesc{static_cast<const unsigned short*>(b), s1, s0};
}

namespace ws {
// y and rstd for rows of x (row stride ldx) into a contiguous y, with the eager rounding
// y = r(r(x rstd) r(w)) or the FP32 product r(x rstd w): the RMSNorm pass before the fused
// input projection (eager), also the standalone RMSNorm forward. Rows of at most 8192
// vector-aligned features stay in registers (x read once).
template <bool EAGER>
static void rmsnorm_rows_eager(const unsigned short* xs, long ldx, const float* w,
                               unsigned short* ys, float* rstd, long m, long k, float eps,
                               int vec, hipStream_t s) {
  const dim3 grid(cdiv(m, 4));
  auto reg = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, xs, ldx, w, ys, rstd, (int)m, (int)k, eps);
  };
  if (vec && k <= 512) reg(rmsnorm_rows_reg_kernel<1, EAGER>);
  else if (vec && k <= 1024) reg(rmsnorm_rows_reg_kernel<2, EAGER>);
  else if (vec && k <= 2048) reg(rmsnorm_rows_reg_kernel<4, EAGER>);
  else if (vec && k <= 4096) reg(rmsnorm_rows_reg_kernel<8, EAGER>);
  else if (vec && k <= 8192) reg(rmsnorm_rows_reg_kernel<16, EAGER>);
  else
    hipLaunchKernelGGL(rmsnorm_rows_kernel<EAGER>, grid, dim3(256), 0, s, xs, ldx, w, ys, rstd,
                       (int)m, (int)k, eps, vec);
}

int launch_rmsnorm_rows(const void* x, long ldx, const float* w, void* y, float* rstd, long m,
                        long k, float eps, bool eager, hipStream_t s) {
  // The vector kernels read x and the FP32 weight, and write y, as 16-byte pieces.
  const int vec = (ldx % 8 == 0) && (k % 8 == 0) && al(x, 16) && al(y, 16) && al(w, 16);
  const auto* xs = static_cast<const unsigned short*>(x);
  auto* ys = static_cast<unsigned short*>(y);
  if (eager)
    rmsnorm_rows_eager<true>(xs, ldx, w, ys, rstd, m, k, eps, vec, s);
  else
    rmsnorm_rows_eager<false>(xs, ldx, w, ys, rstd, m, k, eps, vec, s);
  return hip_check(hipGetLastError(), "rmsnorm rows launch");
}
}  // namespace ws

extern "C" int ws_rmsnorm_gate_mm(const void* x, int64_t x_s0, const float* norm_weight,
                                  float eps, float* rstd, void* normed, const void* b,
                                  int64_t b_s0, int64_t b_s1, void* out, int64_t m, int64_t n,
                                  int64_t k, int64_t gate_begin, int64_t gate_end, void* stream) {
  if (int rc = check_gemm_args(x, x_s0, 1, b, b_s0, b_s1, out, m, n, k)) return rc;
  if (!norm_weight || !rstd || !normed) return set_error(kInvalid, "null RMSNorm pointer");
  if (gate_begin < 0 || gate_end < gate_begin || gate_end > n)
    return set_error(kInvalid, "gate column range [%ld, %ld) outside [0, %ld)", (long)gate_begin,
                     (long)gate_end, (long)n);
  if (x_s0 < k) return set_error(kInvalid, "RMSNorm prologue needs row-contiguous x");
  if (int rc = check_out_stride(n, 2, "output")) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Prologue: one pass over x writes the normalized BF16 operand y and rstd.
  if (int rc = launch_rmsnorm_rows(x, x_s0, norm_weight, normed, rstd, m, k, eps, true, s)) return rc;
  GemmParams p{};
  p.a = desc_a(normed, k, 1);
  p.b = desc_b(b, b_s0, b_s1);
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.c = static_cast<unsigned short*>(out);
  p.ldc = n;
  p.vec_out = (n % 4 == 0) && al(out, 8);
  p.gate_lo = (int)gate_begin;
  p.gate_hi = (int)gate_end;
  int am = operand_mode(p.a, m, k, 256), bm = operand_mode(p.b, n, k, 256);
  if (fast_ok(p, am, bm, false))
    return dispatch_fast<false, FEpiStore<true, false>>(p, am, bm, kFusedCfg, s);
  return dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiStore<true, false>>(p, am, bm,
                                                                                   LaunchCfg{0, 1}, s);
}

extern "C" int ws_residual_mm(const void* a, int64_t a_s0, int64_t a_s1, const void* b,
                              int64_t b_s0, int64_t b_s1, const void* residual,
                              int64_t ld_residual, void* out, int64_t m, int64_t n, int64_t k,
                              void* stream) {
  if (int rc = check_gemm_args(a, a_s0, a_s1, b, b_s0, b_s1, out, m, n, k)) return rc;
  if (!residual || ld_residual < n) return set_error(kInvalid, "invalid residual operand");
  if (int rc = check_out_stride(n, 2, "output")) return rc;
  if (int rc = check_out_stride(ld_residual, 2, "residual")) return rc;
  GemmParams p{};
  p.a = desc_a(a, a_s0, a_s1);
  p.b = desc_b(b, b_s0, b_s1);
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.c = static_cast<unsigned short*>(out);
  p.ldc = n;
  p.aux = static_cast<const unsigned short*>(residual);
  p.ldaux = ld_residual;
  p.vec_out = (n % 4 == 0) && (ld_residual % 4 == 0) && al(out, 8) && al(residual, 8);
  int am = operand_mode(p.a, m, k, 256), bm = operand_mode(p.b, n, k, 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fast_ok(p, am, bm, false))
    return dispatch_fast<false, FEpiStore<false, true>>(p, am, bm, kFusedCfg, s);
  constexpr unsigned mask = kMaskKK | ab_bit(kKContig, kMNContig) | kMaskGG;
  return dispatch<mask, WS_TILE_ARGS_LARGE, false, EpiStore<false, true>>(
      p, am, bm, LaunchCfg{0, 1}, s);
}

extern "C" int ws_swiglu_backward_mm(const void* grad, int64_t g_s0, int64_t g_s1, const void* b,
                                     int64_t b_s0, int64_t b_s1, const void* packed,
                                     void* dpacked, int64_t m, int64_t h, int64_t k,
                                     int eager_rounding, void* stream) {
  if (int rc = check_gemm_args(grad, g_s0, g_s1, b, b_s0, b_s1, dpacked, m, h, k)) return rc;
  if (!packed) return set_error(kInvalid, "null packed projection");
  if (int rc = check_out_stride(2 * h, 2, "packed projection")) return rc;
  GemmParams p{};
  p.a = desc_a(grad, g_s0, g_s1);
  p.b = desc_b(b, b_s0, b_s1);
  p.M = (int)m; p.N = (int)h; p.K = (int)k; p.H = (int)h;
  p.c = static_cast<unsigned short*>(dpacked);
  p.ldc = 2 * h;
  p.aux = static_cast<const unsigned short*>(packed);
  p.ldaux = 2 * h;
  p.eager = eager_rounding ? 1 : 0;
  // The staged fast epilogue moves 8 columns per lane.
  p.vec_out = (h % 8 == 0) && al(dpacked, 16) && al(packed, 16);
  int am = operand_mode(p.a, m, k, 256), bm = operand_mode(p.b, h, k, 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fast_ok(p, am, bm, false))
    return dispatch_fast<false, FEpiSwigluBwd>(p, am, bm, kFusedCfg, s);
  constexpr unsigned mask = kMaskKK | ab_bit(kKContig, kMNContig) | kMaskGG;
  return dispatch<mask, WS_TILE_ARGS_LARGE, false, EpiSwigluBwd>(
      p, am, bm, LaunchCfg{0, 1}, s);
}

namespace {

// Balanced accumulation plan for an [m, n] output with k-reduction k on `workers` CUs:
// whole rounds of 256 x 256 tiles run data-parallel, the other tiles' k-tiles are shared
// evenly (stream-K) by sk_workers = min(workers, units) workers, so that every share holds
// at least one unit, with at most `pieces` pieces per tile.
struct BalancedPlan {
  int tiles_m, tiles_n, tiles, k_tiles, dp_tiles, sk_tiles, pieces, sk_workers;
  long units;
  long workspace_floats() const { return (long)sk_tiles * pieces * kFBM * kFBN; }
};

BalancedPlan balanced_plan_tiles(long tiles, long k, int workers) {
  BalancedPlan b{};
  b.tiles = (int)tiles;
  b.k_tiles = cdiv(k, kFBK);
  b.dp_tiles = b.tiles / workers * workers;
  b.sk_tiles = b.tiles - b.dp_tiles;
  b.units = (long)b.sk_tiles * b.k_tiles;
  b.sk_workers = (int)(b.units < workers ? b.units : workers);
  b.pieces = 0;
  for (long ti = 0; ti < b.sk_tiles; ++ti) {
    const int pc = sk_pieces_of(ti, b.k_tiles, b.units, b.sk_workers);
    if (pc > b.pieces) b.pieces = pc;
  }
  return b;
}

BalancedPlan balanced_plan(long m, long n, long k, int workers) {
  BalancedPlan b = balanced_plan_tiles(cdiv(m, kFBM) * cdiv(n, kFBN), k, workers);
  b.tiles_m = cdiv(m, kFBM);
  b.tiles_n = cdiv(n, kFBN);
  return b;
}

// Outputs of a balanced accumulation: one GEMM, or the members of a grouped launch.
struct SkOutputs {
  int count;
  GemmMember m[kMaxGroup];
};

// G[m, n] += f32(r(sum of the tile's pieces)) (=, G not read, with kAccStore) for the
// stream-K tiles of a balanced accumulation: block (tile ti, chunk) handles 1024 elements
// of tile ti's 256 x 256 block, four consecutive columns per thread; pieces are added in
// k order. Tile ti is launch raster index dp_tiles + ti, in the output of the member whose
// tiles hold it.
__global__ void __launch_bounds__(256) sk_accum_kernel(const float* __restrict__ ws,
                                                       const SkOutputs out, int dp_tiles,
                                                       int k_tiles, long units, int workers,
                                                       int pieces_max, int round_acc, int vec) {
  const long ti = blockIdx.x / 64;
  const int e = (blockIdx.x % 64) * 1024 + threadIdx.x * 4;
  const int r = e / kFBN, c = e % kFBN;
  const int t = dp_tiles + (int)ti;
  GemmMember q = out.m[0];
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i)
    if (i < out.count && t >= out.m[i].tile_base) q = out.m[i];
  int tm, tn;
  tile_position(t - q.tile_base, q.tiles_m, q.tiles_n, tm, tn);
  const int m = tm * kFBM + r, n = tn * kFBN + c;
  const int M = q.M, N = q.N;
  float* __restrict__ g = q.g;
  const long ldg = q.ldg;
  if (m >= M || n >= N) return;
  const int pieces = sk_pieces_of(ti, k_tiles, units, workers);
  const float* src = ws + ti * pieces_max * (long)(kFBM * kFBN) + e;
  f32x4_t s = *reinterpret_cast<const f32x4_t*>(src);
  for (int q = 1; q < pieces; ++q) s += *reinterpret_cast<const f32x4_t*>(src + (long)q * kFBM * kFBN);
  if (round_acc & kAccRound) {
#pragma unroll
    for (int d = 0; d < 4; ++d) s[d] = rbf16(s[d]);
  }
  float* dst = g + (long)m * ldg + n;
  const bool store = round_acc & kAccStore;
  if (vec && n + 3 < N) {
    *reinterpret_cast<f32x4_t*>(dst) = store ? s : *reinterpret_cast<const f32x4_t*>(dst) + s;
  } else {
    for (int d = 0; d < 4 && n + d < N; ++d) dst[d] = store ? s[d] : dst[d] + s[d];
  }
}

}  // namespace

extern "C" int64_t ws_mm_accumulate_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t splits) {
  if (splits <= 1 || m < 1 || n < 1 || k < 1) return 0;
  // Even split-K slices (any operand layout), or the balanced plan (vector layouts).
  const long even = m * n * splits;
  const long balanced = balanced_plan(m, n, k, device_cus()).workspace_floats();
  return even > balanced ? even : balanced;
}

namespace {

// G = or += f32(r(A B)) (`acc`: AccMode bits) through the tile, balanced stream-K or even
// split-K paths; the body of ws_mm_accumulate_f32 and ws_mm_store_f32.
int mm_f32(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0, int64_t b_s1,
           float* g, int64_t ldg, int64_t m, int64_t n, int64_t k, int acc, float* workspace,
           int64_t splits, void* stream) {
  if (int rc = check_gemm_args(a, a_s0, a_s1, b, b_s0, b_s1, g, m, n, k)) return rc;
  if (ldg < n) return set_error(kInvalid, "gradient leading dimension %ld < n", (long)ldg);
  if (splits < 1 || splits > 64) return set_error(kInvalid, "splits must be in [1, 64]");
  if (splits > 1 && !workspace) return set_error(kInvalid, "split-K needs a workspace");
  if (int rc = check_out_stride(ldg, 4, "gradient")) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  GemmParams p{};
  p.a = desc_a(a, a_s0, a_s1);
  p.b = desc_b(b, b_s0, b_s1);
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.round_acc = acc;
  int am = operand_mode(p.a, m, k, 256), bm = operand_mode(p.b, n, k, 256);
  p.g = g;
  p.ldg = ldg;
  p.vec_out = (n % 4 == 0) && (ldg % 4 == 0) && al(g, 16);
  if (splits <= 1) {
    if (fast_ok(p, am, bm, false))
      return dispatch_fast<false, FEpiAccF32<false>>(p, am, bm, LaunchCfg{0, 1}, s);
    return dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiAccF32<false>>(p, am, bm,
                                                                                  LaunchCfg{0, 1}, s);
  }
  const int workers = device_cus();
  const BalancedPlan plan = balanced_plan(m, n, k, workers);
  const bool fast = fast_ok(p, am, bm, false);
  if (fast && plan.sk_tiles == 0)  // whole rounds of tiles: nothing to split
    return dispatch_fast<false, FEpiAccF32<false>>(p, am, bm, LaunchCfg{0, 1}, s);
  if (fast && plan.dp_tiles > 0 && al(workspace, 16)) {
    // Balanced: whole rounds of tiles accumulate directly, the rest is shared stream-K.
    p.balanced = 1;
    p.dp_tiles = plan.dp_tiles;
    p.sk_tiles = plan.sk_tiles;
    p.k_tiles = plan.k_tiles;
    p.sk_units = plan.units;
    p.sk_pieces = plan.pieces;
    p.sk_ws = workspace;
    if (int rc = dispatch_fast<false, FEpiAccF32<false>>(p, am, bm, LaunchCfg{1, 1, workers}, s))
      return rc;
    SkOutputs out{};
    out.count = 1;
    out.m[0] = GemmMember{p.a, p.b, (int)m, (int)n, plan.tiles_m, plan.tiles_n, 0, g, (long)ldg};
    hipLaunchKernelGGL(sk_accum_kernel, dim3((unsigned)(plan.sk_tiles * 64)), dim3(256), 0, s,
                       workspace, out, plan.dp_tiles, plan.k_tiles, plan.units, plan.sk_workers,
                       plan.pieces, acc, p.vec_out);
    return hip_check(hipGetLastError(), "stream-K reduce launch");
  }
  // Fewer tiles than compute units, or generic layouts: even split-K slices through the
  // workspace, then one reduction pass.
  p.g = workspace;
  p.ldg = n;
  p.split_stride = m * n;
  p.vec_out = (n % 4 == 0) && al(workspace, 16);
  if (fast && p.vec_out) {
    if (int rc = dispatch_fast<false, FEpiAccF32<true>>(p, am, bm, LaunchCfg{0, (int)splits}, s))
      return rc;
  } else if (int rc = dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiAccF32<true>>(
                 p, am, bm, LaunchCfg{0, (int)splits}, s)) {
    return rc;
  }
  const int vec = (n % 4 == 0) && (ldg % 4 == 0) && al(g, 16) && al(workspace, 16);
  const long threads = vec ? m * n / 4 : m * n;
  hipLaunchKernelGGL(splitk_accum_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     workspace, (int)splits, (long)(m * n), g, (long)ldg, (int)m, (int)n,
                     acc, vec);
  return hip_check(hipGetLastError(), "split-K reduce launch");
}

}  // namespace

extern "C" int ws_mm_accumulate_f32(const void* a, int64_t a_s0, int64_t a_s1, const void* b,
                                    int64_t b_s0, int64_t b_s1, float* g, int64_t ldg, int64_t m,
                                    int64_t n, int64_t k, int round_bf16, float* workspace,
                                    int64_t splits, void* stream) {
  return mm_f32(a, a_s0, a_s1, b, b_s0, b_s1, g, ldg, m, n, k, round_bf16 ? kAccRound : 0,
                workspace, splits, stream);
}

extern "C" int ws_mm_store_f32(const void* a, int64_t a_s0, int64_t a_s1, const void* b,
                               int64_t b_s0, int64_t b_s1, float* g, int64_t ldg, int64_t m,
                               int64_t n, int64_t k, int round_bf16, float* workspace,
                               int64_t splits, void* stream) {
  return mm_f32(a, a_s0, a_s1, b, b_s0, b_s1, g, ldg, m, n, k,
                kAccStore | (round_bf16 ? kAccRound : 0), workspace, splits, stream);
}

namespace {

// Split count for one GEMM of a grouped call that falls back to single launches: the one
// (fewest on ties, at most 4, each split at least 16 k-tiles) that best fills the last
// round of 256 x 256 tiles.
int auto_splits(long m, long n, long k, int cus) {
  const long tiles = cdiv(m, kFBM) * cdiv(n, kFBN);
  int best = 1;
  double best_eff = 0.0;
  for (int s = 1; s <= 4; ++s) {
    if (s > 1 && cdiv(k, kFBK) / s < 16) break;
    const long work = tiles * s;
    const double eff = (double)work / (double)(cdiv(work, cus) * cus);
    if (eff > best_eff + 1e-9) {
      best = s;
      best_eff = eff;
    }
  }
  return best;
}

long group_tiles(const ws_accumulate_problem* pr, int count) {
  long t = 0;
  for (int i = 0; i < count; ++i) t += cdiv(pr[i].m, kFBM) * cdiv(pr[i].n, kFBN);
  return t;
}

}  // namespace

extern "C" int64_t ws_mm_accumulate_group_workspace_floats(const ws_accumulate_problem* problems,
                                                           int count, int64_t k) {
  if (!problems || count < 1 || count > kMaxGroup || k < 1) return 0;
  const int workers = device_cus();
  // The one-launch plan (used only when its tiles fill at least one round), or a fallback
  // single call's split.
  const BalancedPlan plan = balanced_plan_tiles(group_tiles(problems, count), k, workers);
  long need = plan.dp_tiles > 0 ? plan.workspace_floats() : 0;
  for (int i = 0; i < count; ++i) {
    const long m = problems[i].m, n = problems[i].n;
    if (m < 1 || n < 1) return 0;
    const long one = ws_mm_accumulate_workspace_floats(m, n, k, auto_splits(m, n, k, workers));
    if (one > need) need = one;
  }
  return need;
}

namespace {

int mm_f32_group(const ws_accumulate_problem* problems, int count, int64_t k, int acc,
                 float* workspace, void* stream) {
  if (!problems) return set_error(kInvalid, "null problem table");
  if (count < 1 || count > kMaxGroup)
    return set_error(kInvalid, "group size %d outside [1, %d]", count, kMaxGroup);
  for (int i = 0; i < count; ++i) {
    const ws_accumulate_problem& q = problems[i];
    if (int rc = check_gemm_args(q.a, q.a_s0, q.a_s1, q.b, q.b_s0, q.b_s1, q.g, q.m, q.n, k))
      return rc;
    if (q.ldg < q.n) return set_error(kInvalid, "gradient %d leading dimension %ld < n", i, (long)q.ldg);
    if (int rc = check_out_stride(q.ldg, 4, "gradient")) return rc;
  }
  // The gradients are updated in place by different workgroups: they must not overlap.
  for (int i = 0; i < count; ++i)
    for (int j = i + 1; j < count; ++j) {
      const char* bi = reinterpret_cast<const char*>(problems[i].g);
      const char* bj = reinterpret_cast<const char*>(problems[j].g);
      const long si = ((problems[i].m - 1) * problems[i].ldg + problems[i].n) * 4;
      const long sj = ((problems[j].m - 1) * problems[j].ldg + problems[j].n) * 4;
      if (bi < bj + sj && bj < bi + si)
        return set_error(kInvalid, "gradients %d and %d overlap", i, j);
    }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int workers = device_cus();
  const BalancedPlan plan = balanced_plan_tiles(group_tiles(problems, count), k, workers);

  // One launch when every GEMM takes the fast loader with the same operand layouts and
  // vector outputs, and the tiles fill at least one round.
  GemmParams p{};
  p.K = (int)k;
  p.round_acc = acc;
  p.vec_out = 1;
  int am = -1, bm = -1;
  bool one_launch = plan.dp_tiles > 0 && (plan.sk_tiles == 0 || (workspace && al(workspace, 16)));
  int base = 0;
  for (int i = 0; i < count && one_launch; ++i) {
    const ws_accumulate_problem& q = problems[i];
    GemmParams pi{};
    pi.a = desc_a(q.a, q.a_s0, q.a_s1);
    pi.b = desc_b(q.b, q.b_s0, q.b_s1);
    pi.vec_out = (q.n % 4 == 0) && (q.ldg % 4 == 0) && al(q.g, 16);
    const int ami = operand_mode(pi.a, q.m, k, 256), bmi = operand_mode(pi.b, q.n, k, 256);
    if (i == 0) {
      am = ami;
      bm = bmi;
    }
    if (ami != am || bmi != bm || !fast_ok(pi, ami, bmi, false)) {
      one_launch = false;
      break;
    }
    const int tm = cdiv(q.m, kFBM), tn = cdiv(q.n, kFBN);
    p.grp[i] = GemmMember{pi.a, pi.b, (int)q.m, (int)q.n, tm, tn, base, q.g, (long)q.ldg};
    base += tm * tn;
  }
  if (!one_launch) {
    for (int i = 0; i < count; ++i) {
      const ws_accumulate_problem& q = problems[i];
      const int splits = workspace ? auto_splits(q.m, q.n, k, workers) : 1;
      if (int rc = mm_f32(q.a, q.a_s0, q.a_s1, q.b, q.b_s0, q.b_s1, q.g, q.ldg, q.m, q.n, k, acc,
                          workspace, splits, stream))
        return rc;
    }
    return kOk;
  }
  p.group_count = count;
  p.a = p.grp[0].a;
  p.b = p.grp[0].b;
  p.M = p.grp[0].M;
  p.N = p.grp[0].N;
  p.balanced = 1;
  p.dp_tiles = plan.dp_tiles;
  p.sk_tiles = plan.sk_tiles;
  p.k_tiles = plan.k_tiles;
  p.sk_units = plan.units;
  p.sk_pieces = plan.pieces;
  p.sk_ws = workspace;
  if (int rc = dispatch_fast<false, FEpiAccF32<false>>(p, am, bm, LaunchCfg{1, 1, workers}, s))
    return rc;
  if (plan.sk_tiles == 0) return kOk;
  SkOutputs out{};
  out.count = count;
  for (int i = 0; i < count; ++i) out.m[i] = p.grp[i];
  hipLaunchKernelGGL(sk_accum_kernel, dim3((unsigned)(plan.sk_tiles * 64)), dim3(256), 0, s,
                     workspace, out, plan.dp_tiles, plan.k_tiles, plan.units, plan.sk_workers,
                     plan.pieces, acc, 1);
  return hip_check(hipGetLastError(), "stream-K reduce launch");
}

}  // namespace

extern "C" int ws_mm_accumulate_f32_group(const ws_accumulate_problem* problems, int count,
                                          int64_t k, int round_bf16, float* workspace,
                                          void* stream) {
  return mm_f32_group(problems, count, k, round_bf16 ? kAccRound : 0, workspace, stream);
}

extern "C" int ws_mm_store_f32_group(const ws_accumulate_problem* problems, int count, int64_t k,
                                     int round_bf16, float* workspace, void* stream) {
  return mm_f32_group(problems, count, k, kAccStore | (round_bf16 ? kAccRound : 0), workspace,
                      stream);
}
