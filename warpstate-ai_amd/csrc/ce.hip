// C ABI: LM-head GEMM with fused cross-entropy (forward statistics and dHidden).
#include "../../include/warpstate_hip.h"
#include "launch.h"
#include "rowops.h"

namespace ws {
int operand_mode(const OperandDesc& d, long rows, long k, int tile_rows);
}

using namespace ws;

namespace {

constexpr int kCeTileN = 256;  // vocab columns per logits tile (large tile)
constexpr int kCeWavesN = 2;   // waves across those columns, one partial each

int check_ce(const void* hidden, long ld_hidden, const void* weight, long ld_weight,
             const void* targets, long rows, long vocab, long d) {
  if (!hidden || !weight || !targets) return set_error(kInvalid, "null operand pointer");
  if (rows < 1 || vocab < 1 || d < 1 || !fits_i32(rows) || !fits_i32(vocab) || !fits_i32(d))
    return set_error(kInvalid, "invalid LM-head sizes rows=%ld vocab=%ld d=%ld", rows, vocab, d);
  if (ld_hidden < d || ld_weight < d) return set_error(kInvalid, "leading dimension < d");
  return kOk;
}

}  // namespace

extern "C" int64_t ws_linear_ce_parts(int64_t vocab) {
  return (int64_t)cdiv(vocab, kCeTileN) * kCeWavesN;
}

extern "C" int ws_linear_ce_forward(const void* hidden, int64_t ld_hidden, const void* weight,
                                    int64_t ld_weight, const int64_t* targets, int64_t rows,
                                    int64_t vocab, int64_t d, float* part_max, float* part_sum,
                                    float* target_logit, float* lse, float* loss, float* mean,
                                    float* count, void* stream) {
  if (int rc = check_ce(hidden, ld_hidden, weight, ld_weight, targets, rows, vocab, d)) return rc;
  if (!part_max || !part_sum || !target_logit || !lse || !loss || !mean || !count)
    return set_error(kInvalid, "null output pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  GemmParams p{};
  p.a = OperandDesc{static_cast<const unsigned short*>(hidden), ld_hidden, 1};
  p.b = OperandDesc{static_cast<const unsigned short*>(weight), ld_weight, 1};  // B = W^T
  p.M = (int)rows; p.N = (int)vocab; p.K = (int)d;
  p.targets = reinterpret_cast<const long*>(targets);
  p.part_max = part_max;
  p.part_sum = part_sum;
  p.tgt_logit = target_logit;
  p.parts_per_row = (int)ws_linear_ce_parts(vocab);
  int am = operand_mode(p.a, rows, d, 256), bm = operand_mode(p.b, vocab, d, 256);
  if (int rc = dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, false, false, EpiCEStats>(
          p, am, bm, LaunchCfg{0, 1}, s))
    return rc;
  hipLaunchKernelGGL(ce_combine_kernel, dim3(cdiv(rows, 4)), dim3(256), 0, s, part_max, part_sum,
                     p.parts_per_row, target_logit, reinterpret_cast<const long*>(targets), lse,
                     loss, (int)rows, (int)vocab);
  if (int rc = hip_check(hipGetLastError(), "ce combine launch")) return rc;
  hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(1024), 0, s, loss,
                     reinterpret_cast<const long*>(targets), (int)rows, mean, count);
  return hip_check(hipGetLastError(), "ce mean launch");
}

extern "C" int ws_linear_ce_backward(const void* hidden, int64_t ld_hidden, const void* weight,
                                     int64_t ld_weight, const int64_t* targets, const float* lse,
                                     const float* count, const float* grad_mean, int64_t rows,
                                     int64_t vocab, int64_t d, void* grad_logits_ws,
                                     int64_t chunk_rows, float* scale_ws, void* dhidden,
                                     int64_t ld_dhidden, void* stream) {
  if (int rc = check_ce(hidden, ld_hidden, weight, ld_weight, targets, rows, vocab, d)) return rc;
  if (!lse || !count || !grad_mean || !grad_logits_ws || !scale_ws || !dhidden)
    return set_error(kInvalid, "null pointer");
  if (chunk_rows < 1 || !fits_i32(chunk_rows * vocab / 1)) return set_error(kInvalid, "bad chunk_rows");
  if (ld_dhidden < d) return set_error(kInvalid, "dhidden leading dimension < d");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ce_scale_kernel, dim3(1), dim3(64), 0, s, grad_mean, count, scale_ws);
  if (int rc = hip_check(hipGetLastError(), "ce scale launch")) return rc;
  auto* gl = static_cast<unsigned short*>(grad_logits_ws);
  for (long start = 0; start < rows; start += chunk_rows) {
    const long r = rows - start < chunk_rows ? rows - start : chunk_rows;
    // Logit gradients of this row chunk, r(scale * (softmax - onehot)), BF16.
    GemmParams p{};
    p.a = OperandDesc{static_cast<const unsigned short*>(hidden) + start * ld_hidden, ld_hidden, 1};
    p.b = OperandDesc{static_cast<const unsigned short*>(weight), ld_weight, 1};
    p.M = (int)r; p.N = (int)vocab; p.K = (int)d;
    p.c = gl;
    p.ldc = vocab;
    p.vec_out = (vocab % 4 == 0) && (reinterpret_cast<unsigned long>(gl) % 8 == 0);
    p.targets = reinterpret_cast<const long*>(targets) + start;
    p.lse = lse + start;
    p.grad_scale = scale_ws;
    int am = operand_mode(p.a, r, d, 256), bm = operand_mode(p.b, vocab, d, 256);
    if (int rc = dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, false, false, EpiCEGrad>(
            p, am, bm, LaunchCfg{0, 1}, s))
      return rc;
    // dHidden of the chunk: r(G [r, vocab] @ W [vocab, d]).
    GemmParams q{};
    q.a = OperandDesc{gl, vocab, 1};
    q.b = OperandDesc{static_cast<const unsigned short*>(weight), 1, ld_weight};
    q.M = (int)r; q.N = (int)d; q.K = (int)vocab;
    q.c = static_cast<unsigned short*>(dhidden) + start * ld_dhidden;
    q.ldc = ld_dhidden;
    q.vec_out = (d % 4 == 0) && (ld_dhidden % 4 == 0) &&
                (reinterpret_cast<unsigned long>(q.c) % 8 == 0);
    int qa = operand_mode(q.a, r, vocab, 128), qb = operand_mode(q.b, d, vocab, 128);
    if (int rc = dispatch<kMaskMM, WS_TILE_ARGS_SMALL, false, false, EpiStore<false, false>>(
            q, qa, qb, LaunchCfg{0, 1}, s))
      return rc;
  }
  return kOk;
}
