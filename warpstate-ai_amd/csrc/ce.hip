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
                                    int64_t* count, void* logits, void* stream) {
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
  p.vec_out = 1;  // the statistics epilogue stores no output tile
  int am = operand_mode(p.a, rows, d, 256), bm = operand_mode(p.b, vocab, d, 256);
  if (logits) {
    // The logits are kept for the backward: [rows, vocab] BF16, written by the fast path's
    // staged epilogue.
    if (vocab % 4 || reinterpret_cast<unsigned long>(logits) % 16)
      return set_error(kInvalid, "stored logits need vocab %% 4 == 0 and a 16-byte aligned buffer");
    if (int rc = check_out_stride(vocab, 2, "logits")) return rc;
    if (!fast_ok(p, am, bm, false))
      return set_error(kInvalid, "stored logits need row-contiguous hidden and weight operands");
    p.c = static_cast<unsigned short*>(logits);
    p.ldc = vocab;
    if (int rc = dispatch_fast<false, FEpiCEStatsLogits>(p, am, bm, LaunchCfg{0, 1}, s)) return rc;
  } else if (fast_ok(p, am, bm, false)) {
    if (int rc = dispatch_fast<false, FEpiCEStats>(p, am, bm, LaunchCfg{0, 1}, s)) return rc;
  } else if (int rc = dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, false, EpiCEStats>(
                 p, am, bm, LaunchCfg{0, 1}, s)) {
    return rc;
  }
  hipLaunchKernelGGL(ce_combine_kernel, dim3(cdiv(rows, 4)), dim3(256), 0, s, part_max, part_sum,
                     p.parts_per_row, target_logit, reinterpret_cast<const long*>(targets), lse,
                     loss, (int)rows, (int)vocab);
  if (int rc = hip_check(hipGetLastError(), "ce combine launch")) return rc;
  hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(1024), 0, s, loss,
                     reinterpret_cast<const long*>(targets), (int)rows, mean,
                     reinterpret_cast<long*>(count));
  return hip_check(hipGetLastError(), "ce mean launch");
}

// Workspace of the backward: [scale, 256 B][chunk x vocab BF16 logit gradients]
// [splits x chunk x d FP32 dHidden partials], each part 256-byte aligned.
static inline long round256(long b) { return (b + 255) / 256 * 256; }

// Split-K factor of a chunk's dHidden GEMM: enough workgroups to cover the CUs.
static inline int ce_dh_splits(long chunk, long d, long vocab) {
  const long tiles = (long)cdiv(chunk, 256) * cdiv(d, 256);
  long splits = (256 + tiles - 1) / tiles;
  const long k_tiles = cdiv(vocab, 64);
  if (splits > 8) splits = 8;
  if (splits > k_tiles / 4) splits = k_tiles / 4;
  return splits < 1 ? 1 : (int)splits;
}

extern "C" int64_t ws_linear_ce_workspace_bytes(int64_t rows, int64_t vocab, int64_t d,
                                                int64_t chunk_rows) {
  const long chunk = chunk_rows < rows ? chunk_rows : rows;
  const int splits = ce_dh_splits(chunk, d, vocab);
  return 256 + round256(chunk * vocab * 2) + (splits > 1 ? round256((long)splits * chunk * d * 4) : 0);
}

extern "C" int ws_linear_ce_backward(const void* hidden, int64_t ld_hidden, const void* weight,
                                     int64_t ld_weight, const void* weight_t,
                                     const int64_t* targets, const float* lse,
                                     const int64_t* count, const float* grad_mean, int64_t rows,
                                     int64_t vocab, int64_t d, void* workspace,
                                     int64_t chunk_rows, void* dhidden, int64_t ld_dhidden,
                                     float* dweight, int64_t ld_dweight, const void* logits,
                                     void* stream) {
  if (int rc = check_ce(hidden, ld_hidden, weight, ld_weight, targets, rows, vocab, d)) return rc;
  if (!lse || !count || !grad_mean || !workspace || !dhidden) return set_error(kInvalid, "null pointer");
  if (chunk_rows < 1 || !fits_i32(chunk_rows * vocab)) return set_error(kInvalid, "bad chunk_rows");
  if (ld_dhidden < d) return set_error(kInvalid, "dhidden leading dimension < d");
  if (dweight && ld_dweight < d) return set_error(kInvalid, "dweight leading dimension < d");
  if (reinterpret_cast<unsigned long>(workspace) % 256) return set_error(kInvalid, "workspace must be 256-byte aligned");
  if (int rc = check_out_stride(vocab, 2, "logit-gradient chunk")) return rc;
  if (logits && (vocab % 4 || reinterpret_cast<unsigned long>(logits) % 16))
    return set_error(kInvalid, "stored logits need vocab %% 4 == 0 and a 16-byte aligned buffer");
  if (int rc = check_out_stride(ld_dhidden, 2, "dhidden")) return rc;
  if (int rc = check_out_stride(d, 4, "dhidden partial")) return rc;
  if (dweight) {
    if (int rc = check_out_stride(ld_dweight, 4, "dweight")) return rc;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long chunk = chunk_rows < rows ? chunk_rows : rows;
  const int splits = ce_dh_splits(chunk, d, vocab);
  auto* base = static_cast<unsigned char*>(workspace);
  float* scale_ws = reinterpret_cast<float*>(base);
  auto* gl = reinterpret_cast<unsigned short*>(base + 256);
  float* partials = reinterpret_cast<float*>(base + 256 + round256(chunk * vocab * 2));
  hipLaunchKernelGGL(ce_scale_kernel, dim3(1), dim3(64), 0, s, grad_mean,
                     reinterpret_cast<const long*>(count), scale_ws);
  if (int rc = hip_check(hipGetLastError(), "ce scale launch")) return rc;
  for (long start = 0; start < rows; start += chunk) {
    const long r = rows - start < chunk ? rows - start : chunk;
    // Logit gradients of this row chunk, r(scale * (softmax - onehot)), BF16.
    GemmParams p{};
    p.a = OperandDesc{static_cast<const unsigned short*>(hidden) + start * ld_hidden, ld_hidden, 1};
    p.b = OperandDesc{static_cast<const unsigned short*>(weight), ld_weight, 1};
    p.M = (int)r; p.N = (int)vocab; p.K = (int)d;
    p.c = gl;
    p.ldc = vocab;
    p.vec_out = (vocab % 4 == 0);
    p.targets = reinterpret_cast<const long*>(targets) + start;
    p.lse = lse + start;
    p.grad_scale = scale_ws;
    int am = operand_mode(p.a, r, d, 256), bm = operand_mode(p.b, vocab, d, 256);
    if (logits) {
      // Logit gradients from the stored logits: one elementwise pass instead of the GEMM.
      const long blocks = r * (long)cdiv(vocab, 2048);
      hipLaunchKernelGGL(ce_grad_logits_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                         static_cast<const unsigned short*>(logits) + start * vocab, (long)vocab,
                         p.targets, p.lse, scale_ws, gl, (long)vocab, (int)r, (int)vocab);
      if (int rc = hip_check(hipGetLastError(), "ce gradient launch")) return rc;
    } else if (fast_ok(p, am, bm, false)) {
      if (int rc = dispatch_fast<false, FEpiCEGrad>(p, am, bm, LaunchCfg{0, 1}, s)) return rc;
    } else if (int rc = dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, false, EpiCEGrad>(
                   p, am, bm, LaunchCfg{0, 1}, s)) {
      return rc;
    }
    // Head weight gradient of the chunk: dW [vocab, d] += f32(r(G^T @ hidden_chunk)).
    if (dweight) {
      GemmParams w{};
      w.a = OperandDesc{gl, 1, vocab};  // G^T [vocab, r]: vocab contiguous
      w.b = OperandDesc{static_cast<const unsigned short*>(hidden) + start * ld_hidden, 1, ld_hidden};
      w.M = (int)vocab; w.N = (int)d; w.K = (int)r;
      w.g = dweight;
      w.ldg = ld_dweight;
      w.round_acc = 1;
      w.vec_out = (d % 4 == 0) && (ld_dweight % 4 == 0) && (reinterpret_cast<unsigned long>(dweight) % 16 == 0);
      const int wa = operand_mode(w.a, vocab, r, 256), wb = operand_mode(w.b, d, r, 256);
      if (fast_ok(w, wa, wb, false)) {
        if (int rc = dispatch_fast<false, FEpiAccF32<false>>(w, wa, wb, LaunchCfg{0, 1}, s)) return rc;
      } else if (int rc = dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiAccF32<false>>(
                     w, wa, wb, LaunchCfg{0, 1}, s)) {
        return rc;
      }
    }
    // dHidden of the chunk: r(G [r, vocab] @ W [vocab, d]), split over the vocab.
    GemmParams q{};
    q.a = OperandDesc{gl, vocab, 1};
    // B [vocab, d]: the head weight (d contiguous) or its transpose (vocab contiguous).
    q.b = weight_t ? OperandDesc{static_cast<const unsigned short*>(weight_t), vocab, 1}
                   : OperandDesc{static_cast<const unsigned short*>(weight), 1, ld_weight};
    q.M = (int)r; q.N = (int)d; q.K = (int)vocab;
    unsigned short* out = static_cast<unsigned short*>(dhidden) + start * ld_dhidden;
    int qa = operand_mode(q.a, r, vocab, 256), qb = operand_mode(q.b, d, vocab, 256);
    q.vec_out = (d % 4 == 0) && (ld_dhidden % 4 == 0) && (reinterpret_cast<unsigned long>(out) % 8 == 0);
    const bool fast = fast_ok(q, qa, qb, false);
    if (splits > 1 && fast) {
      q.g = partials;
      q.ldg = d;
      q.split_stride = chunk * d;
      q.vec_out = (d % 4 == 0);
      if (int rc = dispatch_fast<false, FEpiAccF32<true>>(q, qa, qb, LaunchCfg{0, splits}, s)) return rc;
      const long total = r * d;
      hipLaunchKernelGGL(splitk_bf16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                         partials, splits, (long)(chunk * d), out, (long)ld_dhidden, (int)r, (int)d);
      if (int rc = hip_check(hipGetLastError(), "split-K reduce launch")) return rc;
    } else {
      q.c = out;
      q.ldc = ld_dhidden;
      q.vec_out = (d % 4 == 0) && (ld_dhidden % 4 == 0) && (reinterpret_cast<unsigned long>(out) % 8 == 0);
      if (fast) {
        if (int rc = dispatch_fast<false, FEpiStore<false, false>>(q, qa, qb, LaunchCfg{0, 1}, s)) return rc;
      } else if (int rc = dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiStore<false, false>>(
                     q, qa, qb, LaunchCfg{0, 1}, s)) {
        return rc;
      }
    }
  }
  return kOk;
}
