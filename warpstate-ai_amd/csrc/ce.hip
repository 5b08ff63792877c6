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
    if (int rc = dispatch_fast<false, FEpiCEStatsLogits>(p, am, bm, kFusedCfg, s)) return rc;
  } else if (fast_ok(p, am, bm, false)) {
    if (int rc = dispatch_fast<false, FEpiCEStats>(p, am, bm, kFusedCfg, s)) return rc;
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

// --- per-chunk pieces shared by the backward and the fused pass -------------------------

// Operand descriptors of one row chunk [start, start + r) of the LM head.
struct CeChunk {
  const unsigned short* hidden;  // first row of the chunk
  long ld_hidden;
  long start, r;
};

// Logit gradients of the chunk, r(scale * (softmax - onehot)), BF16 into gl [r, vocab]:
// recomputing GEMM with the gradient epilogue, or, with `logits` (the chunk's stored BF16
// logits, row stride vocab, may equal gl), one elementwise pass over them.
static int ce_chunk_gradients(const CeChunk& c, const void* weight, long ld_weight, long vocab,
                              long d, const int64_t* targets, const float* lse,
                              const float* scale, const unsigned short* logits,
                              unsigned short* gl, const int* skip, hipStream_t s) {
  const long* tg = reinterpret_cast<const long*>(targets) + c.start;
  if (logits) {
    const long blocks = c.r * (long)cdiv(vocab, 2048);
    hipLaunchKernelGGL(ce_grad_logits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, logits,
                       (long)vocab, tg, lse + c.start, scale, gl, (long)vocab, (int)c.r,
                       (int)vocab);
    return hip_check(hipGetLastError(), "ce gradient launch");
  }
  GemmParams p{};
  p.a = OperandDesc{c.hidden, c.ld_hidden, 1};
  p.b = OperandDesc{static_cast<const unsigned short*>(weight), ld_weight, 1};
  p.M = (int)c.r; p.N = (int)vocab; p.K = (int)d;
  p.c = gl;
  p.ldc = vocab;
  p.vec_out = (vocab % 4 == 0);
  p.targets = tg;
  p.lse = lse + c.start;
  p.grad_scale = scale;
  p.skip_if = skip;
  int am = operand_mode(p.a, c.r, d, 256), bm = operand_mode(p.b, vocab, d, 256);
  if (fast_ok(p, am, bm, false)) return dispatch_fast<false, FEpiCEGrad>(p, am, bm, kFusedCfg, s);
  return dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, false, EpiCEGrad>(p, am, bm,
                                                                          LaunchCfg{0, 1}, s);
}

// Head weight gradient of the chunk: dW [vocab, d] += f32(r(G^T @ hidden_chunk)).
static int ce_chunk_weight_grad(const CeChunk& c, const unsigned short* gl, long vocab, long d,
                                float* dweight, long ld_dweight, const int* skip, hipStream_t s) {
  GemmParams w{};
  w.a = OperandDesc{gl, 1, vocab};  // G^T [vocab, r]: vocab contiguous
  w.b = OperandDesc{c.hidden, 1, c.ld_hidden};
  w.M = (int)vocab; w.N = (int)d; w.K = (int)c.r;
  w.g = dweight;
  w.ldg = ld_dweight;
  w.round_acc = 1;
  w.skip_if = skip;
  w.vec_out = (d % 4 == 0) && (ld_dweight % 4 == 0) && (reinterpret_cast<unsigned long>(dweight) % 16 == 0);
  const int wa = operand_mode(w.a, vocab, c.r, 256), wb = operand_mode(w.b, d, c.r, 256);
  if (fast_ok(w, wa, wb, false))
    return dispatch_fast<false, FEpiAccF32<false>>(w, wa, wb, LaunchCfg{0, 1}, s);
  return dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiAccF32<false>>(w, wa, wb,
                                                                       LaunchCfg{0, 1}, s);
}

// dHidden of the chunk: r(G [r, vocab] @ W [vocab, d]) into out (row stride ld_out), split
// over the vocabulary through FP32 partials when one chunk alone would not fill the GPU.
static int ce_chunk_dhidden(const CeChunk& c, const unsigned short* gl, const void* weight,
                            long ld_weight, const void* weight_t, long vocab, long d,
                            int splits, long chunk, float* partials, unsigned short* out,
                            long ld_out, const int* skip, hipStream_t s) {
  GemmParams q{};
  q.a = OperandDesc{gl, vocab, 1};
  // B [vocab, d]: the head weight (d contiguous) or its transpose (vocab contiguous).
  q.b = weight_t ? OperandDesc{static_cast<const unsigned short*>(weight_t), vocab, 1}
                 : OperandDesc{static_cast<const unsigned short*>(weight), 1, ld_weight};
  q.M = (int)c.r; q.N = (int)d; q.K = (int)vocab;
  q.skip_if = skip;
  int qa = operand_mode(q.a, c.r, vocab, 256), qb = operand_mode(q.b, d, vocab, 256);
  if (splits > 1) {
    // FP32 slices of the vocabulary through the workspace, on the fast kernel when the
    // operands allow it and on the generic one otherwise (a vocabulary that is not a
    // multiple of 8 leaves the logit-gradient rows without 16-byte alignment): with few
    // row tiles an unsplit launch would run the whole vocabulary on a handful of CUs.
    q.g = partials;
    q.ldg = d;
    q.split_stride = chunk * d;
    q.vec_out = (d % 4 == 0);
    const int rc = fast_ok(q, qa, qb, false)
                       ? dispatch_fast<false, FEpiAccF32<true>>(q, qa, qb, LaunchCfg{0, splits}, s)
                       : dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiAccF32<true>>(
                             q, qa, qb, LaunchCfg{0, splits}, s);
    if (rc) return rc;
    const long total = c.r * d;
    hipLaunchKernelGGL(splitk_bf16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       partials, splits, (long)(chunk * d), out, ld_out, (int)c.r, (int)d, skip);
    return hip_check(hipGetLastError(), "split-K reduce launch");
  }
  q.vec_out = (d % 4 == 0) && (ld_out % 4 == 0) && (reinterpret_cast<unsigned long>(out) % 8 == 0);
  q.c = out;
  q.ldc = ld_out;
  if (fast_ok(q, qa, qb, false)) return dispatch_fast<false, FEpiStore<false, false>>(q, qa, qb, kFusedCfg, s);
  return dispatch<kMaskMM, WS_TILE_ARGS_LARGE, false, EpiStore<false, false>>(q, qa, qb,
                                                                             LaunchCfg{0, 1}, s);
}

static int check_backward_args(long rows, long vocab, long d, long chunk_rows,
                               const void* workspace, long ld_dhidden, const float* dweight,
                               long ld_dweight) {
  if (chunk_rows < 1 || !fits_i32(chunk_rows * vocab)) return set_error(kInvalid, "bad chunk_rows");
  if (ld_dhidden < d) return set_error(kInvalid, "dhidden leading dimension < d");
  if (dweight && ld_dweight < d) return set_error(kInvalid, "dweight leading dimension < d");
  if (reinterpret_cast<unsigned long>(workspace) % 256) return set_error(kInvalid, "workspace must be 256-byte aligned");
  if (int rc = check_out_stride(vocab, 2, "logit-gradient chunk")) return rc;
  if (int rc = check_out_stride(ld_dhidden, 2, "dhidden")) return rc;
  if (int rc = check_out_stride(d, 4, "dhidden partial")) return rc;
  if (dweight) {
    if (int rc = check_out_stride(ld_dweight, 4, "dweight")) return rc;
  }
  return kOk;
}

// The two-pass backward's chunk loop; with `skip` (a device flag) every kernel of it exits
// at once when the flag is set.
static int ce_backward_chunks(const void* hidden, long ld_hidden, const void* weight,
                              long ld_weight, const void* weight_t, const int64_t* targets,
                              const float* lse, const int64_t* count, const float* grad_mean,
                              long rows, long vocab, long d, void* workspace, long chunk_rows,
                              void* dhidden, long ld_dhidden, float* dweight, long ld_dweight,
                              const void* logits, const int* skip, hipStream_t s) {
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
    const CeChunk c{static_cast<const unsigned short*>(hidden) + start * ld_hidden, ld_hidden,
                    start, rows - start < chunk ? rows - start : chunk};
    const auto* stored = logits ? static_cast<const unsigned short*>(logits) + start * vocab : nullptr;
    if (int rc = ce_chunk_gradients(c, weight, ld_weight, vocab, d, targets, lse, scale_ws,
                                    stored, gl, skip, s))
      return rc;
    if (dweight) {
      if (int rc = ce_chunk_weight_grad(c, gl, vocab, d, dweight, ld_dweight, skip, s)) return rc;
    }
    if (int rc = ce_chunk_dhidden(c, gl, weight, ld_weight, weight_t, vocab, d, splits, chunk,
                                  partials, static_cast<unsigned short*>(dhidden) + start * ld_dhidden,
                                  ld_dhidden, skip, s))
      return rc;
  }
  return kOk;
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
  if (int rc = check_backward_args(rows, vocab, d, chunk_rows, workspace, ld_dhidden, dweight,
                                   ld_dweight))
    return rc;
  if (logits && (vocab % 4 || reinterpret_cast<unsigned long>(logits) % 16))
    return set_error(kInvalid, "stored logits need vocab %% 4 == 0 and a 16-byte aligned buffer");
  return ce_backward_chunks(hidden, ld_hidden, weight, ld_weight, weight_t, targets, lse, count,
                            grad_mean, rows, vocab, d, workspace, chunk_rows, dhidden, ld_dhidden,
                            dweight, ld_dweight, logits, nullptr, static_cast<hipStream_t>(stream));
}

// Loss, mean and the gradient of the mean for a unit upstream gradient, one row chunk at a
// time: the chunk's logits GEMM keeps its BF16 logits in the workspace chunk (the whole
// [rows, vocab] logits never exist), their row statistics give the chunk's lse and loss,
// one elementwise pass turns the stored logits into r((softmax - onehot) / count) in place,
// and those feed the chunk's dHidden (and head-weight) GEMMs. Operands that the stored
// logits' epilogue cannot take recompute the chunk's logits instead.
extern "C" int ws_linear_ce_fused(const void* hidden, int64_t ld_hidden, const void* weight,
                                  int64_t ld_weight, const void* weight_t, const int64_t* targets,
                                  int64_t rows, int64_t vocab, int64_t d, float* part_max,
                                  float* part_sum, float* target_logit, float* lse, float* loss,
                                  float* mean, int64_t* count, void* workspace,
                                  int64_t chunk_rows, void* dhidden, int64_t ld_dhidden,
                                  float* dweight, int64_t ld_dweight, void* stream) {
  if (int rc = check_ce(hidden, ld_hidden, weight, ld_weight, targets, rows, vocab, d)) return rc;
  if (!part_max || !part_sum || !target_logit || !lse || !loss || !mean || !count || !workspace ||
      !dhidden)
    return set_error(kInvalid, "null pointer");
  if (int rc = check_backward_args(rows, vocab, d, chunk_rows, workspace, ld_dhidden, dweight,
                                   ld_dweight))
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long chunk = chunk_rows < rows ? chunk_rows : rows;
  const int splits = ce_dh_splits(chunk, d, vocab);
  const int parts = (int)ws_linear_ce_parts(vocab);
  auto* base = static_cast<unsigned char*>(workspace);
  float* scale_ws = reinterpret_cast<float*>(base);
  auto* gl = reinterpret_cast<unsigned short*>(base + 256);
  float* partials = reinterpret_cast<float*>(base + 256 + round256(chunk * vocab * 2));
  const long* tg = reinterpret_cast<const long*>(targets);
  // 1 / max(1, count) first: every chunk's gradients need the whole batch's count.
  hipLaunchKernelGGL(ce_count_kernel, dim3(1), dim3(1024), 0, s, tg, (int)rows,
                     reinterpret_cast<long*>(count), scale_ws);
  if (int rc = hip_check(hipGetLastError(), "ce count launch")) return rc;
  for (long start = 0; start < rows; start += chunk) {
    const CeChunk c{static_cast<const unsigned short*>(hidden) + start * ld_hidden, ld_hidden,
                    start, rows - start < chunk ? rows - start : chunk};
    GemmParams p{};
    p.a = OperandDesc{c.hidden, ld_hidden, 1};
    p.b = OperandDesc{static_cast<const unsigned short*>(weight), ld_weight, 1};
    p.M = (int)c.r; p.N = (int)vocab; p.K = (int)d;
    p.targets = tg + start;
    p.part_max = part_max + start * parts;
    p.part_sum = part_sum + start * parts;
    p.tgt_logit = target_logit + start;
    p.parts_per_row = parts;
    p.vec_out = 1;
    const int am = operand_mode(p.a, c.r, d, 256), bm = operand_mode(p.b, vocab, d, 256);
    const bool store = vocab % 4 == 0 && fast_ok(p, am, bm, false);
    if (store) {
      p.c = gl;
      p.ldc = vocab;
      if (int rc = dispatch_fast<false, FEpiCEStatsLogits>(p, am, bm, kFusedCfg, s)) return rc;
    } else if (fast_ok(p, am, bm, false)) {
      if (int rc = dispatch_fast<false, FEpiCEStats>(p, am, bm, kFusedCfg, s)) return rc;
    } else if (int rc = dispatch<kMaskKK | kMaskGG, WS_TILE_ARGS_LARGE, false, EpiCEStats>(
                   p, am, bm, LaunchCfg{0, 1}, s)) {
      return rc;
    }
    hipLaunchKernelGGL(ce_combine_kernel, dim3(cdiv(c.r, 4)), dim3(256), 0, s, p.part_max,
                       p.part_sum, parts, p.tgt_logit, p.targets, lse + start, loss + start,
                       (int)c.r, (int)vocab);
    if (int rc = hip_check(hipGetLastError(), "ce combine launch")) return rc;
    if (int rc = ce_chunk_gradients(c, weight, ld_weight, vocab, d, targets, lse, scale_ws,
                                    store ? gl : nullptr, gl, nullptr, s))
      return rc;
    if (dweight) {
      if (int rc = ce_chunk_weight_grad(c, gl, vocab, d, dweight, ld_dweight, nullptr, s)) return rc;
    }
    if (int rc = ce_chunk_dhidden(c, gl, weight, ld_weight, weight_t, vocab, d, splits, chunk,
                                  partials, static_cast<unsigned short*>(dhidden) + start * ld_dhidden,
                                  ld_dhidden, nullptr, s))
      return rc;
  }
  hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(1024), 0, s, loss, tg, (int)rows, mean,
                     reinterpret_cast<long*>(count));
  return hip_check(hipGetLastError(), "ce mean launch");
}

// Backward of the fused pass. When grad_mean is a power of two, scaling commutes with every
// rounding of the gradients, so dhidden = grad_mean * dhidden_unit and dweight += grad_mean *
// dweight_unit are the two-pass backward's results bit for bit (dweight up to the order in
// which its chunk sums meet a nonzero buffer). Otherwise the two-pass backward runs. The
// choice is made on the device (ce_exact_scale_kernel): both paths are launched and the
// one not taken exits at once, so the call never synchronises with the host.
extern "C" int ws_linear_ce_fused_backward(
    const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
    const void* weight_t, const int64_t* targets, const float* lse, const int64_t* count,
    const float* grad_mean, int64_t rows, int64_t vocab, int64_t d, void* workspace,
    int64_t chunk_rows, const void* dhidden_unit, int64_t ld_unit, const float* dweight_unit,
    void* dhidden, int64_t ld_dhidden, float* dweight, void* stream) {
  if (int rc = check_ce(hidden, ld_hidden, weight, ld_weight, targets, rows, vocab, d)) return rc;
  if (!lse || !count || !grad_mean || !workspace || !dhidden || !dhidden_unit)
    return set_error(kInvalid, "null pointer");
  if ((dweight == nullptr) != (dweight_unit == nullptr))
    return set_error(kInvalid, "dweight and dweight_unit come together");
  if (ld_unit < d) return set_error(kInvalid, "dhidden_unit leading dimension < d");
  if (int rc = check_backward_args(rows, vocab, d, chunk_rows, workspace, ld_dhidden, dweight, d))
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int* exact = reinterpret_cast<int*>(static_cast<unsigned char*>(workspace) + 64);
  hipLaunchKernelGGL(ce_exact_scale_kernel, dim3(1), dim3(64), 0, s, grad_mean, exact);
  if (int rc = hip_check(hipGetLastError(), "ce exact-scale check launch")) return rc;
  const unsigned long al16 = reinterpret_cast<unsigned long>(dhidden_unit) |
                             reinterpret_cast<unsigned long>(dhidden);
  const int vec = d % 8 == 0 && ld_unit % 8 == 0 && ld_dhidden % 8 == 0 && al16 % 16 == 0;
  const long threads = vec ? rows * (d / 8) : rows * d;
  hipLaunchKernelGGL(scale_bf16_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     s, grad_mean, static_cast<const unsigned short*>(dhidden_unit), (long)ld_unit,
                     static_cast<unsigned short*>(dhidden), (long)ld_dhidden, (int)rows, (int)d,
                     vec, exact);
  if (int rc = hip_check(hipGetLastError(), "dhidden scale launch")) return rc;
  if (dweight) {
    const long wt = vocab * d;
    hipLaunchKernelGGL(scale_add_f32_kernel, dim3((unsigned)((wt + 255) / 256)), dim3(256), 0, s,
                       grad_mean, dweight_unit, dweight, wt, exact);
    if (int rc = hip_check(hipGetLastError(), "dweight scale launch")) return rc;
  }
  return ce_backward_chunks(hidden, ld_hidden, weight, ld_weight, weight_t, targets, lse, count,
                            grad_mean, rows, vocab, d, workspace, chunk_rows, dhidden, ld_dhidden,
                            dweight, d, nullptr, exact, s);
}

// The forward's second phase alone: per-row lse and loss from the statistics partials, then
// the mean over valid tokens and their count (what ws_linear_ce_forward runs after its
// logits GEMM; also the step after an exchange of partials between vocabulary shards).
extern "C" int ws_linear_ce_combine(const float* part_max, const float* part_sum,
                                    const float* target_logit, const int64_t* targets,
                                    float* lse, float* loss, float* mean, int64_t* count,
                                    int64_t rows, int64_t vocab, void* stream) {
  if (!part_max || !part_sum || !target_logit || !targets || !lse || !loss || !mean || !count)
    return set_error(kInvalid, "null pointer");
  if (rows < 1 || vocab < 1 || !fits_i32(rows) || !fits_i32(vocab))
    return set_error(kInvalid, "invalid LM-head sizes rows=%ld vocab=%ld", (long)rows, (long)vocab);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long* tg = reinterpret_cast<const long*>(targets);
  hipLaunchKernelGGL(ce_combine_kernel, dim3(cdiv(rows, 4)), dim3(256), 0, s, part_max, part_sum,
                     (int)ws_linear_ce_parts(vocab), target_logit, tg, lse, loss, (int)rows,
                     (int)vocab);
  if (int rc = hip_check(hipGetLastError(), "ce combine launch")) return rc;
  hipLaunchKernelGGL(ce_mean_kernel, dim3(1), dim3(1024), 0, s, loss, tg, (int)rows, mean,
                     reinterpret_cast<long*>(count));
  return hip_check(hipGetLastError(), "ce mean launch");
}

// Logit gradients from BF16 logits [rows, vocab] (row stride ld_logits, may be `out`):
// out = r(scale * (exp(l - lse) - onehot)), zero rows for ignored targets; `scale` is a
// device scalar (grad_mean / max(1, count)). The elementwise pass of the fused loss.
extern "C" int ws_linear_ce_logit_grad(const void* logits, int64_t ld_logits,
                                       const int64_t* targets, const float* lse,
                                       const float* scale, void* out, int64_t ld_out,
                                       int64_t rows, int64_t vocab, void* stream) {
  if (!logits || !targets || !lse || !scale || !out) return set_error(kInvalid, "null pointer");
  if (rows < 1 || vocab < 1 || !fits_i32(rows) || !fits_i32(vocab) || ld_logits < vocab ||
      ld_out < vocab)
    return set_error(kInvalid, "invalid logit shape");
  const unsigned long a = reinterpret_cast<unsigned long>(logits) | reinterpret_cast<unsigned long>(out);
  if (vocab % 4 || ld_logits % 8 || ld_out % 8 || a % 16)
    return set_error(kInvalid, "logit gradients need vocab %% 4 == 0, 16-byte rows and buffers");
  const long blocks = rows * (long)cdiv(vocab, 2048);
  hipLaunchKernelGGL(ce_grad_logits_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(logits),
                     (long)ld_logits, reinterpret_cast<const long*>(targets), lse, scale,
                     static_cast<unsigned short*>(out), (long)ld_out, (int)rows, (int)vocab);
  return hip_check(hipGetLastError(), "ce gradient launch");
}
