/*
 * warpstate_hip.h -- C ABI of the MI355X (gfx950) BF16 matmul hot path of WarpState.
 *
 * Every entry point takes raw device pointers, element strides and sizes, plus the
 * hipStream_t to launch on (passed as void*; from Python it is
 * torch.cuda.current_stream().cuda_stream of the calling thread). The library launches
 * work on that stream and returns; it never allocates, frees or synchronises. The caller
 * allocates every output and workspace. Outputs must not alias inputs, except the FP32
 * gradient buffers of ws_mm_accumulate_f32 and ws_mm_accumulate_f32_group (updated in
 * place) and the output of
 * ws_sigmoid_backward_cols (which may be its dout).
 *
 * Return value: 0 on success, 1 for an invalid argument (nothing was launched), 2 for a
 * HIP runtime error. ws_last_error() returns the calling thread's last message.
 *
 * Size limits: sizes are positive 32-bit integers. Kernels address a 256-row output tile
 * with 32-bit offsets from the tile's first row, so 256 rows of every output must span
 * less than 2 GiB (a BF16 row stride below 4,194,303 elements, an FP32 one below
 * 2,097,151); wider outputs are rejected with status 1. Operands past the corresponding
 * bound take a slower loader with 64-bit addresses instead.
 *
 * Numerics: BF16 operands, FP32 accumulation in MFMA, BF16 round-to-nearest-even
 * outputs, at the rounding points of the reference's PyTorch path.
 *
 * `algorithm` (GEMM entry points): 0 = "tiled" (one workgroup per output tile),
 * 1 = "persistent" (one resident workgroup per CU slot striding over tiles),
 * 2 = "persistent_tma" (persistent, with the reference's TMA preconditions checked by the
 * caller). `tile`: 0 = 256x256 macro-tile (8 waves), 1 = 128x128 macro-tile (4 waves).
 *
 * Reference citations are path:line in gtausa197-svg/WarpState-AI.
 */
#ifndef WARPSTATE_HIP_H
#define WARPSTATE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" if none). */
const char* ws_last_error(void);

/* Library version string. */
const char* ws_version(void);

/*
 * C[m,n] = bf16(A[m,k] @ B[k,n]), C row-contiguous with leading dimension n.
 * A element (i,j) at a + i*a_s0 + j*a_s1, B element (i,j) at b + i*b_s0 + j*b_s1; any
 * positive strides. Replaces the kernel launches of launch_mm
 * (ops/matmul_kernels.py:167-205): `_matmul_kernel` (:81-108) for "tiled"/"persistent"
 * and `warpstate::persistent_tma_mm` (:135-159) for "persistent_tma".
 */
int ws_mm(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0, int64_t b_s1,
          void* c, int64_t m, int64_t n, int64_t k, int algorithm, int tile, void* stream);

/*
 * Paired up/gate projection with SwiGLU epilogue: packed[m, 2h] = bf16(A @ B) (up in
 * columns [0,h), gate in [h,2h)), act[m,h] = bf16(r?(silu(gate)) * up), where silu runs
 * on the BF16-rounded gate and is itself rounded iff eager_rounding. Replaces the launch
 * of `_paired_swiglu_mm_kernel` in launch_swiglu_mm (ops/matmul_epilogue.py:86-142).
 */
int ws_swiglu_mm(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0,
                 int64_t b_s1, void* packed, void* act, int64_t m, int64_t h, int64_t k,
                 int eager_rounding, int algorithm, int tile, void* stream);

/* Standalone SwiGLU of a contiguous packed [rows, 2h] BF16 projection; replaces
 * bf16_swiglu (ops/activation_execution.py:58-70). */
int ws_swiglu_forward(const void* packed, void* out, int64_t rows, int64_t h, int eager_rounding,
                      void* stream);

/* SwiGLU backward: out[rows, 2h] = (dUp | dGate) from packed [rows, 2h] and contiguous
 * grad [rows, h]; replaces `_swiglu_backward` (ops/activation_execution.py:73-81). */
int ws_swiglu_backward(const void* packed, const void* grad, void* out, int64_t rows, int64_t h,
                       int eager_rounding, void* stream);

/* BF16 RMSNorm forward of contiguous x [rows, d] with FP32 weight; writes y and the FP32
 * row rsqrt; replaces bf16_rmsnorm (ops/activation_execution.py:161-173). */
int ws_rmsnorm_forward(const void* x, const float* weight, void* y, float* rstd, int64_t rows,
                       int64_t d, float eps, int eager_rounding, void* stream);

/* Floats of the `partial` workspace ws_rmsnorm_backward needs: one partial row of d floats
 * per 32 rows up to d = 2048, per 4 to 32 rows (depending on the row count) above. */
int64_t ws_rmsnorm_backward_partial_floats(int64_t rows, int64_t d);

/* RMSNorm backward: dx [rows, d] BF16 and dweight [d] FP32 from x, weight, rstd and a
 * contiguous grad; replaces `_rms_backward` (ops/activation_execution.py:176-194). Any
 * width d <= 8192 and any buffer alignment (d % 8 == 0 with 16-byte aligned x, grad and dx
 * takes the vector kernel, everything else a generic one with the same arithmetic). */
int ws_rmsnorm_backward(const void* x, const float* weight, const float* rstd, const void* grad,
                        void* dx, float* dweight, float* partial, int64_t rows, int64_t d,
                        int eager_rounding, void* stream);

/* Allocation-free variant of ws_rmsnorm_backward: the same kernels and results, with the
 * weight-gradient partials in a static 4 MiB device array of the library instead of a
 * caller workspace. No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It calls no allocator, and none of its row kernels uses runtime-allocated
 * private memory. Limits: d <= 8192 and ws_rmsnorm_backward_partial_floats(rows, d) <=
 * ws_rmsnorm_backward_static_max_partial_floats() (2^20; e.g. 16384 x 2048); larger
 * sizes return an error. Each GPU holds its own copy of the array until the process
 * ends; calls that overlap on one GPU share it and race. */
int ws_rmsnorm_backward_static(const void* x, const float* weight, const float* rstd,
                               const void* grad, void* dx, float* dweight, int64_t rows,
                               int64_t d, int eager_rounding, void* stream);

/* Partial floats the static scratch of ws_rmsnorm_backward_static holds. */
int64_t ws_rmsnorm_backward_static_max_partial_floats(void);

/* out[cols, rows] = transpose(in[rows, cols]) for BF16 (in has row stride ld_in, out is
 * contiguous). Used to give weight-side GEMM operands a contiguous reduction dimension:
 * the input gradient dX = dY @ W (ops/matmul_execution.py:239) then reads W^T rows.
 * No reference counterpart (a layout step of this implementation). */
int ws_transpose_bf16(const void* in, int64_t ld_in, void* out, int64_t rows, int64_t cols,
                      void* stream);

/*
 * RMSNorm-prologue projection with gate sigmoid: out[m,n] = bf16(y @ B) with
 * y = r(r(x * rstd) * r(norm_weight)), then out[:, gate_begin:gate_end] = r(sigmoid(out)).
 * The prologue is one pass over x that writes y into `normed` [m, k] (row-contiguous,
 * caller-allocated; it is also the saved input of the projection's weight gradient) and
 * rstd [m]; the GEMM then reads y. Restates RMSNorm.forward (warpstate/model.py:22-28) ->
 * in_proj (warpstate/model.py:93, 109) -> torch.sigmoid on the gate slice
 * (warpstate/model.py:174). x needs a unit column stride.
 */
int ws_rmsnorm_gate_mm(const void* x, int64_t x_s0, const float* norm_weight, float eps,
                       float* rstd, void* normed, const void* b, int64_t b_s0, int64_t b_s1,
                       void* out, int64_t m, int64_t n, int64_t k, int64_t gate_begin,
                       int64_t gate_end, void* stream);

/* Gradient through the gate sigmoid of ws_rmsnorm_gate_mm's output: dp = dout, except
 * columns [gate_begin, gate_end) where dp = r(dout * (1 - out) * out) with `out` the forward
 * output (torch.sigmoid's backward, warpstate/model.py:174). dp may be dout itself (then
 * only the gate columns are rewritten). */
int ws_sigmoid_backward_cols(const void* dout, int64_t ld_dout, const void* out, int64_t ld_out,
                             void* dp, int64_t ld_dp, int64_t rows, int64_t cols,
                             int64_t gate_begin, int64_t gate_end, void* stream);

/* Down projection with residual add: out[m,n] = r(residual[m,n] + r(A @ B)), residual
 * row stride ld_residual (warpstate/model.py:178 under BF16 residuals,
 * ops/residual_experiment.py:25-58). */
int ws_residual_mm(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0,
                   int64_t b_s1, const void* residual, int64_t ld_residual, void* out, int64_t m,
                   int64_t n, int64_t k, void* stream);

/*
 * Down-projection dgrad with SwiGLU-backward epilogue: dact = r(grad @ B) (grad [m,k] =
 * dY, B [k,h] = W_down of nn.Linear layout [k,h]) is never stored; from the saved packed
 * [m,2h] projection it writes dpacked [m,2h] = (dUp | dGate). Restates `_mm_backward`'s
 * dX (ops/matmul_execution.py:239) followed by `_swiglu_backward_kernel`
 * (ops/activation_execution.py:36-55).
 */
int ws_swiglu_backward_mm(const void* grad, int64_t g_s0, int64_t g_s1, const void* b,
                          int64_t b_s0, int64_t b_s1, const void* packed, void* dpacked,
                          int64_t m, int64_t h, int64_t k, int eager_rounding, void* stream);

/* Floats of the workspace ws_mm_accumulate_f32 needs for an [m, n] gradient with
 * reduction k and `splits` (0 when splits <= 1), on the current device. */
int64_t ws_mm_accumulate_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t splits);

/*
 * Weight-gradient GEMM accumulated into an FP32 buffer: G[m,n] += f32(r(A @ B)) when
 * round_bf16 (the BF16 dW then AccumulateGrad of test_gradient_execution.py:243-246 and
 * ops/matmul_execution.py:243), or G += A @ B in FP32 otherwise (the "direct_fp32_addmm"
 * variant of ops/benchmark_gradient_accumulation.py:141-144). splits > 1 lets the
 * reduction be split through `workspace`: for operands with a contiguous reduction or row
 * dimension the 256 x 256 tiles that fill whole rounds of the GPU accumulate directly and
 * the remaining tiles' k-range is shared evenly by all compute units (FP32 partial sums,
 * added in k order, rounded once); other layouts use `splits` even k-slices.
 */
int ws_mm_accumulate_f32(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0,
                         int64_t b_s1, float* g, int64_t ldg, int64_t m, int64_t n, int64_t k,
                         int round_bf16, float* workspace, int64_t splits, void* stream);

/* One weight gradient of a grouped accumulation: G[m, n] (row stride ldg) += A[m, k] B[k, n],
 * with A and B given by pointer and (row, column) element strides as in ws_mm. */
typedef struct ws_accumulate_problem {
  const void* a;
  int64_t a_s0, a_s1;
  const void* b;
  int64_t b_s0, b_s1;
  float* g;
  int64_t ldg;
  int64_t m, n;
} ws_accumulate_problem;

/* Floats of the workspace ws_mm_accumulate_f32_group needs for these problems (0 when
 * none), on the current device. */
int64_t ws_mm_accumulate_group_workspace_floats(const ws_accumulate_problem* problems, int count,
                                                int64_t k);

/*
 * Up to four weight-gradient accumulations with the same reduction length k (the token
 * count) in one launch, each with the numerics of ws_mm_accumulate_f32 (round_bf16 as
 * there): the weight gradients of one backward stage, computed together instead of as
 * separate AccumulateGrad steps (ops/matmul_execution.py:243 once per weight; fused, new).
 * Their 256 x 256 tiles form one raster: whole rounds of the GPU run directly, the rest
 * is shared evenly by all compute units through `workspace`, so a gradient with fewer
 * tiles than compute units fills the GPU together with the others. The gradients must not
 * overlap. When the problems' operand layouts differ or do not take the fast loader, the
 * call runs ws_mm_accumulate_f32 per problem (split-K through `workspace` when given).
 */
int ws_mm_accumulate_f32_group(const ws_accumulate_problem* problems, int count, int64_t k,
                               int round_bf16, float* workspace, void* stream);

/*
 * G = f32(r(A @ B)) (or the FP32 product when round_bf16 is 0): ws_mm_accumulate_f32 and
 * ws_mm_accumulate_f32_group with the gradient buffers written instead of updated, so
 * they need no clearing and are never read. Same arguments, workspace sizes
 * (ws_mm_accumulate_workspace_floats, ws_mm_accumulate_group_workspace_floats) and
 * paths. This is the BF16 weight gradient of F.linear under autocast widened to FP32,
 * the value AccumulateGrad adds to an FP32 master's .grad
 * (ops/matmul_execution.py:243; test_gradient_execution.py:243-246), produced in one
 * FP32 pass for an adapter that returns it through autograd (new).
 */
int ws_mm_store_f32(const void* a, int64_t a_s0, int64_t a_s1, const void* b, int64_t b_s0,
                    int64_t b_s1, float* g, int64_t ldg, int64_t m, int64_t n, int64_t k,
                    int round_bf16, float* workspace, int64_t splits, void* stream);
int ws_mm_store_f32_group(const ws_accumulate_problem* problems, int count, int64_t k,
                          int round_bf16, float* workspace, void* stream);

/* Number of per-row partials (floats per row of part_max / part_sum) for `vocab`. */
int64_t ws_linear_ce_parts(int64_t vocab);

/*
 * Fused LM-head cross-entropy forward. hidden [rows, d] (row stride ld_hidden, unit column
 * stride), weight [vocab, d] (nn.Embedding / tied head layout, row stride ld_weight),
 * int64 targets with -100 ignored. Writes per-token FP32 loss, lse, the target logit,
 * mean = sum(loss) / max(1, count) and the int64 valid-token count. `logits` (nullable): when given, the rounded
 * BF16 logits are also stored there ([rows, vocab], row stride vocab; vocab % 4 == 0,
 * 16-byte aligned; both operands row-contiguous) for a backward that reads them instead
 * of recomputing the GEMM. Without it the logits exist only in registers.
 * Restates the chunked head of WarpStateLM.forward (warpstate/model.py:316-334) and
 * `_full_loss` (ops/loss_experiment.py:14-19).
 */
int ws_linear_ce_forward(const void* hidden, int64_t ld_hidden, const void* weight,
                         int64_t ld_weight, const int64_t* targets, int64_t rows, int64_t vocab,
                         int64_t d, float* part_max, float* part_sum, float* target_logit,
                         float* lse, float* loss, float* mean, int64_t* count, void* logits,
                         void* stream);

/* Bytes of the workspace ws_linear_ce_backward needs for `chunk_rows`-row chunks. */
int64_t ws_linear_ce_workspace_bytes(int64_t rows, int64_t vocab, int64_t d, int64_t chunk_rows);

/*
 * Fused LM-head cross-entropy backward: dhidden [rows, d] = r(r(g (softmax - onehot)) @ W)
 * with g = grad_mean / max(1, count), zero rows for ignored targets. Rows are processed
 * chunk_rows at a time: the BF16 logit gradients of one chunk ([chunk_rows, vocab], never
 * the whole batch) go to the 256-byte aligned `workspace` and feed that chunk's dHidden
 * GEMM, split over the vocab with FP32 partials when the chunk alone would not fill the
 * GPU. `weight_t` (nullable) is the head weight transposed, [d, vocab] contiguous; when
 * given, the dHidden GEMM reads it instead of `weight`. `dweight` (nullable, FP32
 * [vocab, d], row stride ld_dweight) receives the tied head weight's gradient, accumulated
 * per chunk as dweight += f32(r(G_chunk^T @ hidden_chunk)): the BF16 weight gradient of the
 * chunk's F.linear followed by FP32 accumulation (warpstate/model.py:321-331 under BF16
 * autocast, test_gradient_execution.py:243-246). `logits` (nullable): the logits the
 * forward stored; each chunk's logit gradients then come from one elementwise pass over
 * them (same arithmetic, same bits) instead of a recomputing GEMM. Restates autograd of
 * warpstate/model.py:321-334.
 */
int ws_linear_ce_backward(const void* hidden, int64_t ld_hidden, const void* weight,
                          int64_t ld_weight, const void* weight_t, const int64_t* targets,
                          const float* lse, const int64_t* count, const float* grad_mean,
                          int64_t rows, int64_t vocab, int64_t d, void* workspace,
                          int64_t chunk_rows, void* dhidden, int64_t ld_dhidden, float* dweight,
                          int64_t ld_dweight, const void* logits, void* stream);

/*
 * Fused LM-head cross-entropy in one pass: the outputs of ws_linear_ce_forward plus the
 * gradients for a unit upstream gradient of the mean, dhidden [rows, d] BF16 and (nullable)
 * dweight [vocab, d] FP32 (+=), with the numerics of ws_linear_ce_backward at grad_mean = 1.
 * Rows go chunk_rows at a time through the workspace of ws_linear_ce_workspace_bytes: the
 * chunk's logits GEMM stores its BF16 logits in the workspace chunk (the whole [rows, vocab]
 * logits never exist), the chunk's row statistics give its lse and loss, one elementwise
 * pass turns the stored logits into the logit gradients in place, and they feed the
 * chunk's dHidden and head-weight GEMMs: one logits GEMM per row instead of the forward's
 * and the backward's. `weight_t` as in ws_linear_ce_backward. Restates
 * warpstate/model.py:316-334 with its autograd.
 */
int ws_linear_ce_fused(const void* hidden, int64_t ld_hidden, const void* weight,
                       int64_t ld_weight, const void* weight_t, const int64_t* targets,
                       int64_t rows, int64_t vocab, int64_t d, float* part_max, float* part_sum,
                       float* target_logit, float* lse, float* loss, float* mean, int64_t* count,
                       void* workspace, int64_t chunk_rows, void* dhidden, int64_t ld_dhidden,
                       float* dweight, int64_t ld_dweight, void* stream);

/*
 * Backward of ws_linear_ce_fused for the actual upstream gradient grad_mean (device FP32
 * scalar): dhidden [rows, d] BF16 (row stride ld_dhidden) and, when given, dweight
 * [vocab, d] FP32 (contiguous, +=). When grad_mean is +-2^e with |e| <= 32, scaling
 * commutes with every rounding that stays in the normal range, and the results are
 * grad_mean * dhidden_unit and dweight + grad_mean * dweight_unit: the two-pass backward's
 * results bit for bit (dweight up to summation order into a nonzero buffer), except for
 * elements that are subnormal before or after the scaling. Otherwise it runs the two-pass
 * backward (ws_linear_ce_backward's arguments). The choice is made on the device, without a host synchronisation: both paths
 * are launched and the kernels of the one not taken exit at once.
 */
int ws_linear_ce_fused_backward(const void* hidden, int64_t ld_hidden, const void* weight,
                                int64_t ld_weight, const void* weight_t, const int64_t* targets,
                                const float* lse, const int64_t* count, const float* grad_mean,
                                int64_t rows, int64_t vocab, int64_t d, void* workspace,
                                int64_t chunk_rows, const void* dhidden_unit, int64_t ld_unit,
                                const float* dweight_unit, void* dhidden, int64_t ld_dhidden,
                                float* dweight, void* stream);

/*
 * The second phase of ws_linear_ce_forward on its own: lse and loss per row from the
 * statistics partials part_max / part_sum ([rows, ws_linear_ce_parts(vocab)]) and the
 * target logits, then mean = sum(loss) / max(1, count) and the int64 count (the combine
 * step of the chunked head, warpstate/model.py:326-334, ops/loss_experiment.py:18-19).
 */
int ws_linear_ce_combine(const float* part_max, const float* part_sum, const float* target_logit,
                         const int64_t* targets, float* lse, float* loss, float* mean,
                         int64_t* count, int64_t rows, int64_t vocab, void* stream);

/*
 * Logit gradients from BF16 logits: out = r(scale (exp(l - lse) - onehot)), zero rows for
 * ignored targets, `scale` a device FP32 scalar; `out` may be `logits` (in place). vocab % 4
 * == 0, row strides multiples of 8, 16-byte aligned buffers. The elementwise pass of the
 * fused loss (autograd of F.cross_entropy on BF16 logits, warpstate/model.py:328-334).
 */
int ws_linear_ce_logit_grad(const void* logits, int64_t ld_logits, const int64_t* targets,
                            const float* lse, const float* scale, void* out, int64_t ld_out,
                            int64_t rows, int64_t vocab, void* stream);

/*
 * Packed attention-backward gradient layout: out [B, N*C, 5*H*D] BF16 (token-major rows of
 * [q | k | v | gate | u], each H*D wide) from the saved head-major [B, N, H, C, D] BF16
 * tensors q_memory, q_local, tanh_k, k_local, v_local, memory, local, gate, u_write, tanh_u,
 * k_write [B, N, H, D, C], grad_y [B, N*C, H*D] and FP32 rope tables sin, cos [C, D]; all
 * contiguous. `scale` multiplies memory in the gate gradient (head_dim^-0.5).
 * `algorithm`: 0 = "profile" (two passes through the caller's head-major BF16 scratch_q and
 * scratch_k, the reference's profiled two-kernel baseline), 1 = "paired" (q/k pass, then
 * v/gate/u pass), 2 = "single" (one pass). All three give identical bits. Replaces the
 * launches of prepare_layout (ops/backward_layout.py:213-276) of the kernels at :116-210.
 */
int ws_backward_layout(const void* q_memory, const void* q_local, const float* sin,
                       const float* cos, const void* k_write, const void* tanh_k,
                       const void* k_local, const void* v_local, const void* grad_y,
                       const void* memory, const void* local, const void* gate,
                       const void* u_write, const void* tanh_u, void* out, int64_t batch,
                       int64_t chunks, int64_t heads, int64_t chunk_size, int64_t head_dim,
                       float scale, int algorithm, void* scratch_q, void* scratch_k,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WARPSTATE_HIP_H */
