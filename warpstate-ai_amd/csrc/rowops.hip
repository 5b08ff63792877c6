// C ABI: standalone SwiGLU and RMSNorm kernels (ops/activation_execution.py).
#include <mutex>

#include "../../include/warpstate_hip.h"
#include "launch.h"
#include "rowops.h"

namespace ws {
int launch_rmsnorm_rows(const void* x, long ldx, const float* w, void* y, float* rstd, long m,
                        long k, float eps, bool eager, hipStream_t s);
}

using namespace ws;

extern "C" int ws_swiglu_forward(const void* packed, void* out, int64_t rows, int64_t h,
                                 int eager_rounding, void* stream) {
  if (!packed || !out) return set_error(kInvalid, "null pointer");
  if (rows < 0 || h < 1 || !fits_i32(h)) return set_error(kInvalid, "invalid SwiGLU shape");
  const long total = rows * h;
  if (total == 0) return kOk;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (h % 8 == 0 && al(packed, 16) && al(out, 16)) {
    const long chunks = total / 8;
    const dim3 grid((unsigned)((chunks + 255) / 256));
    const auto* pk = static_cast<const unsigned short*>(packed);
    auto* o = static_cast<unsigned short*>(out);
    if (eager_rounding)
      hipLaunchKernelGGL(swiglu_fwd_vec_kernel<true>, grid, dim3(256), 0, s, pk, o, chunks, (int)h);
    else
      hipLaunchKernelGGL(swiglu_fwd_vec_kernel<false>, grid, dim3(256), 0, s, pk, o, chunks, (int)h);
    return hip_check(hipGetLastError(), "swiglu forward launch");
  }
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(packed),
                     static_cast<unsigned short*>(out), total, (int)h, eager_rounding ? 1 : 0);
  return hip_check(hipGetLastError(), "swiglu forward launch");
}

extern "C" int ws_swiglu_backward(const void* packed, const void* grad, void* out, int64_t rows,
                                  int64_t h, int eager_rounding, void* stream) {
  if (!packed || !grad || !out) return set_error(kInvalid, "null pointer");
  if (rows < 0 || h < 1 || !fits_i32(h)) return set_error(kInvalid, "invalid SwiGLU shape");
  const long total = rows * h;
  if (total == 0) return kOk;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (h % 8 == 0 && al(packed, 16) && al(grad, 16) && al(out, 16)) {
    const long chunks = total / 8;
    const dim3 grid((unsigned)((chunks + 255) / 256));
    const auto* pk = static_cast<const unsigned short*>(packed);
    const auto* g = static_cast<const unsigned short*>(grad);
    auto* o = static_cast<unsigned short*>(out);
    if (eager_rounding)
      hipLaunchKernelGGL(swiglu_bwd_vec_kernel<true>, grid, dim3(256), 0, s, pk, g, o, chunks, (int)h);
    else
      hipLaunchKernelGGL(swiglu_bwd_vec_kernel<false>, grid, dim3(256), 0, s, pk, g, o, chunks, (int)h);
    return hip_check(hipGetLastError(), "swiglu backward launch");
  }
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(packed),
                     static_cast<const unsigned short*>(grad), static_cast<unsigned short*>(out),
                     total, (int)h, eager_rounding ? 1 : 0);
  return hip_check(hipGetLastError(), "swiglu backward launch");
}

extern "C" int ws_rmsnorm_forward(const void* x, const float* weight, void* y, float* rstd,
                                  int64_t rows, int64_t d, float eps, int eager_rounding,
                                  void* stream) {
  if (!x || !weight || !y || !rstd) return set_error(kInvalid, "null pointer");
  if (rows < 0 || d < 1 || !fits_i32(rows) || !fits_i32(d)) return set_error(kInvalid, "invalid RMSNorm shape");
  if (rows == 0) return kOk;
  // The kernels of the fused projection's row pass (eager rounding), in either mode.
  return launch_rmsnorm_rows(x, d, weight, y, rstd, rows, d, eps, eager_rounding != 0,
                             static_cast<hipStream_t>(stream));
}

// Rows per block of the RMSNorm backward: 32 for rows of up to 2048 columns (8 waves, one
// row each at a time); for wider rows (one row per block at a time) the largest power of two
// from 4 to 32 that still gives at least 512 blocks (measured against 256 and 1024 at
// 4096 to 8192 columns: 512 blocks was fastest or tied at every shape).
static int rms_rows_per_block(int64_t rows, int64_t d) {
  if (d <= 2048) return kRmsRowsPerBlock;
  int rpb = 4;
  while (rpb < 32 && rows / (2 * rpb) >= 512) rpb *= 2;
  return rpb;
}

extern "C" int64_t ws_rmsnorm_backward_partial_floats(int64_t rows, int64_t d) {
  return (int64_t)cdiv(rows, rms_rows_per_block(rows, d)) * d;
}

template <int SEGS>
static int launch_rms_bwd(const void* x, const float* weight, const float* rstd, const void* grad,
                          void* dx, float* partial, int rows, int d, int eager, hipStream_t s) {
  // The waves' partial rows, and for the vector kernel the weight row.
  const int lds = (kRmsWaves + (SEGS > 0 ? 1 : 0)) * d * (int)sizeof(float);
  auto launch = [&](auto kernel) {
    if (int rc = ensure_lds(reinterpret_cast<const void*>(kernel), lds)) return rc;
    hipLaunchKernelGGL(kernel, dim3(cdiv(rows, kRmsRowsPerBlock)), dim3(64 * kRmsWaves), lds, s,
                       static_cast<const unsigned short*>(x), weight, rstd,
                       static_cast<const unsigned short*>(grad), static_cast<unsigned short*>(dx),
                       partial, rows, d);
    return hip_check(hipGetLastError(), "rmsnorm backward launch");
  };
  if constexpr (SEGS == 0)
    return eager ? launch(&rmsnorm_bwd_generic_kernel<true>) : launch(&rmsnorm_bwd_generic_kernel<false>);
  else
    return eager ? launch(&rmsnorm_bwd_kernel<SEGS, true>) : launch(&rmsnorm_bwd_kernel<SEGS, false>);
}

template <typename Kernel>
static int launch_rms_bwd_wide(Kernel kernel, const void* x, const float* weight,
                               const float* rstd, const void* grad, void* dx, float* partial,
                               int rows, int d, int rpb, hipStream_t s) {
  hipLaunchKernelGGL(kernel, dim3(cdiv(rows, rpb)), dim3(256), 0, s,
                     static_cast<const unsigned short*>(x), weight, rstd,
                     static_cast<const unsigned short*>(grad), static_cast<unsigned short*>(dx),
                     partial, rows, d, rpb);
  return hip_check(hipGetLastError(), "rmsnorm backward launch");
}

// The row kernels for a width. Up to 2048 columns: one wave per row, the vector kernel
// (SEGS 512-column segments) when d % 8 == 0 and x, grad and dx are 16-byte aligned, else
// the generic one. Wider rows: one block per row, the vector kernel (V 2048-column chunks)
// or the generic one (J columns per thread).
template <bool EAGER>
static int rms_bwd_wide(const void* x, const float* weight, const float* rstd, const void* grad,
                        void* dx, float* partial, int rows, int d, bool vec, hipStream_t s) {
  const int rpb = rms_rows_per_block(rows, d);
  auto run = [&](auto kernel) {
    return launch_rms_bwd_wide(kernel, x, weight, rstd, grad, dx, partial, rows, d, rpb, s);
  };
  if (vec) return d <= 4096 ? run(&rmsnorm_bwd_wide_kernel<2, EAGER>) : run(&rmsnorm_bwd_wide_kernel<4, EAGER>);
  return d <= 4096 ? run(&rmsnorm_bwd_wide_generic_kernel<16, EAGER>)
                   : run(&rmsnorm_bwd_wide_generic_kernel<32, EAGER>);
}

static int rmsnorm_backward(const void* x, const float* weight, const float* rstd,
                            const void* grad, void* dx, float* dweight, float* partial,
                            int64_t rows, int64_t d, int eager_rounding, void* stream) {
  if (!x || !weight || !rstd || !grad || !dx || !dweight || !partial)
    return set_error(kInvalid, "null pointer");
  if (rows < 1 || d < 1 || !fits_i32(rows) || !fits_i32(d)) return set_error(kInvalid, "invalid RMSNorm shape");
  if (d > 8192) return set_error(kInvalid, "RMSNorm backward takes rows of at most 8192 columns (got %ld)", (long)d);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int e = eager_rounding ? 1 : 0;
  // The vector kernels read x and grad and write dx as 16-byte pieces of 8 columns.
  const unsigned long a = reinterpret_cast<unsigned long>(x) | reinterpret_cast<unsigned long>(grad) |
                          reinterpret_cast<unsigned long>(dx);
  const bool vec = d % 8 == 0 && a % 16 == 0;
  const int r = (int)rows, w = (int)d, segs = cdiv(d, 512);
  int rc;
  if (d > 2048)
    rc = e ? rms_bwd_wide<true>(x, weight, rstd, grad, dx, partial, r, w, vec, s)
           : rms_bwd_wide<false>(x, weight, rstd, grad, dx, partial, r, w, vec, s);
  else if (!vec) rc = launch_rms_bwd<0>(x, weight, rstd, grad, dx, partial, r, w, e, s);
  else if (segs <= 1) rc = launch_rms_bwd<1>(x, weight, rstd, grad, dx, partial, r, w, e, s);
  else if (segs <= 2) rc = launch_rms_bwd<2>(x, weight, rstd, grad, dx, partial, r, w, e, s);
  else rc = launch_rms_bwd<4>(x, weight, rstd, grad, dx, partial, r, w, e, s);
  if (rc) return rc;
  const int groups = cdiv(rows, rms_rows_per_block(rows, d));
  const bool vec_reduce = d % 4 == 0 && reinterpret_cast<unsigned long>(partial) % 16 == 0;
  hipLaunchKernelGGL(vec_reduce ? rms_weight_reduce_kernel<true> : rms_weight_reduce_kernel<false>,
                     dim3(cdiv(d, kRmsReduceCols)), dim3(256), 0, s, partial, dweight, groups,
                     (int)d, e);
  return hip_check(hipGetLastError(), "rmsnorm weight reduce launch");
}

extern "C" int ws_rmsnorm_backward(const void* x, const float* weight, const float* rstd,
                                   const void* grad, void* dx, float* dweight, float* partial,
                                   int64_t rows, int64_t d, int eager_rounding, void* stream) {
  return rmsnorm_backward(x, weight, rstd, grad, dx, dweight, partial, rows, d, eager_rounding,
                          stream);
}

// ---------------------------------------------------------------------------------------
// Allocation-free RMSNorm backward. Its weight-gradient partials live in `scratch`, a
// file-scope device array that every GPU the library runs on holds until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory: its device address
// comes from hipGetSymbolAddress, once per device (with that device current), and only
// that address is passed to kernels. The kernels write every partial they later read, so
// the array needs no clearing; calls that overlap on one GPU share it and race.
namespace {

constexpr long kStaticPartialFloats = 1L << 20;  // 4 MiB: rows x d up to 2^25 at d % 8 == 0
constexpr int kStaticMaxWidth = 8192;  // the widest row any RMSNorm backward kernel takes
__device__ __align__(256) float scratch[kStaticPartialFloats];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices];

int scratch_partials(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(kHipError, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kScratchDevices) return set_error(kInvalid, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(kHipError, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

}  // namespace

extern "C" int64_t ws_rmsnorm_backward_static_max_partial_floats(void) {
  return kStaticPartialFloats;
}

extern "C" int ws_rmsnorm_backward_static(const void* x, const float* weight, const float* rstd,
                                          const void* grad, void* dx, float* dweight,
                                          int64_t rows, int64_t d, int eager_rounding,
                                          void* stream) {
  if (rows < 1 || d < 1 || !fits_i32(rows) || !fits_i32(d))
    return set_error(kInvalid, "invalid RMSNorm shape");
  // Checked here, before any device call (the row kernels take at most 8192 columns; none
  // of them uses private scratch memory, which the HIP runtime would have to allocate).
  if (d > kStaticMaxWidth)
    return set_error(kInvalid,
                     "the allocation-free RMSNorm backward takes rows of at most %d columns "
                     "(got %ld)",
                     kStaticMaxWidth, (long)d);
  const long need = ws_rmsnorm_backward_partial_floats(rows, d);
  if (need > kStaticPartialFloats)
    return set_error(kInvalid,
                     "RMSNorm backward of %ld x %ld needs %ld partial floats; the static scratch "
                     "holds %ld (use ws_rmsnorm_backward with a workspace)",
                     (long)rows, (long)d, need, kStaticPartialFloats);
  float* partial = nullptr;
  if (int rc = scratch_partials(&partial)) return rc;
  return rmsnorm_backward(x, weight, rstd, grad, dx, dweight, partial, rows, d, eager_rounding,
                          stream);
}

extern "C" int ws_transpose_bf16(const void* in, int64_t ld_in, void* out, int64_t rows,
                                 int64_t cols, void* stream) {
  if (!in || !out) return set_error(kInvalid, "null pointer");
  if (rows < 1 || cols < 1 || !fits_i32(rows) || !fits_i32(cols) || ld_in < cols)
    return set_error(kInvalid, "invalid transpose shape");
  // Row blocks of 64 run along the grid's y dimension (at most 65535 blocks).
  if (cdiv(rows, 64) > 65535)
    return set_error(kInvalid, "transpose of %ld rows exceeds 4194240", (long)rows);
  const unsigned long pi = reinterpret_cast<unsigned long>(in), po = reinterpret_cast<unsigned long>(out);
  const int vec = rows % 8 == 0 && cols % 8 == 0 && ld_in % 8 == 0 && pi % 16 == 0 && po % 16 == 0;
  if (vec) {
    hipLaunchKernelGGL(transpose_bf16_reg_kernel, dim3(cdiv(cols, 256), cdiv(rows, 64)), dim3(256),
                       0, static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(in),
                       (long)ld_in, static_cast<unsigned short*>(out), (int)rows, (int)cols);
    return hip_check(hipGetLastError(), "transpose launch");
  }
  hipLaunchKernelGGL(transpose_bf16_kernel, dim3(cdiv(cols, 64), cdiv(rows, 64)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(in),
                     (long)ld_in, static_cast<unsigned short*>(out), (int)rows, (int)cols);
  return hip_check(hipGetLastError(), "transpose launch");
}

extern "C" int ws_sigmoid_backward_cols(const void* dout, int64_t ld_dout, const void* out,
                                        int64_t ld_out, void* dp, int64_t ld_dp, int64_t rows,
                                        int64_t cols, int64_t gate_begin, int64_t gate_end,
                                        void* stream) {
  if (!dout || !out || !dp) return set_error(kInvalid, "null pointer");
  if (rows < 1 || cols < 1 || !fits_i32(rows) || !fits_i32(cols) || ld_dout < cols ||
      ld_out < cols || ld_dp < cols)
    return set_error(kInvalid, "invalid gradient shape");
  if (gate_begin < 0 || gate_end < gate_begin || gate_end > cols)
    return set_error(kInvalid, "gate column range [%ld, %ld) outside [0, %ld)", (long)gate_begin,
                     (long)gate_end, (long)cols);
  // In place only the gate columns change; otherwise every column is written.
  const bool in_place = dp == dout && ld_dp == ld_dout;
  long c0 = in_place ? gate_begin : 0, c1 = in_place ? gate_end : cols;
  if (in_place) {  // widen to whole 8-column groups so the vector path applies
    c0 = c0 / 8 * 8;
    c1 = (c1 + 7) / 8 * 8 < cols ? (c1 + 7) / 8 * 8 : cols;
  }
  if (c1 <= c0) return kOk;
  const unsigned long a = reinterpret_cast<unsigned long>(dout) | reinterpret_cast<unsigned long>(out) |
                          reinterpret_cast<unsigned long>(dp);
  const int vec = a % 16 == 0 && ld_dout % 8 == 0 && ld_out % 8 == 0 && ld_dp % 8 == 0 &&
                  c0 % 8 == 0 && (c1 - c0) % 8 == 0;
  const long threads = vec ? rows * ((c1 - c0) / 8) : rows * (c1 - c0);
  hipLaunchKernelGGL(sigmoid_backward_cols_kernel, dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const unsigned short*>(dout), (long)ld_dout,
                     static_cast<const unsigned short*>(out), (long)ld_out,
                     static_cast<unsigned short*>(dp), (long)ld_dp, (int)rows, (int)c0, (int)c1,
                     (int)gate_begin, (int)gate_end, vec);
  return hip_check(hipGetLastError(), "sigmoid backward launch");
}
