// C ABI: standalone SwiGLU and RMSNorm kernels (ops/activation_execution.py).
#include "../../include/warpstate_hip.h"
#include "launch.h"
#include "rowops.h"

using namespace ws;

extern "C" int ws_swiglu_forward(const void* packed, void* out, int64_t rows, int64_t h,
                                 int eager_rounding, void* stream) {
  if (!packed || !out) return set_error(kInvalid, "null pointer");
  if (rows < 0 || h < 1 || !fits_i32(h)) return set_error(kInvalid, "invalid SwiGLU shape");
  const long total = rows * h;
  if (total == 0) return kOk;
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
  hipLaunchKernelGGL(rmsnorm_fwd_kernel, dim3(cdiv(rows, 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(x), weight,
                     static_cast<unsigned short*>(y), rstd, (int)rows, (int)d, eps,
                     eager_rounding ? 1 : 0);
  return hip_check(hipGetLastError(), "rmsnorm forward launch");
}

extern "C" int64_t ws_rmsnorm_backward_partial_floats(int64_t rows, int64_t d) {
  return (int64_t)cdiv(rows, 4) * d;
}

extern "C" int ws_rmsnorm_backward(const void* x, const float* weight, const float* rstd,
                                   const void* grad, void* dx, float* dweight, float* partial,
                                   int64_t rows, int64_t d, int eager_rounding, void* stream) {
  if (!x || !weight || !rstd || !grad || !dx || !dweight || !partial)
    return set_error(kInvalid, "null pointer");
  if (rows < 1 || d < 1 || !fits_i32(rows) || !fits_i32(d)) return set_error(kInvalid, "invalid RMSNorm shape");
  if (d * 4 * 4 > 160 * 1024) return set_error(kInvalid, "RMSNorm width %ld exceeds the LDS budget", (long)d);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int groups = cdiv(rows, 4);
  const int lds = (int)(4 * d * sizeof(float));
  if (int rc = ensure_lds(reinterpret_cast<const void*>(&rmsnorm_bwd_kernel), lds)) return rc;
  hipLaunchKernelGGL(rmsnorm_bwd_kernel, dim3(groups), dim3(256), lds, s,
                     static_cast<const unsigned short*>(x), weight, rstd,
                     static_cast<const unsigned short*>(grad), static_cast<unsigned short*>(dx),
                     partial, (int)rows, (int)d, eager_rounding ? 1 : 0);
  if (int rc = hip_check(hipGetLastError(), "rmsnorm backward launch")) return rc;
  hipLaunchKernelGGL(rms_weight_reduce_kernel, dim3(cdiv(d, 256)), dim3(256), 0, s, partial,
                     dweight, groups, (int)d, eager_rounding ? 1 : 0);
  return hip_check(hipGetLastError(), "rmsnorm weight reduce launch");
}

extern "C" int ws_transpose_bf16(const void* in, int64_t ld_in, void* out, int64_t rows,
                                 int64_t cols, void* stream) {
  if (!in || !out) return set_error(kInvalid, "null pointer");
  if (rows < 1 || cols < 1 || !fits_i32(rows) || !fits_i32(cols) || ld_in < cols)
    return set_error(kInvalid, "invalid transpose shape");
  const unsigned long pi = reinterpret_cast<unsigned long>(in), po = reinterpret_cast<unsigned long>(out);
  const int vec = rows % 8 == 0 && cols % 8 == 0 && ld_in % 8 == 0 && pi % 16 == 0 && po % 16 == 0;
  hipLaunchKernelGGL(transpose_bf16_kernel, dim3(cdiv(cols, 64), cdiv(rows, 64)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned short*>(in),
                     (long)ld_in, static_cast<unsigned short*>(out), (int)rows, (int)cols, vec);
  return hip_check(hipGetLastError(), "transpose launch");
}
