// Shared device helpers for the gfx950 (CDNA4) kernels of the BF16 matmul hot path.
//
// Numerics contract (WarpState ops/matmul_kernels.py:1-8, ops/matmul_epilogue.py:70-83):
// BF16 operands, FP32 accumulation, BF16 round-to-nearest-even outputs. Rounding to
// BF16 uses the hardware v_cvt_pk_bf16_f32 conversion (RNE), and exponentials use the
// hardware base-2 exponential v_exp_f32 scaled by log2(e).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef long i64x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

namespace ws {

constexpr int kWave = 64;
// FP32 accumulation mode bits (GemmParams::round_acc and the split-K reductions):
// kAccRound rounds each product to BF16 before it is added, kAccStore stores f32(.) into
// G instead of adding it (G is not read).
enum AccMode { kAccRound = 1, kAccStore = 2 };
// Byte offset that is always beyond a buffer resource's num_records: loads through it
// return zero and stores through it are dropped by the buffer unit.
constexpr unsigned kOOB = 0x80000000u;
// gfx9 raw buffer resource, DATA_FORMAT 32 (the value every gfx9 raw buffer access uses).
constexpr int kRsrcFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes,
                                           kRsrcFlags);
}

__device__ __forceinline__ float bf16_bits_to_f32(unsigned bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float lo_bf16(unsigned word) { return __uint_as_float(word << 16); }
__device__ __forceinline__ float hi_bf16(unsigned word) { return __uint_as_float(word & 0xffff0000u); }

// Two FP32 values -> packed BF16 pair (lo in bits 0..15), RNE.
__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned short to_bf16_bits(float x) {
  __bf16 b = (__bf16)x;
  return __builtin_bit_cast(unsigned short, b);
}
// Round an FP32 value to the nearest BF16 and return it widened back to FP32.
__device__ __forceinline__ float rbf16(float x) { return bf16_bits_to_f32(to_bf16_bits(x)); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// e^x through the hardware 2^x.
__device__ __forceinline__ float exp_e(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
// Natural log through the hardware log2.
__device__ __forceinline__ float log_e(float x) { return __builtin_amdgcn_logf(x) * kLn2; }

// Logistic sigmoid 1 / (1 + e^-x) (ops/activation_execution.py:45) with the hardware
// reciprocal v_rcp_f32 (1 ulp) in place of an IEEE division; the difference is far below
// the BF16 rounding every result of it goes through.
__device__ __forceinline__ float sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + exp_e(-x));
}
// SiLU g / (1 + e^-g) (ops/matmul_epilogue.py:80), as g times that reciprocal.
__device__ __forceinline__ float silu(float g) { return g * sigmoid(g); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__host__ __device__ constexpr int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

}  // namespace ws
