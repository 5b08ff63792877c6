// Row-wise and elementwise kernels of the hot path: RMSNorm forward / backward,
// standalone SwiGLU forward / backward, cross-entropy reductions and split-K reductions.
// All are HBM-bound; each reads and writes its operands once.
#pragma once

#include "common.h"

namespace ws {

// ---------------------------------------------------------------------------------------
// RMSNorm of x (row stride ldx) into a contiguous BF16 y; also stores rstd
// (warpstate/model.py:25-28, ops/activation_execution.py:96-110). EAGER is the eager
// rounding of RMSNorm.forward, y = r(r(x * rstd) * r(w)); without it y = r(x * rstd * w)
// with the product in FP32 (the compiled path). One wave per row; with `vec`, 16-byte loads
// and stores of 8 elements per lane. EAGER is a template argument: tested at run time, the
// compiler computes every element both ways and selects.
template <bool EAGER>
__device__ __forceinline__ float rms_out(float xv, float r, float wv) {
  return EAGER ? rbf16(xv * r) * rbf16(wv) : (xv * r) * wv;
}

template <bool EAGER>
static __global__ void __launch_bounds__(256) rmsnorm_rows_kernel(
    const unsigned short* __restrict__ x, long ldx, const float* __restrict__ w,
    unsigned short* __restrict__ y, float* __restrict__ rstd, int rows, int D, float eps,
    int vec) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const unsigned short* xr = x + (long)row * ldx;
  unsigned short* yr = y + (long)row * D;
  float acc = 0.0f;
  if (vec) {
    for (int c = lane * 8; c < D; c += 64 * 8) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xr + c);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float a = lo_bf16(v[d]), b = hi_bf16(v[d]);
        acc += a * a;
        acc += b * b;
      }
    }
  } else {
    for (int c = lane; c < D; c += 64) {
      const float a = bf16_bits_to_f32(xr[c]);
      acc += a * a;
    }
  }
  acc = wave_sum(acc);
  const float r = 1.0f / sqrtf(acc / (float)D + eps);
  if (vec) {
    for (int c = lane * 8; c < D; c += 64 * 8) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xr + c);
      const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(w + c);
      const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(w + c + 4);
      const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
      u32x4_t o;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        o[d] = pack_bf16x2(rms_out<EAGER>(lo_bf16(v[d]), r, wv[2 * d]),
                           rms_out<EAGER>(hi_bf16(v[d]), r, wv[2 * d + 1]));
      *reinterpret_cast<u32x4_t*>(yr + c) = o;
    }
  } else {
    for (int c = lane; c < D; c += 64)
      yr[c] = to_bf16_bits(rms_out<EAGER>(bf16_bits_to_f32(xr[c]), r, w[c]));
  }
  if (lane == 0) rstd[row] = r;
}

// rmsnorm_rows_kernel for vector rows of at most 512 NC elements: each lane keeps its NC
// 16-byte chunks of the row in registers (all loads in flight at once), so x is read
// once. Same sums in the same order, so the same bits as rmsnorm_rows_kernel.
template <int NC, bool EAGER>
static __global__ void __launch_bounds__(256) rmsnorm_rows_reg_kernel(
    const unsigned short* __restrict__ x, long ldx, const float* __restrict__ w,
    unsigned short* __restrict__ y, float* __restrict__ rstd, int rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const unsigned short* xr = x + (long)row * ldx;
  unsigned short* yr = y + (long)row * D;
  u32x4_t v[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane * 8 + i * 512;
    v[i] = c < D ? *reinterpret_cast<const u32x4_t*>(xr + c) : u32x4_t{0, 0, 0, 0};
  }
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = lo_bf16(v[i][d]), b = hi_bf16(v[i][d]);
      acc += a * a;
      acc += b * b;
    }
  acc = wave_sum(acc);
  const float r = 1.0f / sqrtf(acc / (float)D + eps);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane * 8 + i * 512;
    if (c >= D) break;
    const f32x4_t w0 = *reinterpret_cast<const f32x4_t*>(w + c);
    const f32x4_t w1 = *reinterpret_cast<const f32x4_t*>(w + c + 4);
    const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      o[d] = pack_bf16x2(rms_out<EAGER>(lo_bf16(v[i][d]), r, wv[2 * d]),
                         rms_out<EAGER>(hi_bf16(v[i][d]), r, wv[2 * d + 1]));
    *reinterpret_cast<u32x4_t*>(yr + c) = o;
  }
  if (lane == 0) rstd[row] = r;
}

// RMSNorm backward (ops/activation_execution.py:113-141): per row
//   z = r?(x r), dz = r?(dy r?(w)), dr = sum(dz x), dx = dz r + (-0.5 dr r^3 / D) * 2x,
// and the weight-gradient partial sum over this block's rows of r?(dy z) (r? = BF16
// rounding when eager). Rows of up to 2048 columns: one wave per row, 16-byte loads: lane
// l owns columns 8 l + 512 s (s < SEGS), and keeps its x and dy chunks in registers between
// the two passes over the row. A block of kRmsWaves waves takes kRmsRowsPerBlock
// consecutive rows (wave w the rows w, w + kRmsWaves, ...); each wave's weight-gradient
// partial builds up in its own LDS row, and the waves' rows are added in wave order into
// one partial row per block. Wider rows take the block-per-row kernels below.
constexpr int kRmsRowsPerBlock = 32;
constexpr int kRmsWaves = 8;

// The block's partial row: the waves' LDS rows added in wave order.
__device__ __forceinline__ void rms_block_partial(const float* lds_part, float* dw_part, int D) {
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    float v = lds_part[c];
#pragma unroll
    for (int q = 1; q < kRmsWaves; ++q) v += lds_part[q * D + c];
    dw_part[(long)blockIdx.x * D + c] = v;
  }
}

// The partials and the (rounded) weight stay in LDS, not registers, so that the kernel fits
// 128 VGPRs without spills: four waves per SIMD (two blocks per CU) keep twice the rows in
// flight of a 4-wave block holding them in registers. EAGER (the rounding mode) is a
// template argument: tested at run time, the compiler computes every element both ways and
// selects.
template <int SEGS, bool EAGER>
static __global__ void __launch_bounds__(64 * kRmsWaves) __attribute__((amdgpu_waves_per_eu(4)))
rmsnorm_bwd_kernel(const unsigned short* __restrict__ x, const float* __restrict__ w,
                   const float* __restrict__ rstd, const unsigned short* __restrict__ dy,
                   unsigned short* __restrict__ dx, float* __restrict__ dw_part, int rows, int D) {
  extern __shared__ float lds_part[];  // [kRmsWaves][D] partials, then [D] weight
  // The wave index as a scalar, so that row addresses are scalar bases plus one lane offset.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* mine = lds_part + wave * D;
  float* wl = lds_part + kRmsWaves * D;
  for (int c = threadIdx.x; c < D; c += blockDim.x) wl[c] = EAGER ? rbf16(w[c]) : w[c];
#pragma unroll
  for (int s = 0; s < SEGS; ++s) {
    const int c = 8 * lane + 512 * s;
    if (c < D) {
      *reinterpret_cast<f32x4_t*>(mine + c) = f32x4_t{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<f32x4_t*>(mine + c + 4) = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  }
  __syncthreads();

  const int row_end = min(rows, (blockIdx.x + 1) * kRmsRowsPerBlock);
  // One row ahead: the next row's x and dy are requested before this row's reduction.
  // (row is wave-uniform: the row bases are scalar and each lane adds its column offset.)
  auto load = [&](int row, u32x4_t (&xv)[SEGS], u32x4_t (&gv)[SEGS]) {
    const unsigned short* xr = x + (long)row * D;
    const unsigned short* gr = dy + (long)row * D;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      const int c = 8 * lane + 512 * s;
      const bool ok = c < D && row < row_end;
      xv[s] = ok ? *reinterpret_cast<const u32x4_t*>(xr + c) : u32x4_t{0u, 0u, 0u, 0u};
      gv[s] = ok ? *reinterpret_cast<const u32x4_t*>(gr + c) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  // dz = dy * w (rounded when EAGER) for the 8 columns of segment s, evaluated in both
  // passes; columns past D read weight 0 (their dy is 0 too).
  auto dz8 = [&](const u32x4_t& g, int s, float (&dz)[8]) {
    const int c = 8 * lane + 512 * s;
    f32x4_t w0 = {0.f, 0.f, 0.f, 0.f}, w1 = {0.f, 0.f, 0.f, 0.f};
    if (c < D) {
      w0 = *reinterpret_cast<const f32x4_t*>(wl + c);
      w1 = *reinterpret_cast<const f32x4_t*>(wl + c + 4);
    }
    const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      dz[2 * d] = lo_bf16(g[d]) * wv[2 * d];
      dz[2 * d + 1] = hi_bf16(g[d]) * wv[2 * d + 1];
      if (EAGER) { dz[2 * d] = rbf16(dz[2 * d]); dz[2 * d + 1] = rbf16(dz[2 * d + 1]); }
    }
  };
  u32x4_t xn[SEGS], gn[SEGS];
  load(blockIdx.x * kRmsRowsPerBlock + wave, xn, gn);
  for (int row = blockIdx.x * kRmsRowsPerBlock + wave; row < row_end; row += kRmsWaves) {
    const float r = rstd[row];
    u32x4_t xv[SEGS], gv[SEGS];
#pragma unroll
    for (int s = 0; s < SEGS; ++s) { xv[s] = xn[s]; gv[s] = gn[s]; }
    load(row + kRmsWaves, xn, gn);
    float dr = 0.0f;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      float dz[8];
      dz8(gv[s], s, dz);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        dr += dz[2 * d] * lo_bf16(xv[s][d]);
        dr += dz[2 * d + 1] * hi_bf16(xv[s][d]);
      }
    }
    dr = wave_sum(dr);
    const float dsq = (-0.5f * dr * (r * r * r)) / (float)D;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      const int c = 8 * lane + 512 * s;
      if (c >= D) continue;
      float dz[8];
      dz8(gv[s], s, dz);
      f32x4_t p0 = *reinterpret_cast<const f32x4_t*>(mine + c);
      f32x4_t p1 = *reinterpret_cast<const f32x4_t*>(mine + c + 4);
      u32x4_t o;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float v2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float xs = h ? hi_bf16(xv[s][d]) : lo_bf16(xv[s][d]);
          const float gs = h ? hi_bf16(gv[s][d]) : lo_bf16(gv[s][d]);
          v2[h] = dz[2 * d + h] * r + dsq * (2.0f * xs);
          float z = xs * r;
          if (EAGER) z = rbf16(z);
          float pv = gs * z;
          if (EAGER) pv = rbf16(pv);
          const int e = 2 * d + h;
          if (e < 4) p0[e] += pv;
          else p1[e - 4] += pv;
        }
        o[d] = pack_bf16x2(v2[0], v2[1]);
      }
      *reinterpret_cast<f32x4_t*>(mine + c) = p0;
      *reinterpret_cast<f32x4_t*>(mine + c + 4) = p1;
      *reinterpret_cast<u32x4_t*>(dx + (long)row * D + c) = o;
      // One segment's LDS reads at a time: hoisting the next segments' reads would take
      // registers past the 128 of four waves per SIMD.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  rms_block_partial(lds_part, dw_part, D);
}

// The same RMSNorm backward for rows of up to 2048 columns with any width and alignment
// (rows whose width is not a multiple of 8, views at odd offsets): lanes take columns lane,
// lane + 64, ... with 2-byte loads. The arithmetic, the rows of each wave, the order of the
// partial sums and of the waves' addition are the vector kernel's. Only dr, each row's dot
// product, is summed in another order (by column residue instead of by 8-column chunk).
template <bool EAGER>
static __global__ void __launch_bounds__(64 * kRmsWaves) rmsnorm_bwd_generic_kernel(
    const unsigned short* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, const unsigned short* __restrict__ dy,
    unsigned short* __restrict__ dx, float* __restrict__ dw_part, int rows, int D) {
  extern __shared__ float lds_part[];  // [kRmsWaves][D]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* mine = lds_part + wave * D;
  for (int c = lane; c < D; c += 64) mine[c] = 0.0f;
  const int row_end = min(rows, (blockIdx.x + 1) * kRmsRowsPerBlock);
  for (int row = blockIdx.x * kRmsRowsPerBlock + wave; row < row_end; row += kRmsWaves) {
    const float r = rstd[row];
    const unsigned short* xr = x + (long)row * D;
    const unsigned short* gr = dy + (long)row * D;
    float dr = 0.0f;
    for (int c = lane; c < D; c += 64) {
      const float wc = EAGER ? rbf16(w[c]) : w[c];
      float dz = bf16_bits_to_f32(gr[c]) * wc;
      if (EAGER) dz = rbf16(dz);
      dr += dz * bf16_bits_to_f32(xr[c]);
    }
    dr = wave_sum(dr);
    const float dsq = (-0.5f * dr * (r * r * r)) / (float)D;
    for (int c = lane; c < D; c += 64) {
      const float xs = bf16_bits_to_f32(xr[c]), gs = bf16_bits_to_f32(gr[c]);
      const float wc = EAGER ? rbf16(w[c]) : w[c];
      float dz = gs * wc;
      if (EAGER) dz = rbf16(dz);
      dx[(long)row * D + c] = to_bf16_bits(dz * r + dsq * (2.0f * xs));
      float z = xs * r;
      if (EAGER) z = rbf16(z);
      float pv = gs * z;
      if (EAGER) pv = rbf16(pv);
      mine[c] += pv;
    }
  }
  rms_block_partial(lds_part, dw_part, D);
}

// The RMSNorm backward of rows wider than 2048 columns (same arithmetic): a block of 256
// threads takes `rpb` consecutive rows one at a time. Each thread holds its own columns of
// the row; the row's dot product dr is summed per thread, across each wave's lanes and then
// over the four waves (in that order, through LDS); each thread keeps its columns'
// weight-gradient partials in registers over the block's rows (summed in row order) and
// writes them once as the block's partial row. `rpb` (rows per block) is chosen by the
// host from the row count, so that a call has enough blocks to fill the GPU.

// The four waves' lane sums of one row, added in wave order. `red` holds two rows' slots
// (row parity), so one barrier per row suffices: a wave writes a row's slot only after the
// barrier of the previous row, which every wave passes only after reading the slot of the
// row before that.
__device__ __forceinline__ float rms_block_sum(float v, float (*red)[4], int parity, int lane,
                                               int wave) {
  v = wave_sum(v);
  if (lane == 0) red[parity][wave] = v;
  __syncthreads();
  return ((red[parity][0] + red[parity][1]) + red[parity][2]) + red[parity][3];
}

// Wide rows whose width is a multiple of 8, 16-byte aligned x, dy and dx: thread t holds the
// 8-column chunks starting at 8 t + 2048 v (v < V, D <= 2048 V) as 16-byte vectors, and
// the next row's chunks are requested before the current row is reduced. EAGER (the
// rounding mode) is a template argument: tested at run time, the compiler computes every
// element both ways and selects.
template <int V, bool EAGER>
static __global__ void __launch_bounds__(256) rmsnorm_bwd_wide_kernel(
    const unsigned short* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, const unsigned short* __restrict__ dy,
    unsigned short* __restrict__ dx, float* __restrict__ dw_part, int rows, int D,
    int rpb) {
  __shared__ float red[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float wb[V][8], part[V][8];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c = 8 * threadIdx.x + 2048 * v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float wv = c + e < D ? w[c + e] : 0.0f;
      wb[v][e] = EAGER ? rbf16(wv) : wv;
      part[v][e] = 0.0f;
    }
  }
  const int r0 = blockIdx.x * rpb, r1 = min(rows, r0 + rpb);
  auto load = [&](int row, u32x4_t (&xv)[V], u32x4_t (&gv)[V], float& rv) {
    const bool live = row < r1;
    rv = live ? rstd[row] : 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = 8 * threadIdx.x + 2048 * v;
      const bool ok = live && c < D;
      xv[v] = ok ? *reinterpret_cast<const u32x4_t*>(x + (long)row * D + c) : u32x4_t{0u, 0u, 0u, 0u};
      gv[v] = ok ? *reinterpret_cast<const u32x4_t*>(dy + (long)row * D + c) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto reduce_row = [&](int row, const u32x4_t (&xv)[V], const u32x4_t (&gv)[V], float r) {
    float dz[V][8];
    float d = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float dz0 = lo_bf16(gv[v][q]) * wb[v][2 * q], dz1 = hi_bf16(gv[v][q]) * wb[v][2 * q + 1];
        if (EAGER) { dz0 = rbf16(dz0); dz1 = rbf16(dz1); }
        dz[v][2 * q] = dz0;
        dz[v][2 * q + 1] = dz1;
        d += dz0 * lo_bf16(xv[v][q]);
        d += dz1 * hi_bf16(xv[v][q]);
      }
    const float dr = rms_block_sum(d, red, row & 1, lane, wave);
    const float dsq = (-0.5f * dr * (r * r * r)) / (float)D;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = 8 * threadIdx.x + 2048 * v;
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float xs = h ? hi_bf16(xv[v][q]) : lo_bf16(xv[v][q]);
          const float gs = h ? hi_bf16(gv[v][q]) : lo_bf16(gv[v][q]);
          v2[h] = dz[v][2 * q + h] * r + dsq * (2.0f * xs);
          float z = xs * r;
          if (EAGER) z = rbf16(z);
          float pv = gs * z;
          if (EAGER) pv = rbf16(pv);
          part[v][2 * q + h] += pv;
        }
        o[q] = pack_bf16x2(v2[0], v2[1]);
      }
      if (c < D && row < r1) *reinterpret_cast<u32x4_t*>(dx + (long)row * D + c) = o;
    }
  };
  // Two row buffers, used alternately (the loop takes rows in pairs, so each buffer keeps
  // a fixed register name).
  u32x4_t xa[V], ga[V], xb[V], gb[V];
  float ra, rb;
  load(r0, xa, ga, ra);
  for (int row = r0; row < r1; row += 2) {
    load(row + 1, xb, gb, rb);
    reduce_row(row, xa, ga, ra);
    if (row + 1 >= r1) break;  // uniform over the block
    load(row + 2, xa, ga, ra);
    reduce_row(row + 1, xb, gb, rb);
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c = 8 * threadIdx.x + 2048 * v;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (c + e < D) dw_part[(long)blockIdx.x * D + c + e] = part[v][e];
  }
}

// The same for wide rows of any width up to 8192 and any buffer alignment (rows whose
// width is not a multiple of 8, views at odd offsets): thread t takes columns t, t + 256,
// ... (J per thread, D <= 256 J) with 2-byte accesses. The arithmetic and the order of the
// weight-gradient sums are the vector kernel's; only dr, each row's dot product, is summed
// in another order within each thread (by column residue instead of by 8-column chunk).
template <int J, bool EAGER>
static __global__ void __launch_bounds__(256) rmsnorm_bwd_wide_generic_kernel(
    const unsigned short* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, const unsigned short* __restrict__ dy,
    unsigned short* __restrict__ dx, float* __restrict__ dw_part, int rows, int D,
    int rpb) {
  __shared__ float red[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float wb[J], part[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = threadIdx.x + 256 * j;
    const float wv = c < D ? w[c] : 0.0f;
    wb[j] = EAGER ? rbf16(wv) : wv;
    part[j] = 0.0f;
  }
  const int r0 = blockIdx.x * rpb, r1 = min(rows, r0 + rpb);
  for (int row = r0; row < r1; ++row) {
    const float r = rstd[row];
    const unsigned short* xr = x + (long)row * D;
    const unsigned short* gr = dy + (long)row * D;
    float xs[J], gs[J], dz[J];
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = threadIdx.x + 256 * j;
      xs[j] = c < D ? bf16_bits_to_f32(xr[c]) : 0.0f;
      gs[j] = c < D ? bf16_bits_to_f32(gr[c]) : 0.0f;
      dz[j] = gs[j] * wb[j];
      if (EAGER) dz[j] = rbf16(dz[j]);
      d += dz[j] * xs[j];
    }
    const float dr = rms_block_sum(d, red, row & 1, lane, wave);
    const float dsq = (-0.5f * dr * (r * r * r)) / (float)D;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = threadIdx.x + 256 * j;
      float z = xs[j] * r;
      if (EAGER) z = rbf16(z);
      float pv = gs[j] * z;
      if (EAGER) pv = rbf16(pv);
      part[j] += pv;
      if (c < D) dx[(long)row * D + c] = to_bf16_bits(dz[j] * r + dsq * (2.0f * xs[j]));
    }
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = threadIdx.x + 256 * j;
    if (c < D) dw_part[(long)blockIdx.x * D + c] = part[j];
  }
}

// Column sum of the weight-gradient partials (ops/activation_execution.py:144-158). A
// block owns 32 columns: thread (lane g, quad q) sums columns 4q..4q+3 over the partial
// rows g, g + 32, g + 64, ... in order, then the 32 lane sums are added in a fixed
// pairwise tree, so the result is deterministic. VEC reads the four columns as one 16-byte
// vector (D % 4 == 0, part 16-byte aligned); otherwise one at a time, in the same order.
constexpr int kRmsReduceCols = 32, kRmsReduceLanes = 32;
template <bool VEC>
static __global__ void __launch_bounds__(256) rms_weight_reduce_kernel(const float* __restrict__ part,
                                                                float* __restrict__ dw, int groups,
                                                                int D, int eager) {
  __shared__ f32x4_t sums[kRmsReduceLanes][kRmsReduceCols / 4];
  const int q = threadIdx.x & 7, g0 = threadIdx.x >> 3;
  const int c = blockIdx.x * kRmsReduceCols + 4 * q;
  f32x4_t total = {0.0f, 0.0f, 0.0f, 0.0f};
  if (VEC && c < D) {
#pragma unroll 8
    for (int g = g0; g < groups; g += kRmsReduceLanes)
      total += *reinterpret_cast<const f32x4_t*>(part + (long)g * D + c);
  } else if (!VEC) {
    for (int g = g0; g < groups; g += kRmsReduceLanes) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c + e < D) total[e] += part[(long)g * D + c + e];
    }
  }
  sums[g0][q] = total;
  __syncthreads();
#pragma unroll
  for (int width = kRmsReduceLanes / 2; width >= 1; width >>= 1) {
    if (g0 < width) sums[g0][q] += sums[g0 + width][q];
    __syncthreads();
  }
  if (g0 == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < D) dw[c + e] = eager ? rbf16(sums[0][q][e]) : sums[0][q][e];
  }
}

// ---------------------------------------------------------------------------------------
// Standalone SwiGLU forward over a packed [rows, 2H] projection
// (ops/activation_execution.py:22-33): out = r?(silu(gate)) * up.
static __global__ void __launch_bounds__(256) swiglu_fwd_kernel(const unsigned short* __restrict__ packed,
                                                         unsigned short* __restrict__ out,
                                                         long total, int H, int eager) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  long row = i / H, col = i % H;
  long p = row * 2 * H + col;
  float up = bf16_bits_to_f32(packed[p]);
  float gate = bf16_bits_to_f32(packed[p + H]);
  float s = silu(gate);
  if (eager) s = rbf16(s);
  out[i] = to_bf16_bits(s * up);
}

// Standalone SwiGLU backward (ops/activation_execution.py:36-55).
static __global__ void __launch_bounds__(256) swiglu_bwd_kernel(const unsigned short* __restrict__ packed,
                                                         const unsigned short* __restrict__ dyv,
                                                         unsigned short* __restrict__ dx,
                                                         long total, int H, int eager) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  long row = i / H, col = i % H;
  long p = row * 2 * H + col;
  float up = bf16_bits_to_f32(packed[p]);
  float gate = bf16_bits_to_f32(packed[p + H]);
  float dy = bf16_bits_to_f32(dyv[i]);
  float sg = sigmoid(gate);
  float s = silu(gate);
  if (eager) s = rbf16(s);
  float dsilu = dy * up;
  if (eager) dsilu = rbf16(dsilu);
  float dgate = (dsilu * sg) * (1.0f + gate * (1.0f - sg));
  dx[p] = to_bf16_bits(dy * s);
  dx[p + H] = to_bf16_bits(dgate);
}

// The two standalone SwiGLU kernels above with 8 consecutive columns per thread (16-byte
// loads and stores; H % 8 == 0 and 16-byte aligned buffers): the same arithmetic per
// element, so the same bits.
template <bool EAGER>
static __global__ void __launch_bounds__(256) swiglu_fwd_vec_kernel(const unsigned short* __restrict__ packed,
                                                             unsigned short* __restrict__ out,
                                                             long chunks, int H) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= chunks) return;
  const int per_row = H / 8;
  const long row = i / per_row;
  const int c = 8 * (int)(i - row * per_row);
  const unsigned short* pr = packed + row * 2 * H + c;
  const u32x4_t up = *reinterpret_cast<const u32x4_t*>(pr);
  const u32x4_t gate = *reinterpret_cast<const u32x4_t*>(pr + H);
  u32x4_t o;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float s0 = silu(lo_bf16(gate[d])), s1 = silu(hi_bf16(gate[d]));
    if (EAGER) { s0 = rbf16(s0); s1 = rbf16(s1); }
    o[d] = pack_bf16x2(s0 * lo_bf16(up[d]), s1 * hi_bf16(up[d]));
  }
  *reinterpret_cast<u32x4_t*>(out + row * H + c) = o;
}

template <bool EAGER>
static __global__ void __launch_bounds__(256) swiglu_bwd_vec_kernel(const unsigned short* __restrict__ packed,
                                                             const unsigned short* __restrict__ dyv,
                                                             unsigned short* __restrict__ dx,
                                                             long chunks, int H) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= chunks) return;
  const int per_row = H / 8;
  const long row = i / per_row;
  const int c = 8 * (int)(i - row * per_row);
  const long p = row * 2 * H + c;
  const u32x4_t up = *reinterpret_cast<const u32x4_t*>(packed + p);
  const u32x4_t gate = *reinterpret_cast<const u32x4_t*>(packed + p + H);
  const u32x4_t dyw = *reinterpret_cast<const u32x4_t*>(dyv + row * H + c);
  u32x4_t du, dg;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float r_up[2], r_dg[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float u = h ? hi_bf16(up[d]) : lo_bf16(up[d]);
      const float g = h ? hi_bf16(gate[d]) : lo_bf16(gate[d]);
      const float y = h ? hi_bf16(dyw[d]) : lo_bf16(dyw[d]);
      const float sg = sigmoid(g);
      float sl = g * sg;
      if (EAGER) sl = rbf16(sl);
      float dsilu = y * u;
      if (EAGER) dsilu = rbf16(dsilu);
      r_up[h] = y * sl;
      r_dg[h] = (dsilu * sg) * (1.0f + g * (1.0f - sg));
    }
    du[d] = pack_bf16x2(r_up[0], r_up[1]);
    dg[d] = pack_bf16x2(r_dg[0], r_dg[1]);
  }
  *reinterpret_cast<u32x4_t*>(dx + p) = du;
  *reinterpret_cast<u32x4_t*>(dx + p + H) = dg;
}

// ---------------------------------------------------------------------------------------
// Cross-entropy, pass 1 combine: lse[r] = M + log(sum_p s_p e^(m_p - M)) over the
// per-(row, column block) partials; loss[r] = lse - logit[target] for targets != -100,
// else 0 (F.cross_entropy(..., ignore_index=-100, reduction="none") semantics); NaN for a
// target outside [0, vocab) that is not -100.
static __global__ void __launch_bounds__(256) ce_combine_kernel(const float* __restrict__ part_max,
                                                         const float* __restrict__ part_sum,
                                                         int parts, const float* __restrict__ tgt_logit,
                                                         const long* __restrict__ targets,
                                                         float* __restrict__ lse,
                                                         float* __restrict__ loss, int rows,
                                                         int vocab) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* pm = part_max + (long)row * parts;
  const float* ps = part_sum + (long)row * parts;
  float mx = -INFINITY, s = 0.0f;
  // Rows of up to 1024 parts in 16-byte pieces: each lane requests all of its maxima and
  // sums at once (4 consecutive parts per load), so a row costs one memory round trip and
  // the sum runs on the registers. Other rows take one part per lane.
  constexpr int kVec = 4;
  const bool vec = (parts & 3) == 0 && parts <= 256 * kVec &&
                   ((reinterpret_cast<unsigned long>(part_max) |
                     reinterpret_cast<unsigned long>(part_sum)) & 15) == 0;
  if (vec) {
    f32x4_t m4[kVec], s4[kVec];
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int q = 4 * lane + 256 * i;
      const bool ok = q < parts;
      m4[i] = ok ? *reinterpret_cast<const f32x4_t*>(pm + q) : f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      s4[i] = ok ? *reinterpret_cast<const f32x4_t*>(ps + q) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int i = 0; i < kVec; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) mx = fmaxf(mx, m4[i][e]);
    mx = wave_max(mx);
#pragma unroll
    for (int i = 0; i < kVec; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += s4[i][e] * exp_e(m4[i][e] - mx);
  } else {
    for (int q = lane; q < parts; q += 64) mx = fmaxf(mx, pm[q]);
    mx = wave_max(mx);
    for (int q = lane; q < parts; q += 64) s += ps[q] * exp_e(pm[q] - mx);
  }
  s = wave_sum(s);
  if (lane == 0) {
    float l = mx + log_e(s);
    lse[row] = l;
    long t = targets[row];
    // A target outside [0, vocab) that is not -100 has no logit: report NaN.
    loss[row] = (t == -100) ? 0.0f : (t < 0 || t >= vocab) ? __builtin_nanf("") : l - tgt_logit[row];
  }
}

// Mean over valid tokens, sum(loss) / max(1, count(target != -100)) (warpstate/model.py:334,
// ops/loss_experiment.py:18-19). One block; a fixed reduction order makes the FP32 sum
// deterministic. The valid-token count is an integer, exact for any row count; like the
// reference's FP32 / int64 division it is converted to FP32 for the quotient.
static __global__ void __launch_bounds__(1024) ce_mean_kernel(const float* __restrict__ loss,
                                                       const long* __restrict__ targets, int rows,
                                                       float* __restrict__ mean,
                                                       long* __restrict__ count_out) {
  __shared__ float ssum[1024];
  __shared__ long scnt[1024];
  float s = 0.0f;
  long c = 0;
  // Thread t takes rows 4t + 4096 u + 16384 j (u < 4): 16-byte loads of 4 losses and 2 x 2
  // targets, all four pieces of a round requested before any is added, so 16384 rows cost
  // one memory round trip. Rows past the end of a piece are read one by one.
  const bool vec = ((reinterpret_cast<unsigned long>(loss) |
                     reinterpret_cast<unsigned long>(targets)) & 15) == 0;
  for (int base = 4 * (int)threadIdx.x; base < rows; base += 4 * 4096) {
    f32x4_t lv[4];
    long tv[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + 4096 * u;
      if (vec && i + 3 < rows) {
        lv[u] = *reinterpret_cast<const f32x4_t*>(loss + i);
        const i64x2_t t0 = *reinterpret_cast<const i64x2_t*>(targets + i);
        const i64x2_t t1 = *reinterpret_cast<const i64x2_t*>(targets + i + 2);
        tv[u][0] = t0[0]; tv[u][1] = t0[1]; tv[u][2] = t1[0]; tv[u][3] = t1[1];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = i + e < rows;
          lv[u][e] = ok ? loss[i + e] : 0.0f;
          tv[u][e] = ok ? targets[i + e] : -100;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s += lv[u][e];
        c += tv[u][e] != -100 ? 1 : 0;
      }
  }
  ssum[threadIdx.x] = s;
  scnt[threadIdx.x] = c;
  __syncthreads();
  for (int stride = 512; stride > 0; stride >>= 1) {
    if (threadIdx.x < stride) {
      ssum[threadIdx.x] += ssum[threadIdx.x + stride];
      scnt[threadIdx.x] += scnt[threadIdx.x + stride];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const long cnt = scnt[0];
    mean[0] = ssum[0] / (float)(cnt > 1 ? cnt : 1);
    count_out[0] = cnt;
  }
}

// The valid-token count of the whole batch and the unit-upstream-gradient scale
// 1 / max(1, count), before any chunk of the fused pass forms its gradients. One block;
// the targets are read as in ce_mean_kernel.
static __global__ void __launch_bounds__(1024) ce_count_kernel(const long* __restrict__ targets,
                                                        int rows, long* __restrict__ count_out,
                                                        float* __restrict__ scale) {
  __shared__ long scnt[1024];
  long c = 0;
  const bool vec = (reinterpret_cast<unsigned long>(targets) & 15) == 0;
  for (int base = 4 * (int)threadIdx.x; base < rows; base += 4 * 4096) {
    long tv[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + 4096 * u;
      if (vec && i + 3 < rows) {
        const i64x2_t t0 = *reinterpret_cast<const i64x2_t*>(targets + i);
        const i64x2_t t1 = *reinterpret_cast<const i64x2_t*>(targets + i + 2);
        tv[u][0] = t0[0]; tv[u][1] = t0[1]; tv[u][2] = t1[0]; tv[u][3] = t1[1];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) tv[u][e] = i + e < rows ? targets[i + e] : -100;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) c += tv[u][e] != -100 ? 1 : 0;
  }
  scnt[threadIdx.x] = c;
  __syncthreads();
  for (int stride = 512; stride > 0; stride >>= 1) {
    if (threadIdx.x < stride) scnt[threadIdx.x] += scnt[threadIdx.x + stride];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    count_out[0] = scnt[0];
    scale[0] = 1.0f / (float)(scnt[0] > 1 ? scnt[0] : 1);
  }
}

// out = r(g * f32(in)) elementwise over [rows, d] BF16 (row strides ld_in, ld_out); runs
// only when run_if (nullable) is set. With `vec` (d, ld_in, ld_out multiples of 8, 16-byte
// aligned rows) each thread moves 8 elements as 16-byte vectors.
static __global__ void __launch_bounds__(256) scale_bf16_rows_kernel(
    const float* __restrict__ g, const unsigned short* __restrict__ in, long ld_in,
    unsigned short* __restrict__ out, long ld_out, int rows, int d, int vec,
    const int* __restrict__ run_if) {
  if (run_if != nullptr && *run_if == 0) return;
  const float scale = *g;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    const int per_row = d / 8;
    if (i >= (long)rows * per_row) return;
    const long r = i / per_row, c = (i - r * per_row) * 8;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(in + r * ld_in + c);
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(scale * lo_bf16(v[e]), scale * hi_bf16(v[e]));
    *reinterpret_cast<u32x4_t*>(out + r * ld_out + c) = o;
    return;
  }
  if (i >= (long)rows * d) return;
  const long r = i / d, c = i - r * d;
  out[r * ld_out + c] = to_bf16_bits(scale * bf16_bits_to_f32(in[r * ld_in + c]));
}

// acc += g * x elementwise over n FP32 values.
static __global__ void __launch_bounds__(256) scale_add_f32_kernel(const float* __restrict__ g,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ acc, long n,
                                                             const int* __restrict__ run_if) {
  if (run_if != nullptr && *run_if == 0) return;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) acc[i] += *g * x[i];
}

// exact[0] = 1 when g is +-2^e with |e| <= 32 (a normal FP32 number with an all-zero
// mantissa, exponent within 32 of 1): scaling by g then commutes with every BF16 and FP32
// rounding of the LM-head gradients that stays in the normal range, so the fused pass's
// unit gradients scaled by g are the gradients the two-pass backward computes for g, bit
// for bit, except for elements that are subnormal before or after the scaling (where
// r(g r(x)) and r(g x) can differ). The window keeps the scaled gradients of ordinary
// magnitude normal and far from overflow; other values take the two-pass backward.
static __global__ void ce_exact_scale_kernel(const float* __restrict__ g, int* __restrict__ exact) {
  if (threadIdx.x == 0) {
    const unsigned bits = __float_as_uint(g[0]);
    const int expo = (int)((bits >> 23) & 0xff) - 127;
    exact[0] = (bits & 0x7fffff) == 0 && expo >= -32 && expo <= 32;
  }
}

// Backward scale of the summed cross-entropy: dmean / max(1, count).
static __global__ void ce_scale_kernel(const float* __restrict__ dmean, const long* __restrict__ count,
                                float* __restrict__ scale) {
  if (threadIdx.x == 0) scale[0] = dmean[0] / (float)(count[0] > 1 ? count[0] : 1);
}

// ---------------------------------------------------------------------------------------
// Split-K reductions. Partials are [splits][M][N] FP32 slices of one GEMM output.
// G[m, n] += f32(r(sum_s P_s)) (round) or G += sum_s P_s; with kAccStore, G = the same
// sum (G not read). With `vec` (N and ldg multiples of 4, 16-byte aligned buffers) each
// thread moves four columns with 16-byte accesses.
static __global__ void __launch_bounds__(256) splitk_accum_kernel(const float* __restrict__ part,
                                                           int splits, long split_stride,
                                                           float* __restrict__ g, long ldg, int M,
                                                           int N, int round_acc, int vec) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    const long total4 = (long)M * N / 4;
    if (i >= total4) return;
    const long e = 4 * i, m = e / N, n = e % N;
    f32x4_t s = *reinterpret_cast<const f32x4_t*>(part + e);
    for (int q = 1; q < splits; ++q) s += *reinterpret_cast<const f32x4_t*>(part + q * split_stride + e);
    if (round_acc & kAccRound) {
#pragma unroll
      for (int d = 0; d < 4; ++d) s[d] = rbf16(s[d]);
    }
    f32x4_t* dst = reinterpret_cast<f32x4_t*>(g + m * ldg + n);
    *dst = (round_acc & kAccStore) ? s : *dst + s;
    return;
  }
  const long total = (long)M * N;
  if (i >= total) return;
  const long m = i / N, n = i % N;
  float s = 0.0f;
  for (int q = 0; q < splits; ++q) s += part[q * split_stride + m * N + n];
  const float v = (round_acc & kAccRound) ? rbf16(s) : s;
  g[m * ldg + n] = (round_acc & kAccStore) ? v : g[m * ldg + n] + v;
}

// out[m, n] = r(sum_s P_s) as BF16.
static __global__ void __launch_bounds__(256) splitk_bf16_kernel(const float* __restrict__ part,
                                                          int splits, long split_stride,
                                                          unsigned short* __restrict__ out,
                                                          long ldo, int M, int N,
                                                          const int* __restrict__ skip_if) {
  if (skip_if != nullptr && *skip_if != 0) return;
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long total = (long)M * N;
  if (i >= total) return;
  long m = i / N, n = i % N;
  float s = 0.0f;
  for (int q = 0; q < splits; ++q) s += part[q * split_stride + m * N + n];
  out[m * ldo + n] = to_bf16_bits(s);
}

}  // namespace ws

namespace ws {

// BF16 transpose out[c, r] = in[r, c] of a [rows, cols] matrix with row stride ld_in into a
// contiguous [cols, rows] result, for any shape: 64 x 64 tiles through LDS (rows padded by 8
// elements so the column reads do not collide), one element per access. Shapes whose rows,
// columns and stride are multiples of 8 take transpose_bf16_reg_kernel below. HBM-bound.
static __global__ void __launch_bounds__(256) transpose_bf16_kernel(
    const unsigned short* __restrict__ in, long ld_in, unsigned short* __restrict__ out,
    int rows, int cols) {
  __shared__ unsigned short tile[64][72];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int t = threadIdx.x;
  for (int idx = t; idx < 64 * 64; idx += 256) {
    const int r = idx >> 6, c = idx & 63;
    tile[r][c] = (r0 + r < rows && c0 + c < cols) ? in[(long)(r0 + r) * ld_in + c0 + c] : 0;
  }
  __syncthreads();
  for (int idx = t; idx < 64 * 64; idx += 256) {
    const int c = idx >> 6, r = idx & 63;
    if (c0 + c < cols && r0 + r < rows) out[(long)(c0 + c) * rows + r0 + r] = tile[r][c];
  }
}

// The transpose held in registers (rows, cols and ld_in multiples of 8, both pointers
// 16-byte aligned): each lane moves one 8 x 8 block, read as eight 16-byte row pieces and
// written as eight 16-byte column pieces after an in-register transpose (one byte
// permutation per output word). The 64 lanes of a wave cover a 64 x 64 tile (lane
// 8 * br + bc holds block (br, bc)), so every load instruction reads, and every store
// writes, eight whole 128-byte lines. No LDS and no barrier. Streaming (non-temporal)
// stores: 5.5 -> 6.0-6.4 TB/s on the weight shapes of the layer step.
static __global__ void __launch_bounds__(256) transpose_bf16_reg_kernel(
    const unsigned short* __restrict__ in, long ld_in, unsigned short* __restrict__ out,
    int rows, int cols) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.y * 64 + 8 * (lane >> 3);
  const int c = (blockIdx.x * 4 + wave) * 64 + 8 * (lane & 7);
  if (r >= rows || c >= cols) return;  // whole blocks: rows and cols are multiples of 8
  u32x4_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    w[j] = *reinterpret_cast<const u32x4_t*>(in + (long)(r + j) * ld_in + c);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    // Output row c + q: column q of the block, from word q / 2 of each input row (low half
    // for even q), rows 2p and 2p + 1 packed into word p.
    u32x4_t o;
#pragma unroll
    for (int p = 0; p < 4; ++p)
      o[p] = __builtin_amdgcn_perm(w[2 * p + 1][q >> 1], w[2 * p][q >> 1],
                                   (q & 1) ? 0x07060302u : 0x05040100u);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(out + (long)(c + q) * rows + r));
  }
}

}  // namespace ws

namespace ws {

// Gradient through the gate sigmoid of the fused input projection: for columns
// [col_lo, col_hi) of a [rows, *] gradient, dp = r(dout * (1 - s) * s) with s the BF16
// sigmoid output (torch's sigmoid backward, evaluated in FP32), other columns in
// [c0, c1) are copied. Processes columns [c0, c1) of every row; 8 columns per thread
// with 16-byte accesses when `vec`.
static __global__ void __launch_bounds__(256) sigmoid_backward_cols_kernel(
    const unsigned short* __restrict__ dout, long ld_dout, const unsigned short* __restrict__ s,
    long ld_s, unsigned short* dp, long ld_dp, int rows, int c0, int c1, int col_lo, int col_hi,
    int vec) {
  const int width = c1 - c0;
  if (vec) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = width / 8;
    if (idx >= (long)rows * per_row) return;
    const long r = idx / per_row;
    const int c = c0 + 8 * (int)(idx % per_row);
    u32x4_t g = *reinterpret_cast<const u32x4_t*>(dout + r * ld_dout + c);
    if (c + 8 > col_lo && c < col_hi) {
      const u32x4_t sv = *reinterpret_cast<const u32x4_t*>(s + r * ld_s + c);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float lo = lo_bf16(g[d]), hi = hi_bf16(g[d]);
        const float slo = lo_bf16(sv[d]), shi = hi_bf16(sv[d]);
        if (c + 2 * d >= col_lo && c + 2 * d < col_hi) lo = (lo * (1.0f - slo)) * slo;
        if (c + 2 * d + 1 >= col_lo && c + 2 * d + 1 < col_hi) hi = (hi * (1.0f - shi)) * shi;
        g[d] = pack_bf16x2(lo, hi);
      }
    }
    *reinterpret_cast<u32x4_t*>(dp + r * ld_dp + c) = g;
    return;
  }
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * width) return;
  const long r = idx / width;
  const int c = c0 + (int)(idx % width);
  float g = bf16_bits_to_f32(dout[r * ld_dout + c]);
  if (c >= col_lo && c < col_hi) {
    const float sv = bf16_bits_to_f32(s[r * ld_s + c]);
    g = (g * (1.0f - sv)) * sv;
  }
  dp[r * ld_dp + c] = to_bf16_bits(g);
}

}  // namespace ws

namespace ws {

// Logit gradients of one chunk from stored BF16 logits, with the arithmetic of the
// LM-head pass 2 epilogue: g = r(scale * exp(l - lse) - [n == target] scale), scale = 0 for
// ignored rows (target -100). Thread (row, 8-column piece) reads and writes 16 bytes;
// vocab % 4 == 0, a last half piece moves 8 bytes.
// `g` may be `logits` itself (in place): each thread reads its 16 bytes before writing them.
static __global__ void __launch_bounds__(256) ce_grad_logits_kernel(
    const unsigned short* logits, long ld_logits, const long* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ grad_scale,
    unsigned short* g, long ldg, int rows, int vocab) {
  const int per_row = (vocab + 2047) / 2048;  // blocks per row
  const int m = blockIdx.x / per_row;
  const int n = ((blockIdx.x % per_row) * 256 + threadIdx.x) * 8;
  if (m >= rows || n >= vocab) return;
  const long tgt = targets[m];
  const float l0 = lse[m];
  const float scale = (tgt == -100) ? 0.0f : *grad_scale;
  const unsigned short* src = logits + (long)m * ld_logits + n;
  unsigned short* dst = g + (long)m * ldg + n;
  const bool full = n + 7 < vocab;
  u32x4_t vl;
  if (full) {
    vl = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src));
  } else {
    const u32x2_t h = *reinterpret_cast<const u32x2_t*>(src);
    vl = u32x4_t{h[0], h[1], 0u, 0u};
  }
  u32x4_t o;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const long e = n + 2 * d;
    const float v0 = scale * exp_e(lo_bf16(vl[d]) - l0) - (e == tgt ? scale : 0.0f);
    const float v1 = scale * exp_e(hi_bf16(vl[d]) - l0) - (e + 1 == tgt ? scale : 0.0f);
    o[d] = pack_bf16x2(v0, v1);
  }
  if (full) *reinterpret_cast<u32x4_t*>(dst) = o;
  else *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{o[0], o[1]};
}

}  // namespace ws
