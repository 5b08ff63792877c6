// C ABI: the packed attention-backward gradient layout (ops/backward_layout.py).
//
// From the saved [B, N, H, C, D] activations/gradients of one attention core, build the
// token-major packed gradient out[B, N*C, 5*H*D] = [q | k | v | gate | u] that feeds the
// input projection's dgrad/wgrad GEMMs:
//   q  = bf16(inverse RoPE of (q_memory + q_local))
//   k  = bf16(inverse RoPE of (k_write^T (1 - tanh_k^2) + k_local)), with the rotated
//        half-term rounded to BF16 before the cosine term is added
//   v  = v_local
//   gate = bf16((dy (local) - dy (memory * scale)) * gate (1 - gate))
//   u  = bf16(u_write (1 - tanh_u^2))
// (ops/backward_layout.py:84-111 for the expression, :116-186 for the kernel arithmetic).
//
// FP32 arithmetic is evaluated exactly as written below (the library compiles with
// -ffp-contract=off); the four multiply-adds the reference's fused kernels contract are
// explicit fmaf calls:
//   q_e = fma(q_e, cos_e, r(q_o sin_o) + 0),  q_o = fma(q_o, cos_o, r(-q_e sin_e) + 0)
//   k   = fma(k_write, fma(-tanh_k, tanh_k, 1), k_local)
//   k_e = fma(k_e, cos_e, bf16(r(k_o sin_o) + 0)),  likewise k_o
//   gate: fma(dy, local, -r(dy r(memory scale)))
//   u:    u_write * fma(-tanh_u, tanh_u, 1)
// where r() is FP32 rounding and (e, o) = (2i, 2i + 1) is a rotary lane pair.
//
// Layout: one workgroup per (b, n, h) and block of CB tokens. Head-major operands are
// read as D-contiguous rows (16-byte vectors when D % 8 == 0), the transposed k_write
// [D, C] tile is staged once in LDS as [D][CB + 2] (row pitch = 1 word mod 64 banks, so
// both the staging writes and the per-token column reads are conflict-free), and each
// token's five output segments are written as whole D-element runs of its packed row.
#include "../../include/warpstate_hip.h"
#include "launch.h"

using namespace ws;

namespace {

enum LayoutMode {
  kAllSections = 0,     // "single": every section in one pass
  kRotarySections = 1,  // "paired", first launch: q and k
  kOtherSections = 2,   // "paired", second launch: v, gate and u
  kProfileRotary = 3,   // "profile", first launch: q and the rounded k half-term to scratch
  kProfilePack = 4,     // "profile", second launch: every section from the scratch
};

constexpr int kLayoutThreads = 256;
constexpr int kLayoutMaxLds = 64 * 1024;

struct LayoutParams {
  const unsigned short *qm, *ql, *kw, *tk, *kl, *vl, *dy, *mem, *loc, *gate, *uw, *tu;
  const float *sin, *cos;
  unsigned short* out;
  unsigned short* sq;   // profile scratch: final q, head-major
  unsigned short* skr;  // profile scratch: BF16 rotated half-term of k, head-major
  int H, C, D, CB, blocks_c, kw_vec;
  float scale;
};

// VEC consecutive BF16 elements <-> FP32 registers.
template <int VEC>
struct Run;

template <>
struct Run<8> {
  static __device__ __forceinline__ void load(const unsigned short* p, long off, float (&x)[8]) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = lo_bf16(w[i]);
      x[2 * i + 1] = hi_bf16(w[i]);
    }
  }
  static __device__ __forceinline__ void store(unsigned short* p, long off, const float (&x)[8]) {
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    *reinterpret_cast<u32x4_t*>(p + off) = w;
  }
  static __device__ __forceinline__ void copy(const unsigned short* s, long so, unsigned short* d,
                                              long doff) {
    *reinterpret_cast<u32x4_t*>(d + doff) = *reinterpret_cast<const u32x4_t*>(s + so);
  }
  static __device__ __forceinline__ void load_f32(const float* p, long off, float (&x)[8]) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p + off);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + off + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  }
};

template <>
struct Run<2> {
  static __device__ __forceinline__ void load(const unsigned short* p, long off, float (&x)[2]) {
    x[0] = bf16_bits_to_f32(p[off]);
    x[1] = bf16_bits_to_f32(p[off + 1]);
  }
  static __device__ __forceinline__ void store(unsigned short* p, long off, const float (&x)[2]) {
    p[off] = to_bf16_bits(x[0]);
    p[off + 1] = to_bf16_bits(x[1]);
  }
  static __device__ __forceinline__ void copy(const unsigned short* s, long so, unsigned short* d,
                                              long doff) {
    d[doff] = s[so];
    d[doff + 1] = s[so + 1];
  }
  static __device__ __forceinline__ void load_f32(const float* p, long off, float (&x)[2]) {
    x[0] = p[off];
    x[1] = p[off + 1];
  }
};

// x + 0 turns a -0 product into +0 (the reference adds the inactive rotary lane's zero).
__device__ __forceinline__ float plus_zero(float x) { return x + 0.0f; }

template <int VEC, int MODE>
__global__ void __launch_bounds__(kLayoutThreads) backward_layout_kernel(const LayoutParams p) {
  extern __shared__ unsigned short kwt[];  // [D][CB + 2] transposed k_write tile
  constexpr bool kNeedK = MODE != kOtherSections;
  constexpr bool kRotary = MODE != kOtherSections;
  constexpr bool kOther = MODE == kAllSections || MODE == kOtherSections || MODE == kProfilePack;

  const int H = p.H, C = p.C, D = p.D;
  const int g = blockIdx.x / p.blocks_c;  // (b, n, h)
  const int c0 = (blockIdx.x % p.blocks_c) * p.CB;
  const int ncb = min(p.CB, C - c0);
  const int h = g % H;
  const int pitch = p.CB + 2;
  const long hm0 = ((long)g * C + c0) * D;     // head-major offset of (g, c0, 0)
  const long tok0 = (long)(g / H) * C + c0;    // token row of (b, n, c0)
  const long HD = (long)H * D;

  if (kNeedK) {
    const unsigned short* kw = p.kw + (long)g * D * C + c0;  // row d at kw + d * C
    if (p.kw_vec) {  // C % 8 == 0, CB % 8 == 0, 16-byte aligned base
      const int per_row = ncb / 8;
      for (int i = threadIdx.x; i < D * per_row; i += kLayoutThreads) {
        const int d = i / per_row, cc = 8 * (i % per_row);
        const u32x4_t w = *reinterpret_cast<const u32x4_t*>(kw + (long)d * C + cc);
        unsigned* row = reinterpret_cast<unsigned*>(kwt + d * pitch + cc);
#pragma unroll
        for (int j = 0; j < 4; ++j) row[j] = w[j];
      }
    } else {
      for (int i = threadIdx.x; i < D * ncb; i += kLayoutThreads) {
        const int d = i / ncb, cc = i % ncb;
        kwt[d * pitch + cc] = kw[(long)d * C + cc];
      }
    }
    __syncthreads();
  }

  const int runs = D / VEC;
  for (int w = threadIdx.x; w < ncb * runs; w += kLayoutThreads) {
    const int cc = w / runs, d0 = (w % runs) * VEC;
    const long hm = hm0 + (long)cc * D + d0;
    const long tok = tok0 + cc;
    const long o = tok * 5 * HD + (long)h * D + d0;  // section 0 of this run

    if (kRotary) {
      float sn[VEC], cs[VEC];
      Run<VEC>::load_f32(p.sin, (long)(c0 + cc) * D + d0, sn);
      Run<VEC>::load_f32(p.cos, (long)(c0 + cc) * D + d0, cs);
      // q
      if (MODE == kProfilePack) {
        Run<VEC>::copy(p.sq, hm, p.out, o);
      } else {
        float a[VEC], b[VEC], q[VEC];
        Run<VEC>::load(p.qm, hm, a);
        Run<VEC>::load(p.ql, hm, b);
#pragma unroll
        for (int i = 0; i < VEC; ++i) a[i] = a[i] + b[i];
#pragma unroll
        for (int i = 0; i < VEC; i += 2) {
          q[i] = __builtin_fmaf(a[i], cs[i], plus_zero(a[i + 1] * sn[i + 1]));
          q[i + 1] = __builtin_fmaf(a[i + 1], cs[i + 1], plus_zero(-a[i] * sn[i]));
        }
        if (MODE == kProfileRotary) Run<VEC>::store(p.sq, hm, q);
        else Run<VEC>::store(p.out, o, q);
      }
      // k
      float t[VEC], l[VEC], k[VEC], kr[VEC];
      Run<VEC>::load(p.tk, hm, t);
      Run<VEC>::load(p.kl, hm, l);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float kw = bf16_bits_to_f32(kwt[(d0 + i) * pitch + cc]);
        k[i] = __builtin_fmaf(kw, __builtin_fmaf(-t[i], t[i], 1.0f), l[i]);
      }
      if (MODE == kProfilePack) {
        Run<VEC>::load(p.skr, hm, kr);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; i += 2) {
          kr[i] = rbf16(plus_zero(k[i + 1] * sn[i + 1]));
          kr[i + 1] = rbf16(plus_zero(-k[i] * sn[i]));
        }
      }
      if (MODE == kProfileRotary) {
        Run<VEC>::store(p.skr, hm, kr);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) k[i] = __builtin_fmaf(k[i], cs[i], kr[i]);
        Run<VEC>::store(p.out, o + HD, k);
      }
    }

    if (kOther) {
      // v
      Run<VEC>::copy(p.vl, hm, p.out, o + 2 * HD);
      // gate
      float dy[VEC], m[VEC], lc[VEC], gt[VEC];
      Run<VEC>::load(p.dy, tok * HD + (long)h * D + d0, dy);
      Run<VEC>::load(p.mem, hm, m);
      Run<VEC>::load(p.loc, hm, lc);
      Run<VEC>::load(p.gate, hm, gt);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float scaled = dy[i] * (m[i] * p.scale);
        const float pre = __builtin_fmaf(dy[i], lc[i], -scaled);
        m[i] = pre * (gt[i] * (1.0f - gt[i]));
      }
      Run<VEC>::store(p.out, o + 3 * HD, m);
      // u
      float uw[VEC], tu[VEC];
      Run<VEC>::load(p.uw, hm, uw);
      Run<VEC>::load(p.tu, hm, tu);
#pragma unroll
      for (int i = 0; i < VEC; ++i) uw[i] = uw[i] * __builtin_fmaf(-tu[i], tu[i], 1.0f);
      Run<VEC>::store(p.out, o + 4 * HD, uw);
    }
  }
}

template <int VEC>
int launch_layout(const LayoutParams& p, int mode, unsigned blocks, hipStream_t s) {
  const size_t lds = mode == kOtherSections ? 0 : (size_t)p.D * (p.CB + 2) * 2;
  switch (mode) {
    case kAllSections:
      hipLaunchKernelGGL((backward_layout_kernel<VEC, kAllSections>), dim3(blocks),
                         dim3(kLayoutThreads), lds, s, p);
      break;
    case kRotarySections:
      hipLaunchKernelGGL((backward_layout_kernel<VEC, kRotarySections>), dim3(blocks),
                         dim3(kLayoutThreads), lds, s, p);
      break;
    case kOtherSections:
      hipLaunchKernelGGL((backward_layout_kernel<VEC, kOtherSections>), dim3(blocks),
                         dim3(kLayoutThreads), lds, s, p);
      break;
    case kProfileRotary:
      hipLaunchKernelGGL((backward_layout_kernel<VEC, kProfileRotary>), dim3(blocks),
                         dim3(kLayoutThreads), lds, s, p);
      break;
    default:
      hipLaunchKernelGGL((backward_layout_kernel<VEC, kProfilePack>), dim3(blocks),
                         dim3(kLayoutThreads), lds, s, p);
      break;
  }
  return hip_check(hipGetLastError(), "backward layout launch");
}

bool aligned16(const void* ptr) { return reinterpret_cast<unsigned long>(ptr) % 16 == 0; }

}  // namespace

extern "C" int ws_backward_layout(const void* q_memory, const void* q_local, const float* sin,
                                  const float* cos, const void* k_write, const void* tanh_k,
                                  const void* k_local, const void* v_local, const void* grad_y,
                                  const void* memory, const void* local, const void* gate,
                                  const void* u_write, const void* tanh_u, void* out,
                                  int64_t batch, int64_t chunks, int64_t heads,
                                  int64_t chunk_size, int64_t head_dim, float scale, int algorithm,
                                  void* scratch_q, void* scratch_k, void* stream) {
  const void* bf16_inputs[] = {q_memory, q_local, k_write, tanh_k, k_local, v_local, grad_y,
                               memory, local, gate, u_write, tanh_u};
  for (const void* ptr : bf16_inputs)
    if (!ptr) return set_error(kInvalid, "null pointer");
  if (!sin || !cos || !out) return set_error(kInvalid, "null pointer");
  if (batch < 1 || chunks < 1 || heads < 1 || chunk_size < 1 || head_dim < 2 || head_dim % 2)
    return set_error(kInvalid, "Expected positive [B,N,H,C,D] with an even head dimension");
  if (head_dim > 8192) return set_error(kInvalid, "head dimension %ld exceeds 8192", (long)head_dim);
  if (algorithm < 0 || algorithm > 2)
    return set_error(kInvalid, "Unknown backward layout algorithm code %d", algorithm);
  if (algorithm == 0 && (!scratch_q || !scratch_k))
    return set_error(kInvalid, "The profile baseline needs two contiguous BF16 scratch tensors");
  const long groups = batch * chunks * heads;
  const long elements = groups * chunk_size * head_dim;
  if (elements / head_dim / chunk_size != groups || 5 * heads * head_dim > 0x7fffffffL)
    return set_error(kInvalid, "backward layout shape too large");

  LayoutParams p;
  p.qm = static_cast<const unsigned short*>(q_memory);
  p.ql = static_cast<const unsigned short*>(q_local);
  p.kw = static_cast<const unsigned short*>(k_write);
  p.tk = static_cast<const unsigned short*>(tanh_k);
  p.kl = static_cast<const unsigned short*>(k_local);
  p.vl = static_cast<const unsigned short*>(v_local);
  p.dy = static_cast<const unsigned short*>(grad_y);
  p.mem = static_cast<const unsigned short*>(memory);
  p.loc = static_cast<const unsigned short*>(local);
  p.gate = static_cast<const unsigned short*>(gate);
  p.uw = static_cast<const unsigned short*>(u_write);
  p.tu = static_cast<const unsigned short*>(tanh_u);
  p.sin = sin;
  p.cos = cos;
  p.out = static_cast<unsigned short*>(out);
  p.sq = static_cast<unsigned short*>(scratch_q);
  p.skr = static_cast<unsigned short*>(scratch_k);
  p.H = (int)heads;
  p.C = (int)chunk_size;
  p.D = (int)head_dim;
  // Token block: up to 16 tokens, and small enough that the [D][CB + 2] tile fits 64 KiB.
  // Many small blocks overlap one another's k_write staging and token work: at
  // [4,16,32,128,64] 16-token blocks ran 10 % faster than 128-token blocks (108.7 against
  // 120.2 us), 32 and 8 tokens in between.
  int cb = chunk_size < 16 ? (int)chunk_size : 16;
  while (cb > 2 && (long)head_dim * (cb + 2) * 2 > kLayoutMaxLds) cb = (cb / 2 + 1) & ~1;
  p.CB = cb;
  p.blocks_c = cdiv(chunk_size, cb);
  p.scale = scale;
  const long blocks = groups * p.blocks_c;
  if (blocks > 0x7fffffffL) return set_error(kInvalid, "backward layout grid too large");

  bool vec = head_dim % 8 == 0 && aligned16(sin) && aligned16(cos) && aligned16(out);
  for (const void* ptr : bf16_inputs) vec = vec && aligned16(ptr);
  if (algorithm == 0) vec = vec && aligned16(scratch_q) && aligned16(scratch_k);
  p.kw_vec = chunk_size % 8 == 0 && cb % 8 == 0 && aligned16(k_write);

  hipStream_t s = static_cast<hipStream_t>(stream);
  auto run = [&](int mode) {
    return vec ? launch_layout<8>(p, mode, (unsigned)blocks, s)
               : launch_layout<2>(p, mode, (unsigned)blocks, s);
  };
  int rc = kOk;
  if (algorithm == 2) {  // "single"
    rc = run(kAllSections);
  } else if (algorithm == 1) {  // "paired"
    rc = run(kRotarySections);
    if (rc == kOk) rc = run(kOtherSections);
  } else {  // "profile"
    rc = run(kProfileRotary);
    if (rc == kOk) rc = run(kProfilePack);
  }
  return rc;
}
