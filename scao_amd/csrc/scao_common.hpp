// Shared device helpers for the gfx950 SCAO kernels.
//
// Arithmetic is compiled with -ffp-contract=off: every fused multiply-add in
// these kernels is an explicit fmaf() placed where the reference's CPU path
// (ATen vectorised kernels) rounds once, and everything else rounds per op.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/scao_amd.h"

typedef float v4f __attribute__((ext_vector_type(4)));

#define SCAO_WAVE 64

namespace scao {

// ---------------------------------------------------------------- MFMA ---
// v_mfma_f32_16x16x4_f32.  Lane l supplies A[l%16][l/16] and B[l/16][l%16];
// the accumulator holds D[4*(l/16)+r][l%16] in element r (checked on gfx950).
__device__ __forceinline__ v4f mfma16(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16.  Lane l supplies A[l%16][8*(l/16)+e] and
// B[8*(l/16)+e][l%16] in element e; the accumulator layout is mfma16's
// (checked on gfx950).  Products of two bf16 are exact in fp32.
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v4f mfma16bf(v8bf a, v8bf b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// fp32 products on the bf16 matrix cores: x = h + m + l exactly for every
// finite x above ~1e-33 in magnitude (h rounds x to 8 significant bits, m the
// remainder, and the second remainder has at most 8 bits left, so l holds it
// exactly; both subtractions are exact).  A product x*y is then the sum of
// nine exact bf16 products; the six kept by mfma_x6 drop m*l, l*m and l*l,
// at most about 2^-23 |x y| together, the size of fp32's own rounding of
// the product.
struct bf3 {
  v8bf h, m, l;
};
typedef float v2f_t __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
// a and b rounded to bf16 (nearest even) by one v_cvt_pk_bf16_f32, a in the
// low half of the word
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f_t){a, b}, v2bf_t));
}
// The three-way split of a pair, packed as the MFMA operands and LDS planes
// hold it: word h holds a's and b's leading parts, m and l the remainders.
// Per element it is (__bf16)x, then x - h, and so on: the same bits as one
// scalar conversion at a time, at three conversions per two elements.
__device__ __forceinline__ void split3_pk(float a, float b, uint32_t& h, uint32_t& m,
                                          uint32_t& l) {
  h = pk_bf16(a, b);
  const float ra = a - __uint_as_float(h << 16), rb = b - __uint_as_float(h & 0xffff0000u);
  m = pk_bf16(ra, rb);
  l = pk_bf16(ra - __uint_as_float(m << 16), rb - __uint_as_float(m & 0xffff0000u));
}
__device__ __forceinline__ bf3 split_bf3(const float (&x)[8]) {
  v4u_t h, m, l;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    uint32_t a, b, c;
    split3_pk(x[2 * p], x[2 * p + 1], a, b, c);
    h[p] = a;
    m[p] = b;
    l[p] = c;
  }
  return bf3{__builtin_bit_cast(v8bf, h), __builtin_bit_cast(v8bf, m), __builtin_bit_cast(v8bf, l)};
}
// c + A B for fp32 A and B given as bf3 splits: six bf16 MFMAs (small terms
// first).
__device__ __forceinline__ v4f mfma_x6(const bf3& a, const bf3& b, v4f c) {
  c = mfma16bf(a.m, b.m, c);
  c = mfma16bf(a.h, b.l, c);
  c = mfma16bf(a.l, b.h, c);
  c = mfma16bf(a.h, b.m, c);
  c = mfma16bf(a.m, b.h, c);
  return mfma16bf(a.h, b.h, c);
}

// ------------------------------------------------------------- dtypes ---
__device__ __forceinline__ float bf16_to_f(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t f_to_bf16(float f) {  // round to nearest even
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_to_f(uint16_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, h);
  return (float)x;
}
__device__ __forceinline__ uint16_t f_to_f16(float f) {
  _Float16 x = (_Float16)f;
  return __builtin_bit_cast(uint16_t, x);
}

// round a float to the storage dtype and back (the reference's .to(dtype))
__device__ __forceinline__ float round_to(int dt, float x) {
  if (dt == SCAO_BF16) return bf16_to_f(f_to_bf16(x));
  if (dt == SCAO_F16) return f16_to_f(f_to_f16(x));
  return x;
}

// All tensors these kernels touch live in device global memory; loads and
// stores go through address-space-1 pointers so the compiler emits global_*
// instructions (pointers read from descriptor tables are otherwise generic
// and become flat_* accesses).
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) uint16_t gu16;
typedef __attribute__((address_space(1))) v4f gv4f;
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) v2u gv2u;

__device__ __forceinline__ v4f gld4(const float* p) { return *(const gv4f*)p; }
__device__ __forceinline__ void gst4(float* p, v4f x) { *(gv4f*)p = x; }
// streaming (read or written once per step): non-temporal cache policy
__device__ __forceinline__ v4f gld4_nt(const float* p) {
  return __builtin_nontemporal_load((const gv4f*)p);
}
__device__ __forceinline__ void gst4_nt(float* p, v4f x) {
  __builtin_nontemporal_store(x, (gv4f*)p);
}
__device__ __forceinline__ float gld1(const float* p) { return *(const gfloat*)p; }
__device__ __forceinline__ void gst1(float* p, float x) { *(gfloat*)p = x; }
// 16-byte alignment for fp32 float4 access, 8-byte for a 16-bit dtype's 4-pack
__device__ __forceinline__ bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
__device__ __forceinline__ bool al_dt(const void* p, int dt) {
  return dt == SCAO_F32 ? al16(p) : (((uintptr_t)p & 7u) == 0);
}
typedef __attribute__((address_space(1))) uint32_t gu32;
__device__ __forceinline__ uint32_t gld1(const uint32_t* p) { return *(const gu32*)p; }
__device__ __forceinline__ void gst1(uint32_t* p, uint32_t x) { *(gu32*)p = x; }

__device__ __forceinline__ float ld1(const void* base, int dt, int64_t i) {
  if (dt == SCAO_F32) return gld1((const float*)base + i);
  uint16_t h = ((const gu16*)base)[i];
  return dt == SCAO_BF16 ? bf16_to_f(h) : f16_to_f(h);
}
__device__ __forceinline__ void st1(void* base, int dt, int64_t i, float x) {
  if (dt == SCAO_F32) {
    gst1((float*)base + i, x);
  } else {
    ((gu16*)base)[i] = dt == SCAO_BF16 ? f_to_bf16(x) : f_to_f16(x);
  }
}

// Four consecutive elements starting at element i.  `vec` promises 16-byte
// (fp32) / 8-byte (16-bit) alignment and that all four are in bounds; else
// element t is loaded only when mask bit t is set (zero otherwise).
__device__ __forceinline__ v4f ld4(const void* base, int dt, int64_t i, bool vec, int mask) {
  v4f r = {0.f, 0.f, 0.f, 0.f};
  if (vec) {
    if (dt == SCAO_F32) {
      r = gld4((const float*)base + i);
    } else {
      const v2u x = *(const gv2u*)((const uint16_t*)base + i);
      uint16_t h[4] = {(uint16_t)(x[0] & 0xffff), (uint16_t)(x[0] >> 16), (uint16_t)(x[1] & 0xffff),
                       (uint16_t)(x[1] >> 16)};
      for (int t = 0; t < 4; ++t) r[t] = dt == SCAO_BF16 ? bf16_to_f(h[t]) : f16_to_f(h[t]);
    }
  } else {
    for (int t = 0; t < 4; ++t)
      if (mask & (1 << t)) r[t] = ld1(base, dt, i + t);
  }
  return r;
}
__device__ __forceinline__ void st4(void* base, int dt, int64_t i, v4f x, bool vec, int mask) {
  if (vec) {
    if (dt == SCAO_F32) {
      gst4((float*)base + i, x);
    } else {
      uint16_t h[4];
      for (int t = 0; t < 4; ++t) h[t] = dt == SCAO_BF16 ? f_to_bf16(x[t]) : f_to_f16(x[t]);
      const v2u y = {(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
      *(gv2u*)((uint16_t*)base + i) = y;
    }
  } else {
    for (int t = 0; t < 4; ++t)
      if (mask & (1 << t)) st1(base, dt, i + t, x[t]);
  }
}
// fp32-only variants (optimizer state is always float32)
__device__ __forceinline__ v4f ldf4(const float* base, int64_t i, bool vec, int mask) {
  if (vec) return gld4(base + i);
  v4f r = {0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t < 4; ++t)
    if (mask & (1 << t)) r[t] = gld1(base + i + t);
  return r;
}
__device__ __forceinline__ void stf4(float* base, int64_t i, v4f x, bool vec, int mask) {
  if (vec) {
    gst4(base + i, x);
    return;
  }
  for (int t = 0; t < 4; ++t)
    if (mask & (1 << t)) gst1(base + i + t, x[t]);
}

// the gradient the moments use: raw p.grad in its dtype, or a float32 buffer
// ---- gradient noise: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel
// random numbers: as easy as 1, 2, 3", SC'11): ten rounds of the published
// multiply/xor network with the Weyl key schedule; Box-Muller turns the four
// words of counter (element index / 4) into four N(0,1) values.
__device__ __forceinline__ void philox(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * c[0], hi0 = __umulhi(0xD2511F53u, c[0]);
    const uint32_t lo1 = 0xCD9E8D57u * c[2], hi1 = __umulhi(0xCD9E8D57u, c[2]);
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// N(0,1) values of elements e .. e+3 for e a multiple of 4.  Box-Muller on
// the hardware transcendentals: -2 ln u = -2 ln2 * v_log_f32(u) (log2),
// v_sqrt_f32, and v_sin_f32 / v_cos_f32, which take the angle in
// revolutions -- u2 in (0, 1] already is one.
__device__ __forceinline__ v4f normals4(uint64_t key, int64_t e) {
  const uint64_t ctr = (uint64_t)e >> 2;
  uint32_t c[4] = {(uint32_t)ctr, (uint32_t)(ctr >> 32), 0u, 0u};
  philox(c, (uint32_t)key, (uint32_t)(key >> 32));
  v4f z;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    // uniforms in (0, 1): 24 bits plus half a step
    const float u1 = ((float)(c[2 * j] >> 8) + 0.5f) * 5.9604645e-8f;
    const float u2 = ((float)(c[2 * j + 1] >> 8) + 0.5f) * 5.9604645e-8f;
    const float rad = __builtin_amdgcn_sqrtf(-1.3862944f * __builtin_amdgcn_logf(u1));
    z[2 * j] = rad * __builtin_amdgcn_cosf(u2);
    z[2 * j + 1] = rad * __builtin_amdgcn_sinf(u2);
  }
  return z;
}

// The moment gradient of elements e .. e+3 from their raw values and, with
// SCAO_PF_FMASK, the filter's EMA values `em` (loaded by the caller with its
// other streams): fp32(g) * (em >= t), then + fp32(fnoise * z) with
// SCAO_PF_FNOISE -- the values scao_sparse_filter's output pass would write.
// Lanes outside `mask` are left as they are.
// keep: bit t set when the filter keeps element t (EMA >= threshold); all
// set when the parameter has no filter mask.
__device__ __forceinline__ v4f finish_mgrad_bits(const scao_param_desc& P, int64_t e,
                                                 const v4f& gr, uint32_t keep, int mask) {
  v4f o = gr;
  if (P.flags & SCAO_PF_FMASK) {
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = gr[t] * (((keep >> t) & 1u) ? 1.0f : 0.0f);
  }
  if (P.flags & SCAO_PF_FNOISE) {
    const uint64_t key = *P.fseed;
    if ((e & 3) == 0) {
      const v4f z = normals4(key, e);
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] = o[t] + z[t] * P.fnoise;
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (!(mask & (1 << t))) continue;
        const int64_t i = e + t;
        const v4f z = normals4(key, i & ~(int64_t)3);
        o[t] = o[t] + z[(int)(i & 3)] * P.fnoise;
      }
    }
  }
  return o;
}

__device__ __forceinline__ v4f finish_mgrad(const scao_param_desc& P, int64_t e, const v4f& gr,
                                            const v4f& em, int mask) {
  uint32_t keep = 15u;
  if (P.flags & SCAO_PF_FMASK) {
    const float thr = *P.fthr;
    keep = 0u;
#pragma unroll
    for (int t = 0; t < 4; ++t) keep |= (em[t] >= thr ? 1u : 0u) << t;
  }
  return finish_mgrad_bits(P, e, gr, keep, mask);
}

// true when the moment gradient is formed in-kernel from graw (+ the EMA)
__device__ __forceinline__ bool fused_mgrad(const scao_param_desc& P) {
  return (P.flags & (SCAO_PF_FMASK | SCAO_PF_FNOISE)) != 0;
}

__device__ __forceinline__ v4f ld_mgrad(const scao_param_desc& P, int64_t i, bool vec, int mask) {
  if (P.flags & SCAO_PF_GF32) return ldf4((const float*)P.g, i, vec, mask);
  return ld4(P.g, P.dtype, i, vec, mask);
}

// ---------------------------------------------------------- reductions ---
__device__ __forceinline__ double wave_sum(double x) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, SCAO_WAVE);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, SCAO_WAVE));
  return x;
}
// Sum over a 256-thread block, deterministic order; result valid in thread 0.
template <int NQ>
__device__ __forceinline__ void block_sum(double (&x)[NQ], double* lds /* >= 4*NQ */) {
  const int w = threadIdx.x / SCAO_WAVE, l = threadIdx.x % SCAO_WAVE;
#pragma unroll
  for (int q = 0; q < NQ; ++q) x[q] = wave_sum(x[q]);
  __syncthreads();
  if (l == 0)
    for (int q = 0; q < NQ; ++q) lds[w * NQ + q] = x[q];
  __syncthreads();
  if (threadIdx.x == 0)
    for (int q = 0; q < NQ; ++q) x[q] = ((lds[q] + lds[NQ + q]) + lds[2 * NQ + q]) + lds[3 * NQ + q];
}
// The same over an NT-thread block (waves added in order); lds >= NQ*NT/64.
template <int NQ, int NT>
__device__ __forceinline__ void block_sum_n(double (&x)[NQ], double* lds) {
  constexpr int NW = NT / SCAO_WAVE;
  const int w = threadIdx.x / SCAO_WAVE, l = threadIdx.x % SCAO_WAVE;
#pragma unroll
  for (int q = 0; q < NQ; ++q) x[q] = wave_sum(x[q]);
  __syncthreads();
  if (l == 0)
    for (int q = 0; q < NQ; ++q) lds[w * NQ + q] = x[q];
  __syncthreads();
  if (threadIdx.x == 0)
    for (int q = 0; q < NQ; ++q) {
      double s = lds[q];
      for (int v = 1; v < NW; ++v) s += lds[v * NQ + q];
      x[q] = s;
    }
}
__device__ __forceinline__ float block_max(float x, float* lds) {
  const int w = threadIdx.x / SCAO_WAVE, l = threadIdx.x % SCAO_WAVE;
  x = wave_max(x);
  __syncthreads();
  if (l == 0) lds[w] = x;
  __syncthreads();
  float r = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
  return r;
}

// clamp(S, 1e-8)^(-1/4) for the eigenvalue scaling (torch: pow(-0.25)); the
// double evaluation is correctly rounded, torch's CPU path is within 1 ulp.
__device__ __forceinline__ float inv4(float s) {
  float c = fmaxf(s, 1e-8f);
  return (float)pow((double)c, -0.25);
}
// clamp(S, eps)^(-1/2) = 1/sqrt (torch lowers pow(-0.5) to a reciprocal sqrt)
__device__ __forceinline__ float inv2(float s, float eps) {
  float c = fmaxf(s, eps);
  return 1.0f / sqrtf(c);
}

// The optimizer's elementwise tail for four elements (scao/optimizer.py:606-645):
// clip -> blend -> Adan moments -> bias-corrected update (-> gSNR mask).
// Writes m, v, d, prev; returns the fp32 update u.
__device__ __forceinline__ v4f adan_tail(const scao_param_desc& P, const scao_param_stat& S,
                                         int64_t e, v4f g, v4f gp, bool vec, int mask) {
  const int dt = P.dtype;
  if (P.flags & SCAO_PF_CLIP) {
    for (int t = 0; t < 4; ++t) gp[t] = round_to(dt, gp[t] * S.clip);
  }
  v4f m = ldf4(P.exp_avg, e, vec, mask);
  v4f v = ldf4(P.exp_avg_sq, e, vec, mask);
  v4f d = ldf4(P.exp_avg_diff, e, vec, mask);
  v4f pv = ldf4(P.prev_grad, e, vec, mask);
  v4f u;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float geff = P.blend * gp[t] + P.omblend * g[t];
    const float delta = g[t] - pv[t];
    m[t] = fmaf(geff, P.omb1, m[t] * P.beta1);
    d[t] = fmaf(delta, P.omb3, d[t] * P.beta3);
    const float gad = geff + P.omb3 * delta;
    v[t] = fmaf(P.omb2 * gad, gad, v[t] * P.beta2);
    const float mh = m[t] / P.bc1;
    const float dh = d[t] / P.bc3;
    const float vh = v[t] / P.bc2;
    float x = (mh + P.omb3 * dh) / (sqrtf(vh) + P.eps);
    if (P.flags & SCAO_PF_GSNR) {
      const float snr = fabsf(m[t]) / (sqrtf(v[t]) + P.eps);
      x = x * (snr >= P.gsnr ? 1.0f : 0.0f);
    }
    u[t] = x;
  }
  stf4(P.exp_avg, e, m, vec, mask);
  stf4(P.exp_avg_sq, e, v, vec, mask);
  stf4(P.exp_avg_diff, e, d, vec, mask);
  stf4(P.prev_grad, e, g, vec, mask);
  return u;
}

// Final write of four elements: LARS params stage u, others update p at once.
__device__ __forceinline__ float write_update(const scao_param_desc& P, int64_t e, v4f u,
                                              bool vec, int mask) {
  const int dt = P.dtype;
  float u2 = 0.f;
  if (P.flags & SCAO_PF_LARS) {
    stf4(P.upd, e, u, vec, mask);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (mask & (1 << t)) u2 = fmaf(u[t], u[t], u2);
  } else {
    const float alpha = round_to(dt, (float)(-P.lr));
    v4f p = ld4(P.p, dt, e, vec, mask);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float pd = (P.flags & SCAO_PF_DECAY) ? round_to(dt, p[t] * P.decay) : p[t];
      p[t] = round_to(dt, fmaf(round_to(dt, u[t]), alpha, pd));
    }
    st4(P.p, dt, e, p, vec, mask);
  }
  return u2;
}

}  // namespace scao

// ------------------------------------------------------------- errors ---
void scao_set_error(const char* fmt, ...);
#define SCAO_CHECK_ARG(cond, ...)         \
  do {                                    \
    if (!(cond)) {                        \
      scao_set_error(__VA_ARGS__);        \
      return SCAO_ERR_INVALID;            \
    }                                     \
  } while (0)
#define SCAO_LAUNCH_CHECK(name)                                                     \
  do {                                                                              \
    hipError_t e_ = hipGetLastError();                                              \
    if (e_ != hipSuccess) {                                                         \
      scao_set_error("%s: launch failed: %s", name, hipGetErrorString(e_));        \
      return SCAO_ERR_HIP;                                                          \
    }                                                                               \
  } while (0)
