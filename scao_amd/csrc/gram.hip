// Curvature-refresh kernels on gfx950 (scao/preconditioner.py:297-361, 381-406).
//
// gram_ema   C = X X^T for X = G (L side, dim m) or X = G^T (R side, dim n) on
//            fp32 MFMA, 128x128 output tiles staged through LDS in 16-deep
//            K chunks, fused with the EMA
//               int8:  x = fp32(fp32(fp32(q*s)*rho) + fp32(alpha*C))
//               fp32:  ema = fp32(fp32(ema*rho) + fp32(alpha*C))  (in place)
//            (reference: dequantize_sym_int8(...).mul_(rho).add_(alpha*(g@g.T)),
//            scao/preconditioner.py:344-353) and a per-tile |x| maximum.
// requant    scale' = max|x| / 127 (double, as the reference's Python float),
//            q' = clamp(rint(x / fp32(scale')), +-127); zeros and scale 1.0
//            when max|x| < 1e-30 (scao/utils.py:170-189).  The global maximum
//            comes from the per-tile maxima, so no host round trip.
// eig_prep   the eigh input (scao/preconditioner.py:383-406): dequantise,
//            divide by fp32(bias), add fp32(max(1e-8, 1e-4*tr/dim)) on the
//            diagonal; the trace is accumulated in double and rounded to fp32
//            as torch's CPU trace does.
// int8_ema_update  the reference operator (scao/cuda/__init__.py:122-142).
#include "scao_common.hpp"

using namespace scao;

namespace {

constexpr int GT = SCAO_GRAM_TILE;  // 128
constexpr int KC = 16;              // K chunk
constexpr int LP = GT + 4;          // padded LDS row

__device__ __forceinline__ float gload(const scao_gram_desc& D, int i, int k) {
  // X[i][k]
  const int64_t e = D.side == 0 ? D.off + (int64_t)i * D.ld + k : D.off + (int64_t)k * D.ld + i;
  return ld1(D.g, D.dtype, e);
}

// Stage X[r0:r0+128][kb:kb+16] into lds[k][r] (zero outside dim x K).
__device__ __forceinline__ void stage(const scao_gram_desc& D, int dim, int K, int r0, int kb,
                                      float (*lds)[LP], bool vec) {
  const int tid = threadIdx.x;
  if (D.side == 0) {
    // rows contiguous in k: thread -> (row, 4 k's)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = tid / 4 + 64 * h, kq = (tid % 4) * 4;
      const int i = r0 + r;
      int mk = 0;
      for (int t = 0; t < 4; ++t) mk |= (i < dim && kb + kq + t < K) ? (1 << t) : 0;
      v4f x = mk ? ld4(D.g, D.dtype, D.off + (int64_t)i * D.ld + kb + kq, vec && mk == 15, mk)
                 : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) lds[kq + t][r] = x[t];
    }
  } else {
    // k rows contiguous in i: thread -> (k, 4 i's)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kr = tid / 32 + 8 * h, iq = (tid % 32) * 4;
      const int kk = kb + kr;
      int mk = 0;
      for (int t = 0; t < 4; ++t) mk |= (kk < K && r0 + iq + t < dim) ? (1 << t) : 0;
      v4f x = mk ? ld4(D.g, D.dtype, D.off + (int64_t)kk * D.ld + r0 + iq, vec && mk == 15, mk)
                 : v4f{0.f, 0.f, 0.f, 0.f};
      *(v4f*)&lds[kr][iq] = x;
    }
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gram_ema(const scao_task* __restrict__ tasks,
                                                  const scao_gram_desc* __restrict__ descs) {
  __shared__ __attribute__((aligned(16))) float As[2][KC][LP];
  __shared__ __attribute__((aligned(16))) float Bs[2][KC][LP];
  __shared__ float red[4];
  const scao_task tk = tasks[blockIdx.x];
  const scao_gram_desc D = descs[tk.idx];
  const int dim = D.side == 0 ? D.rows : D.cols;
  const int K = D.side == 0 ? D.cols : D.rows;
  const int i0 = tk.a * GT, j0 = tk.b * GT;
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int wr = (w / 2) * 64, wc = (w % 2) * 64;
  const bool vec = ((D.off | D.ld) % 4 == 0) &&
                   (((uintptr_t)D.g & (D.dtype == SCAO_F32 ? 15u : 7u)) == 0);

  // Two-level sum: the MFMAs accumulate FOLD consecutive K values in acc,
  // which is then added to tot and cleared.  One fp32 accumulator over all
  // of K (2048-4096 here, K/4 dependent MFMA adds) drifts by about
  // sqrt(K/4) ulps, above the reference's own float32 GEMM; two levels of
  // sqrt(FOLD/4) and sqrt(K/FOLD) bring that under it.  Both sums are exact
  // sums of the same products, so only rounding changes.
  constexpr int FOLD = 128;
  v4f acc[4][4], tot[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = tot[a][b] = v4f{0.f, 0.f, 0.f, 0.f};

  stage(D, dim, K, i0, 0, As[0], vec);
  stage(D, dim, K, j0, 0, Bs[0], vec);
  __syncthreads();
  int buf = 0;
  for (int kb = 0; kb < K; kb += KC) {
    if (kb + KC < K) {
      stage(D, dim, K, i0, kb + KC, As[buf ^ 1], vec);
      stage(D, dim, K, j0, kb + KC, Bs[buf ^ 1], vec);
    }
#pragma unroll
    for (int ks = 0; ks < KC / 4; ++ks) {
      const int kr = 4 * ks + l / 16;
      float af[4], bf[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) af[a] = As[buf][kr][wr + 16 * a + (l % 16)];
#pragma unroll
      for (int b = 0; b < 4; ++b) bf[b] = Bs[buf][kr][wc + 16 * b + (l % 16)];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16(af[a], bf[b], acc[a][b]);
    }
    __syncthreads();
    buf ^= 1;
    if ((kb + KC) % FOLD == 0 || kb + KC >= K) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          tot[a][b] += acc[a][b];
          acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    }
  }

  // EMA epilogue: element (i, j) = tot[a][b][r],
  // i = i0 + wr + 16a + 4*(l/16) + r, j = j0 + wc + 16b + l%16
  const float sf = D.q ? (float)(*D.scale) : 0.f;
  float amax = 0.f;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + wr + 16 * a + 4 * (l / 16) + r;
      if (i >= dim) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int j = j0 + wc + 16 * b + (l % 16);
        if (j >= dim) continue;
        const int64_t e = (int64_t)i * dim + j;
        const float add = D.alpha * tot[a][b][r];
        if (D.q) {
          const float old = ((float)D.q[e] * sf) * D.rho;
          const float x = old + add;
          D.ema[e] = x;
          amax = fmaxf(amax, fabsf(x));
        } else {
          D.ema[e] = D.ema[e] * D.rho + add;
        }
      }
    }
  // the transposed tile (b, a) of a symmetric factor: element (j, i) takes
  // the same product as (i, j).  Staged through LDS (the operand buffers are
  // free after the K loop), one 64 x 64 wave sub-tile per buffer, two waves at
  // a time, so the global accesses run along rows of the transposed tile.
  const bool mirror = (D.flags & SCAO_GRAM_SYM) && tk.a != tk.b;
  if (mirror) {
    static_assert(sizeof(As) >= 64 * 65 * sizeof(float), "staging");
    float* S = (w % 2 == 0) ? &As[0][0][0] : &Bs[0][0][0];
    for (int half = 0; half < 2; ++half) {
      const bool mine = (w / 2) == half;
      if (mine) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int b = 0; b < 4; ++b)
              S[(16 * b + (l % 16)) * 65 + 16 * a + 4 * (l / 16) + r] = tot[a][b][r];
      }
      __syncthreads();
      if (mine) {
        const int i = i0 + wr + l;             // column of the transposed tile
        for (int jj = 0; jj < 64; ++jj) {
          const int j = j0 + wc + jj;          // row of the transposed tile
          if (i >= dim || j >= dim) continue;
          const int64_t e = (int64_t)j * dim + i;
          const float add = D.alpha * S[jj * 65 + l];
          if (D.q) {
            const float old = ((float)D.q[e] * sf) * D.rho;
            const float x = old + add;
            D.ema[e] = x;
            amax = fmaxf(amax, fabsf(x));
          } else {
            D.ema[e] = D.ema[e] * D.rho + add;
          }
        }
      }
      __syncthreads();
    }
  }
  if (D.q) {
    const float mx = block_max(amax, red);
    if (threadIdx.x == 0) {
      D.amax[tk.slot] = mx;
      if (mirror) {
        const int nt = (dim + GT - 1) / GT;
        D.amax[tk.b * nt + tk.a] = mx;
      }
    }
  }
}

// Requantise x[0:n) given the per-tile maxima; divide (utils.quantize_sym_int8)
// or multiply by the fp32 reciprocal (the int8_ema_update operator).
// Code for one value: rint(y) clamped to +-127 (rintf rounds half to even,
// as torch.round does).
__device__ __forceinline__ uint32_t code_of(float y) {
  return (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(rintf(y), -127.f), 127.f);
}

// Requantise one SCAO_FLAT_CHUNK-element chunk of x into q.  The scale is
// max|x| / 127 in double from the per-tile maxima amax[0..nparts); `recip`
// selects the reference operator's reciprocal multiply
// (scao/cuda/__init__.py:122-142) instead of quantize_sym_int8's division
// (scao/utils.py:170-189).  Whole, aligned chunks stream 4 values per load
// and store 4 codes per 32-bit write, each wave covering 1 KB of x per
// instruction; other chunks go element by element.
__device__ __forceinline__ void requant_chunk(const float* x, int64_t n, const float* amax, int nparts,
                              int8_t* q, double* scale_out, int chunk, bool recip) {
  __shared__ float red[4];
  const int64_t base = (int64_t)chunk * SCAO_FLAT_CHUNK;
  const bool vec = base + SCAO_FLAT_CHUNK <= n && (((uintptr_t)x | (uintptr_t)q) & 15) == 0;
  v4f v[4];
  if (vec) {   // the chunk's loads go out before the scale is known
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = gld4_nt(x + base + 4 * (threadIdx.x + 256 * j));
  }
  float mx = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 256) mx = fmaxf(mx, amax[i]);
  mx = block_max(mx, red);
  const double amax_d = (double)mx;
  double scale;
  float mul = 0.f, div = 1.f;
  bool zero;
  if (recip) {
    scale = amax_d > 1e-30 ? amax_d / 127.0 : 1.0;
    const double inv = scale > 1e-30 ? 1.0 / scale : 0.0;
    mul = (float)inv;
    zero = false;
  } else {
    zero = amax_d < 1e-30;
    scale = zero ? 1.0 : amax_d / 127.0;
    div = (float)scale;
  }
  if (chunk == 0 && threadIdx.x == 0) *scale_out = scale;
  if (vec) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t w = 0;
      if (!zero) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          w |= code_of(recip ? v[j][t] * mul : v[j][t] / div) << (8 * t);
      }
      gst1((uint32_t*)(q + base) + threadIdx.x + 256 * j, w);
    }
    return;
  }
  for (int t = threadIdx.x; t < SCAO_FLAT_CHUNK; t += 256) {
    const int64_t e = base + t;
    if (e >= n) break;
    q[e] = zero ? (int8_t)0 : (int8_t)code_of(recip ? x[e] * mul : x[e] / div);
  }
}

__global__ __launch_bounds__(256) void k_requant(const scao_task* __restrict__ tasks,
                                                 const scao_gram_desc* __restrict__ descs,
                                                 double* const* __restrict__ scale_out) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_gram_desc D = descs[tk.idx];
  const int dim = D.side == 0 ? D.rows : D.cols;
  requant_chunk(D.ema, (int64_t)dim * dim, D.amax, D.ntiles, D.q, scale_out[tk.idx], tk.a, false);
}

// eigh input, pass 1 (one block per factor): shift = fp32(max(1e-8,
// 1e-4 * fp32(tr X) / dim)), the trace summed in double in a fixed order.
__device__ __forceinline__ float prep_val(const scao_prep_desc& D, float sf, int64_t e) {
  const float x = D.q ? (float)D.q[e] * sf : D.ema[e];
  return x / D.bias;
}
__global__ __launch_bounds__(256) void k_eig_trace(const scao_prep_desc* __restrict__ descs) {
  __shared__ double red[16];
  const scao_prep_desc D = descs[blockIdx.x];
  const int dim = D.dim;
  const float sf = D.q ? (float)(*D.scale) : 0.f;
  double tr = 0.0;
  for (int i = threadIdx.x; i < dim; i += 256) tr += (double)prep_val(D, sf, (int64_t)i * dim + i);
  double x[1] = {tr};
  block_sum<1>(x, red);
  if (threadIdx.x == 0) {
    const float tr_f = (float)x[0];
    double eps = 1e-4 * (double)tr_f / (double)dim;
    if (eps < 1e-8) eps = 1e-8;
    *D.shift = (float)eps;
  }
}

// eigh input, pass 2: X = deq / fp32(bias) (+ shift on the diagonal), one
// SCAO_FLAT_CHUNK-element chunk per block.  Whole aligned chunks of a
// dim % 4 == 0 factor read 4 codes (or 4 fp32) per load and write a float4,
// each wave covering a contiguous stretch per instruction.
__global__ __launch_bounds__(256) void k_eig_prep(const scao_task* __restrict__ tasks,
                                                  const scao_prep_desc* __restrict__ descs) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_prep_desc D = descs[tk.idx];
  const int dim = D.dim;
  const int64_t n = (int64_t)dim * dim;
  const int64_t base = (int64_t)tk.a * SCAO_FLAT_CHUNK;
  const uintptr_t src = D.q ? (uintptr_t)D.q : (uintptr_t)D.ema;
  const bool vec = dim % 4 == 0 && base + SCAO_FLAT_CHUNK <= n && n < (1LL << 31) &&
                   ((src | (uintptr_t)D.out) & 15) == 0;
  if (vec) {
    // the chunk's loads go out before the scale and shift are read
    v4f x[4];
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t e = base + 4 * (threadIdx.x + 256 * j);
      if (D.q)
        w[j] = gld1((const uint32_t*)(D.q + e));
      else
        x[j] = gld4_nt(D.ema + e);
    }
    const float sf = D.q ? (float)(*D.scale) : 0.f;
    const float eps = *D.shift;
    if (D.q) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) x[j][t] = (float)(int8_t)(w[j] >> (8 * t)) * sf;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = (int)(base + 4 * (threadIdx.x + 256 * j));
      const int row = e / dim, col = e - row * dim;
      v4f y;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        y[t] = x[j][t] / D.bias;
        if (col + t == row) y[t] = y[t] + eps;
      }
      gst4_nt(D.out + e, y);
    }
    return;
  }
  const float sf = D.q ? (float)(*D.scale) : 0.f;
  const float eps = *D.shift;
  for (int t = threadIdx.x; t < SCAO_FLAT_CHUNK; t += 256) {
    const int64_t e = base + t;
    if (e >= n) break;
    float y = prep_val(D, sf, e);
    if (e / dim == e % dim) y = y + eps;
    D.out[e] = y;
  }
}

// int8_ema_update pass 1: x = fp32(fp32(q*s)*rho) + v, per-block |x| max
__global__ __launch_bounds__(256) void k_ema_pass1(const int8_t* __restrict__ q, float sf,
                                                   float rho, const float* __restrict__ v,
                                                   int64_t n, float* __restrict__ x,
                                                   float* __restrict__ amax) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * SCAO_FLAT_CHUNK;
  float mx = 0.f;
  for (int t = threadIdx.x; t < SCAO_FLAT_CHUNK; t += 256) {
    const int64_t e = base + t;
    if (e >= n) break;
    const float y = ((float)q[e] * sf) * rho + v[e];
    x[e] = y;
    mx = fmaxf(mx, fabsf(y));
  }
  mx = block_max(mx, red);
  if (threadIdx.x == 0) amax[blockIdx.x] = mx;
}

__global__ __launch_bounds__(256) void k_ema_pass2(const float* __restrict__ x, int64_t n,
                                                   const float* __restrict__ amax, int nparts,
                                                   int8_t* __restrict__ q, double* scale_out) {
  requant_chunk(x, n, amax, nparts, q, scale_out, blockIdx.x, true);
}

}  // namespace

// ------------------------------------------------------------- C ABI ---
extern "C" int scao_gram_ema(const scao_task* tasks, int ntasks, const scao_gram_desc* descs,
                             void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_gram_ema: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && descs, "scao_gram_ema: null pointer");
  hipLaunchKernelGGL(k_gram_ema, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, descs);
  SCAO_LAUNCH_CHECK("scao_gram_ema");
  return SCAO_OK;
}

extern "C" int scao_requant(const scao_task* tasks, int ntasks, const scao_gram_desc* descs,
                            double* const* scale_out, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_requant: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && descs && scale_out, "scao_requant: null pointer");
  hipLaunchKernelGGL(k_requant, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, descs,
                     scale_out);
  SCAO_LAUNCH_CHECK("scao_requant");
  return SCAO_OK;
}

extern "C" int scao_eig_prep(const scao_task* tasks, int ntasks, const scao_prep_desc* descs,
                             int ndescs, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0 && ndescs >= 0, "scao_eig_prep: negative count");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && descs && ndescs > 0, "scao_eig_prep: null pointer");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_eig_trace, dim3(ndescs), dim3(256), 0, s, descs);
  hipLaunchKernelGGL(k_eig_prep, dim3(ntasks), dim3(256), 0, s, tasks, descs);
  SCAO_LAUNCH_CHECK("scao_eig_prep");
  return SCAO_OK;
}

extern "C" int64_t scao_int8_ema_scratch_bytes(int64_t n) {
  if (n <= 0) return 0;
  const int64_t parts = (n + SCAO_FLAT_CHUNK - 1) / SCAO_FLAT_CHUNK;
  return (n + parts) * (int64_t)sizeof(float);
}

extern "C" int scao_int8_ema_update(int8_t* q, double scale_in, const float* new_val, double rho,
                                    int64_t n, double* scale_out, void* scratch, void* stream) {
  SCAO_CHECK_ARG(n >= 0, "scao_int8_ema_update: n < 0");
  SCAO_CHECK_ARG(n < (int64_t)SCAO_FLAT_CHUNK * 0x7fffffffLL, "scao_int8_ema_update: n too large");
  if (n == 0) return SCAO_OK;
  SCAO_CHECK_ARG(q && new_val && scale_out && scratch, "scao_int8_ema_update: null pointer");
  const int parts = (int)((n + SCAO_FLAT_CHUNK - 1) / SCAO_FLAT_CHUNK);
  float* x = (float*)scratch;
  float* amax = x + n;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_ema_pass1, dim3(parts), dim3(256), 0, s, q, (float)scale_in, (float)rho,
                     new_val, n, x, amax);
  SCAO_LAUNCH_CHECK("scao_int8_ema_update/pass1");
  hipLaunchKernelGGL(k_ema_pass2, dim3(parts), dim3(256), 0, s, x, n, amax, parts, q, scale_out);
  SCAO_LAUNCH_CHECK("scao_int8_ema_update/pass2");
  return SCAO_OK;
}
