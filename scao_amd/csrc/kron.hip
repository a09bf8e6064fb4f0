// Kronecker-block kernels of the SCAO step on gfx950 (fp32 MFMA 16x16x4).
//
// Per block (m x n, rank k) the reference computes, in
// scao/cuda/__init__.py:78-99 (the path scao/preconditioner.py:519 takes):
//     P = (U_l^T G) U_r ;  Delta = (s_l s_r^T - 1) * P ;  out = G + (U_l Delta) U_r^T
// and, for the curvature clip (scao/preconditioner.py:558-564), the Frobenius
// norm of clamp(S_l,eps)^-1/2 * P * clamp(S_r,eps)^-1/2.  Here that is four
// kernels so every block of every parameter runs in one launch per stage:
//   project  T = U_l^T G                 (4mnk/2 flops, reads G once; MFMA)
//   delta    P = T U_r, Delta, nu^2      (k x k per block)
//   lift     W = U_l Delta               (m x k per block)
//   apply    out = G + W U_r^T, fused with the optimizer's elementwise tail
//
// Lane layouts.  For v_mfma_f32_16x16x4_f32 lane l supplies A[l%16][l/16],
// B[l/16][l%16] and receives D[4*(l/16)+r][l%16].  Two index permutations keep
// global accesses vectorised:
//   * output columns: MFMA tile t, column jj maps to matrix column
//     j0 + 4*jj + t, so one float4 per lane feeds (or receives) four tiles;
//   * reduction index: K-step s of a 16-wide chunk uses index
//     kb + 4*(l/16) + s, so one float4 per lane feeds four K-steps.
// Both only reorder an exact sum, so they change rounding order, never terms.
#include "scao_common.hpp"

using namespace scao;

namespace {

// ----------------------------------------------------------- project ---
// T[c0:c0+64, j0:j0+256] = U_l^T G over all m rows.  Wave w owns 64 columns.
// Chunk 0 tasks also reduce ||g||^2 and ||p*decay||^2 over their columns.
__device__ __forceinline__ void project_tile(const scao_leaf_desc& L, const scao_param_desc& P, int j0,
                             int c0, int slot, double* slots) {
  __shared__ double red[16];
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, n = L.n, k = L.k;
  const int64_t ld = L.ld;
  const int dt = P.dtype;
  const int jl = j0 + 64 * w + 4 * (l % 16);
  const int kk = l / 16;
  const int cl = c0 + (l % 16);
  int cmask = 0;
  for (int t = 0; t < 4; ++t) cmask |= (jl + t < n) ? (1 << t) : 0;
  const bool vec = (L.flags & SCAO_LF_VEC4) && cmask == 15;
  const bool do_norms = (c0 == 0) && slot >= 0;
  const bool do_p = do_norms && (P.flags & SCAO_PF_LARS);
  const bool decay = P.flags & SCAO_PF_DECAY;
  const float* Ul = L.Ul;

  v4f acc[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[q][t] = v4f{0.f, 0.f, 0.f, 0.f};
  double g2 = 0.0, p2 = 0.0;

  // two-stage register pipeline over 16-row groups
  v4f bq[4], bn[4];
  float aq[4][4], an[4][4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bn[s] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) an[s][q] = 0.f;
  }
  auto load_stage = [&](int i0, v4f (&b)[4], float (&a)[4][4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = i0 + 4 * s + kk;
      const bool rok = i < m;
      b[s] = rok && cmask ? ld4(P.graw, dt, L.off + (int64_t)i * ld + jl, vec, cmask)
                          : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = cl + 16 * q;
        a[s][q] = (rok && c < k) ? Ul[(int64_t)i * k + c] : 0.f;
      }
    }
  };
  load_stage(0, bq, aq);
  for (int i0 = 0; i0 < m; i0 += 16) {
    if (i0 + 16 < m) load_stage(i0 + 16, bn, an);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[q][t] = mfma16(aq[s][q], bq[s][t], acc[q][t]);
    if (do_norms) {
      float part = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) part = fmaf(bq[s][t], bq[s][t], part);
      g2 += (double)part;
      if (do_p) {
        float pp = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int i = i0 + 4 * s + kk;
          if (i < m && cmask) {
            v4f pv = ld4(P.p, dt, L.off + (int64_t)i * ld + jl, vec, cmask);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              float x = decay ? round_to(dt, pv[t] * P.decay) : pv[t];
              pp = fmaf(x, x, pp);
            }
          }
        }
        p2 += (double)pp;
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bq[s] = bn[s];
#pragma unroll
      for (int q = 0; q < 4; ++q) aq[s][q] = an[s][q];
    }
  }
  // T[c][j] for c = c0 + 16q + 4*(l/16) + r, j = jl + t
  const bool tvec = (L.flags & SCAO_LF_VEC4) && cmask == 15;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = c0 + 16 * q + 4 * kk + r;
      if (c < k && cmask) {
        v4f o = {acc[q][0][r], acc[q][1][r], acc[q][2][r], acc[q][3][r]};
        stf4(L.T, (int64_t)c * n + jl, o, tvec, cmask);
      }
    }
  if (do_norms) {
    double x[2] = {g2, p2};
    block_sum<2>(x, red);
    if (threadIdx.x == 0) {
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = x[0];
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = x[1];
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = 0.0;
    }
  }
}

// ------------------------------------------------------------- delta ---
// P[c0:c0+64, d0:d0+64] = T U_r; Delta and the natural-norm partial.
__device__ __forceinline__ void delta_tile(const scao_leaf_desc& L, float eps, int c0, int d0, int slot,
                           double* slots) {
  __shared__ double red[16];
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int n = L.n, k = L.k;
  const int kk = l / 16;
  const int crow = c0 + 16 * w + (l % 16);  // A row supplied by this lane
  const bool tvec = (L.flags & SCAO_LF_VEC4) != 0;
  const float* T = L.T;
  const float* Ur = L.Ur;
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int jb = 0; jb < n; jb += 16) {
    const int j = jb + 4 * kk;
    int jm = 0;
    for (int s = 0; s < 4; ++s) jm |= (j + s < n) ? (1 << s) : 0;
    v4f a = (crow < k && jm) ? ldf4(T, (int64_t)crow * n + j, tvec && jm == 15, jm)
                             : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int d = d0 + 16 * t + (l % 16);
        const float b = ((jm >> s) & 1) && d < k ? Ur[(int64_t)(j + s) * k + d] : 0.f;
        acc[t] = mfma16(a[s], b, acc[t]);
      }
    }
  }
  const bool sinv4 = L.flags & SCAO_LF_SINV4;
  double nu2 = 0.0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = c0 + 16 * w + 4 * kk + r;
    if (c >= k) continue;
    const float sl = L.Sl[c];
    const float sl4 = sinv4 ? sl : inv4(sl);
    const float il2 = sinv4 ? 0.f : inv2(sl, eps);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = d0 + 16 * t + (l % 16);
      if (d >= k) continue;
      const float sr = L.Sr[d];
      const float sr4 = sinv4 ? sr : inv4(sr);
      const float pv = acc[t][r];
      L.Delta[(int64_t)c * k + d] = (sl4 * sr4 - 1.0f) * pv;
      if (!sinv4) {
        const float x = (il2 * pv) * inv2(sr, eps);
        nu2 += (double)x * (double)x;
      }
    }
  }
  if (slot >= 0) {
    double x[1] = {nu2};
    block_sum<1>(x, red);
    if (threadIdx.x == 0) {
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = 0.0;
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = 0.0;
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = x[0];
    }
  }
}

// -------------------------------------------------------------- lift ---
// W[i0:i0+64, d0:d0+64] = U_l Delta.
__device__ __forceinline__ void lift_tile(const scao_leaf_desc& L, int i0, int d0) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, k = L.k;
  const int kk = l / 16;
  const int irow = i0 + 16 * w + (l % 16);
  const bool kvec = (k % 4) == 0;
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int cb = 0; cb < k; cb += 16) {
    const int c = cb + 4 * kk;
    int cm = 0;
    for (int s = 0; s < 4; ++s) cm |= (c + s < k) ? (1 << s) : 0;
    v4f a = (irow < m && cm) ? ldf4(L.Ul, (int64_t)irow * k + c, kvec && cm == 15, cm)
                             : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int d = d0 + 16 * t + (l % 16);
        const float b = ((cm >> s) & 1) && d < k ? L.Delta[(int64_t)(c + s) * k + d] : 0.f;
        acc[t] = mfma16(a[s], b, acc[t]);
      }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = i0 + 16 * w + 4 * kk + r;
    if (i >= m) continue;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = d0 + 16 * t + (l % 16);
      if (d < k) L.W[(int64_t)i * k + d] = acc[t][r];
    }
  }
}

// ------------------------------------------------------------- apply ---
// corr[i0:i0+64, j0:j0+64] = W U_r^T; the caller's epilogue consumes it.
// Returns, per lane, corr for rows i0+16w+4*(l/16)+r and columns jl..jl+3.
__device__ __forceinline__ void corr_tile(const scao_leaf_desc& L, int i0, int jl, v4f (&acc)[4]) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, n = L.n, k = L.k;
  const int kk = l / 16;
  const int irow = i0 + 16 * w + (l % 16);
  const bool kvec = (k % 4) == 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int cb = 0; cb < k; cb += 16) {
    const int c = cb + 4 * kk;
    int cm = 0;
    for (int s = 0; s < 4; ++s) cm |= (c + s < k) ? (1 << s) : 0;
    const v4f a = (irow < m && cm) ? ldf4(L.W, (int64_t)irow * k + c, kvec && cm == 15, cm)
                                   : v4f{0.f, 0.f, 0.f, 0.f};
    v4f b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = jl + t;
      b[t] = (j < n && cm) ? ldf4(L.Ur, (int64_t)j * k + c, kvec && cm == 15, cm)
                           : v4f{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = mfma16(a[s], b[t][s], acc[t]);
  }
}

}  // namespace

namespace {

__device__ __forceinline__ void apply_tile(const scao_leaf_desc& L, const scao_param_desc& P,
                           const scao_param_stat& S, int i0, int j0, int slot, double* slots) {
  __shared__ double red[16];
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, n = L.n;
  const int dt = P.dtype;
  const int jl = j0 + 4 * (l % 16);
  v4f acc[4];
  corr_tile(L, i0, jl, acc);
  int cmask = 0;
  for (int t = 0; t < 4; ++t) cmask |= (jl + t < n) ? (1 << t) : 0;
  const bool vec = (L.flags & SCAO_LF_VEC4) && cmask == 15;
  double u2 = 0.0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = i0 + 16 * w + 4 * (l / 16) + r;
    if (i >= m || !cmask) continue;
    const int64_t e = L.off + (int64_t)i * L.ld + jl;
    const v4f graw = ld4(P.graw, dt, e, vec, cmask);
    const v4f g = (P.flags & SCAO_PF_GF32) ? ld_mgrad(P, e, vec, cmask) : graw;
    v4f gp;
#pragma unroll
    for (int t = 0; t < 4; ++t) gp[t] = round_to(dt, graw[t] + acc[t][r]);
    const v4f u = adan_tail(P, S, e, g, gp, vec, cmask);
    u2 += (double)write_update(P, e, u, vec, cmask);
  }
  if (slot >= 0) {
    double x[1] = {u2};
    block_sum<1>(x, red);
    if (threadIdx.x == 0) {
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = 0.0;
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = 0.0;
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = x[0];
    }
  }
}

// Reference operator: out = G + W U_r^T (dense m x n output).
__device__ __forceinline__ void apply_out_tile(const scao_leaf_desc& L, const float* G, float* out, int i0,
                               int j0) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, n = L.n;
  const int jl = j0 + 4 * (l % 16);
  v4f acc[4];
  corr_tile(L, i0, jl, acc);
  int cmask = 0;
  for (int t = 0; t < 4; ++t) cmask |= (jl + t < n) ? (1 << t) : 0;
  const bool gvec = (L.flags & SCAO_LF_VEC4) && cmask == 15;
  const bool ovec = (n % 4 == 0) && cmask == 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = i0 + 16 * w + 4 * (l / 16) + r;
    if (i >= m || !cmask) continue;
    const v4f g = ldf4(G, (int64_t)i * L.ld + jl, gvec, cmask);
    v4f o;
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = g[t] + acc[t][r];
    stf4(out, (int64_t)i * n + jl, o, ovec, cmask);
  }
}

// ---------------------------------------------------------- kernels ---
__global__ __launch_bounds__(256) void k_project(const scao_task* __restrict__ tasks,
                                                 const scao_leaf_desc* __restrict__ leaves,
                                                 const scao_param_desc* __restrict__ params,
                                                 double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  project_tile(L, params[L.param], tk.a, tk.b, tk.slot, slots);
}
__global__ __launch_bounds__(256) void k_delta(const scao_task* __restrict__ tasks,
                                               const scao_leaf_desc* __restrict__ leaves,
                                               const scao_param_desc* __restrict__ params,
                                               double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  delta_tile(L, params[L.param].eps, tk.a, tk.b, tk.slot, slots);
}
__global__ __launch_bounds__(256) void k_lift(const scao_task* __restrict__ tasks,
                                              const scao_leaf_desc* __restrict__ leaves) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  lift_tile(L, tk.a, tk.b);
}
__global__ __launch_bounds__(256) void k_apply(const scao_task* __restrict__ tasks,
                                               const scao_leaf_desc* __restrict__ leaves,
                                               const scao_param_desc* __restrict__ params,
                                               const scao_param_stat* __restrict__ stat,
                                               double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  apply_tile(L, params[L.param], stat[L.param], tk.a, tk.b, tk.slot, slots);
}

// single-block reference operator (descriptors by value, tiles from blockIdx)
__global__ __launch_bounds__(256) void k_project_one(scao_leaf_desc L, scao_param_desc P) {
  const int strips = (L.n + SCAO_PROJ_COLS - 1) / SCAO_PROJ_COLS;
  project_tile(L, P, (blockIdx.x % strips) * SCAO_PROJ_COLS, (blockIdx.x / strips) * 64, -1,
               nullptr);
}
__global__ __launch_bounds__(256) void k_delta_one(scao_leaf_desc L) {
  const int tiles = (L.k + 63) / 64;
  delta_tile(L, 1e-8f, (blockIdx.x / tiles) * 64, (blockIdx.x % tiles) * 64, -1, nullptr);
}
__global__ __launch_bounds__(256) void k_lift_one(scao_leaf_desc L) {
  const int tiles = (L.k + 63) / 64;
  lift_tile(L, (blockIdx.x / tiles) * 64, (blockIdx.x % tiles) * 64);
}
__global__ __launch_bounds__(256) void k_apply_out_one(scao_leaf_desc L, const float* G,
                                                      float* out) {
  const int tiles = (L.n + 63) / 64;
  apply_out_tile(L, G, out, (blockIdx.x / tiles) * 64, (blockIdx.x % tiles) * 64);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// ------------------------------------------------------------- C ABI ---
extern "C" int scao_kron_project(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                                 const scao_param_desc* params, double* slots, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_kron_project: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && leaves && params && slots, "scao_kron_project: null pointer");
  hipLaunchKernelGGL(k_project, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, leaves,
                     params, slots);
  SCAO_LAUNCH_CHECK("scao_kron_project");
  return SCAO_OK;
}

extern "C" int scao_kron_delta(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                               const scao_param_desc* params, double* slots, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_kron_delta: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && leaves && params && slots, "scao_kron_delta: null pointer");
  hipLaunchKernelGGL(k_delta, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, leaves,
                     params, slots);
  SCAO_LAUNCH_CHECK("scao_kron_delta");
  return SCAO_OK;
}

extern "C" int scao_kron_lift(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                              void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_kron_lift: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && leaves, "scao_kron_lift: null pointer");
  hipLaunchKernelGGL(k_lift, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, leaves);
  SCAO_LAUNCH_CHECK("scao_kron_lift");
  return SCAO_OK;
}

extern "C" int scao_kron_apply(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                               const scao_param_desc* params, const scao_param_stat* stat,
                               double* slots, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_kron_apply: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && leaves && params && stat && slots, "scao_kron_apply: null pointer");
  hipLaunchKernelGGL(k_apply, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, leaves,
                     params, stat, slots);
  SCAO_LAUNCH_CHECK("scao_kron_apply");
  return SCAO_OK;
}

extern "C" int64_t scao_fused_kronecker_workspace(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return (k * n + k * k + m * k) * (int64_t)sizeof(float);
}

extern "C" int scao_fused_kronecker_precond(const float* U_l, const float* s_l_inv4,
                                            const float* U_r, const float* s_r_inv4,
                                            const float* G, int64_t ldG, float* out, int64_t m,
                                            int64_t n, int64_t k, void* workspace,
                                            void* stream) {
  SCAO_CHECK_ARG(U_l && s_l_inv4 && U_r && s_r_inv4 && G && out && workspace,
                 "scao_fused_kronecker_precond: null pointer");
  SCAO_CHECK_ARG(m > 0 && n > 0 && k > 0 && ldG >= n,
                 "scao_fused_kronecker_precond: bad shape m=%lld n=%lld k=%lld ldG=%lld",
                 (long long)m, (long long)n, (long long)k, (long long)ldG);
  SCAO_CHECK_ARG(m < (1LL << 31) && n < (1LL << 31) && k <= 4096,
                 "scao_fused_kronecker_precond: dimension too large");
  float* ws = (float*)workspace;
  scao_leaf_desc L = {};
  L.Ul = U_l;
  L.Ur = U_r;
  L.Sl = s_l_inv4;
  L.Sr = s_r_inv4;
  L.T = ws;
  L.Delta = ws + k * n;
  L.W = ws + k * n + k * k;
  L.off = 0;
  L.ld = ldG;
  L.param = 0;
  L.m = (int)m;
  L.n = (int)n;
  L.k = (int)k;
  L.flags = SCAO_LF_SINV4;
  if (ldG % 4 == 0 && n % 4 == 0 && aligned16(G) && aligned16(ws) && aligned16(L.T))
    L.flags |= SCAO_LF_VEC4;
  scao_param_desc P = {};
  P.g = G;
  P.graw = G;
  P.dtype = SCAO_F32;
  hipStream_t s = (hipStream_t)stream;
  const int strips = (int)((n + SCAO_PROJ_COLS - 1) / SCAO_PROJ_COLS);
  const int kt = (int)((k + 63) / 64);
  hipLaunchKernelGGL(k_project_one, dim3(strips * kt), dim3(256), 0, s, L, P);
  SCAO_LAUNCH_CHECK("scao_fused_kronecker_precond/project");
  hipLaunchKernelGGL(k_delta_one, dim3(kt * kt), dim3(256), 0, s, L);
  SCAO_LAUNCH_CHECK("scao_fused_kronecker_precond/delta");
  hipLaunchKernelGGL(k_lift_one, dim3((int)((m + 63) / 64) * kt), dim3(256), 0, s, L);
  SCAO_LAUNCH_CHECK("scao_fused_kronecker_precond/lift");
  hipLaunchKernelGGL(k_apply_out_one, dim3((int)((m + 63) / 64) * (int)((n + 63) / 64)),
                     dim3(256), 0, s, L, G, out);
  SCAO_LAUNCH_CHECK("scao_fused_kronecker_precond/apply");
  return SCAO_OK;
}
