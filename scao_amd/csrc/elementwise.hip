// Bandwidth-bound kernels of the SCAO step on gfx950: every parameter of a
// launch is cut into SCAO_FLAT_CHUNK-element chunks, one 256-thread block per
// chunk, float4 accesses (4 x 1024 contiguous elements per block).
//
//   adam_step     Phase 1 (scao/optimizer.py:567-578): decay, Adam moments,
//                 bias-corrected step, prev_grad copy, ||g||^2   -- 32 B/elem
//   diag_reduce   Phase 2 diagonal preconditioner reductions
//                 (scao/preconditioner.py:554-556, optimizer.py:534, 371-377)
//   diag_apply    Phase 2 diagonal precondition (preconditioner.py:506-510)
//                 + the shared Adan tail
//   lars_write    p = fma(u, -(lr*trust), p*decay) (optimizer.py:642-645)
//   diag_ema      1-D curvature EMA (preconditioner.py:332-339)
//   step_finalize per-parameter norms, clip factor, LARS trust, and the
//                 global grad-norm EMA (optimizer.py:439-446, 667-678, 371-377)
#include "scao_common.hpp"

using namespace scao;

namespace {

// element range of a flat task and this thread's 4 groups of 4 elements
struct Chunk {
  int64_t base, end;
  __device__ Chunk(const scao_task& tk, int64_t numel) {
    base = (int64_t)tk.a * SCAO_FLAT_CHUNK;
    end = base + SCAO_FLAT_CHUNK < numel ? base + SCAO_FLAT_CHUNK : numel;
  }
  __device__ int64_t elem(int grp) const { return base + grp * 1024 + threadIdx.x * 4; }
  __device__ int mask(int64_t e) const {
    int mk = 0;
    for (int t = 0; t < 4; ++t) mk |= (e + t < end) ? (1 << t) : 0;
    return mk;
  }
};

__device__ __forceinline__ void write_slot(double* slots, int slot, double a, double b, double c) {
  if (slot < 0) return;
  slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = a;
  slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = b;
  slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = c;
}

// --------------------------------------------------------------- adam ---
// FAST: fp32 data, 16-byte aligned, a full 4096-element chunk -- straight-line
// non-temporal float4 traffic with every load of the thread issued first.
template <bool FAST>
__device__ __forceinline__ void adam_chunk(const scao_task& tk, const scao_param_desc& P,
                                           double* slots) {
  __shared__ double red[16];
  const int dt = FAST ? SCAO_F32 : P.dtype;
  const Chunk ch(tk, P.numel);
  const bool gf32 = P.flags & SCAO_PF_GF32;
  const bool fused = fused_mgrad(P);
  const bool fmask = P.flags & SCAO_PF_FMASK;
  const bool aligned = FAST || (al_dt(P.p, dt) && al16(P.g) && al_dt(P.graw, dt) &&
                                al16(P.exp_avg) && al16(P.exp_avg_sq) && al16(P.prev_grad) &&
                                (!fmask || al16(P.fema)));
  const bool decay = P.flags & SCAO_PF_DECAY;
  const float alpha = round_to(dt, P.adam_alpha);
  v4f g[4], gr[4], p[4], m[4], v[4];
  int mk[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t e = ch.elem(grp);
    if (FAST) {
      mk[grp] = 15;
      if (fused) {   // g holds the filter's EMA until finish_mgrad below
        gr[grp] = gld4_nt((const float*)P.graw + e);
        g[grp] = fmask ? gld4_nt(P.fema + e) : gr[grp];
      } else {
        g[grp] = gld4_nt((const float*)P.g + e);
        gr[grp] = gf32 ? gld4_nt((const float*)P.graw + e) : g[grp];
      }
      p[grp] = gld4_nt((const float*)P.p + e);
      m[grp] = gld4_nt(P.exp_avg + e);
      v[grp] = gld4_nt(P.exp_avg_sq + e);
    } else {
      mk[grp] = ch.mask(e);
      const bool vec = aligned && mk[grp] == 15;
      const v4f z = {0.f, 0.f, 0.f, 0.f};
      if (fused) {
        gr[grp] = mk[grp] ? ld4(P.graw, dt, e, vec, mk[grp]) : z;
        g[grp] = (mk[grp] && fmask) ? ldf4(P.fema, e, vec, mk[grp]) : gr[grp];
      } else {
        g[grp] = mk[grp] ? ld_mgrad(P, e, vec, mk[grp]) : z;
        gr[grp] = (mk[grp] && gf32) ? ld4(P.graw, dt, e, vec, mk[grp]) : g[grp];
      }
      p[grp] = mk[grp] ? ld4(P.p, dt, e, vec, mk[grp]) : z;
      m[grp] = mk[grp] ? ldf4(P.exp_avg, e, vec, mk[grp]) : z;
      v[grp] = mk[grp] ? ldf4(P.exp_avg_sq, e, vec, mk[grp]) : z;
    }
  }
  if (fused) {
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
      if (mk[grp]) g[grp] = finish_mgrad(P, ch.elem(grp), gr[grp], g[grp], mk[grp]);
  }
  float part = 0.f;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      part = fmaf(gr[grp][t], gr[grp][t], part);
      const float pd = decay ? round_to(dt, p[grp][t] * P.decay) : p[grp][t];
      m[grp][t] = fmaf(g[grp][t], P.omb1, m[grp][t] * P.beta1);
      v[grp][t] = fmaf(P.omb2 * g[grp][t], g[grp][t], v[grp][t] * P.beta2);
      const float den = sqrtf(v[grp][t]) / P.adam_sqrt_bc2 + P.eps;
      const float u = round_to(dt, m[grp][t] / den);
      p[grp][t] = round_to(dt, fmaf(u, alpha, pd));
    }
    const int64_t e = ch.elem(grp);
    if (FAST) {
      gst4_nt(P.exp_avg + e, m[grp]);
      gst4_nt(P.exp_avg_sq + e, v[grp]);
      gst4_nt(P.prev_grad + e, g[grp]);
      gst4_nt((float*)P.p + e, p[grp]);
    } else if (mk[grp]) {
      const bool vec = aligned && mk[grp] == 15;
      stf4(P.exp_avg, e, m[grp], vec, mk[grp]);
      stf4(P.exp_avg_sq, e, v[grp], vec, mk[grp]);
      stf4(P.prev_grad, e, g[grp], vec, mk[grp]);
      st4(P.p, dt, e, p[grp], vec, mk[grp]);
    }
  }
  double x[1] = {(double)part};
  block_sum<1>(x, red);
  if (threadIdx.x == 0) write_slot(slots, tk.slot, x[0], 0.0, 0.0);
}

__device__ __forceinline__ bool flat_fast(const scao_task& tk, const scao_param_desc& P) {
  return P.dtype == SCAO_F32 && (P.flags & SCAO_PF_ALIGNED) &&
         (int64_t)(tk.a + 1) * SCAO_FLAT_CHUNK <= P.numel;
}

__global__ __launch_bounds__(256) void k_adam(const scao_task* __restrict__ tasks,
                                              const scao_param_desc* __restrict__ params,
                                              double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_param_desc& P = params[tk.idx];
  if (flat_fast(tk, P))
    adam_chunk<true>(tk, P, slots);
  else
    adam_chunk<false>(tk, P, slots);
}

// ------------------------------------------------------- diag reduce ---
__global__ __launch_bounds__(256) void k_diag_reduce(const scao_task* __restrict__ tasks,
                                                     const scao_param_desc* __restrict__ params,
                                                     double* slots) {
  __shared__ double red[16];
  const scao_task tk = tasks[blockIdx.x];
  const scao_param_desc& P = params[tk.idx];
  const int dt = P.dtype;
  const Chunk ch(tk, P.numel);
  const bool aligned = al_dt(P.p, dt) && al_dt(P.graw, dt) && al16(P.diag_ema);
  const bool decay = P.flags & SCAO_PF_DECAY;
  const bool lars = P.flags & SCAO_PF_LARS;
  double acc[3] = {0.0, 0.0, 0.0};
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t e = ch.elem(grp);
    const int mk = ch.mask(e);
    if (!mk) continue;
    const bool vec = aligned && mk == 15;
    const v4f g = ld4(P.graw, dt, e, vec, mk);
    const v4f dg = ldf4(P.diag_ema, e, vec, mk);
    v4f p = {0.f, 0.f, 0.f, 0.f};
    if (lars) p = ld4(P.p, dt, e, vec, mk);
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (!(mk & (1 << t))) continue;
      a0 = fmaf(g[t], g[t], a0);
      const float pd = decay ? round_to(dt, p[t] * P.decay) : p[t];
      a1 = fmaf(pd, pd, a1);
      a2 += (g[t] * g[t]) / (sqrtf(dg[t]) + P.eps);
    }
    acc[0] += a0;
    acc[1] += a1;
    acc[2] += a2;
  }
  block_sum<3>(acc, red);
  if (threadIdx.x == 0) write_slot(slots, tk.slot, acc[0], acc[1], acc[2]);
}

// -------------------------------------------------------- diag apply ---
__global__ __launch_bounds__(256) void k_diag_apply(const scao_task* __restrict__ tasks,
                                                    const scao_param_desc* __restrict__ params,
                                                    const scao_param_stat* __restrict__ stat,
                                                    double* slots) {
  __shared__ double red[16];
  const scao_task tk = tasks[blockIdx.x];
  const scao_param_desc& P = params[tk.idx];
  const scao_param_stat S = stat[tk.idx];
  const int dt = P.dtype;
  const Chunk ch(tk, P.numel);
  const bool aligned = al_dt(P.p, dt) && al16(P.g) && al_dt(P.graw, dt) && al16(P.diag_ema) &&
                       al16(P.exp_avg) && al16(P.exp_avg_sq) && al16(P.exp_avg_diff) &&
                       al16(P.prev_grad) && (P.upd == nullptr || al16(P.upd)) &&
                       (!(P.flags & SCAO_PF_FMASK) || al16(P.fema));
  double u2 = 0.0;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t e = ch.elem(grp);
    const int mk = ch.mask(e);
    if (!mk) continue;
    const bool vec = aligned && mk == 15;
    const v4f graw = ld4(P.graw, dt, e, vec, mk);
    const v4f g = fused_mgrad(P)
                      ? finish_mgrad(P, e, graw,
                                     (P.flags & SCAO_PF_FMASK) ? ldf4(P.fema, e, vec, mk) : graw, mk)
                      : ((P.flags & SCAO_PF_GF32) ? ld_mgrad(P, e, vec, mk) : graw);
    const v4f dg = ldf4(P.diag_ema, e, vec, mk);
    v4f gp;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float x = dg[t] / P.diag_bias;
      const float den = (float)pow((double)x, 0.25) + 1e-8f;
      gp[t] = round_to(dt, graw[t] / den);
    }
    const v4f u = adan_tail(P, S, e, g, gp, vec, mk);
    u2 += (double)write_update(P, e, u, vec, mk);
  }
  double x[1] = {u2};
  block_sum<1>(x, red);
  if (threadIdx.x == 0) write_slot(slots, tk.slot, 0.0, 0.0, x[0]);
}

// -------------------------------------------------------- lars write ---
template <bool FAST>
__device__ __forceinline__ void lars_chunk(const scao_task& tk, const scao_param_desc& P,
                                           float alpha) {
  const int dt = FAST ? SCAO_F32 : P.dtype;
  const Chunk ch(tk, P.numel);
  const bool aligned = FAST || (al_dt(P.p, dt) && al16(P.upd));
  const bool decay = P.flags & SCAO_PF_DECAY;
  v4f u[4], p[4];
  int mk[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t e = ch.elem(grp);
    if (FAST) {
      mk[grp] = 15;
      u[grp] = gld4(P.upd + e);
      p[grp] = gld4_nt((const float*)P.p + e);
    } else {
      mk[grp] = ch.mask(e);
      const bool vec = aligned && mk[grp] == 15;
      const v4f z = {0.f, 0.f, 0.f, 0.f};
      u[grp] = mk[grp] ? ldf4(P.upd, e, vec, mk[grp]) : z;
      p[grp] = mk[grp] ? ld4(P.p, dt, e, vec, mk[grp]) : z;
    }
  }
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float pd = decay ? round_to(dt, p[grp][t] * P.decay) : p[grp][t];
      p[grp][t] = round_to(dt, fmaf(round_to(dt, u[grp][t]), alpha, pd));
    }
    const int64_t e = ch.elem(grp);
    if (FAST) {
      gst4_nt((float*)P.p + e, p[grp]);
    } else if (mk[grp]) {
      st4(P.p, dt, e, p[grp], aligned && mk[grp] == 15, mk[grp]);
    }
  }
}

__global__ __launch_bounds__(256) void k_lars_write(const scao_task* __restrict__ tasks,
                                                    const scao_param_desc* __restrict__ params,
                                                    const scao_param_stat* __restrict__ stat) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_param_desc& P = params[tk.idx];
  const float alpha = stat[tk.idx].alpha;
  if (flat_fast(tk, P))
    lars_chunk<true>(tk, P, alpha);
  else
    lars_chunk<false>(tk, P, alpha);
}

// ---------------------------------------------------------- diag ema ---
__global__ __launch_bounds__(256) void k_diag_ema(const scao_task* __restrict__ tasks,
                                                  const scao_param_desc* __restrict__ params,
                                                  const float* __restrict__ rho_alpha) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_param_desc& P = params[tk.idx];
  const float rho = rho_alpha[2 * tk.idx], alpha = rho_alpha[2 * tk.idx + 1];
  const int dt = P.dtype;
  float* dg = const_cast<float*>(P.diag_ema);
  const Chunk ch(tk, P.numel);
  const bool aligned = al_dt(P.graw, dt) && al16(dg);
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t e = ch.elem(grp);
    const int mk = ch.mask(e);
    if (!mk) continue;
    const bool vec = aligned && mk == 15;
    const v4f g = ld4(P.graw, dt, e, vec, mk);
    v4f d = ldf4(dg, e, vec, mk);
#pragma unroll
    for (int t = 0; t < 4; ++t) d[t] = d[t] * rho + alpha * (g[t] * g[t]);
    stf4(dg, e, d, vec, mk);
  }
}

// ---------------------------------------------------------- lookahead ---
// slow = slow + fp32(alpha * (p - slow)); p = slow (three roundings in the
// parameter dtype, scao/optimizer.py:363-364).  16 B/elem for fp32.
__global__ __launch_bounds__(256) void k_lookahead(const scao_task* __restrict__ tasks,
                                                   const scao_lookahead_desc* __restrict__ descs,
                                                   float alpha) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_lookahead_desc& D = descs[tk.idx];
  const int dt = D.dtype;
  const Chunk ch(tk, D.numel);
  const bool aligned = al_dt(D.p, dt) && al_dt(D.slow, dt);
  v4f p[4], w[4];
  int mk[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t e = ch.elem(grp);
    mk[grp] = ch.mask(e);
    const bool vec = aligned && mk[grp] == 15;
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    p[grp] = mk[grp] ? ld4(D.p, dt, e, vec, mk[grp]) : z;
    w[grp] = mk[grp] ? ld4(D.slow, dt, e, vec, mk[grp]) : z;
  }
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    if (!mk[grp]) continue;
    const int64_t e = ch.elem(grp);
    const bool vec = aligned && mk[grp] == 15;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float d = round_to(dt, p[grp][t] - w[grp][t]);
      const float a = round_to(dt, alpha * d);
      w[grp][t] = round_to(dt, w[grp][t] + a);
    }
    st4(D.slow, dt, e, w[grp], vec, mk[grp]);
    st4(D.p, dt, e, w[grp], vec, mk[grp]);
  }
}

// ---------------------------------------------------------- finalize ---
__global__ __launch_bounds__(256) void k_finalize_params(const scao_param_desc* __restrict__ params,
                                                         const double* __restrict__ slots,
                                                         scao_param_stat* stat, int phase) {
  __shared__ double red[16];
  const scao_param_desc& P = params[blockIdx.x];
  scao_param_stat& S = stat[blockIdx.x];
  const int l = threadIdx.x;
  const int dt = P.dtype;
  const double* __restrict__ sl = slots;
  if (phase == 0) {
    // four independent partial sums per thread keep four slot loads in
    // flight (an Adam-path embedding has tens of thousands of slots); they
    // are combined in a fixed order
    double a4[3][4] = {};
    int s = P.pre_begin + l;
    for (; s + 768 < P.pre_end; s += 1024)
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < 3; ++q) a4[q][u] += sl[(int64_t)(s + 256 * u) * SCAO_SLOT_WIDTH + q];
    for (; s < P.pre_end; s += 256)
#pragma unroll
      for (int q = 0; q < 3; ++q) a4[q][0] += sl[(int64_t)s * SCAO_SLOT_WIDTH + q];
    double a[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) a[q] = (a4[q][0] + a4[q][1]) + (a4[q][2] + a4[q][3]);
    block_sum<3>(a, red);
    if (l == 0) {
      S.g2 = a[0];
      S.p2 = a[1];
      S.nu2 = a[2];
      S.gnorm = round_to(dt, (float)sqrt(a[0]));
      S.pnorm = round_to(dt, (float)sqrt(a[1]));
      const float nu = (float)sqrt(a[2]);
      S.nu = nu;
      float clip = 1.0f;
      if ((P.flags & SCAO_PF_CLIP) && nu > P.tau) clip = (1.0f / fmaxf(nu, P.eps)) * P.tau;
      S.clip = clip;
      S.u2 = 0.0;
      S.unorm = 0.f;
      S.trust = 1.0f;
      S.alpha = round_to(dt, (float)(-P.lr));
    }
  } else {
    double a4[4] = {0.0, 0.0, 0.0, 0.0};
    int s = P.post_begin + l;
    for (; s + 768 < P.post_end; s += 1024)
#pragma unroll
      for (int u = 0; u < 4; ++u) a4[u] += sl[(int64_t)(s + 256 * u) * SCAO_SLOT_WIDTH + 2];
    for (; s < P.post_end; s += 256) a4[0] += sl[(int64_t)s * SCAO_SLOT_WIDTH + 2];
    double ax[1] = {(a4[0] + a4[1]) + (a4[2] + a4[3])};
    block_sum<1>(ax, red);
    const double a = ax[0];
    if (l == 0) {
      S.u2 = a;
      const float un = (float)sqrt(a);
      S.unorm = un;
      float trust = 1.0f;
      if ((P.flags & SCAO_PF_LARS) && !(S.pnorm == 0.f || un == 0.f)) {
        const float num = round_to(dt, P.lars * S.pnorm);
        const float wdp = round_to(dt, P.wd * S.pnorm);
        trust = num / ((un + wdp) + 1e-8f);
      }
      S.trust = trust;
      S.alpha = round_to(dt, (float)(-(P.lr * (double)trust)));
    }
  }
}

// The average of the per-parameter gradient norms, summed in parameter order
// as the reference's Python sum does; 256 threads stage each batch of norms in
// LDS so that the ordered sum does not wait on one global load per term.
__global__ __launch_bounds__(256) void k_finalize_global(const scao_param_desc* __restrict__ params,
                                                         int nparams, const scao_param_stat* stat,
                                                         double* runtime, int norm_count) {
  constexpr int B = 1024;
  __shared__ double v[B];
  __shared__ int use[B];
  double sum = 0.0;
  int cnt = 0;
  for (int b0 = 0; b0 < nparams; b0 += B) {
    const int nb = nparams - b0 < B ? nparams - b0 : B;
    for (int i = threadIdx.x; i < nb; i += 256) {
      use[i] = params[b0 + i].norm_index >= 0;
      v[i] = (double)stat[b0 + i].gnorm;
    }
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < nb; ++i)
        if (use[i]) {
          sum += v[i];
          ++cnt;
        }
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  if (cnt == 0 || cnt != norm_count) {
    runtime[1] = 0.0;
    return;
  }
  const double avg = sum / (double)cnt;
  runtime[1] = avg;
  runtime[0] = 0.95 * runtime[0] + 0.05 * avg;
}

}  // namespace

// ------------------------------------------------------------- C ABI ---
#define FLAT_LAUNCH(name, kernel, ...)                                                        \
  do {                                                                                        \
    SCAO_CHECK_ARG(ntasks >= 0, name ": ntasks < 0");                                        \
    if (ntasks == 0) return SCAO_OK;                                                          \
    SCAO_CHECK_ARG(tasks && params, name ": null pointer");                                  \
    hipLaunchKernelGGL(kernel, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, __VA_ARGS__); \
    SCAO_LAUNCH_CHECK(name);                                                                  \
    return SCAO_OK;                                                                           \
  } while (0)

extern "C" int scao_adam_step(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                              double* slots, void* stream) {
  SCAO_CHECK_ARG(slots || ntasks == 0, "scao_adam_step: null slots");
  FLAT_LAUNCH("scao_adam_step", k_adam, tasks, params, slots);
}

extern "C" int scao_diag_reduce(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                                double* slots, void* stream) {
  SCAO_CHECK_ARG(slots || ntasks == 0, "scao_diag_reduce: null slots");
  FLAT_LAUNCH("scao_diag_reduce", k_diag_reduce, tasks, params, slots);
}

extern "C" int scao_diag_apply(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                               const scao_param_stat* stat, double* slots, void* stream) {
  SCAO_CHECK_ARG((slots && stat) || ntasks == 0, "scao_diag_apply: null pointer");
  FLAT_LAUNCH("scao_diag_apply", k_diag_apply, tasks, params, stat, slots);
}

extern "C" int scao_lars_write(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                               const scao_param_stat* stat, void* stream) {
  SCAO_CHECK_ARG(stat || ntasks == 0, "scao_lars_write: null stat");
  FLAT_LAUNCH("scao_lars_write", k_lars_write, tasks, params, stat);
}

extern "C" int scao_lookahead(const scao_task* tasks, int ntasks,
                              const scao_lookahead_desc* descs, float alpha, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_lookahead: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && descs, "scao_lookahead: null pointer");
  hipLaunchKernelGGL(k_lookahead, dim3(ntasks), dim3(256), 0, (hipStream_t)stream, tasks, descs,
                     alpha);
  SCAO_LAUNCH_CHECK("scao_lookahead");
  return SCAO_OK;
}

extern "C" int scao_diag_ema(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                             const float* rho_alpha, void* stream) {
  SCAO_CHECK_ARG(rho_alpha || ntasks == 0, "scao_diag_ema: null rho_alpha");
  FLAT_LAUNCH("scao_diag_ema", k_diag_ema, tasks, params, rho_alpha);
}

extern "C" int scao_step_finalize(const scao_param_desc* params, int nparams, const double* slots,
                                  scao_param_stat* stat, double* runtime, int phase,
                                  int update_norm_ema, int norm_count, void* stream) {
  SCAO_CHECK_ARG(nparams >= 0 && (phase == 0 || phase == 1), "scao_step_finalize: bad args");
  if (nparams == 0) return SCAO_OK;
  SCAO_CHECK_ARG(params && slots && stat, "scao_step_finalize: null pointer");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_finalize_params, dim3(nparams), dim3(256), 0, s, params, slots, stat, phase);
  SCAO_LAUNCH_CHECK("scao_step_finalize");
  if (phase == 0 && update_norm_ema) {
    SCAO_CHECK_ARG(runtime != nullptr, "scao_step_finalize: null runtime");
    hipLaunchKernelGGL(k_finalize_global, dim3(1), dim3(256), 0, s, params, nparams, stat, runtime,
                       norm_count);
    SCAO_LAUNCH_CHECK("scao_step_finalize/global");
  }
  return SCAO_OK;
}
