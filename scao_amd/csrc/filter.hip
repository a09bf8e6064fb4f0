// Sparse gradient filter on gfx950 (scao/optimizer.py:42-57, the default
// sparsity=0.7 path): magnitude EMA, exact linear-interpolated quantile of the
// EMA, and the mask, batched over every filtered parameter of a step.
//
//   ema   e = |g| on the first call, else fp32(fp32(e*decay) + fp32(omd*|g|))
//         (mag_ema.mul_(ema).add_((1-ema)*mag): three roundings, no fusion)
//   t     torch.quantile(e, q), interpolation "linear": ranks = fp32(q*(n-1)),
//         lo = trunc(ranks), hi = ceil(ranks), w = ranks - lo, and ATen's lerp
//         fma(w, v_hi - v_lo, v_lo) for |w| < 0.5, else
//         fma(-(v_hi - v_lo), 1 - w, v_hi); NaN when any e is NaN (the
//         reference's rank then points at the sorted NaN)
//   out   g * (e >= t ? 1 : 0) in fp32 (NaN/inf gradients propagate as in
//         the reference's multiply); descs without SCAO_FILTER_MASK pass g
//         through.  With noise > 0, out + fp32(noise * z) (grad +
//         randn_like(grad) * noise_std, :544-545), z from Philox4x32-10
//         (Salmon et al., SC'11) keyed by the desc's seed with the element
//         index / 4 as counter, turned into normals by Box-Muller.
//
// The two order statistics come from an exact radix select on the bit
// patterns of e (e >= 0, so unsigned order is float order): digits of 11, 11
// and 10 bits, each a streaming pass that builds per-block LDS histograms and
// flushes the non-zero bins into the parameter's global histogram with
// vector atomics, followed by a one-block-per-parameter select that scans the
// histogram, narrows both targets and clears the histogram for the next pass.
// The first digit's histogram is built by the EMA pass itself.
#include "scao_common.hpp"

using namespace scao;

namespace {

constexpr int NB = SCAO_FILTER_BINS;   // 2048
constexpr int SHIFT[3] = {21, 10, 0};
constexpr uint32_t DMASK[3] = {2047u, 2047u, 1023u};

// per-parameter scratch: hist[2][NB], then the selection state
struct FState {
  uint32_t prefix[2];   // key bits selected so far (target lo, hi)
  uint32_t rank[2];     // rank still to skip inside the current prefix
  uint32_t nan;         // NaN count of this call (reset by the last select)
  uint32_t split;       // targets have different prefixes (two histograms)
  float w;              // interpolation weight
  float thr;            // the threshold, written by the last select
};
static_assert(sizeof(FState) == 4 * (SCAO_FILTER_WORK_WORDS - 2 * SCAO_FILTER_BINS),
              "state words");

__device__ __forceinline__ uint32_t* hist_of(const scao_filter_desc& D, int t) {
  return D.work + t * NB;
}
__device__ __forceinline__ FState* state_of(const scao_filter_desc& D) {
  return (FState*)(D.work + 2 * NB);
}

struct FChunk {
  int64_t base, end;
  __device__ FChunk(const scao_task& tk, int64_t numel) {
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

__device__ __forceinline__ bool is_nan_key(uint32_t k) { return (k & 0x7fffffffu) > 0x7f800000u; }

__device__ __forceinline__ void zero_lds(uint32_t* h, int n) {
  for (int i = threadIdx.x; i < n; i += 256) h[i] = 0u;
}

// add the block's non-zero bins to the global histogram
__device__ __forceinline__ void flush(const uint32_t* h, uint32_t* g, int n) {
  for (int i = threadIdx.x; i < n; i += 256) {
    const uint32_t c = h[i];
    if (c) atomicAdd(g + i, c);
  }
}

// ---------------------------------------------- pass 0: EMA + digit 0 ---
__global__ __launch_bounds__(256) void k_filter_ema(const scao_task* __restrict__ tasks,
                                                    const scao_filter_desc* __restrict__ descs) {
  __shared__ uint32_t h[NB];
  __shared__ uint32_t nan_s;
  const scao_task tk = tasks[blockIdx.x];
  const scao_filter_desc& D = descs[tk.idx];
  if (!(D.flags & SCAO_FILTER_MASK)) return;
  const bool first = D.flags & SCAO_FILTER_FIRST;
  const FChunk ch(tk, D.numel);
  zero_lds(h, NB);
  if (threadIdx.x == 0) nan_s = 0u;
  const bool vec = ((uintptr_t)D.ema & 15) == 0 && al_dt(D.g, D.dtype);
  v4f g[4], e[4];
  int mk[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t i = ch.elem(grp);
    mk[grp] = ch.mask(i);
    const bool v = vec && mk[grp] == 15;
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    g[grp] = mk[grp] ? ld4(D.g, D.dtype, i, v, mk[grp]) : z;
    e[grp] = (mk[grp] && !first) ? ldf4(D.ema, i, v, mk[grp]) : z;
  }
  __syncthreads();
  uint32_t nans = 0;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    if (!mk[grp]) continue;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float mag = fabsf(g[grp][t]);
      const float x = first ? mag : (e[grp][t] * D.decay) + (D.omd * mag);
      e[grp][t] = x;
      if (mk[grp] & (1 << t)) {
        const uint32_t key = __float_as_uint(x);
        if (is_nan_key(key))
          ++nans;
        else
          atomicAdd(&h[key >> SHIFT[0]], 1u);
      }
    }
    stf4(D.ema, ch.elem(grp), e[grp], vec && mk[grp] == 15, mk[grp]);
  }
  if (nans) atomicAdd(&nan_s, nans);
  __syncthreads();
  flush(h, hist_of(D, 0), NB);
  if (threadIdx.x == 0 && nan_s) atomicAdd(&state_of(D)->nan, nan_s);
}

// -------------------------------------------- passes 1, 2: digits 1, 2 ---
// A block takes FH consecutive tasks.  All their loads go out first (nothing
// they read depends on the selection state); the LDS histograms are flushed
// to the parameter's global ones whenever the next task belongs to another
// parameter, and at the end.
constexpr int FH = 4;

__global__ __launch_bounds__(256) void k_filter_hist(const scao_task* __restrict__ tasks,
                                                     int ntasks,
                                                     const scao_filter_desc* __restrict__ descs,
                                                     int pass) {
  __shared__ uint32_t h[2][NB];
  const int t0 = blockIdx.x * FH;
  const int nt = ntasks - t0 < FH ? ntasks - t0 : FH;
  v4f e[FH][4];
  int mk[FH][4];
#pragma unroll
  for (int c = 0; c < FH; ++c) {
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) mk[c][grp] = 0;
    if (c >= nt) continue;
    const scao_task tk = tasks[t0 + c];
    const scao_filter_desc& D = descs[tk.idx];
    if (!(D.flags & SCAO_FILTER_MASK)) continue;
    const FChunk ch(tk, D.numel);
    const bool vec = ((uintptr_t)D.ema & 15) == 0;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int64_t i = ch.elem(grp);
      mk[c][grp] = ch.mask(i);
      e[c][grp] = mk[c][grp] ? ldf4(D.ema, i, vec && mk[c][grp] == 15, mk[c][grp])
                             : v4f{0.f, 0.f, 0.f, 0.f};
    }
  }
  const int sh_prev = SHIFT[pass - 1], sh = SHIFT[pass];
  const uint32_t dm = DMASK[pass];
  const int nb = (int)dm + 1;
  zero_lds(&h[0][0], 2 * NB);
  int cur = -1;
  uint32_t p0 = 0, p1 = 0;
  bool split = false;
#pragma unroll
  for (int c = 0; c < FH; ++c) {
    if (c >= nt) break;
    const int idx = tasks[t0 + c].idx;
    if (!(descs[idx].flags & SCAO_FILTER_MASK)) continue;
    if (idx != cur) {
      if (cur >= 0) {
        __syncthreads();
        flush(&h[0][0], hist_of(descs[cur], 0), nb);
        if (split) flush(&h[1][0], hist_of(descs[cur], 1), nb);
        __syncthreads();
        zero_lds(&h[0][0], 2 * NB);
      }
      cur = idx;
      const FState* S = state_of(descs[cur]);
      p0 = S->prefix[0];
      p1 = S->prefix[1];
      split = S->split != 0u;
      __syncthreads();
    }
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (!(mk[c][grp] & (1 << t))) continue;
        const uint32_t key = __float_as_uint(e[c][grp][t]);
        const uint32_t top = key >> sh_prev;
        if (top == p0) atomicAdd(&h[0][(key >> sh) & dm], 1u);
        if (split && top == p1) atomicAdd(&h[1][(key >> sh) & dm], 1u);
      }
    }
  }
  __syncthreads();
  if (cur >= 0) {
    flush(&h[0][0], hist_of(descs[cur], 0), nb);
    if (split) flush(&h[1][0], hist_of(descs[cur], 1), nb);
  }
}

// Inclusive prefix sums of NB counts held 8 per thread (256 threads); finds,
// for rank r, the first bin whose running count exceeds r.  Returns the bin
// in *bin_out and the count before it in *before_out (from one thread).
__device__ __forceinline__ void find_bin(const uint32_t* h, uint32_t r, uint32_t* scan,
                                         uint32_t* bin_out, uint32_t* before_out) {
  const int l = threadIdx.x;
  uint32_t c[8], s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c[i] = h[8 * l + i];
    s += c[i];
  }
  scan[l] = s;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {   // Hillis-Steele inclusive scan
    const uint32_t v = l >= off ? scan[l - off] : 0u;
    __syncthreads();
    scan[l] += v;
    __syncthreads();
  }
  uint32_t run = l ? scan[l - 1] : 0u;
  if (run <= r && r < scan[l]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (run <= r && r < run + c[i]) {
        *bin_out = (uint32_t)(8 * l + i);
        *before_out = run;
      }
      run += c[i];
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------- select ---
__global__ __launch_bounds__(256) void k_filter_select(const scao_filter_desc* __restrict__ descs,
                                                       int pass) {
  __shared__ uint32_t h[2][NB];
  __shared__ uint32_t scan[256];
  __shared__ uint32_t bin[2], before[2];
  const scao_filter_desc& D = descs[blockIdx.x];
  if (!(D.flags & SCAO_FILTER_MASK)) return;
  FState* S = state_of(D);
  uint32_t r[2], pre[2];
  bool split;
  if (pass == 0) {
    // ranks = fp32(q * (n - 1)) as torch.quantile computes them
    const float ranks = D.q * (float)(D.numel - 1);
    const uint32_t lo = (uint32_t)ranks;
    const uint32_t hi = (uint32_t)ceilf(ranks);
    r[0] = lo;
    r[1] = hi;
    pre[0] = pre[1] = 0u;
    split = false;
    if (threadIdx.x == 0) S->w = ranks - (float)lo;
  } else {
    r[0] = S->rank[0];
    r[1] = S->rank[1];
    pre[0] = S->prefix[0];
    pre[1] = S->prefix[1];
    split = S->split != 0u;
  }
  if (threadIdx.x < 2) {   // defined result when no bin holds the rank (NaNs present)
    bin[threadIdx.x] = 0u;
    before[threadIdx.x] = 0u;
  }
  uint32_t* g0 = hist_of(D, 0);
  uint32_t* g1 = hist_of(D, 1);
  for (int i = threadIdx.x; i < NB; i += 256) {
    h[0][i] = g0[i];
    h[1][i] = split ? g1[i] : h[0][i];
  }
  __syncthreads();
  // leave the histograms zero for the next pass / call
  for (int i = threadIdx.x; i < NB; i += 256) {
    g0[i] = 0u;
    if (split) g1[i] = 0u;
  }
  for (int t = 0; t < 2; ++t) find_bin(&h[t][0], r[t], scan, &bin[t], &before[t]);
  if (threadIdx.x == 0) {
    const int bits = pass == 2 ? 10 : 11;
    uint32_t np[2];
    for (int t = 0; t < 2; ++t) {
      np[t] = (pre[t] << bits) | bin[t];
      S->prefix[t] = np[t];
      S->rank[t] = r[t] - before[t];
    }
    S->split = np[0] != np[1] ? 1u : 0u;
    if (pass == 2) {
      const float vlo = __uint_as_float(np[0]), vhi = __uint_as_float(np[1]);
      const float w = S->w;
      const float d = vhi - vlo;
      float thr = fabsf(w) < 0.5f ? fmaf(w, d, vlo) : fmaf(-d, 1.0f - w, vhi);
      if (S->nan) thr = __uint_as_float(0x7fc00000u);
      S->thr = thr;
      S->nan = 0u;
      S->split = 0u;
    }
  }
}

// ---------------------------------------------------------------- out ---
__global__ __launch_bounds__(256) void k_filter_out(const scao_task* __restrict__ tasks,
                                                    const scao_filter_desc* __restrict__ descs) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_filter_desc& D = descs[tk.idx];
  if (D.out == nullptr) return;   // the step kernels form the values themselves
  const FChunk ch(tk, D.numel);
  const bool masked = D.flags & SCAO_FILTER_MASK;
  const bool vec = ((((uintptr_t)D.ema) | (uintptr_t)D.out) & 15) == 0 && al_dt(D.g, D.dtype);
  v4f g[4], e[4];
  int mk[4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int64_t i = ch.elem(grp);
    mk[grp] = ch.mask(i);
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    const bool v = vec && mk[grp] == 15;
    g[grp] = mk[grp] ? ld4(D.g, D.dtype, i, v, mk[grp]) : z;
    e[grp] = (masked && mk[grp]) ? ldf4(D.ema, i, v, mk[grp]) : z;
  }
  const float thr = masked ? state_of(D)->thr : 0.f;
  const bool noisy = D.noise > 0.f;
  const uint64_t key = noisy ? *D.seed : 0ull;
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    if (!mk[grp]) continue;
    const int64_t i = ch.elem(grp);
    v4f o;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      o[t] = masked ? g[grp][t] * (e[grp][t] >= thr ? 1.0f : 0.0f) : g[grp][t];
    if (noisy) {
      const v4f z = normals4(key, i);
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] = o[t] + z[t] * D.noise;
    }
    stf4(D.out, i, o, vec && mk[grp] == 15, mk[grp]);
  }
}

}  // namespace

// ------------------------------------------------------------- C ABI ---
extern "C" int scao_sparse_filter(const scao_task* tasks, int ntasks,
                                  const scao_filter_desc* descs, int ndescs, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0 && ndescs >= 0, "scao_sparse_filter: negative count");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && descs && ndescs > 0, "scao_sparse_filter: null pointer");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_filter_ema, dim3(ntasks), dim3(256), 0, s, tasks, descs);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 0);
  const int hblocks = (ntasks + FH - 1) / FH;
  hipLaunchKernelGGL(k_filter_hist, dim3(hblocks), dim3(256), 0, s, tasks, ntasks, descs, 1);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 1);
  hipLaunchKernelGGL(k_filter_hist, dim3(hblocks), dim3(256), 0, s, tasks, ntasks, descs, 2);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 2);
  hipLaunchKernelGGL(k_filter_out, dim3(ntasks), dim3(256), 0, s, tasks, descs);
  SCAO_LAUNCH_CHECK("scao_sparse_filter");
  return SCAO_OK;
}
