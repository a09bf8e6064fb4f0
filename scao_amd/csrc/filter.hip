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
// patterns of e (e >= 0, so unsigned order is float order) with digits of
// 11, 11 and 10 bits: streaming passes build per-block LDS histograms and
// flush their non-zero bins into the parameter's global histogram, and a
// one-block-per-parameter select scans it, narrows both targets and clears
// it for the next pass.
//
// A magnitude EMA's threshold moves slowly from call to call.  After the
// first call the EMA pass therefore assumes the top digit (a quarter octave)
// of the previous threshold, `pred`: instead of the top-digit histogram it
// counts the keys below bin `pred` and histograms the second digit of the
// keys inside it (about a tenth of them, spread over 2048 bins), and copies
// those keys into the desc's candidate buffer.  If both targets fall in bin
// `pred` (a hit) the first select resolves two digits at once and the last
// refinement pass reads the candidates; otherwise (a miss) a top-digit pass
// over the EMA runs first and the refinement passes read the EMA.  Each
// desc's `step` says which digit its next pass builds; every pass is
// launched and skips the descs it does not concern.  The same keys are
// counted either way, so the threshold does not depend on the path.
#include "scao_common.hpp"

using namespace scao;

namespace {

constexpr int NB = SCAO_FILTER_BINS;   // 2048
constexpr int RG = SCAO_FILTER_REGION; // candidate slots per chunk
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
  uint32_t overflow;    // a candidate sub-stream of this call ran out of room
  uint32_t pred;        // top digit of the previous call's lower target
  uint32_t pvalid;      // pred holds a digit: the EMA pass runs predicted
  uint32_t compact;     // the last refinement pass reads the candidates
  uint32_t step;        // the digit the next streaming pass builds (3: done)
  uint32_t pad;
  unsigned long long below;  // predicted EMA pass: keys below bin pred
};
static_assert(sizeof(FState) == 4 * (SCAO_FILTER_WORK_WORDS - 2 * SCAO_FILTER_BINS),
              "state words");

__device__ __forceinline__ uint32_t* hist_of(const scao_filter_desc& D, int t) {
  return D.work + t * NB;
}
__device__ __forceinline__ FState* state_of(const scao_filter_desc& D) {
  return (FState*)(D.work + 2 * NB);
}
// the candidate buffer is usable: RG slots and four count words per chunk
__device__ __forceinline__ int64_t nchunks(const scao_filter_desc& D) {
  return (D.numel + SCAO_FLAT_CHUNK - 1) / SCAO_FLAT_CHUNK;
}
__device__ __forceinline__ bool has_cand(const scao_filter_desc& D) {
  return D.cand != nullptr && D.cap >= nchunks(D) * (RG + 4);
}
// count word of wave w's sub-stream of the segment starting at chunk c
__device__ __forceinline__ uint32_t* cand_count(const scao_filter_desc& D, int64_t c, int w) {
  return (uint32_t*)(D.cand + nchunks(D) * RG) + 4 * c + w;
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

// The EMA pass and the streaming passes run the same grid, a few blocks per
// CU; block b takes the consecutive tasks [b*per, (b+1)*per) and splits them
// into segments, one per desc, so its LDS histograms are zeroed and flushed
// once per segment.  The candidates of a segment of L chunks go to its
// L * RG slots from the first chunk's on, a quarter for each wave: wave w
// appends its keys (wave-level prefix sums, no block barrier) to sub-stream
// w, through a buffer in LDS so that they are stored in whole 2 KB blocks,
// and leaves their count in the first chunk's count word w.  The last
// refinement pass sees the same segments and streams each sub-stream.

// One past the last task of the segment that starts at task t: the desc's
// chunks follow t in order (as the task list is built), up to te.  If the
// list is not in that order the segment is t alone.
__device__ __forceinline__ int seg_end(const scao_task* __restrict__ tasks, int t, int te,
                                       const scao_filter_desc* __restrict__ descs) {
  const scao_task tk = tasks[t];
  const int64_t nch = nchunks(descs[tk.idx]);
  int64_t e = (int64_t)t + (nch - tk.a);
  if (e > te) e = te;
  if (e <= (int64_t)t + 1) return t + 1;
  const scao_task last = tasks[e - 1];
  return (last.idx == tk.idx && (int64_t)last.a == (int64_t)tk.a + (e - 1 - t)) ? (int)e : t + 1;
}

// exclusive prefix sum of v over the wave; *total gets the wave's sum
__device__ __forceinline__ uint32_t wave_offset(uint32_t v, uint32_t* total) {
  const int l = threadIdx.x & 63;
  uint32_t x = v;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (l >= o) x += y;
  }
  *total = __shfl(x, 63, 64);
  return x - v;
}

// add the block's counts of one segment into desc D's global histogram(s)
// and its scalars, then clear them
__device__ __forceinline__ void flush_segment(uint32_t (*h)[NB], int nb, bool two,
                                              uint32_t* nan_s, unsigned long long* below_s,
                                              const scao_filter_desc& D) {
  __syncthreads();   // every update of the segment has landed
  flush(&h[0][0], hist_of(D, 0), nb);
  if (two) flush(&h[1][0], hist_of(D, 1), nb);
  if (threadIdx.x == 0) {
    FState* S = state_of(D);
    if (nan_s && *nan_s) atomicAdd(&S->nan, *nan_s);
    if (below_s && *below_s) atomicAdd(&S->below, *below_s);
  }
  __syncthreads();   // read before cleared
  zero_lds(&h[0][0], two ? 2 * NB : NB);
  if (threadIdx.x == 0) {
    if (nan_s) *nan_s = 0u;
    if (below_s) *below_s = 0ull;
  }
  __syncthreads();
}

// ---------------------------------------------------------- EMA pass ---
__global__ __launch_bounds__(256) void k_filter_ema(const scao_task* __restrict__ tasks,
                                                    int ntasks, int per,
                                                    const scao_filter_desc* __restrict__ descs) {
  __shared__ uint32_t h[1][NB];
  __shared__ uint32_t nan_s;
  __shared__ unsigned long long below_s;
  __shared__ __attribute__((aligned(16))) float stage[4][1536];
  const int tb = blockIdx.x * per;
  const int te = ntasks - tb < per ? ntasks : tb + per;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  zero_lds(&h[0][0], NB);
  if (threadIdx.x == 0) {
    nan_s = 0u;
    below_s = 0ull;
  }
  __syncthreads();
  for (int t = tb; t < te;) {
    const int se = seg_end(tasks, t, te, descs);
    const scao_task tk0 = tasks[t];
    const scao_filter_desc& D = descs[tk0.idx];
    if (!(D.flags & SCAO_FILTER_MASK)) {
      t = se;
      continue;
    }
    const bool first = D.flags & SCAO_FILTER_FIRST;
    FState* S = state_of(D);
    // the same for every block of this desc
    const bool predicted = S->pvalid != 0u;
    const uint32_t pred = S->pred;
    const bool gather = predicted && has_cand(D) && (int64_t)tk0.a < nchunks(D);
    const uint32_t sub = (uint32_t)(se - t) * (uint32_t)(RG / 4);   // slots per sub-stream
    float* slots = D.cand + (int64_t)tk0.a * RG + (int64_t)w * sub;
    const bool vec = ((uintptr_t)D.ema & 15) == 0 && al_dt(D.g, D.dtype);
    uint32_t run = 0;      // this wave's candidates of the segment so far
    // keys wait in the wave's LDS buffer and go out in whole, aligned blocks
    // of 512 (2 KB): a partly written line evicted before the rest of it
    // arrives costs a read-modify-write in HBM
    uint32_t pend = 0, written = 0;
    float* st = &stage[w][0];
    uint32_t nbelow = 0;   // this thread's keys below bin pred
    for (int c = t; c < se; ++c) {
      const scao_task tk = tasks[c];
      const FChunk ch(tk, D.numel);
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
      uint32_t nans = 0, cmask = 0;
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        if (!mk[grp]) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float mag = fabsf(g[grp][k]);
          const float x = first ? mag : (e[grp][k] * D.decay) + (D.omd * mag);
          e[grp][k] = x;
          if (!(mk[grp] & (1 << k))) continue;
          const uint32_t key = __float_as_uint(x);
          if (is_nan_key(key)) {
            ++nans;
          } else if (!predicted) {
            atomicAdd(&h[0][key >> SHIFT[0]], 1u);
          } else {
            const uint32_t top = key >> SHIFT[0];
            nbelow += top < pred ? 1u : 0u;
            if (top == pred) {
              atomicAdd(&h[0][(key >> SHIFT[1]) & DMASK[1]], 1u);
              cmask |= 1u << (4 * grp + k);
            }
          }
        }
        stf4(D.ema, ch.elem(grp), e[grp], vec && mk[grp] == 15, mk[grp]);
      }
      if (nans) atomicAdd(&nan_s, nans);
      if (gather) {
        uint32_t total;
        uint32_t at = pend + wave_offset(__popc(cmask), &total);   // < 512 + 1024
#pragma unroll
        for (int grp = 0; grp < 4; ++grp)
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (cmask & (1u << (4 * grp + k))) st[at++] = e[grp][k];
        pend += total;
        run += total;
        __syncwarp();
        while (pend >= 512u) {
          if (written + 512u <= sub) {
            const v4f a0 = *(const v4f*)&st[4 * l];
            const v4f a1 = *(const v4f*)&st[256 + 4 * l];
            *(v4f*)&slots[written + 4 * l] = a0;
            *(v4f*)&slots[written + 256 + 4 * l] = a1;
          }
          __syncwarp();
          for (uint32_t i = l; i + 512u < pend; i += 64) st[i] = st[i + 512];
          __syncwarp();
          written += 512u;
          pend -= 512u;
        }
      }
    }
    if (gather) {
      for (uint32_t i = l; i < pend; i += 64)
        if (written + i < sub) slots[written + i] = st[i];
      __syncwarp();
    }
    if (gather && l == 0) {
      *cand_count(D, tk0.a, w) = run;
      if (run > sub) atomicOr(&S->overflow, 1u);
    }
    if (predicted) {
      uint32_t wb;
      wave_offset(nbelow, &wb);
      if (l == 0 && wb) atomicAdd(&below_s, (unsigned long long)wb);
    }
    flush_segment(h, NB, false, &nan_s, &below_s, D);
    t = se;
  }
}

// ----------------------------------------------------- streaming pass ---
// Builds digit d's histogram for the descs whose step is d: d = 0 after a
// missed prediction (all keys of the EMA), d = 1 and 2 for the keys that
// carry the selected prefix, from the candidates when the desc is compact
// (d = 2 only), else from the EMA.  The EMA's chunks go FH at a time, all
// their loads first (nothing they read depends on the selection state).
constexpr int FH = 4;

template <int d>
__device__ __forceinline__ void hist_keys(const v4f& x, int mk, uint32_t (*h)[NB], uint32_t p0,
                                          uint32_t p1, bool split) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (!(mk & (1 << k))) continue;
    const uint32_t key = __float_as_uint(x[k]);
    if constexpr (d == 0) {
      if (!is_nan_key(key)) atomicAdd(&h[0][key >> SHIFT[0]], 1u);
    } else {
      const uint32_t top = key >> SHIFT[d - 1];
      const uint32_t dig = (key >> SHIFT[d]) & DMASK[d];
      if (top == p0) atomicAdd(&h[0][dig], 1u);
      if (split && top == p1) atomicAdd(&h[1][dig], 1u);
    }
  }
}

template <int d>
__global__ __launch_bounds__(256) void k_filter_hist(const scao_task* __restrict__ tasks,
                                                     int ntasks, int per,
                                                     const scao_filter_desc* __restrict__ descs) {
  __shared__ uint32_t h[2][NB];
  const int tb = blockIdx.x * per;
  const int te = ntasks - tb < per ? ntasks : tb + per;
  const int nb = (int)DMASK[d] + 1;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  zero_lds(&h[0][0], 2 * NB);
  __syncthreads();
  for (int t = tb; t < te;) {
    const int se = seg_end(tasks, t, te, descs);
    const scao_task tk0 = tasks[t];
    const scao_filter_desc& D = descs[tk0.idx];
    const FState* S = state_of(D);
    if (!(D.flags & SCAO_FILTER_MASK) || S->step != (uint32_t)d) {
      t = se;
      continue;
    }
    const uint32_t p0 = S->prefix[0], p1 = S->prefix[1];
    const bool split = d > 0 && S->split != 0u;
    if (d == 2 && S->compact != 0u && (int64_t)tk0.a < nchunks(D)) {   // folds for d < 2
      // wave w streams sub-stream w; no sub-stream overflowed, so its count
      // is at most the segment's share (clamped anyway: the reads stay in
      // the segment's slots whatever the count word holds)
      const uint32_t sub = (uint32_t)(se - t) * (uint32_t)(RG / 4);
      const float* src = D.cand + (int64_t)tk0.a * RG + (int64_t)w * sub;
      const uint32_t cnt = *cand_count(D, tk0.a, w);
      const int64_t n = cnt < sub ? cnt : sub;
      for (int64_t v0 = 0; v0 < n; v0 += 4 * 256) {
        v4f x[4];
        int mk[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t i = v0 + q * 256 + l * 4;
          int m = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) m |= (i + k < n) ? (1 << k) : 0;
          mk[q] = m;
          x[q] = m ? ldf4(src, i, m == 15, m) : v4f{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) hist_keys<d>(x[q], mk[q], h, p0, p1, split);
      }
    } else {
      const bool vec = ((uintptr_t)D.ema & 15) == 0;
      for (int c0 = t; c0 < se; c0 += FH) {
        const int nt = se - c0 < FH ? se - c0 : FH;
        v4f x[FH][4];
        int mk[FH][4];
#pragma unroll
        for (int c = 0; c < FH; ++c) {
#pragma unroll
          for (int grp = 0; grp < 4; ++grp) mk[c][grp] = 0;
          if (c >= nt) continue;
          const FChunk ch(tasks[c0 + c], D.numel);
#pragma unroll
          for (int grp = 0; grp < 4; ++grp) {
            const int64_t i = ch.elem(grp);
            mk[c][grp] = ch.mask(i);
            x[c][grp] = mk[c][grp] ? ldf4(D.ema, i, vec && mk[c][grp] == 15, mk[c][grp])
                                   : v4f{0.f, 0.f, 0.f, 0.f};
          }
        }
#pragma unroll
        for (int c = 0; c < FH; ++c)
#pragma unroll
          for (int grp = 0; grp < 4; ++grp) hist_keys<d>(x[c][grp], mk[c][grp], h, p0, p1, split);
      }
    }
    flush_segment(h, nb, split, nullptr, nullptr, D);
    t = se;
  }
}

// Inclusive prefix sums of NB counts held 8 per thread (256 threads); finds,
// for rank r, the first bin whose running count exceeds r.  Returns the bin
// in *bin_out and the count before it in *before_out (from one thread), and
// the total in *total_out (every thread).
__device__ __forceinline__ void find_bin(const uint32_t* h, uint64_t r, uint32_t* scan,
                                         uint32_t* bin_out, uint32_t* before_out,
                                         uint32_t* total_out) {
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
      if (run <= r && r < (uint64_t)run + c[i]) {
        *bin_out = (uint32_t)(8 * l + i);
        *before_out = run;
      }
      run += c[i];
    }
  }
  *total_out = scan[255];
  __syncthreads();
}

// ------------------------------------------------------------- select ---
// stage 0 follows the EMA pass; stage d + 1 follows the streaming pass of
// digit d and concerns the descs whose step is d.
__global__ __launch_bounds__(256) void k_filter_select(const scao_filter_desc* __restrict__ descs,
                                                       int stage) {
  __shared__ uint32_t h[2][NB];
  __shared__ uint32_t scan[256];
  __shared__ uint32_t bin[2], before[2];
  const scao_filter_desc& D = descs[blockIdx.x];
  if (!(D.flags & SCAO_FILTER_MASK)) return;
  FState* S = state_of(D);
  const int d = stage == 0 ? -1 : stage - 1;
  if (d >= 0 && S->step != (uint32_t)d) return;
  uint64_t r[2];
  uint32_t pre[2];
  bool split = false;
  // the digit the histogram in hist_of(D, 0 / 1) holds
  int dig;
  bool predicted = false;
  uint64_t below = 0;
  if (d < 0) {
    // ranks = fp32(q * (n - 1)) as torch.quantile computes them
    const float ranks = D.q * (float)(D.numel - 1);
    const uint64_t lo = (uint64_t)ranks;
    const uint64_t hi = (uint64_t)ceilf(ranks);
    r[0] = lo;
    r[1] = hi;
    predicted = S->pvalid != 0u;
    below = S->below;
    pre[0] = pre[1] = predicted ? S->pred : 0u;
    dig = predicted ? 1 : 0;
    __syncthreads();   // every thread has read the state before thread 0 writes it
    if (threadIdx.x == 0) S->w = ranks - (float)lo;
  } else {
    r[0] = S->rank[0];
    r[1] = S->rank[1];
    pre[0] = S->prefix[0];
    pre[1] = S->prefix[1];
    split = d > 0 && S->split != 0u;
    dig = d;
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
  // a predicted EMA pass counted `below` keys under bin pred and histogrammed
  // the second digit inside it: a hit when both targets fall in the bin
  bool hit = true;
  if (predicted) {
    uint32_t inb;
    find_bin(&h[0][0], 0, scan, &bin[0], &before[0], &inb);
    hit = below <= r[0] && r[1] < below + inb;
    if (hit) {
      r[0] -= below;
      r[1] -= below;
    }
    if (threadIdx.x < 2) {
      bin[threadIdx.x] = 0u;
      before[threadIdx.x] = 0u;
    }
    __syncthreads();
  }
  if (!hit) {
    // missed: the next pass builds the top-digit histogram from the EMA
    if (threadIdx.x == 0) {
      S->rank[0] = (uint32_t)r[0];
      S->rank[1] = (uint32_t)r[1];
      S->prefix[0] = S->prefix[1] = 0u;
      S->split = 0u;
      S->compact = 0u;
      S->below = 0ull;
      S->overflow = 0u;
      S->step = 0u;
    }
    return;
  }
  uint32_t tot;
  for (int t = 0; t < 2; ++t) find_bin(&h[t][0], r[t], scan, &bin[t], &before[t], &tot);
  if (threadIdx.x == 0) {
    const int bits = dig == 2 ? 10 : 11;
    uint32_t np[2];
    for (int t = 0; t < 2; ++t) {
      np[t] = (pre[t] << bits) | bin[t];
      S->prefix[t] = np[t];
      S->rank[t] = (uint32_t)(r[t] - before[t]);
    }
    S->split = np[0] != np[1] ? 1u : 0u;
    if (d < 0) {
      // a hit leaves the candidates of bin pred usable if none was dropped
      S->compact = (predicted && has_cand(D) && S->overflow == 0u) ? 1u : 0u;
      S->below = 0ull;
      S->overflow = 0u;
    }
    if (dig == 0) {   // the top digit of the lower target predicts the next call
      S->pred = np[0];
      S->pvalid = 1u;
    }
    S->step = (uint32_t)dig + 1u;
    if (dig == 2) {
      const float vlo = __uint_as_float(np[0]), vhi = __uint_as_float(np[1]);
      const float w = S->w;
      const float dv = vhi - vlo;
      float thr = fabsf(w) < 0.5f ? fmaf(w, dv, vlo) : fmaf(-dv, 1.0f - w, vhi);
      if (S->nan) thr = __uint_as_float(0x7fc00000u);
      S->thr = thr;
      S->nan = 0u;
      S->split = 0u;
    }
  }
}

// ---------------------------------------------------------------- out ---
__global__ __launch_bounds__(256) void k_filter_out(const scao_task* __restrict__ tasks,
                                                    int ntasks, int per,
                                                    const scao_filter_desc* __restrict__ descs) {
  const int tb = blockIdx.x * per;
  const int te = ntasks - tb < per ? ntasks : tb + per;
  for (int ti = tb; ti < te; ++ti) {
    const scao_task tk = tasks[ti];
    const scao_filter_desc& D = descs[tk.idx];
    if (D.out == nullptr) continue;   // the step kernels form the values themselves
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
}

// Blocks for a pass over ntasks tasks taken `unit` at a time: four per CU
// (all resident at once), each with a run of `*per` tasks (a multiple of
// unit).
int filter_grid(int ntasks, int unit, int* per) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = -1;
  int n = dev >= 0 ? cus[dev] : 0;
  if (n <= 0) {
    if (dev < 0 || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                       hipSuccess || n <= 0)
      n = 256;
    if (dev >= 0) cus[dev] = n;
  }
  const int groups = (ntasks + unit - 1) / unit;
  const int want = 4 * n;
  const int nblk = groups < want ? groups : want;
  *per = ((groups + nblk - 1) / nblk) * unit;
  return (ntasks + *per - 1) / *per;
}

}  // namespace

// ------------------------------------------------------------- C ABI ---
extern "C" int scao_sparse_filter(const scao_task* tasks, int ntasks,
                                  const scao_filter_desc* descs, int ndescs, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0 && ndescs >= 0, "scao_sparse_filter: negative count");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && descs && ndescs > 0, "scao_sparse_filter: null pointer");
  hipStream_t s = (hipStream_t)stream;
  // the EMA and refinement passes see the same segments: one grid for both
  int per = 0;
  const int nblk = filter_grid(ntasks, 1, &per);
  hipLaunchKernelGGL(k_filter_ema, dim3(nblk), dim3(256), 0, s, tasks, ntasks, per, descs);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 0);
  hipLaunchKernelGGL(k_filter_hist<0>, dim3(nblk), dim3(256), 0, s, tasks, ntasks, per, descs);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 1);
  hipLaunchKernelGGL(k_filter_hist<1>, dim3(nblk), dim3(256), 0, s, tasks, ntasks, per, descs);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 2);
  hipLaunchKernelGGL(k_filter_hist<2>, dim3(nblk), dim3(256), 0, s, tasks, ntasks, per, descs);
  hipLaunchKernelGGL(k_filter_select, dim3(ndescs), dim3(256), 0, s, descs, 3);
  hipLaunchKernelGGL(k_filter_out, dim3(nblk), dim3(256), 0, s, tasks, ntasks, per, descs);
  SCAO_LAUNCH_CHECK("scao_sparse_filter");
  return SCAO_OK;
}
