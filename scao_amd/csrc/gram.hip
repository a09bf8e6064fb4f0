// Curvature-refresh kernels on gfx950 (scao/preconditioner.py:297-361, 381-406).
//
// gram_ema   C = X X^T for X = G (L side, dim m) or X = G^T (R side, dim n) on
//            fp32 MFMA, 128x128 output tiles, operands staged through LDS in
//            32-deep K chunks (the next chunk's loads in flight under the
//            current chunk's MFMAs), fused with the EMA
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
constexpr int KC = 32;              // K chunk
constexpr int LP = GT + 4;          // padded LDS row of an operand chunk
constexpr int SP = GT + 1;          // LDS row of the staged output tile

// Operand chunks X[r0:r0+128][kb:kb+32], four 4-element loads per thread,
// held in registers (raw, in the gradient's dtype) from chunk_load until
// chunk_store converts them into lds[k][r] (row pitch LP).  DT >= 0: the
// chunk lies inside the factor and is aligned, so the loads are plain vector
// loads in straight-line code (no branch may join before the MFMAs that
// hide them); DT = -1: any chunk, masked at the edges, any dtype.
template <int DT> struct ChunkRaw { typedef v4f T; };
template <> struct ChunkRaw<SCAO_BF16> { typedef v2u T; };
template <> struct ChunkRaw<SCAO_F16> { typedef v2u T; };

template <int DT, int SIDE>
__device__ __forceinline__ void chunk_load(const scao_gram_desc& D, int dim, int K, int r0, int kb,
                                           bool vec, typename ChunkRaw<DT>::T (&x)[4]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    int i, k;
    int64_t e;
    if (SIDE == 0) {
      // rows contiguous in k: thread -> (row, 4 k's)
      i = r0 + tid / 8 + 32 * h;
      k = kb + (tid % 8) * 4;
      e = D.off + (int64_t)i * D.ld + k;
    } else {
      // k rows contiguous in i: thread -> (k, 4 i's)
      k = kb + tid / 32 + 8 * h;
      i = r0 + (tid % 32) * 4;
      e = D.off + (int64_t)k * D.ld + i;
    }
    if constexpr (DT == SCAO_F32) {
      x[h] = gld4((const float*)D.g + e);
    } else if constexpr (DT >= 0) {
      x[h] = *(const gv2u*)((const uint16_t*)D.g + e);
    } else {
      int mk = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        mk |= (SIDE == 0 ? (i < dim && k + t < K) : (k < K && i + t < dim)) ? (1 << t) : 0;
      x[h] = mk ? ld4(D.g, D.dtype, e, vec && mk == 15, mk) : v4f{0.f, 0.f, 0.f, 0.f};
    }
  }
}

template <int DT>
__device__ __forceinline__ v4f chunk_f32(const typename ChunkRaw<DT>::T& x) {
  if constexpr (DT == SCAO_BF16 || DT == SCAO_F16) {
    const uint16_t h[4] = {(uint16_t)(x[0] & 0xffff), (uint16_t)(x[0] >> 16),
                           (uint16_t)(x[1] & 0xffff), (uint16_t)(x[1] >> 16)};
    v4f r;
#pragma unroll
    for (int t = 0; t < 4; ++t) r[t] = DT == SCAO_BF16 ? bf16_to_f(h[t]) : f16_to_f(h[t]);
    return r;
  } else {
    return x;
  }
}

template <int DT, int SIDE>
__device__ __forceinline__ void chunk_store(float* lds, const typename ChunkRaw<DT>::T (&x)[4]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const v4f v = chunk_f32<DT>(x[h]);
    if (SIDE == 0) {
      const int r = tid / 8 + 32 * h, kq = (tid % 8) * 4;
#pragma unroll
      for (int t = 0; t < 4; ++t) lds[(kq + t) * LP + r] = v[t];
    } else {
      *(v4f*)&lds[(tid / 32 + 8 * h) * LP + (tid % 32) * 4] = v;
    }
  }
}

// Two-level sum: the MFMAs accumulate FOLD consecutive K values in acc,
// which is then added to tot and cleared.  One fp32 accumulator over all of
// K (2048-4096 here, K/4 dependent MFMA adds) drifts by about sqrt(K/4) ulps,
// above the reference's own float32 GEMM; two levels of sqrt(FOLD/4) and
// sqrt(K/FOLD) bring that under it.  Both sums are exact sums of the same
// products, so only rounding changes.
constexpr int FOLD = 128;
static_assert(FOLD % KC == 0, "fold");

// The K loop of one 128 x 128 tile: the next chunk's loads go out before
// this chunk's MFMAs and land in LDS after them, so their latency hides
// under the products.  Wave w computes rows wr.., columns wc.. (64 x 64).
template <int DT, int SIDE>
__device__ __forceinline__ void gram_kloop(const scao_gram_desc& D, int dim, int K, int i0, int j0,
                                           bool diag, bool vec, float* As, float* Bs, int wr,
                                           int wc, v4f (&tot)[4][4]) {
  const int l = threadIdx.x % 64;
  v4f acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = tot[a][b] = v4f{0.f, 0.f, 0.f, 0.f};
  typename ChunkRaw<DT>::T xa[4], xb[4];
  chunk_load<DT, SIDE>(D, dim, K, i0, 0, vec, xa);
  if (!diag) chunk_load<DT, SIDE>(D, dim, K, j0, 0, vec, xb);
  chunk_store<DT, SIDE>(As, xa);
  if (!diag) chunk_store<DT, SIDE>(Bs, xb);
  __syncthreads();
  int buf = 0;
  for (int kb = 0; kb < K; kb += KC) {
    const bool more = kb + KC < K;
    if (more) {
      chunk_load<DT, SIDE>(D, dim, K, i0, kb + KC, vec, xa);
      if (!diag) chunk_load<DT, SIDE>(D, dim, K, j0, kb + KC, vec, xb);
    }
    const float* Ab = As + buf * KC * LP + (l / 16) * LP + wr + (l % 16);
    const float* Bb = (diag ? As : Bs) + buf * KC * LP + (l / 16) * LP + wc + (l % 16);
    // operands of step ks + 1 are read from LDS while step ks's MFMAs run
    float af[2][4], bf[2][4];
#pragma unroll
    for (int a = 0; a < 4; ++a) af[0][a] = Ab[16 * a];
#pragma unroll
    for (int b = 0; b < 4; ++b) bf[0][b] = Bb[16 * b];
#pragma unroll
    for (int ks = 0; ks < KC / 4; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KC / 4) {
#pragma unroll
        for (int a = 0; a < 4; ++a) af[cur ^ 1][a] = Ab[4 * (ks + 1) * LP + 16 * a];
#pragma unroll
        for (int b = 0; b < 4; ++b) bf[cur ^ 1][b] = Bb[4 * (ks + 1) * LP + 16 * b];
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16(af[cur][a], bf[cur][b], acc[a][b]);
    }
    // the schedule: step 0's four LDS reads, then per step the next step's
    // four reads ahead of its sixteen MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int ks = 0; ks < KC / 4; ++ks) {
      if (ks + 1 < KC / 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
    }
    if (more) {
      chunk_store<DT, SIDE>(As + (buf ^ 1) * KC * LP, xa);
      if (!diag) chunk_store<DT, SIDE>(Bs + (buf ^ 1) * KC * LP, xb);
    }
    __syncthreads();
    buf ^= 1;
    if ((kb + KC) % FOLD == 0 || !more) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          tot[a][b] += acc[a][b];
          acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    }
  }
}

// The K loop for whole fp32 tiles on the bf16 matrix cores: fp32 products as
// six bf16 MFMAs over three-way splits (mfma_x6), one v_mfma_f32_16x16x32
// covering a whole 32-deep chunk (6 * 16 cycles per output tile against
// 8 * 32 for the fp32 16x16x4 form).  The loader splits each operand value
// once and stores the three bf16 planes row-major with k contiguous (pitch
// XCP = 40: a lane's 8 consecutive k are one 16-byte read, and the 16 lanes
// of a read hit disjoint bank quads); the chunk buffer is single (60 KB for
// both operands, two workgroups per CU) with the next chunk's raw values held
// in registers across the MFMAs.  Side 1 (X = G^T) loads four consecutive k
// of one X row (four G rows at one column: coalesced across the lanes), so
// every plane write is 8 bytes.
constexpr int XCP = 40;
constexpr int XPL = GT * XCP;        // bf16 per plane
static_assert(2 * 3 * XPL * 2 <= 2 * 2 * KC * LP * 4, "x6 planes fit the operand LDS");

template <int SIDE>
__device__ __forceinline__ void chunk_load_x6(const scao_gram_desc& D, int r0, int kb,
                                              v4f (&x)[4]) {
  const int tid = threadIdx.x;
  const float* g = (const float*)D.g;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    if (SIDE == 0) {
      // row tid/8 + 32h, k = kb + 4(tid%8) .. +3
      const int i = r0 + tid / 8 + 32 * h, k = kb + (tid % 8) * 4;
      x[h] = gld4(g + D.off + (int64_t)i * D.ld + k);
    } else {
      // X row i = tid % 128 (a G column), k = kb + 4(tid/128 + 2h) .. +3 (G rows)
      const int i = r0 + tid % 128, k = kb + 4 * (tid / 128 + 2 * h);
#pragma unroll
      for (int u = 0; u < 4; ++u) x[h][u] = g[D.off + (int64_t)(k + u) * D.ld + i];
    }
  }
}

template <int SIDE>
__device__ __forceinline__ void chunk_store_x6(__bf16* P, const v4f (&x)[4]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int row = SIDE == 0 ? tid / 8 + 32 * h : tid % 128;
    const int k = SIDE == 0 ? (tid % 8) * 4 : 4 * (tid / 128 + 2 * h);
    uint32_t pk[3][2];
#pragma unroll
    for (int u = 0; u < 4; u += 2)
      split3_pk(x[h][u], x[h][u + 1], pk[0][u / 2], pk[1][u / 2], pk[2][u / 2]);
#pragma unroll
    for (int pp = 0; pp < 3; ++pp)
      *(v2u*)&P[pp * XPL + row * XCP + k] = v2u{pk[pp][0], pk[pp][1]};
  }
}

template <int SIDE>
__device__ __forceinline__ void gram_kloop_x6(const scao_gram_desc& D, int K, int i0, int j0,
                                              bool diag, __bf16* Ap, __bf16* Bp, int wr, int wc,
                                              v4f (&tot)[4][4]) {
  const int l = threadIdx.x % 64, jj = l % 16, g = l / 16;
  v4f acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = tot[a][b] = v4f{0.f, 0.f, 0.f, 0.f};
  v4f xa[4], xb[4];
  chunk_load_x6<SIDE>(D, i0, 0, xa);
  if (!diag) chunk_load_x6<SIDE>(D, j0, 0, xb);
  const __bf16* Bq = diag ? Ap : Bp;
  for (int kb = 0; kb < K; kb += KC) {
    if (kb) __syncthreads();               // the previous chunk's planes are consumed
    chunk_store_x6<SIDE>(Ap, xa);
    if (!diag) chunk_store_x6<SIDE>(Bp, xb);
    __syncthreads();
    if (kb + KC < K) {                     // in flight during the MFMAs below
      chunk_load_x6<SIDE>(D, i0, kb + KC, xa);
      if (!diag) chunk_load_x6<SIDE>(D, j0, kb + KC, xb);
    }
    bf3 bo[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const __bf16* q = Bq + (wc + 16 * b + jj) * XCP + 8 * g;
      bo[b].h = *(const v8bf*)q;
      bo[b].m = *(const v8bf*)(q + XPL);
      bo[b].l = *(const v8bf*)(q + 2 * XPL);
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const __bf16* q = Ap + (wr + 16 * a + jj) * XCP + 8 * g;
      bf3 ao;
      ao.h = *(const v8bf*)q;
      ao.m = *(const v8bf*)(q + XPL);
      ao.l = *(const v8bf*)(q + 2 * XPL);
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = mfma_x6(ao, bo[b], acc[a][b]);
    }
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
  __syncthreads();                         // the planes' LDS is reused by the epilogue
}

// EMA update of the output tile rows r0.., columns c0.. from the product
// tile staged in S (S[row][col], or S[col][row] when `tr`).  A tile inside
// a factor with dim % 4 == 0 goes 4 elements per thread and pass (one 32-bit
// load of 4 codes or a float4 of the old EMA, a float4 store), each
// wavefront covering two rows; the old values of all 16 passes are loaded
// before any is used.  Other tiles go element by element.
__device__ __forceinline__ float ema_one(const scao_gram_desc& D, float old, float prod, float sf,
                                         float& amax) {
  const float add = D.alpha * prod;
  if (D.q) {
    const float x = (old * sf) * D.rho + add;
    amax = fmaxf(amax, fabsf(x));
    return x;
  }
  return old * D.rho + add;
}

__device__ __forceinline__ void ema_tile(const scao_gram_desc& D, const float* S, int dim, int r0,
                                         int c0, bool tr, float sf, float& amax) {
  const int tid = threadIdx.x;
  const bool vec4 = dim % 4 == 0 && r0 + GT <= dim && c0 + GT <= dim &&
                    (((uintptr_t)D.ema | (uintptr_t)D.q) & 15) == 0;
  if (vec4) {
    constexpr int NP = GT * GT / 4 / 256;   // 16 passes
    uint32_t qv[NP];
    v4f ov[NP];
#pragma unroll
    for (int t = 0; t < NP; ++t) {
      const int idx = t * 256 + tid, row = idx / (GT / 4), col = (idx % (GT / 4)) * 4;
      const int64_t e = (int64_t)(r0 + row) * dim + c0 + col;
      if (D.q)
        qv[t] = gld1((const uint32_t*)(D.q + e));
      else
        ov[t] = gld4(D.ema + e);
    }
#pragma unroll
    for (int t = 0; t < NP; ++t) {
      const int idx = t * 256 + tid, row = idx / (GT / 4), col = (idx % (GT / 4)) * 4;
      const int64_t e = (int64_t)(r0 + row) * dim + c0 + col;
      v4f x;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float prod = tr ? S[(col + u) * SP + row] : S[row * SP + col + u];
        const float old = D.q ? (float)(int8_t)(uint8_t)(qv[t] >> (8 * u)) : ov[t][u];
        x[u] = ema_one(D, old, prod, sf, amax);
      }
      gst4(D.ema + e, x);
    }
    return;
  }
  for (int p0 = 0; p0 < GT * GT / 256; p0 += 16) {
    float old[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int idx = (p0 + t) * 256 + tid, row = idx / GT, col = idx % GT;
      const int i = r0 + row, j = c0 + col;
      const int64_t e = (int64_t)i * dim + j;
      old[t] = 0.f;
      if (i < dim && j < dim) old[t] = D.q ? (float)D.q[e] : D.ema[e];
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int idx = (p0 + t) * 256 + tid, row = idx / GT, col = idx % GT;
      const int i = r0 + row, j = c0 + col;
      if (i >= dim || j >= dim) continue;
      D.ema[(int64_t)i * dim + j] =
          ema_one(D, old[t], tr ? S[col * SP + row] : S[row * SP + col], sf, amax);
    }
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gram_ema(const scao_task* __restrict__ tasks,
                                                  const scao_gram_desc* __restrict__ descs) {
  // two double-buffered operand chunks; after the K loop, the 128 x 128
  // product tile (pitch SP)
  __shared__ __attribute__((aligned(16))) float smem[2 * 2 * KC * LP];
  static_assert(GT * SP <= 2 * 2 * KC * LP, "output tile staging");
  __shared__ float red[4];
  float* As = smem;                 // [2][KC][LP]
  float* Bs = smem + 2 * KC * LP;   // [2][KC][LP]
  const scao_task tk = tasks[blockIdx.x];
  const scao_gram_desc D = descs[tk.idx];
  const int dim = D.side == 0 ? D.rows : D.cols;
  const int K = D.side == 0 ? D.cols : D.rows;
  const int i0 = tk.a * GT, j0 = tk.b * GT;
  const bool diag = tk.a == tk.b;   // both operands are the same rows
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int wr = (w / 2) * 64, wc = (w % 2) * 64;
  const bool vec = ((D.off | D.ld) % 4 == 0) &&
                   (((uintptr_t)D.g & (D.dtype == SCAO_F32 ? 15u : 7u)) == 0);

  v4f tot[4][4];
  const bool whole = vec && K % KC == 0 && i0 + GT <= dim && j0 + GT <= dim;
#define SCAO_GRAM_KLOOP(DT, SIDE) \
  gram_kloop<DT, SIDE>(D, dim, K, i0, j0, diag, vec, As, Bs, wr, wc, tot)
  __bf16* Ap = (__bf16*)smem;
  __bf16* Bp = Ap + 3 * XPL;
  if (whole && D.dtype == SCAO_F32 && D.side == 0)
    gram_kloop_x6<0>(D, K, i0, j0, diag, Ap, Bp, wr, wc, tot);
  else if (whole && D.dtype == SCAO_F32)
    gram_kloop_x6<1>(D, K, i0, j0, diag, Ap, Bp, wr, wc, tot);
  else if (whole && D.dtype == SCAO_BF16 && D.side == 0)
    SCAO_GRAM_KLOOP(SCAO_BF16, 0);
  else if (whole && D.dtype == SCAO_BF16)
    SCAO_GRAM_KLOOP(SCAO_BF16, 1);
  else if (whole && D.dtype == SCAO_F16 && D.side == 0)
    SCAO_GRAM_KLOOP(SCAO_F16, 0);
  else if (whole && D.dtype == SCAO_F16)
    SCAO_GRAM_KLOOP(SCAO_F16, 1);
  else if (D.side == 0)
    SCAO_GRAM_KLOOP(-1, 0);
  else
    SCAO_GRAM_KLOOP(-1, 1);
#undef SCAO_GRAM_KLOOP

  // EMA epilogue.  The product tile goes to LDS (the operand buffers are free
  // after the K loop's last barrier): element (i0 + row, j0 + col) is
  // tot[a][b][r] with row = wr + 16a + 4*(l/16) + r, col = wc + 16b + l%16.
  // A task with a > b of a symmetric factor also updates the transposed tile
  // (b, a): element (j, i) takes the same product as (i, j).
  float* S = smem;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        S[(wr + 16 * a + 4 * (l / 16) + r) * SP + wc + 16 * b + (l % 16)] = tot[a][b][r];
  __syncthreads();
  const float sf = D.q ? (float)(*D.scale) : 0.f;
  float amax = 0.f;
  ema_tile(D, S, dim, i0, j0, false, sf, amax);
  const bool mirror = (D.flags & SCAO_GRAM_SYM) && !diag;
  if (mirror) ema_tile(D, S, dim, j0, i0, true, sf, amax);
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

// ---- exactly diagonal eigh inputs -------------------------------------
// When every off-diagonal entry of a factor is zero, LAPACK's syevd (torch's
// CPU eigh) does no arithmetic on it: the tridiagonal reduction's reflectors
// are all identities, so the tridiagonal is the diagonal itself with zero
// off-diagonal, and divide and conquer (stedc; steqr below 26 rows) only
// orders it.  That ordering is stedc's selection sort: for i = 0 .. n-2, k is
// the first position of the minimum of d[i..n-1] (a strict < scan starting
// from d[i], so k = i when d[i] ties the minimum), then d[i] <-> d[k] and
// columns i <-> k of the identity are swapped.  The eigenvalues are the
// diagonal values exactly and the eigenvectors +e_j.  Ties are common here: an
// int8 EMA of small gradients keeps only its diagonal codes, a handful of
// distinct values over thousands of rows, and the order the sort leaves them
// in decides which unit vectors the top k are.

constexpr int OFFDIAG_WORDS = 4096;   // 32-bit words (16 KB of int8 codes) per block
constexpr int DIAG_MAX = 4096 + 16;   // largest factor the diagonal path takes

// flags[f] |= 1 when factor f has a non-zero off-diagonal entry (int8 code or
// fp32 value).  Grid (chunks, factors); a block covers `per` elements of one
// factor, a 32-bit word of codes (or one float) per thread and iteration.
// The flags must be zero beforehand.
__global__ __launch_bounds__(256) void k_eig_offdiag(const scao_prep_desc* __restrict__ descs,
                                                     int max_dim, int per,
                                                     int* __restrict__ flags) {
  const scao_prep_desc D = descs[blockIdx.y];
  const int dim = D.dim;
  if (dim > max_dim) {   // not covered by the grid: take the general path
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(flags + blockIdx.y, 1);
    return;
  }
  const int64_t n = (int64_t)dim * dim;
  const int64_t e0 = (int64_t)blockIdx.x * per;
  if (e0 >= n) return;
  const int64_t e1 = e0 + per < n ? e0 + per : n;
  const bool vec = D.q ? ((uintptr_t)D.q & 3) == 0 : true;
  bool any = false;
  if (D.q && vec) {
    for (int64_t e = e0 + 4 * threadIdx.x; e < e1 && !any; e += 4 * 256) {
      if (e + 4 <= e1) {
        const uint32_t w = gld1((const uint32_t*)(D.q + e));
        if (w == 0) continue;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if ((w >> (8 * t)) & 0xffu) {
            const int64_t x = e + t;
            any |= x / dim != x % dim;
          }
      } else {
        for (int64_t x = e; x < e1; ++x) any |= D.q[x] != 0 && x / dim != x % dim;
      }
    }
  } else {
    for (int64_t x = e0 + threadIdx.x; x < e1 && !any; x += 256) {
      const bool nz = D.q ? D.q[x] != 0 : D.ema[x] != 0.f;
      any |= nz && x / dim != x % dim;
    }
  }
  if (__syncthreads_or(any) && threadIdx.x == 0) atomicOr(flags + blockIdx.y, 1);
}

__global__ __launch_bounds__(256) void k_flags_clear(int* flags, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) flags[i] = 0;
}

// Eigenpairs of an exactly diagonal eigh input, one block per factor: the
// diagonal of X = deq / fp32(bias) + shift as k_eig_prep forms it (the shift
// from k_eig_trace), ordered by the selection sort above, then flipped to
// descending order as the reference does (scao/preconditioner.py:418-426).
// Writes w[j] (double) and column j of U (n x kq, row-major) = e_{r_j} for the
// kq largest, and total = sum of max(d, 0) in double.
//
// Each thread owns the positions p = tid (mod 256).  A step scans the owned
// positions >= i for the first minimum (increasing p, strict <), reduces
// (value, position) over the block (smaller value, then smaller position: the
// first position of the minimum), and the owner of the winning position k
// records it and moves position i's value and index into k.  Position i is
// never read or written again after step i, and position k is only touched
// by its owner, so one barrier per step suffices (the reduction slots
// alternate between two buffers).
__global__ __launch_bounds__(256) void k_eig_diag(const scao_prep_desc* __restrict__ descs, int dim,
                                                  int kq, double* __restrict__ w, float* __restrict__ U,
                                                  int64_t ustride, double* __restrict__ total) {
  __shared__ float val[DIAG_MAX];
  __shared__ int idx[DIAG_MAX];
  __shared__ int top[DIAG_MAX];   // top[j]: row of the unit vector in column j
  __shared__ float rv[2][4];
  __shared__ int rp[2][4];
  __shared__ double red[4];
  const int f = blockIdx.x;
  const scao_prep_desc D = descs[f];
  const int n = D.dim;
  if (n != dim || n < 1 || n > DIAG_MAX || kq > n) return;   // outside the call's contract
  const int tid = threadIdx.x, lane = tid % 64, wv = tid / 64;
  const float sf = D.q ? (float)(*D.scale) : 0.f;
  const float eps = *D.shift;
  double pos = 0.0;
  for (int i = tid; i < n; i += 256) {
    const float y = prep_val(D, sf, (int64_t)i * n + i) + eps;
    val[i] = y;
    idx[i] = i;
    pos += y > 0.f ? (double)y : 0.0;
  }
  double acc[1] = {pos};
  block_sum<1>(acc, red);   // ends with a barrier: val/idx are complete
  if (tid == 0) total[f] = acc[0];
  double* wf = w + (int64_t)f * kq;
  for (int i = 0; i + 1 < n; ++i) {
    // first owned position >= i
    const int r = i % 256;
    int p = i - r + tid + (tid < r ? 256 : 0);
    float bv = INFINITY;
    int bp = n;
    if (p < n) {
      bv = val[p];
      bp = p;
      for (p += 256; p < n; p += 256) {
        const float v = val[p];
        if (v < bv) {
          bv = v;
          bp = p;
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int op = __shfl_xor(bp, o, 64);
      if (ov < bv || (ov == bv && op < bp)) {
        bv = ov;
        bp = op;
      }
    }
    const int b = i & 1;
    if (lane == 0) {
      rv[b][wv] = bv;
      rp[b][wv] = bp;
    }
    __syncthreads();
    float kv = rv[b][0];
    int k = rp[b][0];
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (rv[b][q] < kv || (rv[b][q] == kv && rp[b][q] < k)) {
        kv = rv[b][q];
        k = rp[b][q];
      }
    if (k < i || k >= n) k = i;   // only reachable with NaN values
    if (k % 256 == tid) {
      const int j = n - 1 - i;    // column after the flip
      if (j < kq) {
        top[j] = idx[k];
        wf[j] = (double)val[k];
      }
      if (k != i) {
        val[k] = val[i];
        idx[k] = idx[i];
      }
    }
  }
  if ((n - 1) % 256 == tid) {   // the last position holds the largest value
    top[0] = idx[n - 1];
    wf[0] = (double)val[n - 1];
  }
  __syncthreads();
  float* Uf = U + (int64_t)f * ustride;
  const int total_e = n * kq;   // <= DIAG_MAX^2
  if (kq % 4 == 0 && ((uintptr_t)Uf & 15) == 0) {
    for (int e = 4 * tid; e < total_e; e += 4 * 256) {
      const int row = e / kq, j = e - row * kq;
      v4f x;
#pragma unroll
      for (int t = 0; t < 4; ++t) x[t] = top[j + t] == row ? 1.f : 0.f;
      gst4(Uf + e, x);
    }
  } else {
    for (int e = tid; e < total_e; e += 256) {
      const int row = e / kq, j = e - row * kq;
      Uf[e] = top[j] == row ? 1.f : 0.f;
    }
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

extern "C" int scao_eig_offdiag(const scao_prep_desc* descs, int ndescs, int max_dim, int codes,
                                int* flags, void* stream) {
  SCAO_CHECK_ARG(ndescs >= 0 && ndescs <= 65535, "scao_eig_offdiag: ndescs=%d outside [0, 65535]",
                 ndescs);
  if (ndescs == 0) return SCAO_OK;
  SCAO_CHECK_ARG(descs && flags, "scao_eig_offdiag: null pointer");
  SCAO_CHECK_ARG(max_dim > 0 && max_dim <= 65535, "scao_eig_offdiag: max_dim=%d", max_dim);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_flags_clear, dim3((ndescs + 255) / 256), dim3(256), 0, s, flags, ndescs);
  const int per = OFFDIAG_WORDS * (codes ? 4 : 1);
  const int64_t nblk = ((int64_t)max_dim * max_dim + per - 1) / per;
  hipLaunchKernelGGL(k_eig_offdiag, dim3((unsigned)nblk, ndescs), dim3(256), 0, s, descs, max_dim,
                     per, flags);
  SCAO_LAUNCH_CHECK("scao_eig_offdiag");
  return SCAO_OK;
}

extern "C" int scao_eig_diag(const scao_prep_desc* descs, int ndescs, int n, int kq, double* w,
                             float* U, int64_t ustride, double* total, void* stream) {
  SCAO_CHECK_ARG(ndescs >= 0 && ndescs <= 65535, "scao_eig_diag: ndescs=%d outside [0, 65535]",
                 ndescs);
  if (ndescs == 0) return SCAO_OK;
  SCAO_CHECK_ARG(descs && w && U && total, "scao_eig_diag: null pointer");
  SCAO_CHECK_ARG(n >= 1 && n <= DIAG_MAX && kq >= 1 && kq <= n && ustride >= (int64_t)n * kq,
                 "scao_eig_diag: bad arguments n=%d kq=%d", n, kq);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_eig_trace, dim3(ndescs), dim3(256), 0, s, descs);
  hipLaunchKernelGGL(k_eig_diag, dim3(ndescs), dim3(256), 0, s, descs, n, kq, w, U, ustride, total);
  SCAO_LAUNCH_CHECK("scao_eig_diag");
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
