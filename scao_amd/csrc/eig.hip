// Eigen stage of the curvature refresh on gfx950: the top-k eigenpairs (and
// the sum of the clamped spectrum) of a batch of symmetric fp32 matrices --
// what scao/preconditioner.py:413-451 obtains from torch.linalg.eigh, whose
// LAPACK/rocSOLVER drivers tridiagonalise with Householder matrix-vector
// products (one pass over the trailing matrix per column).  Here:
//
//   1. dense -> band (SCAO_EIG_BAND = b sub-diagonals): per panel of b
//      columns a Householder QR (k_panel_qr, one workgroup per matrix, the
//      panel in registers); the two-sided trailing update is two plain batched
//      GEMMs issued by the caller (scao_amd/eigen.py);
//   2. band -> tridiagonal by bulge chasing (k_sb2st): sweep s annihilates
//      column s below the sub-diagonal with a reflector of length b and
//      chases the bulge it creates down the band, one task per b-row block;
//      a task touches only its own b rows of band storage (diagonals 0..2b);
//   3. eigenvalues of the tridiagonal by bisection with float64 Sturm counts
//      (k_bisect): the kq largest, and every negative one so that the sum of
//      the clamped spectrum is exact (trace minus the negatives);
//   4. eigenvectors by float64 inverse iteration on the band matrix itself
//      (k_inviter: band LU with partial pivoting in a sliding 17 x 33 window,
//      one wavefront per vector, shifted by the bisection eigenvalue): one
//      solve, a second only when the solution did not grow enough to have
//      converged, then the Rayleigh quotient as the eigenvalue; Gram-Schmidt
//      inside clusters of (nearly) equal eigenvalues (k_cluster_orth) and a
//      transposing float32 write of the vectors (k_vec_out);
//   5. back-transformation with the stage-1 block reflectors: caller GEMMs.
//
// The tridiagonal's reflectors are never stored: the vectors come from the
// band matrix, so only stage 1's reflectors (kept in the panels of A) are
// applied to them.
#include <type_traits>
#include <utility>

#include "scao_common.hpp"

using namespace scao;

namespace {

constexpr int NB = SCAO_EIG_BAND;    // 16
constexpr int BW = SCAO_EIG_BANDW;   // 33: band row pitch (diagonals 0..2b)
constexpr int OW = NB + 1;           // 17: pitch of the original band copy

// ----------------------------------------------------- cross-lane sums ---
// Butterfly levels (every lane adds lane l^o's value) without an LDS round
// trip, for call sites where the whole wavefront is active.  A permlane swap
// of x with itself returns two registers holding, in every lane, the lower
// and the upper lane of its xor-32 (permlane32) or xor-16 (permlane16) pair
// (lane layout checked on gfx950), so their sum is that level.  DPP moves
// give the levels inside a 16-lane row: quad_perm for xor 1 and 2, row_ror:8
// for xor 8, row_ror:4 for xor 4 once values repeat every 8 lanes, and the
// half-row and row mirrors for xor 4 and 8 once values are equal within
// quads.  Each level adds the same two values as the shuffle butterfly and
// fp addition commutes, so the sums are the same bits.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_QUAD0 = 0x00;
constexpr int DPP_ROW_MIRROR = 0x140, DPP_HALF_MIRROR = 0x141;
constexpr int DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return __builtin_amdgcn_update_dpp(0u, x, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __uint_as_float(dpp_u<CTRL>(__float_as_uint(x)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = dpp_u<CTRL>((uint32_t)b), hi = dpp_u<CTRL>((uint32_t)(b >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float xor32_sum_f(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_sum_f(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <bool W32>
__device__ __forceinline__ double xor_sum_d(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
  const auto rl = W32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                      : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto rh = W32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                      : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  const double a = __builtin_bit_cast(double, ((uint64_t)rh[0] << 32) | rl[0]);
  const double c = __builtin_bit_cast(double, ((uint64_t)rh[1] << 32) | rl[1]);
  return a + c;
}
// the sum over the wavefront in every lane, levels xor 32, 16, 8, 4, 2, 1
__device__ __forceinline__ float wave_sum_f(float y) {
  y = xor32_sum_f(y);
  y = xor16_sum_f(y);
  y += dpp_f<DPP_ROR8>(y);
  y += dpp_f<DPP_ROR4>(y);
  y += dpp_f<DPP_XOR2>(y);
  y += dpp_f<DPP_XOR1>(y);
  return y;
}
__device__ __forceinline__ double wave_sum_d(double y) {
  y = xor_sum_d<true>(y);
  y = xor_sum_d<false>(y);
  y += dpp_d<DPP_ROR8>(y);
  y += dpp_d<DPP_ROR4>(y);
  y += dpp_d<DPP_XOR2>(y);
  y += dpp_d<DPP_XOR1>(y);
  return y;
}

// ------------------------------------------------------------ panel QR ---
// Block reduction of NV floats over a workgroup of up to 1024 threads: every thread
// receives the NV sums in out[] (LDS).  (A reduce-scatter across the wave's
// lanes, 28 shuffles for 16 values instead of 96, measured slower: its
// lane-dependent selects cost more than the shuffles they save.)
template <int NV>
__device__ __forceinline__ void block_sum_f(float (&x)[NV], float (*red)[NV + 1], float* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    x[v] = wave_sum_f(x[v]);
  }
  if (lane == 0)
#pragma unroll
    for (int v = 0; v < NV; ++v) red[wid][v] = x[v];
  __syncthreads();
  if (threadIdx.x < NV) {
    float s = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += red[w][threadIdx.x];
    out[threadIdx.x] = s;
  }
  __syncthreads();
}

// f(integral_constant<int, J>) for J = 0, 1, .., in order
template <class F, int... J>
__device__ __forceinline__ void static_for(F& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}

// Householder QR of the panel A[r0:n, c0:c0+NB], r0 = c0 + NB, m = n - r0
// rows (LAPACK geqr2 + larft, forward columnwise).  Thread t holds rows
// t + NT h (h < RPT) of the panel.  Outputs: V (explicit, unit lower
// trapezoidal) over the panel of A, T (NB x NB upper), R into the band.
// NT threads (256 or 512, at least NB * NB for the T write) hold RPT rows
// each: few waves keep the per-column block reductions cheap and let two
// workgroups share a CU (480 panels of 2032 rows: 19.7 -> 11.3 ms for a
// sweep with 256-512 threads of 4 rows instead of 512-1024 of 2).
template <int RPT, int NT>
__global__ __launch_bounds__(NT) void k_panel_qr(float* A, int64_t stride, int n, int c0,
                                                   float* Tout, float* band, int64_t bstride) {
  __shared__ float red[16][NB + 1];
  __shared__ float bc[NB + 2];
  __shared__ float rowj[2][NB];
  __shared__ float Ts[NB][NB];
  __shared__ float betas[NB], taus[NB];
  __shared__ float Ds[NB][NB + 1];
  const int tid = threadIdx.x;
  float* Am = A + (int64_t)blockIdx.x * stride;
  const int r0 = c0 + NB, m = n - r0;
  const int kk = m < NB ? m : NB;
  // a row's 16 floats as four 16-byte accesses when rows are 16-byte aligned
  // (one access instruction then touches 64 lines for 16 bytes each, against
  // 64 lines for 4 bytes each with scalar accesses)
  const bool vec = (n % 4) == 0 && (stride % 4) == 0 && (((uintptr_t)A) & 15) == 0;
  float P[RPT][NB];
#pragma unroll
  for (int h = 0; h < RPT; ++h) {
    const int row = tid + NT * h;
    const float* arow = Am + (int64_t)(r0 + row) * n + c0;
    if (row < m && vec) {
#pragma unroll
      for (int c = 0; c < NB; c += 4) {
        const v4f x = gld4(arow + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) P[h][c + e] = x[e];
      }
    } else {
#pragma unroll
      for (int c = 0; c < NB; ++c) P[h][c] = row < m ? arow[c] : 0.f;
    }
  }
  if (tid < NB * NB) Ts[tid / NB][tid % NB] = 0.f;
  __syncthreads();
  // Column j: one reduction gives G[c] = sum over rows i > j of P[i][j] P[i][c]
  // for every c (G[j] = sigma^2); with v = (1, scale * P[j+1:, j]) every dot
  // v^T P[:, c] is then P[j][c] + scale * G[c] (the trailing columns' w_c and
  // the earlier reflectors' d_c for T alike), so a column costs one block
  // reduction.  Row j comes from thread j through LDS, double-buffered by
  // column parity (a slow thread may still read the previous column's).
  // The columns are expanded at compile time, so every P[h][j] index is a
  // constant and the rows stay in registers (a runtime j puts them in
  // scratch memory once they exceed about 32 floats).
  auto column = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j >= kk) return;
    float* rj = rowj[j & 1];
    if (tid == j) {
#pragma unroll
      for (int c = 0; c < NB; ++c) rj[c] = P[0][c];
    }
    float acc[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) acc[c] = 0.f;
#pragma unroll
    for (int h = 0; h < RPT; ++h) {
      const int row = tid + NT * h;
      if (row > j && row < m) {
        const float pj = P[h][j];
#pragma unroll
        for (int c = 0; c < NB; ++c) acc[c] = fmaf(pj, P[h][c], acc[c]);
      }
    }
    block_sum_f<NB>(acc, red, bc);
    const float alpha = rj[j], sig2 = bc[j];
    float tau = 0.f, beta = alpha, scale = 0.f;
    if (sig2 > 0.f) {
      beta = -copysignf(sqrtf(alpha * alpha + sig2), alpha);
      tau = (beta - alpha) / beta;
      scale = 1.f / (alpha - beta);
    }
    float dot[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) dot[c] = fmaf(scale, bc[c], rj[c]);
    // v (rows > j) replaces column j; P[:, c] -= tau v w_c for c > j
#pragma unroll
    for (int h = 0; h < RPT; ++h) {
      const int row = tid + NT * h;
      if (row >= j && row < m) {
        float v = 1.f;
        if (row > j) {
          v = P[h][j] * scale;
          P[h][j] = v;
        }
#pragma unroll
        for (int c = 0; c < NB; ++c)
          if (c > j) P[h][c] = fmaf(-tau * v, dot[c], P[h][c]);
      }
    }
    if (tid == 0) {
      // the column's dots and tau for T, built after the loop
#pragma unroll
      for (int c = 0; c < NB; ++c) Ds[j][c] = dot[c];
      taus[j] = tau;
      betas[j] = beta;
    }
  };
  static_for(column, std::make_integer_sequence<int, NB>{});
  __syncthreads();
  // T[0:j, j] = T[0:j, 0:j] (-tau_j d_j[0:j]), T[j][j] = tau_j, column by
  // column on one wavefront (lane i: row i; the same sums in the same order
  // as a serial build)
  if (tid < 64) {
    for (int j = 0; j < kk; ++j) {
      if (tid < j) {
        float s = 0.f;
        for (int l = tid; l < j; ++l) s = fmaf(Ts[tid][l], Ds[j][l], s);
        Ts[tid][j] = -taus[j] * s;
      }
      if (tid == j) Ts[j][j] = taus[j];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
  // outputs
  float* Tm = Tout + (int64_t)blockIdx.x * NB * NB;
  if (tid < NB * NB) Tm[tid] = Ts[tid / NB][tid % NB];
  float* Bm = band + (int64_t)blockIdx.x * bstride;
#pragma unroll
  for (int h = 0; h < RPT; ++h) {
    const int row = tid + NT * h;
    if (row >= m) continue;
    float* arow = Am + (int64_t)(r0 + row) * n + c0;
    float o[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) o[c] = row > c ? (c < kk ? P[h][c] : 0.f) : (row == c ? (c < kk ? 1.f : 0.f) : 0.f);
    if (vec) {
#pragma unroll
      for (int c = 0; c < NB; c += 4) gst4(arow + c, v4f{o[c], o[c + 1], o[c + 2], o[c + 3]});
    } else {
#pragma unroll
      for (int c = 0; c < NB; ++c) arow[c] = o[c];
    }
    if (row < NB) {
      // R row `row`: columns c >= row, band diagonal d = NB + row - c
      float* brow = Bm + (int64_t)(r0 + row) * BW;
#pragma unroll
      for (int c = 0; c < NB; ++c)
        if (c >= row) brow[NB + row - c] = c == row ? (row < kk ? betas[row] : P[h][c]) : P[h][c];
    }
  }
}

// ------------------------------------------------------- sy2sb update ---
// One panel step of the dense -> band reduction, on the lower triangle only.
// Region R: rows and columns >= r1 of each matrix (mr of them).  With the
// panel's reflector block V (mr x 16, rows from r1) and its correction W,
//   A <- A - V W^T - W V^T        (elements with row >= column)
// and, when Vn (the next panel's reflectors, rows from r1) is given,
//   Y  = A_new Vn                 (the symmetric matrix A_new)
// Nothing above the diagonal is read or written: a diagonal tile is read from
// its lower half and mirrored (k_sy2sb_update_vec below, for aligned
// operands, also writes the upper half of diagonal tiles; nothing reads it).  64 x 64 tiles; the workgroup of tile-row I
// and chunk c takes tiles (I, J), J in [UCH c, min(UCH (c+1), I+1)); it
// writes its direct product sum_J A(I,J) Vn(J) to Pd[I][c] and, per tile
// below the diagonal, A(I,J)^T Vn(I) to Pt[J][I]; k_sy2sb_reduce sums them
// in a fixed order.  Each tile moves 16 KB in and 16 KB out (half of them on
// the diagonal), against 48 KB for a full-matrix update plus a separate
// A Vn product.
constexpr int UT = 64;           // update tile
constexpr int UCH = 4;           // tiles per workgroup
constexpr int UPT = UT + 4;      // LDS pitch of the A tile
constexpr int UPL = 33;          // LDS pitch of [V | W] rows (conflict-free MFMA reads)
constexpr int UPV = 17;          // LDS pitch of Vn rows

__device__ __forceinline__ void ut_task(int t, int& I, int& c) {
  int before = 0;
  I = 0;
  for (;;) {
    const int nc = I / UCH + 1;
    if (t < before + nc) {
      c = t - before;
      return;
    }
    before += nc;
    ++I;
  }
}

__global__ __launch_bounds__(256) void k_sy2sb_update(float* A, int64_t sA, int ldA, int mr,
                                                      const float* V, int64_t sV, int ldV,
                                                      const float* W, int64_t sW, int ldW,
                                                      const float* Vn, int64_t sVn, int ldVn,
                                                      float* Pd, float* Pt, int nt, int nch) {
  __shared__ __attribute__((aligned(16))) float As[UT][UPT];
  __shared__ float Ls[UT][UPL];   // [V_I | W_I]
  __shared__ float Rs[UT][UPL];   // [W_J | V_J]
  __shared__ float VnI[UT][UPV];
  __shared__ float VnJ[UT][UPV];
  int I, c;
  ut_task(blockIdx.x, I, c);
  const int mat = blockIdx.y;
  float* Am = A + (int64_t)mat * sA;
  V += (int64_t)mat * sV;
  W += (int64_t)mat * sW;
  const bool doY = Vn != nullptr;
  if (doY) Vn += (int64_t)mat * sVn;
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64, kk = l / 16;
  const bool vec = (ldA % 4) == 0;

  for (int idx = tid; idx < UT * 16; idx += 256) {
    const int row = idx / 16, q = idx % 16, gi = UT * I + row;
    const bool ok = gi < mr;
    Ls[row][q] = ok ? V[(int64_t)gi * ldV + q] : 0.f;
    Ls[row][16 + q] = ok ? W[(int64_t)gi * ldW + q] : 0.f;
    if (doY) VnI[row][q] = ok ? Vn[(int64_t)gi * ldVn + q] : 0.f;
  }
  // the next tile's operands, in registers: A (4 x 4 per thread) and the
  // W_J / V_J / Vn_J rows (4 each: thread t holds row t/4, columns 4(t%4)..)
  v4f na[4], nw, nv, nn;
  auto fetch = [&](int J) {
    const bool diag = J == I;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int idx = tid + 256 * h, row = idx / 16, c4 = (idx % 16) * 4;
      const int gi = UT * I + row, gj = UT * J + c4;
      v4f x = {0.f, 0.f, 0.f, 0.f};
      if (gi < mr) {
        const float* src = Am + (int64_t)gi * ldA + gj;
        if (vec && gj + 3 < mr && (!diag || row >= c4 + 3)) {
          x = *(const v4f*)src;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (gj + t < mr && (!diag || row >= c4 + t)) x[t] = src[t];
        }
      }
      na[h] = x;
    }
    const int row = tid / 4, q4 = (tid % 4) * 4, gj = UT * J + row;
    const bool ok = gj < mr;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      nw[t] = ok ? W[(int64_t)gj * ldW + q4 + t] : 0.f;
      nv[t] = ok ? V[(int64_t)gj * ldV + q4 + t] : 0.f;
      nn[t] = (ok && doY) ? Vn[(int64_t)gj * ldVn + q4 + t] : 0.f;
    }
  };
  v4f ay = {0.f, 0.f, 0.f, 0.f};
  const int j0 = UCH * c, j1 = UCH * c + UCH < I + 1 ? UCH * c + UCH : I + 1;
  fetch(j0);
  for (int J = j0; J < j1; ++J) {
    const bool diag = J == I;
    __syncthreads();                 // the previous tile's LDS reads are done
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int idx = tid + 256 * h;
      *(v4f*)&As[idx / 16][(idx % 16) * 4] = na[h];
    }
    {
      const int row = tid / 4, q4 = (tid % 4) * 4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        Rs[row][q4 + t] = nw[t];
        Rs[row][16 + q4 + t] = nv[t];
        VnJ[row][q4 + t] = nn[t];
      }
    }
    __syncthreads();
    if (J + 1 < j1) fetch(J + 1);    // in flight during this tile's work
    if (diag) {                      // mirror the lower half
      for (int idx = tid; idx < UT * UT; idx += 256) {
        const int row = idx / UT, col = idx % UT;
        if (row < col) As[row][col] = As[col][row];
      }
      __syncthreads();
    }
    // A_new = A - [V_I W_I] [W_J V_J]^T: wave w rows 16w.., four 16-column tiles
    v4f d[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) d[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k4 = 0; k4 < 8; ++k4) {
      const int q = 4 * k4 + kk;
      const float a = Ls[16 * w + l % 16][q];
#pragma unroll
      for (int t = 0; t < 4; ++t) d[t] = mfma16(a, Rs[16 * t + l % 16][q], d[t]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * w + 4 * kk + r, col = 16 * t + l % 16;
        As[row][col] = As[row][col] - d[t][r];
      }
    __syncthreads();
    if (diag) {                      // the stored (lower) half defines the matrix
      for (int idx = tid; idx < UT * UT; idx += 256) {
        const int row = idx / UT, col = idx % UT;
        if (row < col) As[row][col] = As[col][row];
      }
      __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int idx = tid + 256 * h, row = idx / 16, c4 = (idx % 16) * 4;
      const int gi = UT * I + row, gj = UT * J + c4;
      if (gi >= mr) continue;
      float* dst = Am + (int64_t)gi * ldA + gj;
      const v4f x = *(const v4f*)&As[row][c4];
      if (vec && gj + 3 < mr && (!diag || row >= c4 + 3)) {
        *(v4f*)dst = x;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (gj + t < mr && (!diag || row >= c4 + t)) dst[t] = x[t];
      }
    }
    if (!doY) continue;
    // direct part: rows 16w.. of A_new(I,J) Vn(J)
#pragma unroll
    for (int k4 = 0; k4 < 16; ++k4) {
      const int j = 4 * k4 + kk;
      ay = mfma16(As[16 * w + l % 16][j], VnJ[j][l % 16], ay);
    }
    if (!diag) {
      // transposed part: rows 16w.. of A_new(I,J)^T Vn(I), for tile-row J
      v4f pt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k4 = 0; k4 < 16; ++k4) {
        const int i = 4 * k4 + kk;
        pt = mfma16(As[i][16 * w + l % 16], VnI[i][l % 16], pt);
      }
      float* dst = Pt + (((int64_t)mat * nt + J) * nt + I) * (UT * 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(16 * w + 4 * kk + r) * 16 + l % 16] = pt[r];
    }
  }
  if (doY) {
    float* dst = Pd + (((int64_t)mat * nt + I) * nch + c) * (UT * 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(16 * w + 4 * kk + r) * 16 + l % 16] = ay[r];
  }
}

// The same update for 16-byte aligned operands (every leading dimension and
// mr a multiple of 4), with the A tile held in registers: lane l of wave w
// keeps rows 16w + 4(l/16) + r, columns 4(l%16) .. 4(l%16)+3 of the tile,
// which is the MFMA output layout once the update's columns are permuted
// (MFMA tile t, lane column jj <-> tile column 4jj + t).  So the rank-32
// update happens in registers and the tile goes back to memory as float4
// rows; LDS holds it only for the two Y products.  The LDS operands are
// double-buffered (the next panel's reflector rows triple-buffered), so one
// block barrier per tile suffices: before barrier J every wave writes tile
// J's updated values and tile J+1's W/V/Vn rows, after it the Y products of
// tile J run while tile J+1's loads are in flight.  The arithmetic is that of
// k_sy2sb_update term by term, so the results are bit-identical.
constexpr int UQ = 3;   // slots of the next panel's reflector rows

__global__ __launch_bounds__(256) void k_sy2sb_update_vec(float* A, int64_t sA, int ldA, int mr,
                                                          const float* V, int64_t sV, int ldV,
                                                          const float* W, int64_t sW, int ldW,
                                                          const float* Vn, int64_t sVn, int ldVn,
                                                          float* Pd, float* Pt, int nt, int nch) {
  __shared__ __attribute__((aligned(16))) float As[2][UT][UPT];
  __shared__ float Ls[UT][UPL];      // [V_I | W_I]
  __shared__ float Rs[2][UT][UPL];   // [W_J | V_J]
  __shared__ float VnI[UT][UPV];
  __shared__ float VnJ[UQ][UT][UPV];
  int I, c;
  ut_task(blockIdx.x, I, c);
  const int mat = blockIdx.y;
  float* Am = A + (int64_t)mat * sA;
  V += (int64_t)mat * sV;
  W += (int64_t)mat * sW;
  const bool doY = Vn != nullptr;
  if (doY) Vn += (int64_t)mat * sVn;
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64, kk = l / 16, jj = l % 16;

  // Tile loads: every address stays inside the region (rows and columns at or
  // beyond mr read row / column 0); such values are replaced by zeros where
  // they are used, not where they land, so no wait follows a load.  The
  // block's (at most UCH) tiles are unrolled, so each prefetch buffer has a
  // fixed register name and nothing is copied between iterations.
  const int gr0 = UT * I + 16 * w + 4 * kk;   // the lane's first tile row
  // Every prefetch is issued whether or not its tile exists (a tile past the
  // block's last reads the region's first element, one line for all lanes):
  // a load issued on one path only would make the compiler wait for all
  // loads at the join.
  const int j0 = UCH * c, j1 = UCH * c + UCH < I + 1 ? UCH * c + UCH : I + 1;
  auto load_a = [&](int J, v4f (&x)[4]) {
    const int gj = UT * J + 4 * jj;
    const bool cok = J < j1 && gj < mr;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = cok && gr0 + r < mr;
      x[r] = gld4(Am + (int64_t)(ok ? gr0 + r : 0) * ldA + (ok ? gj : 0));
    }
  };
  // W_J, V_J, Vn_J rows: thread -> row tid/4, columns 4(tid%4) ..
  const int rrow = tid / 4, rq = (tid % 4) * 4;
  auto load_rows = [&](int J, v4f (&x)[3]) {
    const int gj = UT * J + rrow;
    const int64_t g = J < j1 && gj < mr ? gj : 0;
    x[0] = gld4(W + g * ldW + rq);
    x[1] = gld4(V + g * ldV + rq);
    x[2] = gld4(doY ? Vn + g * ldVn + rq : W + rq);
  };
  auto put_rows = [&](int J, int b, int slot, const v4f (&x)[3]) {
    const bool ok = UT * J + rrow < mr;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      Rs[b][rrow][rq + t] = ok ? x[0][t] : 0.f;
      Rs[b][rrow][16 + rq + t] = ok ? x[1][t] : 0.f;
      VnJ[slot][rrow][rq + t] = ok && doY ? x[2][t] : 0.f;
    }
  };

  v4f ay = {0.f, 0.f, 0.f, 0.f};
  // EDGE: the last tile-row of a region whose size is not a multiple of 64
  // (rows, and the diagonal tile's columns, reach past mr).  Elsewhere every
  // element of every tile exists and the stores are four float4 rows per
  // lane on every path; a diagonal tile then also writes its upper half,
  // which nothing reads (the stored lower half defines the matrix), so that
  // the number of memory operations in flight is the same on every path and
  // each wait is for the one load it needs.
  auto tiles = [&](auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    v4f ab[3][4], rb[2][3], li[3];
    v4f keep[UCH][4], ptk[UCH];   // each tile's new values and transposed partial
    // the tile-row's own V, W, Vn rows and the first two tiles, all in flight
    // together
    {
      const int gi = UT * I + rrow;
      const int64_t g = gi < mr ? gi : 0;
      li[0] = gld4(V + g * ldV + rq);
      li[1] = gld4(W + g * ldW + rq);
      li[2] = gld4(doY ? Vn + g * ldVn + rq : W + rq);
    }
    load_a(j0, ab[0]);
    load_a(j0 + 1, ab[1]);
    load_rows(j0, rb[0]);
    load_rows(j0 + 1, rb[1]);
    {
      const bool ok = UT * I + rrow < mr;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        Ls[rrow][rq + t] = ok ? li[0][t] : 0.f;
        Ls[rrow][16 + rq + t] = ok ? li[1][t] : 0.f;
        VnI[rrow][rq + t] = ok && doY ? li[2][t] : 0.f;
      }
    }
    put_rows(j0, 0, 0, rb[0]);
    __syncthreads();
#pragma unroll
    for (int jt = 0; jt < UCH; ++jt) {
      const int J = j0 + jt;
      if (J >= j1) break;
      const int b = jt & 1, slot = jt % UQ;
      const bool diag = J == I;
      load_a(J + 2, ab[(jt + 2) % 3]);   // two tiles of A in flight
      // A_new = A - [V_I W_I] [W_J V_J]^T, in the lane's own elements
      v4f d[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) d[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k4 = 0; k4 < 8; ++k4) {
        const int q = 4 * k4 + kk;
        const float a = Ls[16 * w + jj][q];
#pragma unroll
        for (int t = 0; t < 4; ++t) d[t] = mfma16(a, Rs[b][4 * jj + t][q], d[t]);
      }
      // the next tile's W/V/Vn rows (loaded one tile ahead)
      if (J + 1 < j1) put_rows(J + 1, b ^ 1, (jt + 1) % UQ, rb[(jt + 1) & 1]);
      const int gj = UT * J + 4 * jj;
      v4f (&an)[4] = keep[jt];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = !EDGE || (gj < mr && gr0 + r < mr);
#pragma unroll
        for (int t = 0; t < 4; ++t) an[r][t] = (ok ? ab[jt % 3][r][t] : 0.f) - d[t][r];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) *(v4f*)&As[b][16 * w + 4 * kk + r][4 * jj] = an[r];
      load_rows(J + 2, rb[jt & 1]);
      __syncthreads();
      if (diag) {                      // the stored (lower) half defines the matrix
#pragma unroll
        for (int h = 0; h < UT * UT / 256; ++h) {
          const int idx = tid + 256 * h, row = idx / UT, col = idx % UT;
          if (row < col) As[b][row][col] = As[b][col][row];
        }
        __syncthreads();
      }
      if (doY) {
        // direct part: rows 16w.. of A_new(I,J) Vn(J); transposed part: rows
        // 16w.. of A_new(I,J)^T Vn(I), for tile-row J
        if (!diag) {
          v4f pt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int k4 = 0; k4 < 16; ++k4) {
            const int j = 4 * k4 + kk;
            ay = mfma16(As[b][16 * w + jj][j], VnJ[slot][j][jj], ay);
            pt = mfma16(As[b][j][16 * w + jj], VnI[j][jj], pt);
          }
          ptk[jt] = pt;
        } else {
#pragma unroll
          for (int k4 = 0; k4 < 16; ++k4) {
            const int j = 4 * k4 + kk;
            ay = mfma16(As[b][16 * w + jj][j], VnJ[slot][j][jj], ay);
          }
        }
      }
    }
    // Every global store of the block goes out here, after the last load:
    // with stores and loads both in flight the compiler can only wait for
    // all of them (vmcnt(0)), which would expose each prefetch's latency.
#pragma unroll
    for (int jt = 0; jt < UCH; ++jt) {
      const int J = j0 + jt;
      if (J >= j1) break;
      const bool diag = J == I;
      const int gj = UT * J + 4 * jj;
      if (!EDGE) {
        // a diagonal tile also writes its upper half, which nothing reads
#pragma unroll
        for (int r = 0; r < 4; ++r) gst4(Am + (int64_t)(gr0 + r) * ldA + gj, keep[jt][r]);
      } else {
        // the lower triangle only, inside the region
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int gi = gr0 + r;
          if (gi >= mr || gj >= mr) continue;
          float* dst = Am + (int64_t)gi * ldA + gj;
          if (!diag) {
            gst4(dst, keep[jt][r]);
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (gi >= gj + t) dst[t] = keep[jt][r][t];
          }
        }
      }
      if (doY && !diag) {
        float* dst = Pt + (((int64_t)mat * nt + J) * nt + I) * (UT * 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[(16 * w + 4 * kk + r) * 16 + jj] = ptk[jt][r];
      }
    }
  };
  if (UT * I + UT <= mr)
    tiles(std::false_type{});
  else
    tiles(std::true_type{});
  if (doY) {
    float* dst = Pd + (((int64_t)mat * nt + I) * nch + c) * (UT * 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(16 * w + 4 * kk + r) * 16 + jj] = ay[r];
  }
}

// The panel's correction W and the next panel's columns, one workgroup of
// 1024 threads per matrix.  V: the panel's reflectors (m x 16, rows r0.. of A
// at column c0), Y = A22 V (m x 16), T (16 x 16 upper):
//   G = V^T Y (four row-quarter partial sums per 256-row chunk, added in a
//       fixed order), M = T^T G T,
//   W = Y T - V M / 2                          (m x 16, to Wout),
// and, with `strip`, the next panel's columns r0..r0+15 of rows r0..:
//   A[r0+i][r0+j] -= V[i] . W[j] + W[i] . V[j]   (j < 16).
// W and the strip take one thread per row (PW_RPT rows per thread), each
// row's 16 floats as four 16-byte accesses when rows are 16-byte aligned.
constexpr int PW_RPT = 2;    // rows per thread: m <= 2048 (larger m loops)
__device__ __forceinline__ void ld16(const float* p, bool vec, float (&x)[16]) {
  if (vec) {
#pragma unroll
    for (int c = 0; c < 16; c += 4) {
      const v4f v = gld4(p + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[c + e] = v[e];
    }
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) x[c] = p[c];
  }
}
__device__ __forceinline__ void st16(float* p, bool vec, const float (&x)[16]) {
  if (vec) {
#pragma unroll
    for (int c = 0; c < 16; c += 4) gst4(p + c, v4f{x[c], x[c + 1], x[c + 2], x[c + 3]});
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) p[c] = x[c];
  }
}
__global__ __launch_bounds__(1024) void k_sy2sb_panel_w(float* A, int64_t sA, int n, int r0, int c0,
                                                        const float* Y, const float* T, float* Wout,
                                                        int strip) {
  __shared__ float Vs[256][17], Ys[256][17];
  __shared__ float Gp[4][16][17];
  __shared__ float Ts[16][17], GTs[16][17], Ms[16][17];
  __shared__ float Vt[16][17], Wt[16][17];
  const int mat = blockIdx.x, tid = threadIdx.x;
  const int m = n - r0;
  float* Am = A + (int64_t)mat * sA;
  const float* Ym = Y + (int64_t)mat * m * 16;
  float* Wm = Wout + (int64_t)mat * m * 16;
  const bool vec = (n % 4) == 0 && (sA % 4) == 0 && (c0 % 4) == 0 && (r0 % 4) == 0 &&
                   ((((uintptr_t)A) | ((uintptr_t)Y) | ((uintptr_t)Wout)) & 15) == 0;
  const int a = (tid / 16) % 16, b = tid % 16, p = tid / 256;
  if (tid < 256) Ts[a][b] = T[(int64_t)mat * 256 + a * 16 + b];
  // G[a][b] = sum_i V[i][a] Y[i][b]: chunks of 256 rows staged in LDS (the
  // next chunk's loads in flight during the current chunk's sums); thread
  // (p, a, b) sums rows 64p .. 64p+63 of each chunk
  const int lr = tid / 4, lq = (tid % 4) * 4;    // loader: row lr, floats lq..lq+3
  auto load = [&](int i0, v4f& xv, v4f& xy) {
    const int i = i0 + lr;
    xv = v4f{0.f, 0.f, 0.f, 0.f};
    xy = xv;
    if (i < m) {
      const float* vp = Am + (int64_t)(r0 + i) * n + c0 + lq;
      const float* yp = Ym + (int64_t)i * 16 + lq;
      if (vec) {
        xv = gld4(vp);
        xy = gld4(yp);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xv[e] = vp[e];
          xy[e] = yp[e];
        }
      }
    }
  };
  float g = 0.f;
  v4f xv, xy;
  load(0, xv, xy);
  for (int i0 = 0; i0 < m; i0 += 256) {
    __syncthreads();                   // the previous chunk is consumed
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Vs[lr][lq + e] = xv[e];
      Ys[lr][lq + e] = xy[e];
    }
    __syncthreads();
    if (i0 + 256 < m) load(i0 + 256, xv, xy);
    const int rows = m - i0 < 256 ? m - i0 : 256;
    const int re = rows < 64 * p + 64 ? rows : 64 * p + 64;
    for (int row = 64 * p; row < re; ++row) g = fmaf(Vs[row][a], Ys[row][b], g);
  }
  Gp[p][a][b] = g;
  __syncthreads();
  if (tid < 256) {
    const float gg = ((Gp[0][a][b] + Gp[1][a][b]) + Gp[2][a][b]) + Gp[3][a][b];
    Gp[0][a][b] = gg;
  }
  __syncthreads();
  if (tid < 256) {
    float x = 0.f;
    for (int c = 0; c < 16; ++c) x = fmaf(Gp[0][a][c], Ts[c][b], x);
    GTs[a][b] = x;
  }
  __syncthreads();
  if (tid < 256) {
    float x = 0.f;
    for (int c = 0; c < 16; ++c) x = fmaf(Ts[c][a], GTs[c][b], x);
    Ms[a][b] = x;
  }
  __syncthreads();
  // W rows, one thread per row
  for (int ib = 0; ib < m; ib += 1024 * PW_RPT) {
    float yr[PW_RPT][16], vr[PW_RPT][16];
#pragma unroll
    for (int h = 0; h < PW_RPT; ++h) {
      const int i = ib + tid + 1024 * h;
      if (i < m) {
        ld16(Ym + (int64_t)i * 16, vec, yr[h]);
        ld16(Am + (int64_t)(r0 + i) * n + c0, vec, vr[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < PW_RPT; ++h) {
      const int i = ib + tid + 1024 * h;
      if (i >= m) continue;
      // T and M are read from LDS per row: hoisted out of the loops they
      // would take 512 registers
      asm volatile("" ::: "memory");
      float w[16];
#pragma unroll
      for (int bb = 0; bb < 16; ++bb) {
        float yt = 0.f, vm = 0.f;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          yt = fmaf(yr[h][c], Ts[c][bb], yt);
          vm = fmaf(vr[h][c], Ms[c][bb], vm);
        }
        w[bb] = yt - 0.5f * vm;
      }
      st16(Wm + (int64_t)i * 16, vec, w);
      if (i < 16) {
#pragma unroll
        for (int bb = 0; bb < 16; ++bb) {
          Wt[i][bb] = w[bb];
          Vt[i][bb] = vr[h][bb];
        }
      }
    }
  }
  if (!strip) return;
  __syncthreads();                   // W (first rows) and the V rows in LDS; W in memory
  for (int ib = 0; ib < m; ib += 1024 * PW_RPT) {
    float vr[PW_RPT][16], wr[PW_RPT][16], ar[PW_RPT][16];
#pragma unroll
    for (int h = 0; h < PW_RPT; ++h) {
      const int i = ib + tid + 1024 * h;
      if (i < m) {
        ld16(Am + (int64_t)(r0 + i) * n + c0, vec, vr[h]);
        ld16(Wm + (int64_t)i * 16, vec, wr[h]);
        ld16(Am + (int64_t)(r0 + i) * n + r0, vec, ar[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < PW_RPT; ++h) {
      const int i = ib + tid + 1024 * h;
      if (i >= m) continue;
      asm volatile("" ::: "memory");   // Wt and Vt read per row, as T and M above
#pragma unroll
      for (int bb = 0; bb < 16; ++bb) {
        float d = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) d = fmaf(vr[h][q], Wt[bb][q], fmaf(wr[h][q], Vt[bb][q], d));
        ar[h][bb] -= d;
      }
      st16(Am + (int64_t)(r0 + i) * n + r0, vec, ar[h]);
    }
  }
}

// Y[J rows] = sum_c Pd[J][c] + sum_{I > J} Pt[J][I], in that order.
__global__ __launch_bounds__(256) void k_sy2sb_reduce(const float* Pd, const float* Pt, float* Y,
                                                      int64_t sY, int mr, int nt, int nch) {
  const int J = blockIdx.x, mat = blockIdx.y;
  const int e0 = threadIdx.x * 4;            // 4 of the 64 x 16 outputs
  const int row = e0 / 16, col = e0 % 16;
  if (UT * J + row >= mr) return;
  v4f s = {0.f, 0.f, 0.f, 0.f};
  // the terms in order; RU loads in flight at a time (one at a time, each
  // block's chain of up to nt tiles waited on the memory latency per term)
  constexpr int RU = 8;
  auto add_run = [&](const float* base, int n_terms) {
    int u0 = 0;
    for (; u0 + RU <= n_terms; u0 += RU) {
      v4f x[RU];
#pragma unroll
      for (int u = 0; u < RU; ++u) x[u] = *(const v4f*)(base + (int64_t)(u0 + u) * (UT * 16) + e0);
#pragma unroll
      for (int u = 0; u < RU; ++u)
#pragma unroll
        for (int t = 0; t < 4; ++t) s[t] += x[u][t];
    }
    for (; u0 < n_terms; ++u0) {
      const v4f x = *(const v4f*)(base + (int64_t)u0 * (UT * 16) + e0);
#pragma unroll
      for (int t = 0; t < 4; ++t) s[t] += x[t];
    }
  };
  add_run(Pd + ((int64_t)mat * nt + J) * nch * (UT * 16), J / UCH + 1);
  add_run(Pt + (((int64_t)mat * nt + J) * nt + J + 1) * (UT * 16), nt - J - 1);
  *(v4f*)(Y + (int64_t)mat * sY + (int64_t)(UT * J + row) * 16 + col) = s;
}

// ---------------------------------------------------------- band finish ---
// Row i: diagonals 0..i-bs from the final diagonal block of A (bs = start of
// i's NB-row block), diagonals above that up to NB were written by the panel
// QR (R), or are left of column 0 (first block: zero); bulge diagonals
// NB+1..2NB zero.  orig keeps diagonals 0..NB.
__global__ __launch_bounds__(256) void k_band_finish(const float* A, int64_t stride, int n,
                                                     const float* band, int64_t bstride,
                                                     float* orig, int64_t ostride, double* band64) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int mat = blockIdx.y;
  const float* Am = A + (int64_t)mat * stride;
  const float* brow = band + (int64_t)mat * bstride + (int64_t)i * BW;
  float* orow = orig + (int64_t)mat * ostride + (int64_t)i * OW;
  double* wrow = band64 + (int64_t)mat * n * BW + (int64_t)i * BW;
  const int bs = (i / NB) * NB;
  for (int d = 0; d <= NB; ++d) {
    float v;
    if (d <= i - bs)
      v = Am[(int64_t)i * n + (i - d)];
    else if (bs == 0)
      v = 0.f;
    else
      v = brow[d];
    orow[d] = v;
    wrow[d] = (double)v;
  }
  for (int d = NB + 1; d < BW; ++d) wrow[d] = 0.0;
}

// --------------------------------------------------------------- sb2st ---
// Bulge chasing in float64, one workgroup of SB_W wavefronts per matrix (the
// per-task chain of LDS round trips and shuffles is latency-bound, and there is
// one matrix per CU: more sweeps in flight are the parallelism there is).
// Task k of sweep s owns band rows q0..q0+LM-1 (q0 = s + 1 + 16k): the block
// E = B[rows, previous block's rows] (for task 0 the single column s) and the
// diagonal block D.  E gets the previous reflector from the right, a new
// reflector annihilates E's first column below its first row and is applied
// to E from the left and to D from both sides.  A task touches only its own
// rows, so:
//   * wavefront w runs sweeps w, w + SB_W, ...; sweep s may run task k once
//     sweep s-1 has finished task k+2 (their rows overlap up to there), and
//     each wavefront publishes its progress (s * 65536 + tasks done) in LDS;
//   * the rows of task k+1 are loaded while task k computes (they need sweep
//     s-1 to have finished task k+3, which it almost always has).
constexpr int SB_W = 16;   // 16 sweeps in flight (8: 75.8 ms, 12: 59.2, 16: 53.3 at 240 x 2048^2)
constexpr int SB_BIG = 1 << 16;

struct Sb2stLds {
  double E[NB][NB + 1];
  double D[NB][NB + 1];
  double v[NB];
  double y[NB];
  double pv[NB];
  double junk;          // target of an interior task's out-of-window scatter
};
// An interior task addresses E, D and junk as offsets from E[0][0].
constexpr int SB_D0 = NB * (NB + 1);
constexpr int SB_JUNK = 2 * NB * (NB + 1) + 3 * NB;

// sum over each quad (xor 1, 2), left in every lane of the quad
__device__ __forceinline__ double sum4(double x) {
  x += dpp_d<DPP_XOR1>(x);
  x += dpp_d<DPP_XOR2>(x);
  return x;
}
// sum over each 16-lane row, left in every lane of the row
__device__ __forceinline__ double sum16(double x) {
  x = sum4(x);
  x += dpp_d<DPP_HALF_MIRROR>(x);
  x += dpp_d<DPP_ROW_MIRROR>(x);
  return x;
}
// LDS traffic of one wavefront is ordered; this keeps the compiler from
// moving its accesses across the point.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int sb_ntasks(int n, int s) { return (n - 1 - s + NB - 1) / NB; }

// Wait until the wavefront running sweep s-1 has finished `tasks` of its tasks.
// The progress words live in LDS and are reached through an LDS-typed
// pointer: a generic (flat) access would count as a vector memory operation,
// and each poll would wait for every load and store of the wave.
typedef __attribute__((address_space(3))) int lds_int;

__device__ __forceinline__ void sb_wait(lds_int* prog, int s, int tasks) {
  if (s == 0) return;
  const int w = (s - 1) % SB_W;
  const int target = (s - 1) * SB_BIG + tasks;
  while (__hip_atomic_load(&prog[w], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
    __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__global__ __launch_bounds__(SB_W * 64) void k_sb2st(double* band, int n, double* dout,
                                                     double* eout) {
  __shared__ Sb2stLds Sall[SB_W];
  __shared__ int prog_s[SB_W];
  lds_int* prog = (lds_int*)prog_s;
  const int wid = threadIdx.x >> 6, l = threadIdx.x & 63;
  Sb2stLds& S = Sall[wid];
  double* Bm = band + (int64_t)blockIdx.x * n * BW;
  if (l == 0) prog[wid] = -SB_BIG;
  __syncthreads();
  const int r = l >> 2, q = l & 3;   // (row or column, quarter) lane roles
  for (int s = wid; s + 2 < n; s += SB_W) {
    const int nt = sb_ntasks(n, s);
    const int ntp = s > 0 ? sb_ntasks(n, s - 1) : 0;
    double cur[8], nxt[8];
    // rows of task 0
    sb_wait(prog, s, min(3, ntp));
    {
      const int q0 = s + 1, LM = min(NB, n - q0);
      for (int t = 0; t < 8; ++t) {
        const int idx = l + 64 * t, row = idx >> 5, d = idx & 31;
        cur[t] = row < LM ? Bm[(int64_t)(q0 + row) * BW + d] : 0.0;
      }
    }
    int q0 = s + 1, LN = 1;          // task 0: E is column s (one column)
    double ptau = 0.0;               // previous reflector (none for task 0)
    for (int k = 0; k < nt; ++k) {
      // an interior task (16 rows, a 16-column E) has every bound fixed:
      // its instantiation drops the per-element edge tests (the kernel is
      // bound by instruction issue)
      auto task = [&](auto full) {
        constexpr bool FULL = decltype(full)::value;
        const int LM = FULL ? NB : min(NB, n - q0);
        const int LNv = FULL ? NB : LN;
        // scatter this task's rows into E / D (an interior task without
        // branches: every element goes to a selected address, out-of-window
        // ones to junk)
        double* const S0 = &S.E[0][0];
        if constexpr (FULL) {
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int idx = l + 64 * t, row = idx >> 5, d = idx & 31;
            const bool inD = d <= row, inE = !inD && d <= row + NB;
            const int a1 = inD ? SB_D0 + row * (NB + 1) + row - d
                               : (inE ? row * (NB + 1) + NB + row - d : SB_JUNK);
            const int a2 = inD ? SB_D0 + (row - d) * (NB + 1) + row : SB_JUNK;
            S0[a1] = cur[t];
            S0[a2] = cur[t];
          }
        } else {
          for (int t = 0; t < 8; ++t) {
            const int idx = l + 64 * t, row = idx >> 5, d = idx & 31;
            if (row < LM) {
              if (d <= row) {
                S.D[row][row - d] = cur[t];
                S.D[row - d][row] = cur[t];
              } else if (d <= row + LNv) {
                S.E[row][LNv + row - d] = cur[t];
              }
            }
          }
        }
        // prefetch the next task's rows
        if (k + 1 < nt) {
          sb_wait(prog, s, min(k + 4, ntp));
          const int q1 = q0 + LM, LM1 = min(NB, n - q1);
          for (int t = 0; t < 8; ++t) {
            const int idx = l + 64 * t, row = idx >> 5, d = idx & 31;
            nxt[t] = row < LM1 ? Bm[(int64_t)(q1 + row) * BW + d] : 0.0;
          }
        }
        wave_sync();
        // 1. E <- E (I - ptau pv pv^T)
        // Steps 1 and 3 read and write only the lane's own four elements
        // (the sums go through DPP), so each keeps them in registers from its
        // read to its write; step 4 does the same with D.
        if (ptau != 0.0) {
          double t = 0.0, e4[4], p4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int c = 4 * q + j;
            e4[j] = S.E[r][c];
            p4[j] = S.pv[c];
            if (r < LM && c < LNv) t = fma(e4[j], p4[j], t);
          }
          t = sum4(t);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int c = 4 * q + j;
            if (r < LM && c < LNv) S.E[r][c] = fma(-ptau * t, p4[j], e4[j]);
          }
          wave_sync();
        }
        // 2. reflector from E[:, 0] (length LM)
        const int rr = l & 15;
        const double x0 = rr < LM ? S.E[rr][0] : 0.0;
        const double alpha = S.E[0][0];
        const double s2 = sum16(rr >= 1 ? x0 * x0 : 0.0);
        double tau = 0.0, beta = alpha, scale = 0.0;
        if (s2 > 0.0) {
          beta = -copysign(sqrt(alpha * alpha + s2), alpha);
          tau = (beta - alpha) / beta;
          scale = 1.0 / (alpha - beta);
        }
        wave_sync();
        if (l < NB) {
          S.v[l] = l == 0 ? 1.0 : (l < LM ? x0 * scale : 0.0);
          if (l < LM) S.E[l][0] = l == 0 ? beta : 0.0;
        }
        wave_sync();
        if (tau != 0.0) {
          // 3. E[:, 1:] <- (I - tau v v^T) E[:, 1:]   (lane: column r, rows 4q..4q+3)
          double w = 0.0, e4[4], v4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int i = 4 * q + j;
            v4[j] = S.v[i];
            e4[j] = S.E[i][r];
            if (r >= 1 && r < LNv && i < LM) w = fma(v4[j], e4[j], w);
          }
          w = sum4(w);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int i = 4 * q + j;
            if (r >= 1 && r < LNv && i < LM) S.E[i][r] = fma(-tau * v4[j], w, e4[j]);
          }
          // 4. D <- H D H: y = tau D v; y -= (tau/2)(y^T v) v; D -= v y^T + y v^T
          double y = 0.0, d4[4], vc[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int c = 4 * q + j;
            d4[j] = S.D[r][c];
            vc[j] = S.v[c];
            if (r < LM && c < LM) y = fma(d4[j], vc[j], y);
          }
          y = tau * sum4(y);
          // y^T v over the 16 rows: lane 4r holds row r's term; copied to its
          // quad, summed over the 16-lane row, then across the four rows
          double a = (q == 0 && r < LM) ? y * S.v[r] : 0.0;
          a = dpp_d<DPP_QUAD0>(a);
          a += dpp_d<DPP_HALF_MIRROR>(a);
          a += dpp_d<DPP_ROW_MIRROR>(a);
          a = xor_sum_d<false>(a);
          a = xor_sum_d<true>(a);
          a *= 0.5 * tau;
          if (q == 0 && r < LM) S.y[r] = fma(-a, S.v[r], y);
          wave_sync();
          const double vr = S.v[r], yr = S.y[r];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int c = 4 * q + j;
            if (r < LM && c < LM) S.D[r][c] = d4[j] - (vr * S.y[c] + yr * vc[j]);
          }
          wave_sync();
        }
        // store the rows back, then publish the task
        if constexpr (FULL) {
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int idx = l + 64 * t, row = idx >> 5, d = idx & 31;
            const bool inD = d <= row;
            const int a1 = inD ? SB_D0 + row * (NB + 1) + row - d : row * (NB + 1) + NB + row - d;
            const double v = S0[d <= row + NB ? a1 : SB_JUNK];
            if (d <= row + NB) Bm[(int64_t)(q0 + row) * BW + d] = v;
          }
        } else {
          for (int t = 0; t < 8; ++t) {
            const int idx = l + 64 * t, row = idx >> 5, d = idx & 31;
            if (row < LM) {
              if (d <= row)
                Bm[(int64_t)(q0 + row) * BW + d] = S.D[row][row - d];
              else if (d <= row + LNv)
                Bm[(int64_t)(q0 + row) * BW + d] = S.E[row][LNv + row - d];
            }
          }
        }
        if (l < NB) S.pv[l] = S.v[l];
        ptau = tau;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (l == 0)
          __hip_atomic_store(&prog[wid], s * SB_BIG + k + 1, __ATOMIC_RELEASE,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
        wave_sync();
        q0 += LM;
        LN = LM;
      };
      if (n - q0 >= NB && LN == NB)
        task(std::true_type{});
      else
        task(std::false_type{});
#pragma unroll
      for (int t = 0; t < 8; ++t) cur[t] = nxt[t];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  for (int i = threadIdx.x; i < n; i += SB_W * 64) {
    dout[(int64_t)blockIdx.x * n + i] = Bm[(int64_t)i * BW];
    if (i + 1 < n) eout[(int64_t)blockIdx.x * n + i] = Bm[(int64_t)(i + 1) * BW + 1];
  }
}

// ------------------------------------------------------------- bisection ---
// Sturm count of T - x: the number of eigenvalues below x (float64, with
// LAPACK's pivmin guard against a zero pivot).
// Number of eigenvalues of T below x (float64 Sturm count with dstebz's
// pivmin guard); e2[i] = e[i]^2.  The coefficients stream in groups of SG,
// the next group's loads issued before the current group's steps, so their
// latency hides under the division chain (the addresses are uniform: scalar
// loads).
constexpr int SG = 8;
__device__ __forceinline__ int sturm(const double* __restrict__ d, const double* __restrict__ e2,
                                     int n, double x, double pivmin) {
  int c = 0;
  double qv = d[0] - x;
  if (fabs(qv) < pivmin) qv = -pivmin;
  c += qv < 0.0;
  int i = 1;
  if (n - 1 >= SG) {
    double dn[SG], en[SG];
#pragma unroll
    for (int t = 0; t < SG; ++t) {
      dn[t] = d[1 + t];
      en[t] = e2[t];
    }
    for (; i + SG <= n; i += SG) {
      double dc[SG], ec[SG];
#pragma unroll
      for (int t = 0; t < SG; ++t) {
        dc[t] = dn[t];
        ec[t] = en[t];
      }
      if (i + 2 * SG <= n) {
#pragma unroll
        for (int t = 0; t < SG; ++t) {
          dn[t] = d[i + SG + t];
          en[t] = e2[i + SG - 1 + t];
        }
      }
#pragma unroll
      for (int t = 0; t < SG; ++t) {
        qv = (dc[t] - x) - ec[t] / qv;
        if (fabs(qv) < pivmin) qv = -pivmin;
        c += qv < 0.0;
      }
    }
  }
  for (; i < n; ++i) {
    qv = (d[i] - x) - e2[i - 1] / qv;
    if (fabs(qv) < pivmin) qv = -pivmin;
    c += qv < 0.0;
  }
  return c;
}

// Per matrix: Gershgorin bounds, pivmin, the trace (float64), the number of
// negative eigenvalues.  info = {lo, hi, pivmin, trace}, nneg.
__global__ __launch_bounds__(256) void k_tri_info(const double* d, const double* e, int n,
                                                  double* info, int* nneg, double* e2) {
  __shared__ double red[16];
  const int mat = blockIdx.x;
  const double* dm = d + (int64_t)mat * n;
  const double* em = e + (int64_t)mat * n;
  double* e2m = e2 + (int64_t)mat * n;
  double lo = 1e300, hi = -1e300, tr = 0.0, e2max = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) {
    const double r = (i > 0 ? fabs(em[i - 1]) : 0.0) + (i + 1 < n ? fabs(em[i]) : 0.0);
    lo = fmin(lo, dm[i] - r);
    hi = fmax(hi, dm[i] + r);
    tr += dm[i];
    if (i + 1 < n) {
      e2m[i] = em[i] * em[i];
      e2max = fmax(e2max, e2m[i]);
    }
  }
  double x[2] = {tr, 0.0};
  block_sum<2>(x, red);
  // min / max / max through the same LDS, one at a time
  __shared__ double mm[3][256];
  mm[0][threadIdx.x] = lo;
  mm[1][threadIdx.x] = hi;
  mm[2][threadIdx.x] = e2max;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int t = 1; t < 256; ++t) {
      lo = fmin(lo, mm[0][t]);
      hi = fmax(hi, mm[1][t]);
      e2max = fmax(e2max, mm[2][t]);
    }
    const double tnorm = fmax(fabs(lo), fabs(hi));
    const double pivmin = 2.2250738585072014e-308 * fmax(1.0, e2max);
    // widen the interval so bisection brackets every eigenvalue
    const double pad = 2.0 * 2.220446049250313e-16 * tnorm * n + 2.0 * pivmin;
    info[4 * mat + 0] = lo - pad;
    info[4 * mat + 1] = hi + pad;
    info[4 * mat + 2] = pivmin;
    info[4 * mat + 3] = x[0];
    nneg[mat] = sturm(dm, e2m, n, 0.0, pivmin);
  }
}

// Multisection.  BL lanes share one eigenvalue index and each runs BS Sturm
// counts at once, so an iteration evaluates BP = BL * BS points and shrinks
// the bracket (BP + 1) times (about 13 iterations to fp64 resolution against
// 53 halvings).  The counts' divisions are reciprocals (v_rcp_f64 and two
// Newton steps, no condition-register chain as in IEEE division), so a lane's
// BS counts interleave.  A quotient with a few ulps of error is a relative
// perturbation of the matrix of that size, as the rounding of the divisions
// already is (dstebz's analysis), so counts and brackets stay those of a
// matrix within a few ulps of T.
constexpr int BL = 4;
constexpr int BS = 4;
constexpr int BP = BL * BS;

__device__ __forceinline__ double recip(double q) {
  double r = __builtin_amdgcn_rcp(q);
  double t = fma(-q, r, 1.0);
  r = fma(r, t, r);
  t = fma(-q, r, 1.0);
  return fma(r, t, r);
}

// Sturm counts of T - x[t] for S points at once (as sturm above).
template <int S>
__device__ __forceinline__ void sturm_ms(const double* __restrict__ d,
                                         const double* __restrict__ e2, int n,
                                         const double (&x)[S], double pivmin, int (&c)[S]) {
  double q[S];
#pragma unroll
  for (int t = 0; t < S; ++t) {
    q[t] = d[0] - x[t];
    if (fabs(q[t]) < pivmin) q[t] = -pivmin;
    c[t] = q[t] < 0.0;
  }
  auto step = [&](double dv, double ev) {
#pragma unroll
    for (int t = 0; t < S; ++t) {
      q[t] = fma(-ev, recip(q[t]), dv - x[t]);
      if (fabs(q[t]) < pivmin) q[t] = -pivmin;
      c[t] += q[t] < 0.0;
    }
  };
  int i = 1;
  if (n - 1 >= SG) {
    double dn[SG], en[SG];
#pragma unroll
    for (int t = 0; t < SG; ++t) {
      dn[t] = d[1 + t];
      en[t] = e2[t];
    }
    for (; i + SG <= n; i += SG) {
      double dc[SG], ec[SG];
#pragma unroll
      for (int t = 0; t < SG; ++t) {
        dc[t] = dn[t];
        ec[t] = en[t];
      }
      if (i + 2 * SG <= n) {
#pragma unroll
        for (int t = 0; t < SG; ++t) {
          dn[t] = d[i + SG + t];
          en[t] = e2[i + SG - 1 + t];
        }
      }
#pragma unroll
      for (int t = 0; t < SG; ++t) step(dc[t], ec[t]);
    }
  }
  for (; i < n; ++i) step(d[i], e2[i - 1]);
}

// The eigenvalues wanted per matrix: the kq largest (indices n-1 .. n-kq),
// and the negative ones not among them (indices 0 .. nneg-1), which only
// enter the sum of the clamped spectrum.  Waves 0 .. WT-1 of a matrix serve
// the largest, 64 / BL per wave by multisection; the rest the negative ones,
// NB2 per lane by bisection (interleaved counts, one point each: with many
// eigenvalues to find, the halving that needs the fewest counts is
// cheapest), bracketed by [lo, 0] and stopped at an absolute width of
// 1e-12 |T| (at most 1e-12 |T| n off in the sum; the largest are resolved
// to a few ulps of themselves).  The matrix is blockIdx.x: workgroups go to
// the XCDs round-robin by linear index, and with the matrix index slowest
// every block with work would land on one XCD.
constexpr int NB2 = 2;
__global__ __launch_bounds__(256) void k_bisect(const double* d, const double* e2, int n, int kq,
                                                const double* info, const int* nneg,
                                                double* wall) {
  const int mat = blockIdx.x;
  const int wv = blockIdx.y * 4 + threadIdx.x / 64;
  const int l = threadIdx.x % 64;
  const int neg = nneg[mat];
  const int nn = neg < n - kq ? neg : n - kq;   // negative ones to find
  const int wt = (kq + 64 / BL - 1) / (64 / BL);
  const double* dm = d + (int64_t)mat * n;
  const double* em = e2 + (int64_t)mat * n;
  const double lo0 = info[4 * mat + 0], hi0 = info[4 * mat + 1];
  const double pivmin = info[4 * mat + 2];
  if (wv < wt) {
    const int sub = l % BL;
    const int slot = wv * (64 / BL) + l / BL;
    const bool act = slot < kq;
    const int j = n - 1 - (act ? slot : 0);
    double lo = lo0, hi = hi0;
    bool done = !act;
    for (int it = 0; it < 40; ++it) {
      if (hi - lo <= 2.0 * 2.220446049250313e-16 * fmax(fabs(lo), fabs(hi)) + pivmin) done = true;
      if (__all(done)) break;
      // points lo + h * (p + 1), p = 0 .. BP-1; this lane's are p = sub * BS + t
      const double h = (hi - lo) / (BP + 1);
      double x[BS];
#pragma unroll
      for (int t = 0; t < BS; ++t) x[t] = lo + h * (double)(sub * BS + t + 1);
      int c[BS];
      sturm_ms<BS>(dm, em, n, x, pivmin, c);
      // r = number of points whose count is <= j (a prefix: counts grow with x)
      int r = 0;
#pragma unroll
      for (int t = 0; t < BS; ++t) r += c[t] <= j;
      r += __shfl_xor(r, 1);
      r += __shfl_xor(r, 2);
      if (!done) {
        const double nlo = r > 0 ? lo + h * (double)r : lo;
        const double nhi = r < BP ? lo + h * (double)(r + 1) : hi;
        lo = nlo;
        hi = nhi;
      }
    }
    if (act && sub == 0) wall[(int64_t)mat * n + j] = 0.5 * (lo + hi);
    return;
  }
  const int base = (wv - wt) * 64 * NB2;
  if (base >= nn) return;                 // the whole wavefront
  const double tol = 1e-12 * fmax(fabs(lo0), fabs(hi0)) + pivmin;
  int j[NB2];
  bool done[NB2];
  double lo[NB2], hi[NB2];
#pragma unroll
  for (int t = 0; t < NB2; ++t) {
    j[t] = base + l + 64 * t;
    done[t] = j[t] >= nn;
    lo[t] = lo0;
    hi[t] = 0.0;
  }
  for (int it = 0; it < 64; ++it) {
    bool all = true;
#pragma unroll
    for (int t = 0; t < NB2; ++t) {
      if (hi[t] - lo[t] <= tol) done[t] = true;
      all = all && done[t];
    }
    if (__all(all)) break;
    double x[NB2];
#pragma unroll
    for (int t = 0; t < NB2; ++t) x[t] = 0.5 * (lo[t] + hi[t]);
    int c[NB2];
    sturm_ms<NB2>(dm, em, n, x, pivmin, c);
#pragma unroll
    for (int t = 0; t < NB2; ++t)
      if (!done[t]) {
        if (c[t] > j[t])
          hi[t] = x[t];
        else
          lo[t] = x[t];
      }
  }
#pragma unroll
  for (int t = 0; t < NB2; ++t)
    if (j[t] < nn) wall[(int64_t)mat * n + j[t]] = 0.5 * (lo[t] + hi[t]);
}

// The kq largest, descending, and total = trace - sum of the negative ones
// (summed in ascending order, fixed), i.e. the sum of the clamped spectrum.
__global__ __launch_bounds__(64) void k_bisect_finish(const double* wall, int n, int kq,
                                                      const double* info, const int* nneg,
                                                      double* w, double* total) {
  const int mat = blockIdx.x;
  const double* wm = wall + (int64_t)mat * n;
  for (int i = threadIdx.x; i < kq; i += 64) w[(int64_t)mat * kq + i] = wm[n - 1 - i];
  if (threadIdx.x == 0) {
    double s = 0.0;
    const int neg = nneg[mat];
    for (int j = 0; j < neg; ++j) s += wm[j];
    total[mat] = info[4 * mat + 3] - s;
  }
}

// ------------------------------------------------------ inverse iteration ---
constexpr int WC = 2 * NB + 1;   // 33 window columns
constexpr int WR = NB + 1;       // 17 window rows

// B[i][c] - (i == c) * sigma for the band matrix (orig: diagonals 0..NB of the
// lower band, row pitch OW), zero outside the band or the matrix.
__device__ __forceinline__ double mval(const float* orig, int n, int i, int c, double sigma) {
  if (i < 0 || c < 0 || i >= n || c >= n) return 0.0;
  const int dd = i - c;
  if (dd > NB || dd < -NB) return 0.0;
  double v = dd >= 0 ? (double)orig[(int64_t)i * OW + dd] : (double)orig[(int64_t)c * OW - dd];
  if (dd == 0) v -= sigma;
  return v;
}


__device__ __forceinline__ double readlane_d(double x, int lane) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Deterministic start vector: a hash of (vector, row) mapped to [-1, 1].
__device__ __forceinline__ double start_val(uint32_t vid, int row) {
  uint32_t h = vid * 0x9E3779B9u ^ (uint32_t)row * 0x85EBCA6Bu;
  h ^= h >> 16;
  h *= 0x7FEB352Du;
  h ^= h >> 15;
  h *= 0x846CA68Bu;
  h ^= h >> 16;
  return (double)(h & 0xFFFFFF) / 8388608.0 - 1.0;
}

// Prefetch distance (steps) of the band solve: the band values entering the
// window and the U rows of the back substitution are loaded this many steps
// before their use (a step takes a few thousand cycles, so 2 cover the memory
// latency).  At 4 the kernel needs more registers than five waves per SIMD
// leave and spills to scratch, whose allocation by the runtime can fail when
// device memory is nearly full; at 2 it spills nothing and runs as fast
// (38.7 ms against 40.5 ms for 4 at four waves, 480 x 2048^2, kq = 64).
constexpr int PF = 2;

__device__ __forceinline__ double enter_rhs(const double* rhs, uint32_t vid, int n, int i) {
  return i < n ? (rhs ? rhs[i] : start_val(vid, i)) : 0.0;
}

// The band solve keeps its global stores out of the prefetch window: a wait
// for loads with stores in flight is a wait for every outstanding operation,
// which would expose each prefetched value's latency at every step.  The U
// rows (and the transformed right-hand side) of UF steps are staged in LDS and
// written out together, the back substitution's solution values likewise;
// and every prefetch is issued unconditionally (an out-of-range one reads a
// valid address; validity and the shift are applied where the value is
// used), since a load issued on one branch only also makes the compiler wait
// for all loads.
constexpr int UF = 8;                 // steps staged between flushes (a multiple of PF)
constexpr int UST = UF * (WC + 1);    // staged doubles per wavefront
static_assert(UF % PF == 0, "flushes at prefetch group boundaries");
typedef __attribute__((address_space(3))) double lds_double;

// A band value about to enter the window: the raw float and its position
// (entering row i, column c), or the right-hand side's (lane WC).
struct Enter {
  float raw;      // orig value (matrix lanes)
  double rv;      // right-hand side value (lane WC)
  bool ok, dg;    // inside the band and the matrix; on the diagonal
};

// Lane L's window column offset at step j: (L - j) mod WC, carried from step
// to step (one less each step, WC - 1 after 0) instead of a division per use.
__device__ __forceinline__ int lane_rot(int L, int j) { return ((L - j) % WC + WC) % WC; }
__device__ __forceinline__ int rot_next(int r) { return r == 0 ? WC - 1 : r - 1; }

// The band value entering step j's window in lane L's column: column
// j + 1 + rot, rot = lane_rot(L, j + 1) (the lane's offset once step j is done).
template <bool HAS_RHS>
__device__ __forceinline__ Enter enter_load(const float* orig, const double* rhs, uint32_t vid,
                                            int n, int j, int L, int rot) {
  // every lane issues the same loads (clamped addresses), no branches
  Enter e;
  const int i = j + WR;
  const int c = j + 1 + rot;
  const int dd = i - c;
  const bool inb = i < n;
  const bool band = L < WC && inb && c < n && dd <= NB && dd >= -NB;
  e.dg = dd == 0;
  e.ok = L < WC ? band : (L == WC && inb);
  e.raw = orig[band ? (dd >= 0 ? i * OW + dd : c * OW - dd) : 0];
  if constexpr (HAS_RHS)
    e.rv = rhs[inb ? i : 0];
  else
    e.rv = start_val(vid, i);
  return e;
}

__device__ __forceinline__ double enter_value(const Enter& e, int L, double sigma) {
  if (!e.ok) return 0.0;
  if (L == WC) return e.rv;
  double v = (double)e.raw;
  if (e.dg) v -= sigma;
  return v;
}

// The window's 17 row slots: slots 0..15 as one 16-double vector (a single
// 1024-bit register tuple), slot 16 beside it.  Slot p (wave-uniform, known
// only at run time) is then read and written in place through the register
// index mode (s_set_gpr_idx_on): two moves per access, no branches.  A plain
// 17-element array indexed at run time would move to scratch memory, and a
// conditional write into the vector makes the compiler copy the whole tuple,
// so every access below is unconditional.
static_assert(WR == 17, "the window is 16 vector slots and one more");
typedef double v16d __attribute__((ext_vector_type(16)));

// Solve (B - sigma I) x = rhs with band LU and partial pivoting; rhs given by
// `rhs` (NULL: start_val).  U rows (WC doubles each) and the transformed rhs
// go to work; x (float64, normalised) to xout.  One wavefront; lanes 0..32
// each own one window column (lane L holds column j + ((L - j) mod 33) at
// step j), lane 33 the right-hand side (an augmented column, so elimination
// updates it with the same instructions); every lane holds the 17 row slots.
// The window's rows are an unordered set: the pivot row is retired as U row
// j and the entering band row takes its slot, so no rows move.  Returns the
// norm of the solution before normalisation.
template <bool HAS_RHS>
__device__ __forceinline__ double band_solve(const float* __restrict__ orig, int n, double sigma,
                                             double bnorm, uint32_t vid,
                                             const double* __restrict__ rhs, double* U,
                                             double* ys, double* xout, lds_double* st) {
  const int L = threadIdx.x & 63;
  const bool act = L < WC;          // a matrix column
  const bool rl = L == WC;          // the right-hand side
  v16d W;          // slots 0..15
  double Wx;       // slot 16
  // initial window: rows 0..16, columns 0..32 (lane L <-> column L)
  auto init = [&](int s) {
    return act ? mval(orig, n, s, L, sigma) : (rl ? enter_rhs(rhs, vid, n, s) : 0.0);
  };
#pragma unroll
  for (int s = 0; s < 16; ++s) W[s] = init(s);
  Wx = init(16);
  Enter qW[PF];
#pragma unroll
  for (int t = 0; t < PF; ++t) qW[t] = enter_load<HAS_RHS>(orig, rhs, vid, n, t, L, lane_rot(L, t + 1));
  int rot_st = lane_rot(L, 0);        // this step's offset (U row staging)
  int rot_ld = lane_rot(L, PF + 1);   // the offset of the load PF steps ahead
  const double tiny = 2.220446049250313e-16 * bnorm + 1e-300;
  int jf = 0;                        // first U row not yet written out
  for (int j0 = 0; j0 < n; j0 += PF) {
#pragma unroll
    for (int t = 0; t < PF; ++t) {
      const int j = j0 + t;
      if (j >= n) break;
      const int lj = j % WC;
      double col[WR];
      // pivot search on the scalar unit: the high word without its sign
      // orders |col[s]| to 20 mantissa bits (a tie keeps the lowest slot; any
      // pivot within 2^-20 of the largest is as stable)
      int p = 0;
      uint32_t best = 0;
#pragma unroll
      for (int s = 0; s < WR; ++s) {
        col[s] = readlane_d(s < 16 ? W[s & 15] : Wx, lj);
        const uint32_t m =
            (uint32_t)(__builtin_bit_cast(uint64_t, col[s]) >> 32) & 0x7fffffffu;
        if (s == 0 || m > best) {
          best = m;
          p = s;
        }
      }
      const int pi = p & 15;
      const bool top = p < 16;
      const double prow = top ? W[pi] : Wx;   // this lane's entry of the pivot row
      double piv = readlane_d(prow, lj);      // == col[p]
      if (fabs(piv) < tiny) piv = piv < 0.0 ? -tiny : tiny;
      // every slot loses col[s] / piv times the pivot row, as col[s] * (row / piv)
      // (the pivot's own slot is overwritten below)
      const double q = prow / piv;
#pragma unroll
      for (int s = 0; s < 16; ++s) W[s] = fma(-col[s], q, W[s]);
      Wx = fma(-col[16], q, Wx);
      // retire the pivot row as U row j (column offset of this lane) and its
      // right-hand side, staged
      const int off = rot_st;
      if (act) st[(j % UF) * (WC + 1) + off] = L == lj ? piv : prow;
      if (rl) st[(j % UF) * (WC + 1) + WC] = prow;
      // row j + 17 (prefetched PF steps ago) takes the pivot's slot; fetch
      // step j + PF's
      const double ent = enter_value(qW[t], L, sigma);
      W[pi] = top ? ent : W[pi];
      Wx = top ? Wx : ent;
      qW[t] = enter_load<HAS_RHS>(orig, rhs, vid, n, j + PF, L, rot_ld);
      rot_st = rot_next(rot_st);
      rot_ld = rot_next(rot_ld);
    }
    const int je = j0 + PF < n ? j0 + PF : n;
    if (je - jf >= UF || je == n) {
      // U rows jf .. je-1 (contiguous in U) and their right-hand sides
      wave_sync();
      for (int e = L; e < (je - jf) * WC; e += 64) {
        const int r = e / WC, off = e % WC;
        U[(int64_t)(jf + r) * WC + off] = st[r * (WC + 1) + off];
      }
      if (L < je - jf) ys[jf + L] = st[L * (WC + 1) + WC];
      jf = je;
    }
  }
  __threadfence_block();
  // back substitution: x[j] = (ys[j] - sum_{c>=1} U[j][c] x[j+c]) / U[j][0];
  // lane L keeps x[row] for the row = L (mod 33) inside the window.  Row j's
  // U entries, diagonal and rhs are loaded PF steps ahead (they do not depend
  // on x); the solution values are staged UF at a time.
  double qU[PF], qD[PF], qS[PF];
  bool qok[PF];
#pragma unroll
  for (int t = 0; t < PF; ++t) {
    const int j = n - 1 - t;
    const int off = j >= 0 ? (L - j % WC + WC) % WC : 0;
    qok[t] = j >= 0 && act && off != 0 && j + off < n;
    qU[t] = U[qok[t] ? (int64_t)j * WC + off : 0];
    qD[t] = U[j >= 0 ? (int64_t)j * WC : 0];
    qS[t] = ys[j >= 0 ? j : 0];
  }
  double xv = 0.0, nrm = 0.0;
  int jx = n;                        // xout rows jx .. n-1 are written out
  for (int j0 = n - 1; j0 >= 0; j0 -= PF) {
#pragma unroll
    for (int t = 0; t < PF; ++t) {
      const int j = j0 - t;
      if (j < 0) break;
      const double sm = wave_sum_d((qok[t] ? qU[t] : 0.0) * xv);
      const double xj = (qS[t] - sm) / qD[t];
      if (L == j % WC) {
        xv = xj;
        nrm = fma(xj, xj, nrm);
        st[(n - 1 - j) % UF] = xj;
      }
      const int jn = j - PF;
      const int off = jn >= 0 ? (L - jn % WC + WC) % WC : 0;
      qok[t] = jn >= 0 && act && off != 0 && jn + off < n;
      qU[t] = U[qok[t] ? (int64_t)jn * WC + off : 0];
      qD[t] = U[jn >= 0 ? (int64_t)jn * WC : 0];   // rows below 0 are never used
      qS[t] = ys[jn >= 0 ? jn : 0];
    }
    const int jl = j0 - PF + 1 > 0 ? j0 - PF + 1 : 0;   // lowest row of the group
    if (jx - jl >= UF || jl == 0) {
      // rows jl .. jx-1: row j sits in slot (n - 1 - j) mod UF
      wave_sync();
      if (L < jx - jl) xout[jx - 1 - L] = st[(n - jx + L) % UF];
      jx = jl;
    }
  }
  nrm = wave_sum_d(nrm);
  __threadfence_block();
  const double sc = 1.0 / sqrt(nrm);
  for (int j = L; j < n; j += 64) xout[j] *= sc;
  __threadfence_block();
  return sqrt(nrm);
}

// Rayleigh quotient x^T B x of a normalised float64 vector (one wavefront).
__device__ double rayleigh(const float* orig, int n, const double* x) {
  const int L = threadIdx.x & 63;
  double acc = 0.0;
  for (int i = L; i < n; i += 64) {
    double bx = 0.0;
    const int c0 = i - NB < 0 ? 0 : i - NB, c1 = i + NB >= n ? n - 1 : i + NB;
    for (int c = c0; c <= c1; ++c) bx = fma(mval(orig, n, i, c, 0.0), x[c], bx);
    acc = fma(x[i], bx, acc);
  }
  return wave_sum_d(acc);
}

// Clusters: consecutive eigenvalues (descending) closer than kClusterTol times
// the largest |B| entry.  Inverse iteration cannot separate them (their
// vectors would converge to one combination), so each member gets its own
// shift, offset by (rank + 1/2) * kShiftStep * |B| -- no exactly singular
// pivot, and the random start vectors stay independent -- and the members are
// made orthonormal afterwards (LAPACK's stein perturbs and orthogonalises
// clustered eigenvalues the same way).
constexpr double kClusterTol = 1e-10;
constexpr double kShiftStep = 1e-13;

// One wavefront per eigenvector; vectors [v0, v0 + gridDim.x * 4) of the
// flattened (matrix, index) list; 4 wavefronts per block.  One solve from a
// pseudo-random start (the shift is a float64 eigenvalue of the float64
// tridiagonal, so one solve converges for any gap far above 1e-15 |B|; a
// second one follows when the solution did not grow as that implies), then
// the Rayleigh quotient into wr.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5, 5))) void k_inviter(const float* orig, int64_t ostride, int n, int kq,
                                                 int nvec, int v0, const double* w,
                                                 const double* bnorm, double* work, double* xall,
                                                 double* wr) {
  __shared__ double stage[4][UST];   // each wavefront's staged U rows / solution
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar registers
  const int vid = v0 + blockIdx.x * 4 + wv;
  if (vid >= nvec) return;
  const int mat = vid / kq, idx = vid % kq;
  const float* om = orig + (int64_t)mat * ostride;
  const int64_t slot = (int64_t)(vid - v0);
  double* U = work + slot * ((int64_t)n * (WC + 1));
  double* ys = U + (int64_t)n * WC;
  double* x = xall + (int64_t)vid * n;
  const double bn = bnorm[mat];
  const double* wm = w + (int64_t)mat * kq;
  const double tol = kClusterTol * bn;
  int rank = 0;
  for (int t = idx; t > 0 && fabs(wm[t - 1] - wm[t]) <= tol; --t) ++rank;
  const bool clustered = rank > 0 || (idx + 1 < kq && fabs(wm[idx] - wm[idx + 1]) <= tol);
  const double sigma = wm[idx] + (clustered ? (rank + 0.5) * kShiftStep * bn : 0.0);
  // the start vector has entries uniform in [-1, 1]: norm about sqrt(n / 3);
  // a solution that grew by less than 1e10 / |B| relative to it had a shift
  // too far from the eigenvalue to have converged: solve once more from it
  lds_double* st = (lds_double*)&stage[wv][0];
  const double growth = band_solve<false>(om, n, sigma, bn, (uint32_t)vid, nullptr, U, ys, x, st);
  if (growth * bn < 1e10 * sqrt(n / 3.0))
    band_solve<true>(om, n, sigma, bn, (uint32_t)vid, x, U, ys, x, st);
  const double rq = rayleigh(om, n, x);
  if ((threadIdx.x & 63) == 0) wr[vid] = rq;
}

// Sum over a 256-thread block, the result returned to every thread.
__device__ __forceinline__ double block_sum_all(double x, double* red /* >= 5 */) {
  double a[1] = {x};
  block_sum<1>(a, red);
  if (threadIdx.x == 0) red[4] = a[0];
  __syncthreads();
  const double r = red[4];
  __syncthreads();
  return r;
}

// Gram-Schmidt (twice) of vectors [cs, ce) of xm against the earlier ones of
// the cluster, in place.
__device__ __forceinline__ void cluster_mgs(double* xm, int n, int cs, int ce, double* red) {
  for (int i = cs + 1; i < ce; ++i) {
    double* xi = xm + (int64_t)i * n;
    for (int pass = 0; pass < 2; ++pass) {
      for (int jv = cs; jv < i; ++jv) {
        const double* xj = xm + (int64_t)jv * n;
        double x = 0.0;
        for (int r = threadIdx.x; r < n; r += 256) x = fma(xj[r], xi[r], x);
        x = block_sum_all(x, red);
        for (int r = threadIdx.x; r < n; r += 256) xi[r] = fma(-x, xj[r], xi[r]);
        __syncthreads();
      }
      double x = 0.0;
      for (int r = threadIdx.x; r < n; r += 256) x = fma(xi[r], xi[r], x);
      x = block_sum_all(x, red);
      const double sc = 1.0 / sqrt(x);
      for (int r = threadIdx.x; r < n; r += 256) xi[r] *= sc;
      __syncthreads();
    }
  }
}

// One Cholesky-QR pass over the c <= CQ vectors [cs, cs+c) of xm: G = X^T X
// (float64, through LDS in chunks of CR rows), G = R^T R, X <- X R^-1 (row by
// row).  In exact arithmetic R is Gram-Schmidt's, so X becomes the same
// orthonormal basis; two passes are as accurate as Gram-Schmidt twice while
// X is far from rank-deficient.  Returns false, with X unchanged, when a pivot
// falls below 1e-10 of its column's squared norm (X too close to
// rank-deficient for the normal equations): the caller then uses cluster_mgs.
constexpr int CQ = 64;   // largest cluster taken through Cholesky QR
constexpr int CR = 32;   // rows per LDS chunk of the Gram pass
struct CholQrLds {
  double G[CQ][CQ + 1];
  double chunk[CR][CQ + 1];
  int fail;
};

__device__ __forceinline__ bool cholqr_pass(double* xm, int n, int cs, int c, CholQrLds& S) {
  const int tid = threadIdx.x;
  // 1. G = X^T X: thread t accumulates cells t, t + 256, ... (a <= b only)
  constexpr int NQ = CQ * CQ / 256;
  double acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = 0.0;
  for (int r0 = 0; r0 < n; r0 += CR) {
    for (int idx = tid; idx < CR * c; idx += 256) {
      const int v = idx / CR, r = idx % CR;
      S.chunk[r][v] = r0 + r < n ? xm[(int64_t)(cs + v) * n + r0 + r] : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int cell = tid + 256 * q, a = cell / c, b = cell % c;
      if (a <= b && a < c) {
        double x = acc[q];
        for (int r = 0; r < CR; ++r) x = fma(S.chunk[r][a], S.chunk[r][b], x);
        acc[q] = x;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int cell = tid + 256 * q, a = cell / c, b = cell % c;
    if (a <= b && a < c) S.G[a][b] = acc[q];
  }
  if (tid == 0) S.fail = 0;
  __syncthreads();
  // 2. G = R^T R (R into G's upper triangle), on wavefront 0: lane j owns
  // column j
  if (tid < 64) {
    const int j = tid;
    const double d0 = j < c ? S.G[j][j] : 1.0;
    for (int k = 0; k < c; ++k) {
      if (j == k) {
        const double d = S.G[k][k];
        if (!(d > 1e-10 * d0)) S.fail = 1;
        S.G[k][k] = sqrt(fmax(d, 0.0));
      }
      wave_sync();
      if (S.fail) break;
      if (j > k && j < c) S.G[k][j] /= S.G[k][k];
      wave_sync();
      if (j > k && j < c)
        for (int i = k + 1; i <= j; ++i) S.G[i][j] = fma(-S.G[k][i], S.G[k][j], S.G[i][j]);
      wave_sync();
    }
  }
  __syncthreads();
  if (S.fail) return false;
  // 3. X <- X R^-1: row r of X, forward substitution against R's columns.
  // The solved entries are read back from xm (this thread wrote them), not
  // held in a private array: a c-long array of doubles would spill to
  // scratch, and the runtime's scratch allocation for it can fail when
  // device memory is nearly full.
  for (int r = tid; r < n; r += 256) {
    double* xr = xm + (int64_t)cs * n + r;
    for (int j = 0; j < c; ++j) {
      double sacc = xr[(int64_t)j * n];
      for (int i = 0; i < j; ++i) sacc = fma(-xr[(int64_t)i * n], S.G[i][j], sacc);
      xr[(int64_t)j * n] = sacc / S.G[j][j];
    }
  }
  __syncthreads();
  return true;
}

// X_b <- X_b - X_p (X_p^T X_b) for the cb vectors [b0, b0 + cb) against the
// cp orthonormal vectors [p0, p0 + cp) (both <= CQ): the cross products
// through LDS, 16 rows of each side per chunk (chunk rows 0-15 hold X_p's,
// 16-31 X_b's), into S.G; then each thread updates its rows, 16 columns of
// X_b at a time (X_p's entries read back from xm).
__device__ __forceinline__ void cluster_project(double* xm, int n, int p0, int cp, int b0, int cb,
                                                CholQrLds& S) {
  static_assert(CR == 32, "two 16-row halves");
  const int tid = threadIdx.x;
  constexpr int NQ = CQ * CQ / 256;
  double acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = 0.0;
  for (int r0 = 0; r0 < n; r0 += 16) {
    for (int idx = tid; idx < 16 * CQ; idx += 256) {
      const int v = idx / 16, r = idx % 16;
      S.chunk[r][v] = r0 + r < n && v < cp ? xm[(int64_t)(p0 + v) * n + r0 + r] : 0.0;
      S.chunk[16 + r][v] = r0 + r < n && v < cb ? xm[(int64_t)(b0 + v) * n + r0 + r] : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int cell = tid + 256 * q, a = cell / CQ, b = cell % CQ;
      double x = acc[q];
      for (int r = 0; r < 16; ++r) x = fma(S.chunk[r][a], S.chunk[16 + r][b], x);
      acc[q] = x;
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int cell = tid + 256 * q;
    S.G[cell / CQ][cell % CQ] = acc[q];
  }
  __syncthreads();
  for (int r = tid; r < n; r += 256) {
    const double* xp = xm + (int64_t)p0 * n + r;
    double* xb = xm + (int64_t)b0 * n + r;
    for (int j0 = 0; j0 < cb; j0 += 16) {
      double u[16];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) u[jj] = 0.0;
      for (int i = 0; i < cp; ++i) {
        const double xi = xp[(int64_t)i * n];
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) u[jj] = fma(xi, S.G[i][j0 + jj], u[jj]);
      }
#pragma unroll
      for (int jj = 0; jj < 16; ++jj)
        if (j0 + jj < cb) xb[(int64_t)(j0 + jj) * n] -= u[jj];
    }
  }
  __syncthreads();
}

// A cluster of c > CQ vectors, CQ at a time (block Gram-Schmidt with
// Cholesky QR, twice): each slice is projected against the slices before it
// and made orthonormal, then both steps are repeated.  Returns false, the
// vectors partly updated, when a Cholesky QR fails (the caller then runs
// Gram-Schmidt over the whole cluster).
__device__ __forceinline__ bool cluster_block(double* xm, int n, int cs, int ce, CholQrLds& S) {
  for (int b0 = cs; b0 < ce; b0 += CQ) {
    const int cb = ce - b0 < CQ ? ce - b0 : CQ;
    for (int pass = 0; pass < 2; ++pass) {
      for (int p0 = cs; p0 < b0; p0 += CQ) cluster_project(xm, n, p0, CQ, b0, cb, S);
      if (cb > 1 && !cholqr_pass(xm, n, b0, cb, S)) return false;
      if (cb == 1) {   // one vector: its norm
        __shared__ double red1[16];
        double x = 0.0;
        for (int r = threadIdx.x; r < n; r += 256) x = fma(xm[(int64_t)b0 * n + r], xm[(int64_t)b0 * n + r], x);
        x = block_sum_all(x, red1);
        const double sc = 1.0 / sqrt(x);
        for (int r = threadIdx.x; r < n; r += 256) xm[(int64_t)b0 * n + r] *= sc;
        __syncthreads();
      }
    }
  }
  return true;
}

// Per matrix: the vectors of each cluster -- consecutive eigenvalues whose gaps
// are all below tol * bnorm -- made orthonormal in place in xall (Cholesky QR
// twice up to CQ vectors, block Gram-Schmidt with Cholesky QR above; plain
// Gram-Schmidt as the fallback); matrices without clusters only copy the
// Rayleigh quotients.
__global__ __launch_bounds__(256) void k_cluster_orth(int n, int kq, double* w, const double* wr,
                                                      const double* bnorm, double* xall) {
  __shared__ double red[16];
  __shared__ CholQrLds S;
  const int mat = blockIdx.x;
  double* wm = w + (int64_t)mat * kq;
  double* xm = xall + (int64_t)mat * kq * n;
  const double tol = kClusterTol * bnorm[mat];
  for (int cs = 0; cs < kq;) {
    int ce = cs + 1;
    while (ce < kq && fabs(wm[ce - 1] - wm[ce]) <= tol) ++ce;
    const int c = ce - cs;
    if (c >= 2) {
      bool ok;
      if (c <= CQ) {
        ok = cholqr_pass(xm, n, cs, c, S);
        if (ok) ok = cholqr_pass(xm, n, cs, c, S);
      } else {
        ok = cluster_block(xm, n, cs, ce, S);
      }
      if (!ok) cluster_mgs(xm, n, cs, ce, red);
    }
    cs = ce;
  }
  __syncthreads();
  // the Rayleigh quotients replace the bisection values once the clusters
  // (found from the latter) are done
  for (int i = threadIdx.x; i < kq; i += 256) wm[i] = wr[(int64_t)mat * kq + i];
}

// xall (per matrix kq vectors of n float64, vector-major) -> Z (n x kq
// float32, row-major), through a 64 x 64 LDS tile: reads coalesced along
// rows, writes coalesced along vectors.
__global__ __launch_bounds__(256) void k_vec_out(int n, int kq, const double* xall, float* Z,
                                                 int64_t zstride) {
  __shared__ float tile[64][65];
  const int r0 = blockIdx.x * 64, v0 = blockIdx.y * 64, mat = blockIdx.z;
  const double* xm = xall + (int64_t)mat * kq * n;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int v = ty; v < 64; v += 4)
    if (v0 + v < kq && r0 + tx < n) tile[v][tx] = (float)xm[(int64_t)(v0 + v) * n + r0 + tx];
  __syncthreads();
  float* zm = Z + (int64_t)mat * zstride;
  for (int r = ty; r < 64; r += 4)
    if (r0 + r < n && v0 + tx < kq) zm[(int64_t)(r0 + r) * kq + v0 + tx] = tile[tx][r];
}

// max |B| over the band (float64) per matrix: the scale of the pivot guard
// and of the cluster tolerance.
__global__ __launch_bounds__(256) void k_band_norm(const float* orig, int64_t ostride, int n,
                                                   double* bnorm) {
  __shared__ float mx[256];
  const float* om = orig + (int64_t)blockIdx.x * ostride;
  float m = 0.f;
  for (int64_t t = threadIdx.x; t < (int64_t)n * OW; t += 256) m = fmaxf(m, fabsf(om[t]));
  mx[threadIdx.x] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int t = 1; t < 256; ++t) m = fmaxf(m, mx[t]);
    bnorm[blockIdx.x] = (double)m;
  }
}

// vectors per inverse-iteration launch: two rounds of five wavefronts on every
// SIMD (the band solve is latency-bound: 2 -> 5 waves per SIMD took it from
// 80 to 46 ms at 480 x 2048^2, kq = 64), their U workspace (n x 34 float64
// each) capped
constexpr int kInvChunkMax = 10240;
constexpr int64_t kInvWorkBytes = (int64_t)8 << 30;

__host__ __forceinline__ int inv_chunk(int n, int64_t nvec) {
  int64_t c = kInvWorkBytes / ((int64_t)n * (WC + 1) * (int64_t)sizeof(double));
  c = c < kInvChunkMax ? c : kInvChunkMax;
  c = c < 256 ? 256 : c;
  return (int)(nvec < c ? nvec : c);
}

// ------------------------------------------------------ back-transform ---
// Z <- Q_0 (Q_1 (... Q_last Z)), Q_p = I - V_p T_p V_p^T: the stage-1 panels'
// reflectors (V_p explicit in A[r0:n, c0:c0+16], r0 = c0 + 16, c0 = 16p; T_p
// from the panel QR) applied to the eigenvectors, panel by panel from the
// last, as the batched form Z[r0:] -= V_p (T_p (V_p^T Z[r0:])).  One
// workgroup of 16 wavefronts per (matrix, 16 columns of Z): the slice stays
// in registers for the whole pass, wavefront w holding row tiles w, w+16, ...
// (16 rows each) in the MFMA output layout.  Per panel: each wavefront's
// share G_w of G = V_p^T Z on MFMA (each tile's rows are the reduction index:
// lane row 4(l/16)+r is k-step r) and its share T_p G_w of W = T_p G; the 16
// shares summed in LDS in a fixed order by every lane for the four values it
// needs; then Z -= V_p W on MFMA (reduction over the panel's 16 columns,
// column 4(l/16)+s at k-step s, so a lane's four V values are one float4).
// A panel's first row r0 is a multiple of 16, so tiles never straddle it.
template <int ZT, bool EXACT>
__global__ __launch_bounds__(1024) void k_back_transform(const float* __restrict__ A, int64_t sA,
                                                         int n, int npan, const float* __restrict__ T,
                                                         int64_t sT, float* Z, int64_t sZ, int kq,
                                                         int nmat) {
  __shared__ float Wp[2][16][256];
  // blocks in groups of 8 matrices x the slices: a matrix's slices run close
  // together in dispatch order and on one XCD (workgroups are dealt to the
  // XCDs round-robin by linear index), so they share its V through that L2
  const int nsl = (kq + 15) / 16, grp = blockIdx.x / (8 * nsl), rem = blockIdx.x % (8 * nsl);
  const int mat = 8 * grp + rem % 8, z0 = 16 * (rem / 8);
  if (mat >= nmat) return;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, jj = l & 15;
  const float* Am = A + (int64_t)mat * sA;
  float* Zm = Z + (int64_t)mat * sZ;
  const int nrt = (n + 15) / 16;
  const bool colok = EXACT || z0 + jj < kq;   // EXACT: n % 16 == 0 and kq % 16 == 0
  // V through a buffer resource over the matrix: 32-bit offsets (one register
  // per address instead of two), and rows past n read as zero (out of range)
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)Am, (short)0, n * n * 4, 0x00020000);
  const int n4 = 4 * n, t4 = 1024 * n;         // bytes per row, per 256 rows (16 tiles)
  const int b1 = (16 * w + 4 * g) * n4 + 4 * jj;   // step 1: rows 16w+4g+r, column c0+jj
  const int b2 = (16 * w + jj) * n4 + 16 * g;      // step 2: row 16w+jj, columns c0+4g..
  v4f zr[ZT];
#pragma unroll
  for (int t = 0; t < ZT; ++t) {
    const int tile = w + 16 * t;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * tile + 4 * g + r;
      zr[t][r] = (tile < nrt && (EXACT || row < n) && colok) ? Zm[(int64_t)row * kq + z0 + jj] : 0.f;
    }
  }
  for (int p = npan - 1; p >= 0; --p) {
    const int c0 = 16 * p, ft = p + 1;
    // the lane's offsets, opaque to the compiler: each tile's addresses are
    // formed where they are used instead of being hoisted for the whole pass
    int o1 = b1, o2 = b2;
    asm volatile("" : "+v"(o1), "+v"(o2));
    // T_p as the A operand of W_w = T G_w: lane (g, jj) supplies T[jj][4g + r]
    // at k-step r (the permutation of G's rows in its partials below)
    float ta[4];
    {
      const float* Tp = T + (int64_t)p * sT + (int64_t)mat * 256 + jj * 16 + 4 * g;
#pragma unroll
      for (int r = 0; r < 4; ++r) ta[r] = Tp[r];
    }
    // G partials: A[a][k] = V[row_k][c0 + a], B[k][b] = Z[row_k][b]
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < ZT; ++t) {
      const int tile = w + 16 * t;
      if (tile >= ft && tile < nrt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(rs, o1 + t * t4 + r * n4, 4 * c0, 0));
          acc = mfma16(v, zr[t][r], acc);
        }
      }
      if (t & 1) asm volatile("" ::: "memory");   // two tiles' loads in flight at most
    }
    // W = T G = sum over wavefronts of T G_w: this wavefront's share on MFMA
    // (G_w holds G[4g + r][jj], the B operand of k-step r), partials to LDS
    // (double-buffered by panel parity: one barrier per panel)
    v4f wp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) wp = mfma16(ta[r], acc[r], wp);
    float (*Wb)[256] = Wp[p & 1];
#pragma unroll
    for (int r = 0; r < 4; ++r) Wb[w][(4 * g + r) * 16 + jj] = wp[r];
    __syncthreads();
    // Z -= V W: A[i][k] = V[tile row i][c0 + 4(l/16) + s], B[k][j] = W[4(l/16) + s][j]
    float wb[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int e = (4 * g + s4) * 16 + jj;
      float x = Wb[0][e];
#pragma unroll
      for (int v = 1; v < 16; ++v) x += Wb[v][e];   // fixed order
      wb[s4] = x;
    }
#pragma unroll
    for (int t = 0; t < ZT; ++t) {
      const int tile = w + 16 * t;
      if (tile >= ft && tile < nrt) {
        v4f va;
        if (EXACT) {
          va = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, o2 + t * t4,
                                                                              4 * c0, 0));
        } else {
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4)
            va[s4] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                   rs, o2 + t * t4 + 4 * s4, 4 * c0, 0));
        }
        v4f dv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) dv = mfma16(va[s4], wb[s4], dv);
#pragma unroll
        for (int r = 0; r < 4; ++r) zr[t][r] -= dv[r];
      }
      if (t & 1) asm volatile("" ::: "memory");
    }
  }
  float* Zs = Zm;                  // opaque: the store addresses are not kept live
  asm volatile("" : "+s"(Zs));     // across the pass
#pragma unroll
  for (int t = 0; t < ZT; ++t) {
    const int tile = w + 16 * t;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * tile + 4 * g + r;
      if (tile < nrt && (EXACT || row < n) && colok) Zs[(int64_t)row * kq + z0 + jj] = zr[t][r];
    }
  }
}

}  // namespace

// ------------------------------------------------------------- C ABI ---
extern "C" int scao_eig_panel_qr(float* A, int64_t stride, int n, int c0, int batch, float* T,
                                 float* band, int64_t bstride, void* stream) {
  SCAO_CHECK_ARG(A && T && band, "scao_eig_panel_qr: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && n > 0 && n <= 4096 + NB && c0 >= 0 && c0 % NB == 0 &&
                     c0 + NB < n && stride >= (int64_t)n * n && bstride >= (int64_t)n * BW,
                 "scao_eig_panel_qr: bad arguments n=%d c0=%d", n, c0);
  if (batch == 0) return SCAO_OK;
  const int m = n - c0 - NB;
  hipStream_t s = (hipStream_t)stream;
  float* Am = A;
  if (m <= 512)
    hipLaunchKernelGGL((k_panel_qr<2, 256>), dim3(batch), dim3(256), 0, s, Am, stride, n, c0, T, band, bstride);
  else if (m <= 1024)
    hipLaunchKernelGGL((k_panel_qr<4, 256>), dim3(batch), dim3(256), 0, s, Am, stride, n, c0, T, band, bstride);
  else if (m <= 2048)
    hipLaunchKernelGGL((k_panel_qr<4, 512>), dim3(batch), dim3(512), 0, s, Am, stride, n, c0, T, band, bstride);
  else
    hipLaunchKernelGGL((k_panel_qr<8, 512>), dim3(batch), dim3(512), 0, s, Am, stride, n, c0, T, band, bstride);
  SCAO_LAUNCH_CHECK("scao_eig_panel_qr");
  return SCAO_OK;
}

extern "C" int scao_eig_sy2sb_panel_w(float* A, int64_t sA, int n, int c0, int batch,
                                      const float* Y, const float* T, float* W, int strip,
                                      void* stream) {
  SCAO_CHECK_ARG(A && Y && T && W, "scao_eig_sy2sb_panel_w: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && n > 0 && n <= 4096 + NB && c0 >= 0 && c0 % NB == 0 && c0 + NB < n &&
                     sA >= (int64_t)n * n && (!strip || c0 + 2 * NB <= n),
                 "scao_eig_sy2sb_panel_w: bad arguments n=%d c0=%d", n, c0);
  if (batch == 0) return SCAO_OK;
  hipLaunchKernelGGL(k_sy2sb_panel_w, dim3(batch), dim3(1024), 0, (hipStream_t)stream, A, sA, n,
                     c0 + NB, c0, Y, T, W, strip);
  SCAO_LAUNCH_CHECK("scao_eig_sy2sb_panel_w");
  return SCAO_OK;
}

extern "C" int64_t scao_eig_sy2sb_work(int mr, int batch) {
  if (mr <= 0 || batch <= 0) return 0;
  const int64_t nt = (mr + UT - 1) / UT, nch = (nt - 1) / UCH + 1;
  return (int64_t)batch * nt * (nt + nch) * UT * 16 * (int64_t)sizeof(float);
}

extern "C" int scao_eig_sy2sb_update(float* A, int64_t sA, int ldA, int mr, int batch,
                                     const float* V, int64_t sV, int ldV, const float* W,
                                     int64_t sW, int ldW, const float* Vn, int64_t sVn, int ldVn,
                                     float* Y, int64_t sY, void* work, void* stream) {
  SCAO_CHECK_ARG(A && V && W, "scao_eig_sy2sb_update: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && batch <= 65535 && mr >= 0 && mr <= 4096 + NB && ldA >= mr && ldV >= 16 && ldW >= 16 &&
                     (!Vn || (ldVn >= 16 && Y && work && sY >= (int64_t)mr * 16)),
                 "scao_eig_sy2sb_update: bad arguments mr=%d batch=%d", mr, batch);
  if (batch == 0 || mr == 0) return SCAO_OK;
  const int nt = (mr + UT - 1) / UT, nch = (nt - 1) / UCH + 1;
  int ntask = 0;
  for (int I = 0; I < nt; ++I) ntask += I / UCH + 1;
  float* Pd = (float*)work;
  float* Pt = Pd + (int64_t)batch * nt * nch * UT * 16;
  hipStream_t s = (hipStream_t)stream;
  const auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool vec = mr % 4 == 0 && ldA % 4 == 0 && ldV % 4 == 0 && ldW % 4 == 0 && sA % 4 == 0 &&
                   sV % 4 == 0 && sW % 4 == 0 && al16(A) && al16(V) && al16(W) &&
                   (!Vn || (ldVn % 4 == 0 && sVn % 4 == 0 && al16(Vn)));
  if (vec)
    hipLaunchKernelGGL(k_sy2sb_update_vec, dim3(ntask, batch), dim3(256), 0, s, A, sA, ldA, mr, V,
                       sV, ldV, W, sW, ldW, Vn, sVn, ldVn, Pd, Pt, nt, nch);
  else
    hipLaunchKernelGGL(k_sy2sb_update, dim3(ntask, batch), dim3(256), 0, s, A, sA, ldA, mr, V, sV,
                       ldV, W, sW, ldW, Vn, sVn, ldVn, Pd, Pt, nt, nch);
  SCAO_LAUNCH_CHECK("scao_eig_sy2sb_update");
  if (Vn) {
    hipLaunchKernelGGL(k_sy2sb_reduce, dim3(nt, batch), dim3(256), 0, s, Pd, Pt, Y, sY, mr, nt,
                       nch);
    SCAO_LAUNCH_CHECK("scao_eig_sy2sb_update/reduce");
  }
  return SCAO_OK;
}

extern "C" int scao_eig_band_finish(const float* A, int64_t stride, int n, int batch,
                                    const float* band, int64_t bstride, float* orig,
                                    int64_t ostride, double* band64, void* stream) {
  SCAO_CHECK_ARG(A && band && orig && band64, "scao_eig_band_finish: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && n > 0 && n <= 4096 + NB && stride >= (int64_t)n * n && bstride >= (int64_t)n * BW &&
                     ostride >= (int64_t)n * OW,
                 "scao_eig_band_finish: bad arguments");
  if (batch == 0) return SCAO_OK;
  hipLaunchKernelGGL(k_band_finish, dim3((n + 255) / 256, batch), dim3(256), 0, (hipStream_t)stream,
                     A, stride, n, band, bstride, orig, ostride, band64);
  SCAO_LAUNCH_CHECK("scao_eig_band_finish");
  return SCAO_OK;
}

extern "C" int scao_eig_sb2st(double* band64, int n, int batch, double* d, double* e,
                              void* stream) {
  SCAO_CHECK_ARG(band64 && d && e, "scao_eig_sb2st: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && n > 0 && n <= 4096 + NB, "scao_eig_sb2st: bad arguments n=%d", n);
  if (batch == 0) return SCAO_OK;
  hipLaunchKernelGGL(k_sb2st, dim3(batch), dim3(SB_W * 64), 0, (hipStream_t)stream, band64, n, d,
                     e);
  SCAO_LAUNCH_CHECK("scao_eig_sb2st");
  return SCAO_OK;
}

extern "C" int64_t scao_eig_bisect_work(int n, int batch) {
  if (n <= 0 || batch <= 0) return 0;
  // wall (n), info (4), nneg (one 8-byte slot), e^2 (n) per matrix
  return (int64_t)batch * ((int64_t)n * 8 + 4 * 8 + 8 + (int64_t)n * 8);
}

extern "C" int scao_eig_bisect(const double* d, const double* e, int n, int batch, int kq, double* w,
                               double* total, void* work, void* stream) {
  SCAO_CHECK_ARG(d && e && w && total && work, "scao_eig_bisect: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && n > 0 && n <= 4096 + NB && kq > 0 && kq <= n,
                 "scao_eig_bisect: bad arguments n=%d kq=%d", n, kq);
  if (batch == 0) return SCAO_OK;
  hipStream_t s = (hipStream_t)stream;
  double* wall = (double*)work;
  double* info = wall + (int64_t)batch * n;
  int* nneg = (int*)(info + 4 * (int64_t)batch);
  double* e2 = info + 5 * (int64_t)batch;     // after nneg's batch 8-byte slots
  hipLaunchKernelGGL(k_tri_info, dim3(batch), dim3(256), 0, s, d, e, n, info, nneg, e2);
  SCAO_LAUNCH_CHECK("scao_eig_bisect/info");
  // wavefronts for the kq largest (64 / BL each) and for up to n - kq
  // negative ones (64 * NB2 each)
  const int nwave = (kq + 64 / BL - 1) / (64 / BL) + (n - kq + 64 * NB2 - 1) / (64 * NB2);
  hipLaunchKernelGGL(k_bisect, dim3(batch, (nwave + 3) / 4), dim3(256), 0, s, d, e2, n, kq, info,
                     nneg, wall);
  SCAO_LAUNCH_CHECK("scao_eig_bisect/bisect");
  hipLaunchKernelGGL(k_bisect_finish, dim3(batch), dim3(64), 0, s, wall, n, kq, info, nneg, w,
                     total);
  SCAO_LAUNCH_CHECK("scao_eig_bisect/finish");
  return SCAO_OK;
}

extern "C" int64_t scao_eig_vectors_work(int n, int batch, int kq) {
  if (n <= 0 || batch <= 0 || kq <= 0) return 0;
  const int64_t nvec = (int64_t)batch * kq;
  const int64_t chunk = inv_chunk(n, nvec);
  // per chunk vector: U (n x 33) + ys (n); per vector: x (n) and its Rayleigh
  // quotient; per matrix: |B|
  return (chunk * (int64_t)n * (WC + 1) + nvec * ((int64_t)n + 1) + batch) *
         (int64_t)sizeof(double);
}

extern "C" int scao_eig_vectors(const float* orig, int64_t ostride, int n, int batch, int kq,
                                double* w, float* Z, int64_t zstride, void* work, void* stream) {
  SCAO_CHECK_ARG(orig && w && Z && work, "scao_eig_vectors: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && n > 0 && n <= 4096 + NB && kq > 0 && kq <= n && ostride >= (int64_t)n * OW &&
                     zstride >= (int64_t)n * kq,
                 "scao_eig_vectors: bad arguments");
  if (batch == 0) return SCAO_OK;
  hipStream_t s = (hipStream_t)stream;
  const int nvec = batch * kq;
  const int chunk = inv_chunk(n, nvec);
  double* U = (double*)work;
  double* xall = U + (int64_t)chunk * n * (WC + 1);
  double* wr = xall + (int64_t)nvec * n;
  double* bnorm = wr + nvec;
  hipLaunchKernelGGL(k_band_norm, dim3(batch), dim3(256), 0, s, orig, ostride, n, bnorm);
  SCAO_LAUNCH_CHECK("scao_eig_vectors/norm");
  for (int v0 = 0; v0 < nvec; v0 += chunk) {
    const int cnt = nvec - v0 < chunk ? nvec - v0 : chunk;
    hipLaunchKernelGGL(k_inviter, dim3((cnt + 3) / 4), dim3(256), 0, s, orig, ostride, n, kq, nvec,
                       v0, w, bnorm, U, xall, wr);
    SCAO_LAUNCH_CHECK("scao_eig_vectors/inviter");
  }
  hipLaunchKernelGGL(k_cluster_orth, dim3(batch), dim3(256), 0, s, n, kq, w, wr, bnorm, xall);
  SCAO_LAUNCH_CHECK("scao_eig_vectors/orth");
  hipLaunchKernelGGL(k_vec_out, dim3((n + 63) / 64, (kq + 63) / 64, batch), dim3(256), 0, s, n, kq,
                     xall, Z, zstride);
  SCAO_LAUNCH_CHECK("scao_eig_vectors/out");
  return SCAO_OK;
}

extern "C" int scao_eig_back_transform(const float* A, int64_t stride, int n, int batch,
                                       const float* T, float* Z, int64_t zstride, int kq,
                                       void* stream) {
  SCAO_CHECK_ARG(A && T && Z, "scao_eig_back_transform: null pointer");
  SCAO_CHECK_ARG(batch >= 0 && batch <= 65535 && n > 0 && n <= 4096 + NB && kq > 0 && kq <= n &&
                     stride >= (int64_t)n * n && zstride >= (int64_t)n * kq,
                 "scao_eig_back_transform: bad arguments n=%d kq=%d", n, kq);
  const int npan = n > NB ? (n - NB + NB - 1) / NB : 0;   // panels c0 = 0, 16, .. < n - NB
  if (batch == 0 || npan == 0) return SCAO_OK;
  hipStream_t s = (hipStream_t)stream;
  const int nrt = (n + 15) / 16, zt = (nrt + 15) / 16;
  const int nsl = (kq + 15) / 16;   // 16-column slices of Z per matrix
  const dim3 g((batch + 7) / 8 * 8 * nsl), b(1024);
  const int64_t sT = (int64_t)batch * NB * NB;
  const bool exact = n % 16 == 0 && kq % 16 == 0;
#define SCAO_BT(ZT)                                                                         \
  if (exact)                                                                                \
    hipLaunchKernelGGL((k_back_transform<ZT, true>), g, b, 0, s, A, stride, n, npan, T, sT, Z, \
                       zstride, kq, batch);                                                 \
  else                                                                                      \
    hipLaunchKernelGGL((k_back_transform<ZT, false>), g, b, 0, s, A, stride, n, npan, T, sT, Z, \
                       zstride, kq, batch);
  if (zt <= 2) {
    SCAO_BT(2)
  } else if (zt <= 4) {
    SCAO_BT(4)
  } else if (zt <= 8) {
    SCAO_BT(8)
  } else if (zt <= 16) {
    SCAO_BT(16)
  } else {
    SCAO_BT(17)
  }
#undef SCAO_BT
  SCAO_LAUNCH_CHECK("scao_eig_back_transform");
  return SCAO_OK;
}
