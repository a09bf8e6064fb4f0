// low_rank_precond_mm on gfx950 (scao/cuda/__init__.py:190-228; the reference's
// kernels scao/cuda/low_rank_ops.cu:239-296, its fallback :102-119):
//   left:  out = (U * s) @ (U^T @ G)     U: m x k, G: m x n
//   right: out = (G @ (U * s)) @ U^T     U: n x k, G: m x n
// as two launches of one strided fp32 GEMM on the matrix cores, in the
// fallback's order, with U * s rounded to fp32 as the fallback's elementwise
// product does.  Off the optimizer step: the package never calls it.
#include "scao_common.hpp"

using namespace scao;

namespace {

constexpr int LT = 64;        // output tile
constexpr int LK = 16;        // reduction chunk staged in LDS
constexpr int LP = LT + 4;    // LDS row pitch

// C[r][c] = sum_t A(r, t) B(t, c) for r < R, c < NC, t < T, one 64 x 64 tile
// of C per workgroup, with A(r, t) = A[r*ar + t*at] (* sa[t] when sa) and
// B(t, c) = B[t*bt + c*bc] (* sb[c] when sb).  Four waves: wave w owns rows
// 16w..16w+15 and all 64 columns (four v_mfma_f32_16x16x4_f32 tiles); the
// operands go through LDS 16 reduction steps at a time, zero beyond the edges.
__global__ __launch_bounds__(256) void k_lrmm(const float* __restrict__ A, int64_t ar, int64_t at,
                                              const float* __restrict__ sa,
                                              const float* __restrict__ B, int64_t bt, int64_t bc,
                                              const float* __restrict__ sb, float* __restrict__ C,
                                              int64_t ldc, int R, int NC, int T) {
  __shared__ float As[LK][LP];   // [t][r]
  __shared__ float Bs[LK][LP];   // [t][c]
  const int r0 = blockIdx.y * LT, c0 = blockIdx.x * LT;
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  v4f acc[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) acc[f] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int t0 = 0; t0 < T; t0 += LK) {
#pragma unroll
    for (int e = threadIdx.x; e < LK * LT; e += 256) {
      const int tt = e / LT, x = e % LT, t = t0 + tt;
      float a = 0.f, b = 0.f;
      if (t < T && r0 + x < R) {
        a = A[(int64_t)(r0 + x) * ar + (int64_t)t * at];
        if (sa) a = a * sa[t];
      }
      if (t < T && c0 + x < NC) {
        b = B[(int64_t)t * bt + (int64_t)(c0 + x) * bc];
        if (sb) b = b * sb[c0 + x];
      }
      As[tt][x] = a;
      Bs[tt][x] = b;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < LK / 4; ++s) {
      // lane l supplies A[l%16][l/16] and B[l/16][l%16] of the 16x4 / 4x16 step
      const float a = As[4 * s + l / 16][16 * w + l % 16];
#pragma unroll
      for (int f = 0; f < 4; ++f) acc[f] = mfma16(a, Bs[4 * s + l / 16][16 * f + l % 16], acc[f]);
    }
    __syncthreads();
  }
  // acc[f][r] holds C[16w + 4(l/16) + r][16f + l%16]
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = r0 + 16 * w + 4 * (l / 16) + r, col = c0 + 16 * f + l % 16;
      if (row < R && col < NC) C[(int64_t)row * ldc + col] = acc[f][r];
    }
}

int lrmm(const float* A, int64_t ar, int64_t at, const float* sa, const float* B, int64_t bt,
         int64_t bc, const float* sb, float* C, int64_t ldc, int64_t R, int64_t NC, int64_t T,
         hipStream_t s) {
  const dim3 g((unsigned)((NC + LT - 1) / LT), (unsigned)((R + LT - 1) / LT)), b(256);
  hipLaunchKernelGGL(k_lrmm, g, b, 0, s, A, ar, at, sa, B, bt, bc, sb, C, ldc, (int)R, (int)NC,
                     (int)T);
  SCAO_LAUNCH_CHECK("scao_low_rank_precond_mm");
  return SCAO_OK;
}

}  // namespace

extern "C" int64_t scao_low_rank_precond_mm_workspace(int64_t m, int64_t n, int64_t k, int left) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return (left ? k * n : m * k) * (int64_t)sizeof(float);
}

extern "C" int scao_low_rank_precond_mm(const float* U, const float* s, const float* G, float* out,
                                        int64_t m, int64_t n, int64_t k, int left, float* ws,
                                        void* stream) {
  SCAO_CHECK_ARG(m > 0 && n > 0 && k > 0, "scao_low_rank_precond_mm: empty shape");
  SCAO_CHECK_ARG(U && s && G && out && ws, "scao_low_rank_precond_mm: null pointer");
  SCAO_CHECK_ARG(m < (1 << 30) && n < (1 << 30) && k < (1 << 30),
                 "scao_low_rank_precond_mm: dimension too large");
  // grid rows: the k rows of U^T G, or the m rows of the outputs
  SCAO_CHECK_ARG(((m > k ? m : k) + LT - 1) / LT <= 65535, "scao_low_rank_precond_mm: m too large");
  hipStream_t st = (hipStream_t)stream;
  if (left) {
    // P = U^T G (k x n), then out = (U * s) P (m x n)
    int rc = lrmm(U, 1, k, nullptr, G, n, 1, nullptr, ws, n, k, n, m, st);
    if (rc != SCAO_OK) return rc;
    return lrmm(U, k, 1, s, ws, n, 1, nullptr, out, n, m, n, k, st);
  }
  // P = G (U * s) (m x k), then out = P U^T (m x n)
  int rc = lrmm(G, n, 1, nullptr, U, k, 1, s, ws, k, m, k, n, st);
  if (rc != SCAO_OK) return rc;
  return lrmm(ws, k, 1, nullptr, U, 1, k, nullptr, out, n, m, n, k, st);
}
