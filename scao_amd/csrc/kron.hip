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
#include <mutex>

#include "scao_common.hpp"

using namespace scao;

namespace {

// ----------------------------------------------------------- project ---
// T[c0:c0+CR, j0:j0+256] = U_l^T G over all m rows.  Wave w owns 64 columns.
// Rows are consumed in chunks of PR=32: each chunk of G (32 x 256) and U_l
// (32 x CR) is loaded into registers one chunk ahead (coalesced float4: one
// wave reads one 1 KB row of G), written to LDS, and all four waves run
// 2*CR MFMAs on it.  CR = 64, or 128 for whole tiles of k % 128 == 0 blocks
// (every G chunk staged then feeds twice the MFMAs, and each strip of G is
// read by half as many blocks).  Chunk-0 tasks also reduce ||g||^2 and
// ||p*decay||^2 from the staged registers (every element of the strip passes
// through exactly one thread).
constexpr int PR = 32;           // rows per chunk
// Whole fp32 tiles (the FAST variants) run on the bf16 matrix cores
// (project_tile_x6) with 256 threads for 64 rows of T and 512 for 128 or 256.
constexpr int X6_NT128 = 512;
constexpr int GP = SCAO_PROJ_COLS + 4;  // LDS pitch of the G chunk

template <bool FAST, bool DO_P, int CR = 64>
__device__ __forceinline__ void project_tile(const scao_leaf_desc& L, const scao_param_desc& P,
                                             int j0, int c0, int slot, double* slots) {
  static_assert(CR == 64 || (CR == 128 && FAST), "CR");
  constexpr int UP = CR + 4;       // LDS pitch of the U_l chunk
  constexpr int NQ = CR / 16;      // MFMA tiles down T
  constexpr int NU = CR / 32;      // float4 of U_l per thread and chunk
  __shared__ __attribute__((aligned(16))) float Gs[PR][GP];
  __shared__ __attribute__((aligned(16))) float Us[PR][UP];
  __shared__ double red[16];
  const int tid = threadIdx.x;
  const int w = tid / 64, l = tid % 64;
  const int m = L.m, n = L.n, k = L.k;
  const int64_t ld = L.ld;
  const int dt = FAST ? SCAO_F32 : P.dtype;
  const int kk = l / 16;
  const bool do_norms = (c0 == 0) && slot >= 0;
  constexpr bool do_p = DO_P;
  const bool decay = P.flags & SCAO_PF_DECAY;
  const bool gvec_leaf = FAST || (L.flags & SCAO_LF_VEC4) != 0;
  const bool kvec = FAST || (k % 4) == 0;

  // loader geometry (fixed per thread): G row gr_h = idx/64, 4 columns at gc
  const int gc = (tid % 64) * 4;         // column offset inside the strip
  int gmask = 15;
  if (!FAST)
    for (int t = 0; t < 4; ++t) gmask = (j0 + gc + t < n) ? gmask : (gmask & ~(1 << t));
  const bool gvec = gvec_leaf && gmask == 15;
  const int uc = (tid % (CR / 4)) * 4;   // c offset inside the CR-wide chunk
  int umask = 15;
  if (!FAST)
    for (int t = 0; t < 4; ++t) umask = (c0 + uc + t < k) ? umask : (umask & ~(1 << t));
  const bool uvec = kvec && umask == 15;

  v4f acc[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[q][t] = v4f{0.f, 0.f, 0.f, 0.f};
  double g2 = 0.0, p2 = 0.0;

  v4f rg[8], ru[NU], rp[8];
  auto load_chunk = [&](int i0) {
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const int i = i0 + tid / 64 + 4 * h;     // rows i0 + (0..31)
      const int64_t e = L.off + (int64_t)i * ld + j0 + gc;
      if (FAST) {
        rg[h] = gld4_nt((const float*)P.graw + e);
        if (do_p) rp[h] = gld4_nt((const float*)P.p + e);
      } else {
        const bool ok = i < m && gmask;
        rg[h] = ok ? ld4(P.graw, dt, e, gvec, gmask) : v4f{0.f, 0.f, 0.f, 0.f};
        if (do_p) rp[h] = ok ? ld4(P.p, dt, e, gvec, gmask) : v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int h = 0; h < NU; ++h) {
      const int i = i0 + tid / (CR / 4) + (1024 / CR) * h;
      if (FAST)
        ru[h] = gld4(L.Ul + (int64_t)i * k + c0 + uc);
      else
        ru[h] = (i < m && umask) ? ldf4(L.Ul, (int64_t)i * k + c0 + uc, uvec, umask)
                                 : v4f{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int h = 0; h < 8; ++h) *(v4f*)&Gs[tid / 64 + 4 * h][gc] = rg[h];
#pragma unroll
    for (int h = 0; h < NU; ++h) *(v4f*)&Us[tid / (CR / 4) + (1024 / CR) * h][uc] = ru[h];
    if (do_norms) {
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int h = 0; h < 8; ++h)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          a = fmaf(rg[h][t], rg[h][t], a);
          if (do_p) {
            const float x = decay ? round_to(dt, rp[h][t] * P.decay) : rp[h][t];
            b = fmaf(x, x, b);
          }
        }
      g2 += (double)a;
      p2 += (double)b;
    }
  };

  load_chunk(0);
  for (int i0 = 0; i0 < m; i0 += PR) {
    if (i0) __syncthreads();              // previous chunk fully consumed
    store_chunk();
    __syncthreads();
    if (i0 + PR < m) load_chunk(i0 + PR); // in flight during the MFMAs below
    // operands of step s + 1 are read from LDS while step s's MFMAs run
    v4f b[2];
    float a[2][NQ];
    b[0] = *(const v4f*)&Gs[kk][64 * w + 4 * (l % 16)];
#pragma unroll
    for (int q = 0; q < NQ; ++q) a[0][q] = Us[kk][16 * q + (l % 16)];
#pragma unroll
    for (int s = 0; s < PR / 4; ++s) {
      const int cur = s & 1;
      if (s + 1 < PR / 4) {
        b[cur ^ 1] = *(const v4f*)&Gs[4 * (s + 1) + kk][64 * w + 4 * (l % 16)];
#pragma unroll
        for (int q = 0; q < NQ; ++q) a[cur ^ 1][q] = Us[4 * (s + 1) + kk][16 * q + (l % 16)];
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[q][t] = mfma16(a[cur][q], b[cur][t], acc[q][t]);
    }
    if (FAST && CR == 64) {
      // the schedule: step 0's reads, then per step the next step's reads
      // ahead of its 16 MFMAs (a G float4 and four U_l values: three LDS
      // instructions).  Measured faster at CR = 64 only: the 128-wide tile
      // runs slower with it.
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
      for (int s = 0; s < PR / 4; ++s) {
        if (s + 1 < PR / 4) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
      }
    }
  }
  // T[c][j] for c = c0 + 16q + 4*(l/16) + r, j = jl + t
  const int jl = j0 + 64 * w + 4 * (l % 16);
  int cmask = 15;
  if (!FAST)
    for (int t = 0; t < 4; ++t) cmask = (jl + t < n) ? cmask : (cmask & ~(1 << t));
  const bool tvec = gvec_leaf && cmask == 15;
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = c0 + 16 * q + 4 * kk + r;
      if (FAST || (c < k && cmask)) {
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

// The same tile for whole fp32 tiles (FAST) on the bf16 matrix cores, with
// fp32 products through three-way splits (mfma_x6): one v_mfma_f32_16x16x32
// covers a whole 32-row chunk, so a chunk costs 6 * 16 cycles per output
// tile against 8 * 32 for the fp32 16x16x4 form.  NT threads (NT / 64
// waves) share the CR x 256 tile; wave w owns CW = 256 / (NT / 64) columns
// (NJ = CW / 16 output tiles across) and all CR rows of T.
//   * G does not pass through LDS: lane (jj, g) of wave w loads rows
//     8g..8g+7 of the chunk at the NJ columns j0 + CW*w + NJ*jj + t, which is
//     exactly its B operand of the NJ output tiles t (the column permutation
//     of the fp32 form), and splits it in registers.
//   * U_l (shared by the waves) is split by its loader and stored as three
//     bf16 planes, column-major inside the chunk (column pitch 80 B: the 16
//     lanes of one A-operand read hit 16 disjoint bank quads).
// The next chunk's G, p and U_l are loaded while the current one's MFMAs run.
template <bool DO_P, int CR, int NT>
__device__ __forceinline__ void project_tile_x6(const scao_leaf_desc& L, const scao_param_desc& P,
                                                int j0, int c0, int slot, double* slots) {
  static_assert(CR == 64 || CR == 128 || CR == 256, "CR");
  static_assert(NT == 256 || NT == 512, "NT");
  constexpr int NQ = CR / 16;        // MFMA tiles down T
  constexpr int CW = 256 / (NT / 64);
  constexpr int NJ = CW / 16;        // MFMA tiles across, G columns per lane
  constexpr int UCP = 40;            // bf16 per U_l column in LDS (32 rows + pad)
  constexpr int UG = NT / 8;         // U_l loader threads per 4-row group
  constexpr int UW = CR / UG;        // U_l columns per loader thread
  static_assert(UW == 2 || UW == 4, "U_l loader width");
  typedef float vj __attribute__((ext_vector_type(NJ)));
  typedef __attribute__((address_space(1))) vj gvj;
  __shared__ __attribute__((aligned(16))) __bf16 Us[2][3][CR][UCP];   // by chunk parity
  __shared__ double red[2 * NT / 64];
  const int tid = threadIdx.x;
  const int w = tid / 64, l = tid % 64;
  const int jj = l % 16, g = l / 16;
  const int m = L.m, n = L.n, k = L.k;
  const int64_t ld = L.ld;
  const bool do_norms = (c0 == 0) && slot >= 0;
  // x * 1.0f == x bit for bit, so no per-element select on the decay flag
  const float dec = (P.flags & SCAO_PF_DECAY) ? P.decay : 1.0f;
  const int gcol = j0 + CW * w + NJ * jj;
  // U_l loader: rows 4*ua .. 4*ua+3 of the chunk, columns ub*UW .. +UW-1
  const int ua = tid / UG, ub = tid % UG;
  // Every load address is a row origin shared by the block (scalar
  // registers) plus a 32-bit lane offset fixed for the whole tile: lane
  // (jj, g) reads rows 8g.. of the chunk at column gcol, the U_l loader rows
  // 4ua.. at column c0 + ub*UW.
  const uint32_t g_lane = (uint32_t)((8 * g * ld + (gcol - j0)) * (int64_t)sizeof(float));
  const uint32_t u_lane = (uint32_t)((4 * ua * (int64_t)k + ub * UW) * (int64_t)sizeof(float));
  const int64_t ldb = ld * (int64_t)sizeof(float), kb = k * (int64_t)sizeof(float);

  v4f acc[NQ][NJ];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int t = 0; t < NJ; ++t) acc[q][t] = v4f{0.f, 0.f, 0.f, 0.f};
  double g2 = 0.0, p2 = 0.0;

  vj rg[8], rp[8];
  float ru[4][UW];
  auto load_g = [&](int i0) {
    const int64_t o = L.off + (int64_t)i0 * ld + j0;
    const char* gb = (const char*)((const float*)P.graw + o);
    const char* pb = (const char*)((const float*)P.p + o);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rg[e] = __builtin_nontemporal_load((const gvj*)(gb + e * ldb + g_lane));
      if (DO_P) rp[e] = __builtin_nontemporal_load((const gvj*)(pb + e * ldb + g_lane));
    }
  };
  auto load_u = [&](int i0) {
    const char* ubase = (const char*)(L.Ul + (int64_t)i0 * k + c0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float* src = (const float*)(ubase + r * kb + u_lane);
      if constexpr (UW == 4) {
        const v4f x = gld4(src);
#pragma unroll
        for (int c = 0; c < 4; ++c) ru[r][c] = x[c];
      } else {
        const v2u x = *(const gv2u*)src;
        ru[r][0] = __uint_as_float(x[0]);
        ru[r][1] = __uint_as_float(x[1]);
      }
    }
  };

  // U_l's planes for chunk i sit in Us[i & 1]: chunk i+1's are split and
  // written during chunk i (its raw rows were loaded a chunk earlier), so one
  // barrier per chunk separates a buffer's readers from its next writers
  auto write_u = [&](int buf) {
#pragma unroll
    for (int c = 0; c < UW; ++c) {
      // four rows of one column: one 8-byte write per plane
      v2u pl[3];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t a, b, cc;
        split3_pk(ru[2 * h][c], ru[2 * h + 1][c], a, b, cc);   // rows 2h (low), 2h+1
        pl[0][h] = a;
        pl[1][h] = b;
        pl[2][h] = cc;
      }
      const int col = ub * UW + c;
#pragma unroll
      for (int pp = 0; pp < 3; ++pp) *(v2u*)&Us[buf][pp][col][4 * ua] = pl[pp];
    }
  };
  // CR = 256: the prefetches are unconditional, clamped to the last chunk
  // (m % PR == 0 for these tiles), and pinned ahead of the MFMAs: behind a
  // branch, the join makes the compiler wait for every load in flight, the
  // next chunk's G included, and the scheduler sinks them among the MFMAs.
  // The narrower tiles have half or a quarter of the MFMAs per chunk to hide
  // loads behind and measured faster with the branch (the last chunk loads
  // nothing).
  const int last = m - PR;
  load_g(0);
  load_u(0);
  write_u(0);
  if (CR == 256 || PR < m) load_u(PR < last ? PR : last);
  __syncthreads();
  for (int i0 = 0, cur = 0; i0 < m; i0 += PR, cur ^= 1) {
    // this chunk's G operands, split in registers
    bf3 bg[NJ];
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = rg[e][t];
      bg[t] = split_bf3(x);
    }
    if (do_norms) {
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int t = 0; t < NJ; ++t) {
          a = fmaf(rg[e][t], rg[e][t], a);
          if (DO_P) {
            const float x = rp[e][t] * dec;
            b = fmaf(x, x, b);
          }
        }
      g2 += (double)a;
      p2 += (double)b;
    }
    if constexpr (CR == 256) {
      write_u(cur ^ 1);                   // chunk i+1's planes, read after the barrier below
      // the loads go out after the split (measured faster than letting the
      // scheduler hoist them above it)
      __builtin_amdgcn_sched_barrier(0);
      load_g(i0 + PR < last ? i0 + PR : last);   // in flight during the MFMAs below
      load_u(i0 + 2 * PR < last ? i0 + 2 * PR : last);
      __builtin_amdgcn_sched_barrier(0);
    } else if (i0 + PR < m) {
      write_u(cur ^ 1);
      load_g(i0 + PR);
      if (i0 + 2 * PR < m) load_u(i0 + 2 * PR);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      bf3 au;
      au.h = *(const v8bf*)&Us[cur][0][16 * q + jj][8 * g];
      au.m = *(const v8bf*)&Us[cur][1][16 * q + jj][8 * g];
      au.l = *(const v8bf*)&Us[cur][2][16 * q + jj][8 * g];
#pragma unroll
      for (int t = 0; t < NJ; ++t) acc[q][t] = mfma_x6(au, bg[t], acc[q][t]);
    }
    __syncthreads();
  }
  // T[c][j] for c = c0 + 16q + 4g + r, j = gcol + t
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = c0 + 16 * q + 4 * g + r;
      vj o;
#pragma unroll
      for (int t = 0; t < NJ; ++t) o[t] = acc[q][t][r];
      *(gvj*)(L.T + (int64_t)c * n + gcol) = o;
    }
  if (do_norms) {
    double x[2] = {g2, p2};
    block_sum_n<2, NT>(x, red);
    if (threadIdx.x == 0) {
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = x[0];
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = x[1];
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = 0.0;
    }
  }
}

// ------------------------------------------------------------- delta ---
// P[c0:c0+64, d0:d0+64] = T U_r; Delta and the natural-norm partial.
// The four waves split the n-reduction (one quarter each, 16-column chunks,
// one chunk prefetched); every wave accumulates the whole 64x64 tile
// (16 MFMA tiles) and the four partial tiles are added in LDS in a fixed
// order.  P column d of tile t sits at lane column jj with d = d0 + 4*jj + t,
// so one float4 of a U_r row feeds all four tiles.
constexpr int DP = 64 + 4;   // LDS pitch of a partial tile

// acc[q][t] += sum over j in [jbeg, jend) of A[r0 + 16q + i][j] * B[j][c0 + 4i + t]
// (i = lane % 16) for a 64 x 64 output tile, with the products on the bf16
// matrix cores: six per fp32 product over three-way splits, as the
// projection.  The reduction runs in chunks of 32: lane (i, g) takes A row
// r0 + 16q + i at columns j + 8g .. j + 8g + 7 (the A operand of row tile q)
// and B rows j + 8g .. j + 8g + 7 at columns c0 + 4i .. c0 + 4i + 3 (element t
// of each float4 is the B operand of column tile t), so the accumulator layout
// is the fp32 16x16x4 form's with the same column permutation.  Rows of A and
// B are 16-byte aligned and jend - jbeg is a multiple of 32.
__device__ __forceinline__ void mm64_x6(const float* __restrict__ A, int64_t lda,
                                        const float* __restrict__ B, int64_t ldb, int r0, int c0,
                                        int jbeg, int jend, v4f (&acc)[4][4]) {
  const int l = threadIdx.x % 64, i = l % 16, g = l / 16;
  // each operand's next-chunk load goes out as soon as its current value is
  // split, into the same registers; on the last chunk the loads repeat it
  // (in bounds, unused), so no branch makes the compiler wait for them
  v4f ca[4][2], cb[8];
  auto load_a = [&](int jb, int q, v4f (&a)[2]) {
    const float* ap = A + (int64_t)(r0 + 16 * q + i) * lda + jb + 8 * g;
    a[0] = gld4(ap);
    a[1] = gld4(ap + 4);
  };
  auto load_b = [&](int jb, v4f (&b)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = gld4(B + (int64_t)(jb + 8 * g + e) * ldb + c0 + 4 * i);
  };
  if (jbeg >= jend) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) load_a(jbeg, q, ca[q]);
  load_b(jbeg, cb);
  for (int jb = jbeg; jb < jend; jb += 32) {
    const int jn = jb + 32 < jend ? jb + 32 : jb;
    bf3 bt[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = cb[e][t];
      bt[t] = split_bf3(x);
    }
    load_b(jn, cb);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = ca[q][0][e];
        x[4 + e] = ca[q][1][e];
      }
      const bf3 aq = split_bf3(x);
      load_a(jn, q, ca[q]);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[q][t] = mfma_x6(aq, bt[t], acc[q][t]);
    }
  }
}

// Ps (three partial tiles) and red live in the caller's LDS, so a kernel
// holding both instantiations allocates them once.
template <bool FAST, bool X6 = false>
__device__ __forceinline__ void delta_tile(const scao_leaf_desc& L, float eps, int c0, int d0,
                                           int slot, double* slots, float (*Ps)[64][DP],
                                           double* red) {
  static_assert(FAST || !X6, "X6 needs whole tiles");
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int n = L.n, k = L.k;
  const int kk = l / 16;
  const float* T = L.T;
  const float* Ur = L.Ur;
  const int dl = d0 + 4 * (l % 16);      // this lane's 4 P columns
  int dmask = 15;
  if (!FAST)
    for (int t = 0; t < 4; ++t) dmask = (dl + t < k) ? dmask : (dmask & ~(1 << t));
  const bool uvec = FAST || ((k % 4) == 0 && dmask == 15);
  const bool tvec_leaf = FAST || (L.flags & SCAO_LF_VEC4) != 0;
  const int nq = ((n + 63) / 64) * 16;    // per-wave share of n, multiple of 16
  const int jbeg = w * nq, jend = min(n, jbeg + nq);

  v4f acc[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[q][t] = v4f{0.f, 0.f, 0.f, 0.f};

  if constexpr (X6) {
    // whole tiles, n % 128 == 0: each wave's quarter of n is a multiple of 32
    mm64_x6(T, n, Ur, k, c0, d0, jbeg, jend, acc);
  } else {
    v4f ra[4], rb[4], na[4], nb[4];
    auto load = [&](int jb, v4f (&a)[4], v4f (&b)[4]) {
      const int j = jb + 4 * kk;
      int jm = 15;
      if (!FAST)
        for (int s2 = 0; s2 < 4; ++s2) jm = (j + s2 < jend) ? jm : (jm & ~(1 << s2));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = c0 + 16 * q + (l % 16);
        if (FAST)
          a[q] = gld4(T + (int64_t)c * n + j);
        else
          a[q] = (c < k && jm) ? ldf4(T, (int64_t)c * n + j, tvec_leaf && jm == 15, jm)
                               : v4f{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        if (FAST)
          b[s2] = gld4(Ur + (int64_t)(j + s2) * k + dl);
        else
          b[s2] = (((jm >> s2) & 1) && dmask) ? ldf4(Ur, (int64_t)(j + s2) * k + dl, uvec, dmask)
                                              : v4f{0.f, 0.f, 0.f, 0.f};
      }
    };
    if (jbeg < jend) load(jbeg, ra, rb);
    for (int jb = jbeg; jb < jend; jb += 16) {
      if (jb + 16 < jend) load(jb + 16, na, nb);
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[q][t] = mfma16(ra[q][s2], rb[s2][t], acc[q][t]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ra[q] = na[q];
        rb[q] = nb[q];
      }
    }
  }
  // partial tiles of waves 1..3 go through LDS; wave 0 adds them in order
  // (((w0 + w1) + w2) + w3) and finishes its 64 elements per lane:
  // element (16q + 4*kk + r, 4*(l%16) + t)
  if (w > 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *(v4f*)&Ps[w - 1][16 * q + 4 * kk + r][4 * (l % 16)] =
            v4f{acc[q][0][r], acc[q][1][r], acc[q][2][r], acc[q][3][r]};
  }
  __syncthreads();
  const bool sinv4 = L.flags & SCAO_LF_SINV4;
  double nu2 = 0.0;
  if (w == 0) {
    float sr4[4], ir2[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = dl + t;
      const float sr = d < k ? gld1(L.Sr + d) : 1.f;
      sr4[t] = sinv4 ? sr : inv4(sr);
      ir2[t] = sinv4 ? 0.f : inv2(sr, eps);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * q + 4 * kk + r;
        const int c = c0 + row;
        if (c >= k) continue;
        const float sl = gld1(L.Sl + c);
        const float sl4 = sinv4 ? sl : inv4(sl);
        const float il2 = sinv4 ? 0.f : inv2(sl, eps);
        const v4f p1 = *(const v4f*)&Ps[0][row][4 * (l % 16)];
        const v4f p2 = *(const v4f*)&Ps[1][row][4 * (l % 16)];
        const v4f p3 = *(const v4f*)&Ps[2][row][4 * (l % 16)];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int d = dl + t;
          if (d >= k) continue;
          const float pv = ((acc[q][t][r] + p1[t]) + p2[t]) + p3[t];
          gst1(L.Delta + (int64_t)c * k + d, (sl4 * sr4[t] - 1.0f) * pv);
          if (!sinv4) {
            const float y = (il2 * pv) * ir2[t];
            nu2 += (double)y * (double)y;
          }
        }
      }
  }
  if (slot >= 0) {
    double xs[1] = {nu2};
    block_sum<1>(xs, red);
    if (threadIdx.x == 0) {
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = 0.0;
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = 0.0;
      slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = xs[0];
    }
  }
}

// A diagonal sub-block of a block-diagonal parameter (SCAO_LF_DIAG: a
// remainder block one row or one column wide, reference
// preconditioner.py:142-153, 232-236).  Nothing is projected: one 64x64 tile
// of it contributes ||g||^2, ||p*decay||^2 (LARS params) and the natural-norm
// sum g^2 / (sqrt(diag) + eps) (:542-544) to the task's slot, in the place
// the projection and delta tasks of a Kronecker block write them.
__device__ __forceinline__ void diag_leaf_reduce(const scao_leaf_desc& L,
                                                 const scao_param_desc& P, int i0, int j0,
                                                 int slot, double* slots, double* red) {
  const int dt = P.dtype;
  const bool decay = P.flags & SCAO_PF_DECAY;
  const bool lars = P.flags & SCAO_PF_LARS;
  double acc[3] = {0.0, 0.0, 0.0};
  for (int q = threadIdx.x; q < 64 * 64; q += 256) {
    const int i = i0 + q / 64, j = j0 + q % 64;
    if (i >= L.m || j >= L.n) continue;
    const int64_t e = L.off + (int64_t)i * L.ld + j;
    const float g = ld1(P.graw, dt, e);
    const float dg = gld1(L.Sl + (int64_t)i * L.n + j);
    acc[0] += (double)(g * g);
    if (lars) {
      const float p = ld1(P.p, dt, e);
      const float pd = decay ? round_to(dt, p * P.decay) : p;
      acc[1] += (double)(pd * pd);
    }
    acc[2] += (double)((g * g) / (sqrtf(dg) + P.eps));
  }
  block_sum<3>(acc, red);
  if (threadIdx.x == 0 && slot >= 0) {
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = acc[0];
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = acc[1];
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = acc[2];
  }
}

// -------------------------------------------------------------- lift ---
// W[i0:i0+64, d0:d0+64] = U_l Delta.  Wave w computes rows i0+16w .. +15.
// On whole tiles (k % 16 == 0, 16-byte aligned factors) lane column jj holds
// W columns d0 + 4*jj + t of MFMA tile t, so one float4 of a Delta row feeds
// all four tiles and each row of the result leaves as one float4; the
// reduction runs with NH chunks of operands in flight (fully unrolled for
// k = 16 NC, NC > 0; any multiple of 16 with one chunk of lookahead for
// NC = 0).  Other tiles take the element-wise path.
// W's exact three-way bf16 split (as split_bf3) into the planes h, m, l of
// Wb (plane stride mk elements), at element o: four elements, or one.
__device__ __forceinline__ void split3(float x, __bf16& h, __bf16& m, __bf16& l) {
  h = (__bf16)x;
  const float r = x - (float)h;
  m = (__bf16)r;
  l = (__bf16)(r - (float)m);
}
// four consecutive elements' planes as two packed words each
__device__ __forceinline__ void split4_pk(const v4f& x, v2u& h, v2u& m, v2u& l) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    uint32_t a, b, c;
    split3_pk(x[2 * p], x[2 * p + 1], a, b, c);
    h[p] = a;
    m[p] = b;
    l[p] = c;
  }
}
__device__ __forceinline__ void store_split4(uint16_t* wb, int64_t mk, int64_t o, const v4f& x) {
  v2u h, m, l;
  split4_pk(x, h, m, l);
  *(gv2u*)(wb + o) = h;
  *(gv2u*)(wb + mk + o) = m;
  *(gv2u*)(wb + 2 * mk + o) = l;
}
__device__ __forceinline__ void store_split1(uint16_t* wb, int64_t mk, int64_t o, float x) {
  __bf16 h, m, l;
  split3(x, h, m, l);
  ((gu16*)wb)[o] = __builtin_bit_cast(uint16_t, h);
  ((gu16*)wb)[mk + o] = __builtin_bit_cast(uint16_t, m);
  ((gu16*)wb)[2 * mk + o] = __builtin_bit_cast(uint16_t, l);
}

template <int NC>
__device__ __forceinline__ void lift_chunks(const float* __restrict__ urow,
                                            const float* __restrict__ drow, int k,
                                            v4f (&acc)[4]) {
  // urow: U_l row + 4*kk; drow: Delta row 4*kk, columns dl..dl+3
  if constexpr (NC > 0) {
    constexpr int PD = NC < 4 ? NC : 4;
    v4f A[PD], B[PD][4];
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      A[d] = gld4(urow + 16 * d);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) B[d][s4] = gld4(drow + (int64_t)(16 * d + s4) * (16 * NC));
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c % PD;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(A[d][s4], B[d][s4][t], acc[t]);
      if (c + PD < NC) {
        A[d] = gld4(urow + 16 * (c + PD));
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          B[d][s4] = gld4(drow + (int64_t)(16 * (c + PD) + s4) * (16 * NC));
      }
    }
  } else {
    v4f a = gld4(urow), b[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) b[s4] = gld4(drow + (int64_t)s4 * k);
    for (int cb = 0; cb < k; cb += 16) {
      const bool more = cb + 16 < k;
      v4f an = a, bn[4] = {b[0], b[1], b[2], b[3]};
      if (more) {
        an = gld4(urow + cb + 16);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) bn[s4] = gld4(drow + (int64_t)(cb + 16 + s4) * k);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(a[s4], b[s4][t], acc[t]);
      a = an;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) b[s4] = bn[s4];
    }
  }
}

__device__ __forceinline__ void lift_tile(const scao_leaf_desc& L, int i0, int d0) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, k = L.k;
  const int kk = l / 16;
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const bool whole = k % 16 == 0 && i0 + 64 <= m && d0 + 64 <= k &&
                     (((uintptr_t)L.Ul | (uintptr_t)L.Delta | (uintptr_t)L.W) & 15) == 0 &&
                     ((uintptr_t)L.Wb & 7) == 0;
  if (whole) {
    const int irow = i0 + 16 * w + (l % 16);
    const int dl = d0 + 4 * (l % 16);
    const float* __restrict__ urow = L.Ul + (int64_t)irow * k + 4 * kk;
    const float* __restrict__ drow = L.Delta + (int64_t)(4 * kk) * k + dl;
    if (k == 256)
      lift_chunks<16>(urow, drow, k, acc);
    else if (k == 128)
      lift_chunks<8>(urow, drow, k, acc);
    else if (k == 64)
      lift_chunks<4>(urow, drow, k, acc);
    else
      lift_chunks<0>(urow, drow, k, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t o = (int64_t)(i0 + 16 * w + 4 * kk + r) * k + dl;
      const v4f x = v4f{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
      gst4(L.W + o, x);
      if (L.Wb) store_split4(L.Wb, (int64_t)m * k, o, x);
    }
    return;
  }
  const int irow = i0 + 16 * w + (l % 16);
  const bool kvec = (k % 4) == 0;
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
      if (d < k) {
        L.W[(int64_t)i * k + d] = acc[t][r];
        if (L.Wb) store_split1(L.Wb, (int64_t)m * k, (int64_t)i * k + d, acc[t][r]);
      }
    }
  }
}

// The same tile for k % 128 == 0 on whole, aligned tiles, with the products on
// the bf16 matrix cores (mm64_x6): wave w takes the whole 64 x 64 tile over
// its quarter of k (a multiple of 32), the four partial tiles go through LDS,
// and wave w adds rows 16w .. 16w + 15 of them in order (((w0 + w1) + w2) + w3)
// and writes those rows of W (and Wb).
__device__ __forceinline__ bool lift_x6_ok(const scao_leaf_desc& L, int i0, int d0) {
  return L.k % 128 == 0 && i0 + 64 <= L.m && d0 + 64 <= L.k &&
         (((uintptr_t)L.Ul | (uintptr_t)L.Delta | (uintptr_t)L.W) & 15) == 0 &&
         ((uintptr_t)L.Wb & 7) == 0;
}
__device__ __forceinline__ void lift_tile_x6(const scao_leaf_desc& L, int i0, int d0,
                                             float (*Ps)[64][DP]) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64, jj = l % 16, g = l / 16;
  const int m = L.m, k = L.k, kq = k / 4;
  v4f acc[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[q][t] = v4f{0.f, 0.f, 0.f, 0.f};
  mm64_x6(L.Ul, k, L.Delta, k, i0, d0, w * kq, w * kq + kq, acc);
  // element (16q + 4g + r, 4jj + t) of the wave's partial tile
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *(v4f*)&Ps[w][16 * q + 4 * g + r][4 * jj] =
          v4f{acc[q][0][r], acc[q][1][r], acc[q][2][r], acc[q][3][r]};
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 16 * w + 4 * g + r;
    const v4f p0 = *(const v4f*)&Ps[0][row][4 * jj];
    const v4f p1 = *(const v4f*)&Ps[1][row][4 * jj];
    const v4f p2 = *(const v4f*)&Ps[2][row][4 * jj];
    const v4f p3 = *(const v4f*)&Ps[3][row][4 * jj];
    v4f x;
#pragma unroll
    for (int t = 0; t < 4; ++t) x[t] = ((p0[t] + p1[t]) + p2[t]) + p3[t];
    const int64_t o = (int64_t)(i0 + row) * k + d0 + 4 * jj;
    gst4(L.W + o, x);
    if (L.Wb) store_split4(L.Wb, (int64_t)m * k, o, x);
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

// The Phase-2 elementwise tail for one row of four columns (t = 0..3):
// gp = G + corr -> clip -> blend -> Adan moments -> update.  With LARS the
// update itself is returned in `out` (the write waits for the trust ratio);
// otherwise `out` is the new parameter value.  u2 accumulates u^2 over the
// columns in `cmask`.  Operation order and roundings follow
// scao/optimizer.py:584-645 (see the rounding notes on each line).
template <bool GF32, bool LARS>
__device__ __forceinline__ void adan4(const scao_param_desc& P, const scao_param_stat& S, int dt,
                                      const v4f& gr, const v4f& gm, const v4f& corr, v4f& mm,
                                      v4f& vv, v4f& dd, const v4f& pp, const v4f& par, v4f& out,
                                      float& u2, int cmask, bool direct = false) {
  const bool clip = P.flags & SCAO_PF_CLIP;
  const bool gsnr = P.flags & SCAO_PF_GSNR;
  const bool decay = P.flags & SCAO_PF_DECAY;
  const float alpha_nolars = round_to(dt, (float)(-P.lr));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    // precondition() output in p.dtype; `direct`: corr already is that output
    float gp = round_to(dt, direct ? corr[t] : gr[t] + corr[t]);
    if (clip) gp = round_to(dt, gp * S.clip);           // gp * (tau / nu)
    const float g = GF32 ? gm[t] : gr[t];
    const float geff = P.blend * gp + P.omblend * g;    // b*gp.float() + (1-b)*grad
    const float delta = g - pp[t];
    const float m1 = fmaf(geff, P.omb1, mm[t] * P.beta1);
    const float d1 = fmaf(delta, P.omb3, dd[t] * P.beta3);
    const float gad = geff + P.omb3 * delta;
    const float v1 = fmaf(P.omb2 * gad, gad, vv[t] * P.beta2);
    float x = (m1 / P.bc1 + P.omb3 * (d1 / P.bc3)) / (sqrtf(v1 / P.bc2) + P.eps);
    if (gsnr) x = x * ((fabsf(m1) / (sqrtf(v1) + P.eps)) >= P.gsnr ? 1.0f : 0.0f);
    mm[t] = m1;
    dd[t] = d1;
    vv[t] = v1;
    if (LARS) {
      out[t] = x;
      if (cmask & (1 << t)) u2 = fmaf(x, x, u2);
    } else {
      const float pd = decay ? round_to(dt, par[t] * P.decay) : par[t];
      out[t] = round_to(dt, fmaf(round_to(dt, x), alpha_nolars, pd));
    }
  }
}

__device__ __forceinline__ void write_u2_slot(double* slots, int slot, float u2, double* red) {
  if (slot < 0) return;
  double x[1] = {(double)u2};
  block_sum<1>(x, red);
  if (threadIdx.x == 0) {
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = 0.0;
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = 0.0;
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = x[0];
  }
}

// One 64x64 tile of a block, any shape, dtype or alignment (masked).  Per wave
// 16 rows x 64 columns, 16 elements per lane:
//   1. issue every elementwise load of the tile (g, m, v, d, prev [, p]) --
//      they do not depend on the correction, so HBM latency overlaps step 2;
//   2. corr = W[rows, :] U_r[cols, :]^T on MFMA, with the U_r tile (shared by
//      the four waves) staged once per block through LDS, 64 columns of k at
//      a time;
//   3. the elementwise tail, then the stores.
constexpr int UPAD = 68;   // LDS row pitch (floats) of the staged U_r tile

template <bool GF32, bool LARS>
__device__ __forceinline__ void apply_tile(const scao_leaf_desc& L, const scao_param_desc& P,
                                           const scao_param_stat& S, int i0, int j0, int slot,
                                           double* slots) {
  __shared__ __attribute__((aligned(16))) float Us[64][UPAD];
  __shared__ double red[16];
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int m = L.m, n = L.n, k = L.k;
  const int dt = P.dtype;
  const int kk = l / 16;
  const int jl = j0 + 4 * (l % 16);
  int cmask = 15;
  for (int t = 0; t < 4; ++t) cmask = (jl + t < n) ? cmask : (cmask & ~(1 << t));
  const bool vec = (L.flags & SCAO_LF_VEC4) && cmask == 15;

  // 1) prefetch
  v4f gr[4], gm[4], mm[4], vv[4], dd[4], pp[4], par[4];
  int64_t e[4];
  bool rok[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = i0 + 16 * w + 4 * kk + r;
    e[r] = L.off + (int64_t)i * L.ld + jl;
    rok[r] = i < m && cmask;
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    gr[r] = rok[r] ? ld4(P.graw, dt, e[r], vec, cmask) : z;
    // GF32: the fp32 moment buffer, or (fused) the filter's EMA until finish_mgrad
    gm[r] = (GF32 && rok[r])
                ? (fused_mgrad(P) ? ((P.flags & SCAO_PF_FMASK) ? ldf4(P.fema, e[r], vec, cmask) : gr[r])
                                  : ldf4((const float*)P.g, e[r], vec, cmask))
                : z;
    mm[r] = rok[r] ? ldf4(P.exp_avg, e[r], vec, cmask) : z;
    vv[r] = rok[r] ? ldf4(P.exp_avg_sq, e[r], vec, cmask) : z;
    dd[r] = rok[r] ? ldf4(P.exp_avg_diff, e[r], vec, cmask) : z;
    pp[r] = rok[r] ? ldf4(P.prev_grad, e[r], vec, cmask) : z;
    par[r] = (!LARS && rok[r]) ? ld4(P.p, dt, e[r], vec, cmask) : z;
  }

  // 2) corr = W U_r^T; for a diagonal sub-block the preconditioned gradient
  //    itself, g / (clamp-free (diag / bias)^(1/4) + 1e-8) (reference
  //    preconditioner.py:506-510), with diag element (i, j) at i*n + j
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const bool dleaf = L.flags & SCAO_LF_DIAG;
  if (dleaf) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (!rok[r]) continue;
      const int i = i0 + 16 * w + 4 * kk + r;
      const v4f dg = ldf4(L.Sl, (int64_t)i * n + jl, false, cmask);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float x = dg[t] / L.dbias;
        const float den = (float)pow((double)x, 0.25) + 1e-8f;
        acc[t][r] = gr[r][t] / den;
      }
    }
  }
  const int irow = i0 + 16 * w + (l % 16);
  const bool kvec = (k % 4) == 0;
  for (int cb0 = 0; cb0 < (dleaf ? 0 : k); cb0 += 64) {
    if (cb0) __syncthreads();
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int idx = threadIdx.x + 256 * h;
      const int row = idx / 16, c4 = (idx % 16) * 4;
      const int j = j0 + row, c = cb0 + c4;
      int mk = 0;
      for (int t = 0; t < 4; ++t) mk |= (j < n && c + t < k) ? (1 << t) : 0;
      const v4f x = mk ? ldf4(L.Ur, (int64_t)j * k + c, kvec && mk == 15, mk)
                       : v4f{0.f, 0.f, 0.f, 0.f};
      *(v4f*)&Us[row][c4] = x;
    }
    __syncthreads();
    const int cend = k - cb0 < 64 ? k - cb0 : 64;
    for (int cb = 0; cb < cend; cb += 16) {
      const int c = cb0 + cb + 4 * kk;
      int cm = 15;
      for (int s = 0; s < 4; ++s) cm = (c + s < k) ? cm : (cm & ~(1 << s));
      const v4f a = (irow < m && cm) ? ldf4(L.W, (int64_t)irow * k + c, kvec && cm == 15, cm)
                                     : v4f{0.f, 0.f, 0.f, 0.f};
      v4f b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) b[t] = *(const v4f*)&Us[jl - j0 + t][cb + 4 * kk];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(a[s], b[t][s], acc[t]);
    }
  }

  // 3) elementwise tail
  float u2 = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (!rok[r]) continue;
    const v4f corr = {acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
    if (GF32 && fused_mgrad(P)) gm[r] = finish_mgrad(P, e[r], gr[r], gm[r], cmask);
    v4f out;
    adan4<GF32, LARS>(P, S, dt, gr[r], gm[r], corr, mm[r], vv[r], dd[r], pp[r], par[r], out, u2,
                      cmask, dleaf);
    stf4(P.exp_avg, e[r], mm[r], vec, cmask);
    stf4(P.exp_avg_sq, e[r], vv[r], vec, cmask);
    stf4(P.exp_avg_diff, e[r], dd[r], vec, cmask);
    stf4(P.prev_grad, e[r], GF32 ? gm[r] : gr[r], vec, cmask);
    if (LARS)
      stf4(P.upd, e[r], out, vec, cmask);
    else
      st4(P.p, dt, e[r], out, vec, cmask);
  }
  write_u2_slot(slots, slot, u2, red);
}

// One 16x256 tile, wholly inside an fp32 block whose rows are 16-byte
// aligned, k % 16 == 0.  A 16-row x 1 KB footprint per block streams
// measurably faster than 64 rows x 256 B.  Wave w owns columns
// j0+64w .. j0+64w+63 of all 16 rows; lane l holds rows i0+4*(l/16)+r and
// columns jl..jl+3, jl = j0+64w+4*(l%16).  The correction for those columns
// needs U_r rows private to the wave, so they are read straight from L2 in
// the MFMA B layout; the 16 rows of W are common to the four waves.
template <bool GF32, bool LARS>
__device__ __forceinline__ void apply_wide(const scao_leaf_desc& L, const scao_param_desc& P,
                                           const scao_param_stat& S, int i0, int j0, int slot,
                                           double* slots) {
  __shared__ double red[16];
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  const int k = L.k;
  const int kk = l / 16;
  const int jl = j0 + 64 * w + 4 * (l % 16);

  // 1) the streaming loads (issued in step 2: after the back-projection's
  // operands when k = 64, before them otherwise).  A fused filter's EMA goes
  // first: its keep bits are taken as soon as the back-projection allows,
  // which frees its registers for the rest of the tile.
  v4f gr[4], gm[4], mm[4], vv[4], dd[4], pp[4], par[4];
  int64_t e[4];
  const bool fmask = GF32 && (P.flags & SCAO_PF_FMASK);
  auto load_elem = [&]() {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[r] = L.off + (int64_t)(i0 + 4 * kk + r) * L.ld + jl;
      if (fmask) gm[r] = gld4_nt(P.fema + e[r]);
      gr[r] = gld4_nt((const float*)P.graw + e[r]);
      if (GF32 && !fused_mgrad(P)) gm[r] = gld4_nt((const float*)P.g + e[r]);
      mm[r] = gld4_nt(P.exp_avg + e[r]);
      vv[r] = gld4_nt(P.exp_avg_sq + e[r]);
      dd[r] = gld4_nt(P.exp_avg_diff + e[r]);
      pp[r] = gld4_nt(P.prev_grad + e[r]);
      if (!LARS) par[r] = gld4_nt((const float*)P.p + e[r]);
    }
  };

  // 2) corr = W U_r^T; reduction index c + 4*(l/16) + s for both operands
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const float* __restrict__ wrow = L.W + (int64_t)(i0 + l % 16) * k + 4 * kk;
  const float* __restrict__ urow = L.Ur + (int64_t)jl * k + 4 * kk;
  uint32_t keep = 0xffffu;   // bit 4r+t: the filter keeps element (r, t)
  auto take_keep = [&]() {
    if (fmask) {
      const float thr = *P.fthr;
      keep = 0u;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int t = 0; t < 4; ++t) keep |= (gm[r][t] >= thr ? 1u : 0u) << (4 * r + t);
    }
  };
  if (k == 64) {
    // Every operand of the back-projection goes out before the streaming
    // loads and the four chunks run straight-line, so each MFMA waits for its
    // own operands only, not for the streaming loads queued behind them (the
    // vector-memory counter completes in order).  The tile then takes about
    // 170 registers, two waves per SIMD: faster than the streaming loads
    // first at either two or three waves per SIMD (the same sums in the same
    // order).
    v4f A4[4], B4[4][4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      A4[d] = gld4(wrow + 16 * d);
#pragma unroll
      for (int t = 0; t < 4; ++t) B4[d][t] = gld4(urow + (int64_t)t * 64 + 16 * d);
    }
    load_elem();
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(A4[c][s], B4[c][t][s], acc[t]);
    take_keep();
  } else {
    load_elem();
    // operands of chunk c+16 are loaded while chunk c runs on MFMA
    v4f a = gld4(wrow), b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) b[t] = gld4(urow + (int64_t)t * k);
    take_keep();
    for (int c = 0; c < k; c += 16) {
      const bool more = c + 16 < k;
      v4f an = a, bn[4] = {b[0], b[1], b[2], b[3]};
      if (more) {
        an = gld4(wrow + c + 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) bn[t] = gld4(urow + (int64_t)t * k + c + 16);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(a[s], b[t][s], acc[t]);
      a = an;
#pragma unroll
      for (int t = 0; t < 4; ++t) b[t] = bn[t];
    }
  }

  // 3) elementwise tail
  float u2 = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const v4f corr = {acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
    if (GF32 && fused_mgrad(P)) gm[r] = finish_mgrad_bits(P, e[r], gr[r], (keep >> (4 * r)) & 15u, 15);
    v4f out;
    adan4<GF32, LARS>(P, S, SCAO_F32, gr[r], gm[r], corr, mm[r], vv[r], dd[r], pp[r], par[r], out,
                      u2, 15);
    gst4_nt(P.exp_avg + e[r], mm[r]);
    gst4_nt(P.exp_avg_sq + e[r], vv[r]);
    gst4_nt(P.exp_avg_diff + e[r], dd[r]);
    gst4_nt(P.prev_grad + e[r], GF32 ? gm[r] : gr[r]);
    // the staged update streams past the caches too: it is read back only by
    // k_lars_write, after gigabytes of other traffic, and a caching store
    // evicts the U_r rows the tiles read from L2 (C3 step 12.17 -> 11.98 ms in
    // alternating runs; the strip apply at k = 256 measured slower with it)
    if (LARS)
      gst4_nt(P.upd + e[r], out);
    else
      gst4_nt((float*)P.p + e[r], out);
  }
  write_u2_slot(slots, slot, u2, red);
}

// Wide tiles through a two-role pipeline, for ranks where the back-projection
// no longer hides under the streaming of one-tile blocks (k >= 128; at k = 64
// both kernels measure the same).  A block of eight waves takes
// SCAO_APPLY_GROUP consecutive wide tasks.  Waves 0..3 stream tile s (loads,
// Adan tail, stores) between block barriers s and s+1, then issue tile s+1's
// loads.  Waves 4..7 compute corr = W U_r^T into four LDS tile buffers, two
// tiles at a time: tiles 2q and 2q+1 of one column strip share their U_r
// rows, so one pass over them serves both (the operand loads from L2, not
// the MFMAs, bound this role).  Pair q's reduction is split in two halves,
// computed between barriers 2q-2, 2q-1 and 2q, so each barrier interval holds
// one tile's worth of MFMA work; pair 0 is done before barrier 0.  Tiles of
// different blocks or strips, and ranks other than 128 and 256, are computed
// one per half instead.  Each role
// waits only on its own memory operations (the vector-memory counter is in
// order within a wave, so an operand load queued behind the streaming loads
// would wait for them too).  Both roles use apply_wide's lane <-> element
// mapping, so a streaming wave reads exactly the 16x64 slice its partner
// wrote.  u^2 per tile: four wave partials through LDS, summed in a fixed
// order.
constexpr int CP = SCAO_APPLY_WIDE_COLS + 4;   // LDS pitch of a correction row

// One MFMA wave's 16x64 share of corr = W U_r^T: rows of W from wrow, its 64
// U_r rows from urow (lane layout as in apply_wide).  With NC > 0 (k = 16 NC)
// the reduction is fully unrolled with PD chunks of operands in flight, so
// every wait is for one chunk's loads (a loop's back edge makes the compiler
// wait for all of them); NC = 0 takes any multiple of 16 with one chunk of
// lookahead.
template <int NC>
__device__ __forceinline__ void pipe_corr(const float* __restrict__ wrow,
                                          const float* __restrict__ urow, int k, v4f (&acc)[4]) {
  if constexpr (NC > 0) {
    constexpr int PD = 4;
    v4f A[PD], B[PD][4];
#pragma unroll
    for (int d = 0; d < PD && d < NC; ++d) {
      A[d] = gld4(wrow + 16 * d);
#pragma unroll
      for (int t = 0; t < 4; ++t) B[d][t] = gld4(urow + (int64_t)t * (16 * NC) + 16 * d);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = c % PD;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(A[d][s4], B[d][t][s4], acc[t]);
      if (c + PD < NC) {
        A[d] = gld4(wrow + 16 * (c + PD));
#pragma unroll
        for (int t = 0; t < 4; ++t) B[d][t] = gld4(urow + (int64_t)t * (16 * NC) + 16 * (c + PD));
      }
    }
  } else {
    v4f a = gld4(wrow), b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) b[t] = gld4(urow + (int64_t)t * k);
    for (int c = 0; c < k; c += 16) {
      const bool more = c + 16 < k;
      v4f an = a, bn[4] = {b[0], b[1], b[2], b[3]};
      if (more) {
        an = gld4(wrow + c + 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) bn[t] = gld4(urow + (int64_t)t * k + c + 16);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16(a[s4], b[t][s4], acc[t]);
      a = an;
#pragma unroll
      for (int t = 0; t < 4; ++t) b[t] = bn[t];
    }
  }
}

// The same for two row tiles of one strip (W rows from wa and wb, one U_r
// row set), over NH chunks of a reduction of length K: every U_r load feeds
// both tiles (k = 128 and 256).
// With MID >= 0 a block barrier follows chunk MID's products: the loads of
// the chunks after it are already in flight across the barrier (a block
// barrier waits for LDS operations only), so the second half of a pair starts
// without an operand-latency bubble.
template <int K, int NH, int PD, int MID = -1>
__device__ __forceinline__ void pipe_corr2(const float* __restrict__ wa,
                                           const float* __restrict__ wb,
                                           const float* __restrict__ urow, v4f (&acc)[2][4]) {
  v4f A[PD][2], B[PD][4];
#pragma unroll
  for (int d = 0; d < PD && d < NH; ++d) {
    A[d][0] = gld4(wa + 16 * d);
    A[d][1] = gld4(wb + 16 * d);
#pragma unroll
    for (int t = 0; t < 4; ++t) B[d][t] = gld4(urow + (int64_t)t * K + 16 * d);
  }
#pragma unroll
  for (int c = 0; c < NH; ++c) {
    const int d = c % PD;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[0][t] = mfma16(A[d][0][s4], B[d][t][s4], acc[0][t]);
        acc[1][t] = mfma16(A[d][1][s4], B[d][t][s4], acc[1][t]);
      }
    if (c + PD < NH) {
      A[d][0] = gld4(wa + 16 * (c + PD));
      A[d][1] = gld4(wb + 16 * (c + PD));
#pragma unroll
      for (int t = 0; t < 4; ++t) B[d][t] = gld4(urow + (int64_t)t * K + 16 * (c + PD));
    }
    if (c == MID) __syncthreads();
  }
}

template <bool GF32, bool LARS>
__global__ __launch_bounds__(512) void k_apply_pipe(const scao_task* __restrict__ tasks, int ntasks,
                                                    const scao_leaf_desc* __restrict__ leaves,
                                                    const scao_param_desc* __restrict__ params,
                                                    const scao_param_stat* __restrict__ stat,
                                                    double* slots) {
  __shared__ __attribute__((aligned(16))) float cbuf[4][16][CP];
  __shared__ double part[2][4];
  const int wv = threadIdx.x / 64, l = threadIdx.x % 64;
  const int w = wv & 3;
  const int kk = l / 16;
  const int t0 = blockIdx.x * SCAO_APPLY_GROUP;
  const int nt = ntasks - t0 < SCAO_APPLY_GROUP ? ntasks - t0 : SCAO_APPLY_GROUP;

  if (wv >= 4) {
    // ---- MFMA role: nt + 1 barriers, as the streaming role ----
    if (nt <= 0) {
      __syncthreads();
      return;
    }
    v4f acc[2][4];
    auto zero = [&]() {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[i][t] = v4f{0.f, 0.f, 0.f, 0.f};
    };
    // tiles 2q and 2q+1 share one pass over their U_r rows
    auto paired = [&](int q) {
      if (2 * q + 1 >= nt) return false;
      const scao_task ta = tasks[t0 + 2 * q], tb = tasks[t0 + 2 * q + 1];
      return tb.idx == ta.idx && tb.b == ta.b && (leaves[ta.idx].k == 256 || leaves[ta.idx].k == 128);
    };
    // a pair's chunks (16 at k = 256, 8 at k = 128), with barrier 2q-1 after
    // the first half when MID
    auto pair = [&](int q, auto mid) {
      const scao_task ta = tasks[t0 + 2 * q], tb = tasks[t0 + 2 * q + 1];
      const scao_leaf_desc& L = leaves[ta.idx];
      const int jl = ta.b + 64 * w + 4 * (l % 16);
      zero();
      if (L.k == 256)
        pipe_corr2<256, 16, 4, decltype(mid)::value>(
            L.W + (int64_t)(ta.a + l % 16) * 256 + 4 * kk,
            L.W + (int64_t)(tb.a + l % 16) * 256 + 4 * kk, L.Ur + (int64_t)jl * 256 + 4 * kk, acc);
      else
        pipe_corr2<128, 8, 4, (decltype(mid)::value < 0 ? -1 : 3)>(
            L.W + (int64_t)(ta.a + l % 16) * 128 + 4 * kk,
            L.W + (int64_t)(tb.a + l % 16) * 128 + 4 * kk, L.Ur + (int64_t)jl * 128 + 4 * kk, acc);
    };
    // otherwise tile 2q in the first half and tile 2q+1 (if any) in the second
    auto single = [&](int q, int h) {
      if (h == 0) zero();
      if (h == 1 && 2 * q + 1 >= nt) return;
      const scao_task tk = tasks[t0 + 2 * q + h];
      const scao_leaf_desc& L = leaves[tk.idx];
      const int k = L.k;
      const int jl = tk.b + 64 * w + 4 * (l % 16);
      const float* __restrict__ wrow = L.W + (int64_t)(tk.a + l % 16) * k + 4 * kk;
      const float* __restrict__ urow = L.Ur + (int64_t)jl * k + 4 * kk;
      if (k == 256)
        pipe_corr<16>(wrow, urow, k, acc[h]);
      else if (k == 128)
        pipe_corr<8>(wrow, urow, k, acc[h]);
      else
        pipe_corr<0>(wrow, urow, k, acc[h]);
    };
    auto put = [&](int q) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int s = 2 * q + i;
        if (s < nt) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            *(v4f*)&cbuf[s & 3][4 * kk + r][64 * w + 4 * (l % 16)] =
                v4f{acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
        }
      }
    };
    using NoMid = std::integral_constant<int, -1>;
    using Mid = std::integral_constant<int, 7>;
    if (paired(0)) {
      pair(0, NoMid{});
    } else {
      single(0, 0);
      single(0, 1);
    }
    put(0);
    __syncthreads();                       // barrier 0: tiles 0 and 1 ready
    const int np = (nt + 1) / 2;
    for (int q = 1; q < np; ++q) {
      if (paired(q)) {
        pair(q, Mid{});                    // barrier 2q-1 inside
      } else {
        single(q, 0);
        __syncthreads();                   // barrier 2q-1
        single(q, 1);
      }
      put(q);                              // buffers of tiles 2q-4, 2q-3: consumed
      __syncthreads();                     // barrier 2q: tiles 2q, 2q+1 ready
    }
    for (int b = 2 * np - 1; b < nt + 1; ++b) __syncthreads();
    return;
  }

  // ---- streaming role ----
  v4f gr[4], gm[4], mm[4], vv[4], dd[4], pp[4], par[4];
  int64_t e[4];
  auto prefetch = [&](int s) {
    const scao_task tk = tasks[t0 + s];
    const scao_leaf_desc& L = leaves[tk.idx];
    const scao_param_desc& P = params[L.param];
    const int jl = tk.b + 64 * w + 4 * (l % 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[r] = L.off + (int64_t)(tk.a + 4 * kk + r) * L.ld + jl;
      gr[r] = gld4_nt((const float*)P.graw + e[r]);
      if (GF32) {
        if (!fused_mgrad(P))
          gm[r] = gld4_nt((const float*)P.g + e[r]);
        else
          gm[r] = (P.flags & SCAO_PF_FMASK) ? gld4_nt(P.fema + e[r]) : gr[r];
      }
      mm[r] = gld4_nt(P.exp_avg + e[r]);
      vv[r] = gld4_nt(P.exp_avg_sq + e[r]);
      dd[r] = gld4_nt(P.exp_avg_diff + e[r]);
      pp[r] = gld4_nt(P.prev_grad + e[r]);
      if (!LARS) par[r] = gld4_nt((const float*)P.p + e[r]);
    }
  };
  auto put_slot = [&](int s) {
    const int slot = tasks[t0 + s].slot;
    if (slot < 0) return;
    const double u2 = ((part[s & 1][0] + part[s & 1][1]) + part[s & 1][2]) + part[s & 1][3];
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 0] = 0.0;
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 1] = 0.0;
    slots[(int64_t)slot * SCAO_SLOT_WIDTH + 2] = u2;
  };
  if (nt > 0) prefetch(0);
  for (int s = 0; s < nt; ++s) {
    __syncthreads();     // corr(s) in cbuf[s & 3]; tile s-1's partials in part
    if (s > 0 && w == 0 && l == 0) put_slot(s - 1);
    const scao_task tk = tasks[t0 + s];
    const scao_leaf_desc& L = leaves[tk.idx];
    const scao_param_desc& P = params[L.param];
    const scao_param_stat& S = stat[L.param];
    float u2 = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const v4f corr = *(const v4f*)&cbuf[s & 3][4 * kk + r][64 * w + 4 * (l % 16)];
      if (GF32 && fused_mgrad(P)) gm[r] = finish_mgrad(P, e[r], gr[r], gm[r], 15);
      v4f out;
      adan4<GF32, LARS>(P, S, SCAO_F32, gr[r], gm[r], corr, mm[r], vv[r], dd[r], pp[r], par[r],
                        out, u2, 15);
      gst4_nt(P.exp_avg + e[r], mm[r]);
      gst4_nt(P.exp_avg_sq + e[r], vv[r]);
      gst4_nt(P.exp_avg_diff + e[r], dd[r]);
      gst4_nt(P.prev_grad + e[r], GF32 ? gm[r] : gr[r]);
      if (LARS)
        gst4(P.upd + e[r], out);
      else
        gst4_nt((float*)P.p + e[r], out);
    }
    const double wsum = wave_sum((double)u2);
    if (l == 0) part[s & 1][w] = wsum;
    if (s + 1 < nt) prefetch(s + 1);
  }
  __syncthreads();       // the last tile's partials
  if (nt > 0 && w == 0 && l == 0) put_slot(nt - 1);
}

// ---------------------------------------------- strip-resident apply ---
// Blocks of rank k = 128 or 256.  A task is a run of up to SCAO_APPLY_GROUP
// tiles of one column strip, SW columns x TR rows each (strip_shape: 64 x 128
// at k = 256, 128 x 64 at k = 128), going down the block.  The strip's U_r rows stay in LDS for
// the whole run, so the back-projection reads only W rows from L2 instead of
// every wave refetching U_r per tile.  Per workgroup:
//   waves NS.. (MFMA role): corr(s) = W[rows of tile s, :] U_r[strip, :]^T,
//     32 rows x 64 columns per wave (two 16-row halves sharing each B
//     operand read from LDS), A operands from L2 with chunks of lookahead;
//   waves 0..NS-1 (streaming role, 16 rows x 64 columns each): tile s's loads
//     were issued during tile s-1; once corr(s) is published they run the
//     Phase-2 tail, store, and issue tile s+1's loads.
// The matrix cores and the Phase-2 arithmetic share each SIMD's issue, so the
// products run as six bf16 MFMAs over exact three-way splits (mfma_x6, fp32
// accuracy): W's planes come from scao_kron_lift (Wb), U_r's are split once
// per run into LDS.  Three planes of U_r leave LDS for one correction
// buffer: the streaming waves copy corr(s) to registers and release it (a
// second barrier per tile) before the MFMA waves write corr(s+1).  The GF32
// variants have no registers for that copy; they keep fp32 MFMAs, U_r in
// LDS as fp32 and two correction buffers.
// U_r row r of the strip sits at LDS row 64(r/64) + 16(r%4) + (r%64)/4, so
// that a lane's four B rows (columns 4j + t of its 64-column group) are 16
// rows apart, and the row pitch is 16 bytes past a multiple of 128: a 16-lane
// read phase touches 16 distinct bank groups.
__host__ __device__ constexpr int strip_pitch(int k) { return k + 4 + ((32 - k % 32) % 32); }
__host__ __device__ constexpr int strip_pitch_bf(int k) { return k + 8 + ((64 - k % 64) % 64); }
// Tile shape per rank: SW columns x TR rows (8192 elements), NS = 8
// streaming waves (16 x 64 elements each) and NM = 4 MFMA waves (32 x 64
// each), about 135 KB of LDS: one workgroup per CU.  SW = 64 at k = 256 (what
// LDS holds of U_r), 128 at k = 128: each W row a tile reads then serves 128
// columns.  (64 x 64 tiles at k = 128, two workgroups per CU, measured 10%
// slower: twice the W bytes per element.)
template <int K> struct strip_shape {
  static constexpr int SW = K == 256 ? 64 : 128, TR = 8192 / SW;
  static constexpr int NS = TR * SW / 1024, NM = NS / 2, NT = 64 * (NS + NM);
  // LDS: U_r as three bf16 planes and one correction buffer, or (GF32) as
  // fp32 and two buffers
  static constexpr int lds_bytes(bool bf) {
    return bf ? 3 * SW * strip_pitch_bf(K) * 2 + TR * (SW + 4) * 4
              : SW * strip_pitch(K) * 4 + 2 * TR * (SW + 4) * 4;
  }
};
__device__ __forceinline__ int strip_row(int r) { return 64 * (r / 64) + 16 * (r % 4) + (r % 64) / 4; }

// fp32: corr for rows wa (and wb, 16 rows on) against the LDS strip (lane
// base ub, row pitch pk), k = 16 NC.
template <int NC, int PD>
__device__ __forceinline__ void strip_corr(const float* __restrict__ wa,
                                           const float* __restrict__ wb, const float* ub, int pk,
                                           v4f (&acc)[2][4]) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[h][t] = v4f{0.f, 0.f, 0.f, 0.f};
  v4f A[PD][2], B[2][4];
#pragma unroll
  for (int d = 0; d < PD && d < NC; ++d) {
    A[d][0] = gld4(wa + 16 * d);
    A[d][1] = gld4(wb + 16 * d);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) B[0][t] = *(const v4f*)(ub + 16 * t * pk);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d = c % PD, cur = c & 1;
    if (c + 1 < NC) {
#pragma unroll
      for (int t = 0; t < 4; ++t) B[cur ^ 1][t] = *(const v4f*)(ub + 16 * t * pk + 16 * (c + 1));
    }
    // chunk c+1's LDS reads go out before chunk c's products (a second
    // register set), so their latency hides behind 32 MFMAs
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[0][t] = mfma16(A[d][0][s4], B[cur][t][s4], acc[0][t]);
        acc[1][t] = mfma16(A[d][1][s4], B[cur][t][s4], acc[1][t]);
      }
    if (c + PD < NC) {
      A[d][0] = gld4(wa + 16 * (c + PD));
      A[d][1] = gld4(wb + 16 * (c + PD));
    }
    // keep chunk c+PD's loads here: the scheduler would otherwise sink
    // them next to their use and expose an L2 round trip per chunk
    __builtin_amdgcn_sched_barrier(0);
  }
}

// bf16 planes: the A operands of one 32-k chunk (both halves, three planes).
struct strip_a {
  bf3 a[2];
};
__device__ __forceinline__ v8bf gld8bf(const uint16_t* p) {
  return __builtin_bit_cast(v8bf, gld4((const float*)p));
}
// wp[h][p]: the lane's row of plane p for half h (column 8*(l/16) included)
__device__ __forceinline__ void strip_load_a(strip_a& A, const uint16_t* const (&wp)[2][3], int c) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    A.a[h].h = gld8bf(wp[h][0] + 32 * c);
    A.a[h].m = gld8bf(wp[h][1] + 32 * c);
    A.a[h].l = gld8bf(wp[h][2] + 32 * c);
  }
}
__device__ __forceinline__ bf3 strip_load_b(const uint16_t* ub, int plane, int pk, int t, int c) {
  const uint16_t* p = ub + 16 * t * pk + 32 * c;
  bf3 b;
  b.h = *(const v8bf*)p;
  b.m = *(const v8bf*)(p + plane);
  b.l = *(const v8bf*)(p + 2 * plane);
  return b;
}

// bf16: corr for the rows of wp (two 16-row halves) against the LDS planes
// (lane base ub, plane stride PLC, row pitch PKC), k = K, with the first PD
// chunks of A already in A[0..PD-1]; the chunk loop is unrolled in
// rotations of PD (every address offset a constant).
template <int K, int PKC, int PLC, int PD>
__device__ __forceinline__ void strip_corr_bf(strip_a (&A)[PD], const uint16_t* const (&wp)[2][3],
                                              const uint16_t* ub, v4f (&acc)[2][4]) {
  constexpr int pk = PKC, plane = PLC, nc = K / 32;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[h][t] = v4f{0.f, 0.f, 0.f, 0.f};
  bf3 B[2];
  B[0] = strip_load_b(ub, plane, pk, 0, 0);
#pragma unroll
  for (int c0 = 0; c0 < nc; c0 += PD) {
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      const int c = c0 + d;
      if (c < nc) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int cur = t & 1;
          if (t < 3)
            B[cur ^ 1] = strip_load_b(ub, plane, pk, t + 1, c);
          else if (c + 1 < nc)
            B[cur ^ 1] = strip_load_b(ub, plane, pk, 0, c + 1);
          // the next B goes out before these products (its own registers)
          __builtin_amdgcn_sched_barrier(0);
          acc[0][t] = mfma_x6(A[d].a[0], B[cur], acc[0][t]);
          acc[1][t] = mfma_x6(A[d].a[1], B[cur], acc[1][t]);
        }
        if (c + PD < nc) strip_load_a(A[d], wp, c + PD);
        // chunk c+PD's loads stay here, PD chunks ahead of their use
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

template <bool GF32, bool LARS, int K>
__global__ __launch_bounds__(strip_shape<K>::NT) void k_apply_strip(const scao_task* __restrict__ tasks,
                                                     const scao_leaf_desc* __restrict__ leaves,
                                                     const scao_param_desc* __restrict__ params,
                                                     const scao_param_stat* __restrict__ stat,
                                                     double* slots) {
  constexpr bool BF = !GF32;      // bf16 products, one correction buffer
  using SH = strip_shape<K>;
  constexpr int SW = SH::SW, TR = SH::TR, NS = SH::NS, NM = SH::NM;
  constexpr int CB = SW + 4;      // LDS pitch of a correction row
  constexpr int NBUF = BF ? 1 : 2;
  constexpr int CBYTES = NBUF * TR * CB * 4;
  constexpr int LDSB = SH::lds_bytes(BF);
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDSB];
  __shared__ double part[2][NS];
  float(*cbuf)[TR][CB] = (float(*)[TR][CB])(lds + LDSB - CBYTES);
  const int wv = threadIdx.x / 64, l = threadIdx.x % 64;
  const int kk = l / 16;
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc& L = leaves[tk.idx];
  const int k = L.k;             // == K past the guard below
  constexpr int pk = BF ? strip_pitch_bf(K) : strip_pitch(K);
  const int mw = L.m - L.m % TR;
  int nt = (mw - tk.a) / TR;
  nt = nt < SCAO_APPLY_GROUP ? nt : SCAO_APPLY_GROUP;
  if (nt <= 0) return;   // uniform over the workgroup
  if (k != K || (BF && !L.Wb)) {
    // outside the kernel's contract (the engine never sends this): make the
    // run's norms NaN rather than write anything
    if (threadIdx.x < nt && tk.slot >= 0)
      slots[(int64_t)(tk.slot + threadIdx.x) * SCAO_SLOT_WIDTH + 2] = __builtin_nan("");
    return;
  }

  if (wv >= NS) {
    // ---- MFMA role ----
    constexpr int RP = TR / 32;   // 32-row groups of a tile
    const int mwv = wv - NS, rp = mwv % RP, cg = mwv / RP;
    constexpr int q4 = K / 4;
    auto put = [&](int buf, v4f (&acc)[2][4]) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *(v4f*)&cbuf[buf][32 * rp + 16 * h + 4 * kk + r][64 * cg + 4 * (l % 16)] =
              v4f{acc[h][0][r], acc[h][1][r], acc[h][2][r], acc[h][3][r]};
    };
    if constexpr (BF) {
      // barriers: A, X_0, then (Y_{s-1}, X_s) for s = 1..nt
      uint16_t* urb = (uint16_t*)lds;
      constexpr int plane = SW * pk;
      for (int q = threadIdx.x - 64 * NS; q < SW * q4; q += 64 * NM) {
        const int r = q / q4, c = q - r * q4;
        const v4f x = gld4(L.Ur + (int64_t)(tk.b + r) * K + 4 * c);
        v2u h, m, lo;
        split4_pk(x, h, m, lo);
        uint16_t* d = urb + strip_row(r) * pk + 4 * c;
        *(v2u*)d = h;
        *(v2u*)(d + plane) = m;
        *(v2u*)(d + 2 * plane) = lo;
      }
      const int64_t mk = (int64_t)L.m * K;
      const uint16_t* ub = urb + (64 * cg + l % 16) * pk + 8 * kk;
      constexpr int PD = K == 256 ? 2 : 3;   // chunks of A lookahead (registers)
      strip_a A[PD];
      const uint16_t* wp[2][3];
      auto rows = [&](int s) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int q = 0; q < 3; ++q)
            wp[h][q] = L.Wb + q * mk + (int64_t)(tk.a + s * TR + 32 * rp + 16 * h + l % 16) * K +
                       8 * kk;
      };
      auto first = [&](int s) {
        rows(s);
#pragma unroll
        for (int d = 0; d < PD; ++d) strip_load_a(A[d], wp, d);
      };
      auto corr = [&](int s, v4f (&acc)[2][4]) {
        strip_corr_bf<K, pk, plane, PD>(A, wp, ub, acc);
      };
      first(0);
      __syncthreads();                                        // A: U_r planes in LDS
      {
        v4f acc[2][4];
        corr(0, acc);
        put(0, acc);
      }
      __syncthreads();                                        // X_0: corr(0) published
      for (int s = 1; s <= nt; ++s) {
        if (s < nt) first(s);                                 // loads in flight across Y
        __syncthreads();                                      // Y_{s-1}: corr(s-1) copied
        if (s < nt) {
          v4f acc[2][4];
          corr(s, acc);
          put(0, acc);
        }
        __syncthreads();                                      // X_s: corr(s) published
      }
    } else {
      // barriers: A, then X_s for s = 0..nt
      float* ur = (float*)lds;
      for (int q = threadIdx.x - 64 * NS; q < SW * q4; q += 64 * NM) {
        const int r = q / q4, c = q - r * q4;
        *(v4f*)&ur[strip_row(r) * pk + 4 * c] = gld4(L.Ur + (int64_t)(tk.b + r) * K + 4 * c);
      }
      __syncthreads();                                        // A: U_r strip in LDS
      const float* ub = &ur[(64 * cg + l % 16) * pk + 4 * kk];
      for (int s = 0; s < nt; ++s) {
        v4f acc[2][4];
        const float* __restrict__ wa =
            L.W + (int64_t)(tk.a + s * TR + 32 * rp + l % 16) * K + 4 * kk;
        const float* __restrict__ wb = wa + (int64_t)16 * K;
        strip_corr<K / 16, 6>(wa, wb, ub, pk, acc);
        put(s & 1, acc);
        __syncthreads();                                      // X_s: corr(s) published
      }
      __syncthreads();                                        // X_nt
    }
    return;
  }

  // ---- streaming role ----
  constexpr int RG = TR / 16;     // 16-row groups of a tile
  const int w = wv, rg = w % RG, cg = w / RG;
  const scao_param_desc& P = params[L.param];
  const scao_param_stat& S = stat[L.param];
  v4f gr[4], gm[4], mm[4], vv[4], dd[4], pp[4], par[4];
  int64_t e[4];
  const int jc = tk.b + 64 * cg + 4 * (l % 16);
  auto prefetch = [&](int s) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[r] = L.off + (int64_t)(tk.a + s * TR + 16 * rg + 4 * kk + r) * L.ld + jc;
      gr[r] = gld4_nt((const float*)P.graw + e[r]);
      if (GF32) {
        if (!fused_mgrad(P))
          gm[r] = gld4_nt((const float*)P.g + e[r]);
        else
          gm[r] = (P.flags & SCAO_PF_FMASK) ? gld4_nt(P.fema + e[r]) : gr[r];
      }
      mm[r] = gld4_nt(P.exp_avg + e[r]);
      vv[r] = gld4_nt(P.exp_avg_sq + e[r]);
      dd[r] = gld4_nt(P.exp_avg_diff + e[r]);
      pp[r] = gld4_nt(P.prev_grad + e[r]);
      if (!LARS) par[r] = gld4_nt((const float*)P.p + e[r]);
    }
  };
  auto put_slot = [&](int s) {
    if (tk.slot < 0) return;
    const double* q = part[s & 1];
    double u2 = q[0];
#pragma unroll
    for (int i = 1; i < NS; ++i) u2 += q[i];   // fixed order
    const int64_t slot = tk.slot + s;
    slots[slot * SCAO_SLOT_WIDTH + 0] = 0.0;
    slots[slot * SCAO_SLOT_WIDTH + 1] = 0.0;
    slots[slot * SCAO_SLOT_WIDTH + 2] = u2;
  };
  prefetch(0);
  __syncthreads();                                            // A
  __syncthreads();                                            // X_0: corr(0)
  for (int s = 0; s < nt; ++s) {
    if (s > 0 && w == 0 && l == 0) put_slot(s - 1);
    v4f cr[4];
    if constexpr (BF) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        cr[r] = *(const v4f*)&cbuf[0][16 * rg + 4 * kk + r][64 * cg + 4 * (l % 16)];
      __syncthreads();                                        // Y_s: the buffer is free
    }
    float u2 = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const v4f corr =
          BF ? cr[r] : *(const v4f*)&cbuf[s & 1][16 * rg + 4 * kk + r][64 * cg + 4 * (l % 16)];
      if (GF32 && fused_mgrad(P)) gm[r] = finish_mgrad(P, e[r], gr[r], gm[r], 15);
      v4f out;
      adan4<GF32, LARS>(P, S, SCAO_F32, gr[r], gm[r], corr, mm[r], vv[r], dd[r], pp[r], par[r],
                        out, u2, 15);
      gst4_nt(P.exp_avg + e[r], mm[r]);
      gst4_nt(P.exp_avg_sq + e[r], vv[r]);
      gst4_nt(P.exp_avg_diff + e[r], dd[r]);
      gst4_nt(P.prev_grad + e[r], GF32 ? gm[r] : gr[r]);
      if (LARS)
        gst4(P.upd + e[r], out);
      else
        gst4_nt((float*)P.p + e[r], out);
    }
    const double wsum = wave_sum((double)u2);
    if (l == 0) part[s & 1][w] = wsum;
    if (s + 1 < nt) prefetch(s + 1);
    __syncthreads();                                          // X_{s+1}
  }
  if (w == 0 && l == 0) put_slot(nt - 1);
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
template <bool FAST, bool DO_P, int CR = 64>
__global__ __launch_bounds__(256) void k_project(const scao_task* __restrict__ tasks,
                                                 const scao_leaf_desc* __restrict__ leaves,
                                                 const scao_param_desc* __restrict__ params,
                                                 double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  project_tile<FAST, DO_P, CR>(L, params[L.param], tk.a, tk.b, tk.slot, slots);
}
template <bool DO_P, int CR, int NT>
__global__ __launch_bounds__(NT) void k_project_x6(const scao_task* __restrict__ tasks,
                                                   const scao_leaf_desc* __restrict__ leaves,
                                                   const scao_param_desc* __restrict__ params,
                                                   double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  project_tile_x6<DO_P, CR, NT>(L, params[L.param], tk.a, tk.b, tk.slot, slots);
}
// two waves per SIMD: the bf16-product tiles fit 256 registers without spilling
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_delta(
    const scao_task* __restrict__ tasks, const scao_leaf_desc* __restrict__ leaves,
    const scao_param_desc* __restrict__ params, double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  __shared__ __attribute__((aligned(16))) float Ps[3][64][DP];
  __shared__ double red[16];
  if (L.flags & SCAO_LF_DIAG) {
    diag_leaf_reduce(L, params[L.param], tk.a, tk.b, tk.slot, slots, red);
    return;
  }
  const bool fast = (L.flags & SCAO_LF_VEC4) && (L.k % 4 == 0) && tk.a + 64 <= L.k &&
                    tk.b + 64 <= L.k && (L.n % 64 == 0);
  if (fast && L.n % 128 == 0)
    delta_tile<true, true>(L, params[L.param].eps, tk.a, tk.b, tk.slot, slots, Ps, red);
  else if (fast)
    delta_tile<true>(L, params[L.param].eps, tk.a, tk.b, tk.slot, slots, Ps, red);
  else
    delta_tile<false>(L, params[L.param].eps, tk.a, tk.b, tk.slot, slots, Ps, red);
}
// two waves per SIMD: the bf16-product tiles fit 256 registers without spilling
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_lift(
    const scao_task* __restrict__ tasks, const scao_leaf_desc* __restrict__ leaves) {
  __shared__ __attribute__((aligned(16))) float Ps[4][64][DP];
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  if (lift_x6_ok(L, tk.a, tk.b))
    lift_tile_x6(L, tk.a, tk.b, Ps);
  else
    lift_tile(L, tk.a, tk.b);
}
template <bool GF32, bool LARS, bool FAST>
__global__ __launch_bounds__(256) void k_apply(const scao_task* __restrict__ tasks,
                                               const scao_leaf_desc* __restrict__ leaves,
                                               const scao_param_desc* __restrict__ params,
                                               const scao_param_stat* __restrict__ stat,
                                               double* slots) {
  const scao_task tk = tasks[blockIdx.x];
  const scao_leaf_desc L = leaves[tk.idx];
  if (FAST)
    apply_wide<GF32, LARS>(L, params[L.param], stat[L.param], tk.a, tk.b, tk.slot, slots);
  else
    apply_tile<GF32, LARS>(L, params[L.param], stat[L.param], tk.a, tk.b, tk.slot, slots);
}

// single-block reference operator (descriptors by value, tiles from blockIdx)
__global__ __launch_bounds__(256) void k_project_one(scao_leaf_desc L, scao_param_desc P) {
  const int strips = (L.n + SCAO_PROJ_COLS - 1) / SCAO_PROJ_COLS;
  project_tile<false, false>(L, P, (blockIdx.x % strips) * SCAO_PROJ_COLS,
                             (blockIdx.x / strips) * 64, -1, nullptr);
}
__global__ __launch_bounds__(256) void k_delta_one(scao_leaf_desc L) {
  __shared__ __attribute__((aligned(16))) float Ps[3][64][DP];
  __shared__ double red[16];
  const int tiles = (L.k + 63) / 64;
  delta_tile<false>(L, 1e-8f, (blockIdx.x / tiles) * 64, (blockIdx.x % tiles) * 64, -1, nullptr,
                    Ps, red);
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
                                 const scao_param_desc* params, double* slots, int variant,
                                 void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_kron_project: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && leaves && params && slots, "scao_kron_project: null pointer");
  SCAO_CHECK_ARG(variant >= 0 && variant < 12 && (variant < 4 || (variant & 1)) &&
                     (variant & 12) != 12,
                 "scao_kron_project: bad variant %d", variant);
  hipStream_t s = (hipStream_t)stream;
  dim3 g(ntasks), b(256);
  if (variant & 1) {
    const dim3 b512(512), b128(X6_NT128);
    switch (variant) {
      case 1: hipLaunchKernelGGL((k_project_x6<false, 64, 256>), g, b, 0, s, tasks, leaves, params, slots); break;
      case 3: hipLaunchKernelGGL((k_project_x6<true, 64, 256>), g, b, 0, s, tasks, leaves, params, slots); break;
      case 5: hipLaunchKernelGGL((k_project_x6<false, 128, X6_NT128>), g, b128, 0, s, tasks, leaves, params, slots); break;
      case 7: hipLaunchKernelGGL((k_project_x6<true, 128, X6_NT128>), g, b128, 0, s, tasks, leaves, params, slots); break;
      case 9: hipLaunchKernelGGL((k_project_x6<false, 256, 512>), g, b512, 0, s, tasks, leaves, params, slots); break;
      default: hipLaunchKernelGGL((k_project_x6<true, 256, 512>), g, b512, 0, s, tasks, leaves, params, slots); break;
    }
    SCAO_LAUNCH_CHECK("scao_kron_project");
    return SCAO_OK;
  }
  SCAO_CHECK_ARG(variant < 8, "scao_kron_project: variant %d needs the bf16 projection", variant);
  switch (variant) {
    case 0: hipLaunchKernelGGL((k_project<false, false>), g, b, 0, s, tasks, leaves, params, slots); break;
    case 1: hipLaunchKernelGGL((k_project<true, false>), g, b, 0, s, tasks, leaves, params, slots); break;
    case 2: hipLaunchKernelGGL((k_project<false, true>), g, b, 0, s, tasks, leaves, params, slots); break;
    case 3: hipLaunchKernelGGL((k_project<true, true>), g, b, 0, s, tasks, leaves, params, slots); break;
    case 5: hipLaunchKernelGGL((k_project<true, false, 128>), g, b, 0, s, tasks, leaves, params, slots); break;
    default: hipLaunchKernelGGL((k_project<true, true, 128>), g, b, 0, s, tasks, leaves, params, slots); break;
  }
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
                               double* slots, int variant, void* stream) {
  SCAO_CHECK_ARG(ntasks >= 0, "scao_kron_apply: ntasks < 0");
  if (ntasks == 0) return SCAO_OK;
  SCAO_CHECK_ARG(tasks && leaves && params && stat && slots, "scao_kron_apply: null pointer");
  SCAO_CHECK_ARG(variant >= 0 && variant < 64 && (variant < 8 || (variant & 4)),
                 "scao_kron_apply: bad variant %d", variant);
  hipStream_t s = (hipStream_t)stream;
  if (variant & 16) {
    const dim3 gs(ntasks);
#define SCAO_APPLY_STRIP(GF, LA, KR)                                                          \
  hipLaunchKernelGGL((k_apply_strip<GF, LA, KR>), gs, dim3(strip_shape<KR>::NT), 0, s, tasks, \
                     leaves, params, stat, slots)
    if (variant & 32) {
      switch (variant & 3) {
        case 0: SCAO_APPLY_STRIP(false, false, 128); break;
        case 1: SCAO_APPLY_STRIP(true, false, 128); break;
        case 2: SCAO_APPLY_STRIP(false, true, 128); break;
        default: SCAO_APPLY_STRIP(true, true, 128); break;
      }
    } else {
      switch (variant & 3) {
        case 0: SCAO_APPLY_STRIP(false, false, 256); break;
        case 1: SCAO_APPLY_STRIP(true, false, 256); break;
        case 2: SCAO_APPLY_STRIP(false, true, 256); break;
        default: SCAO_APPLY_STRIP(true, true, 256); break;
      }
    }
#undef SCAO_APPLY_STRIP
    SCAO_LAUNCH_CHECK("scao_kron_apply");
    return SCAO_OK;
  }
  if (variant & 8) {
    const dim3 gp((ntasks + SCAO_APPLY_GROUP - 1) / SCAO_APPLY_GROUP), bp(512);
#define SCAO_APPLY_PIPE(GF, LA) \
  hipLaunchKernelGGL((k_apply_pipe<GF, LA>), gp, bp, 0, s, tasks, ntasks, leaves, params, stat, slots)
    switch (variant & 3) {
      case 0: SCAO_APPLY_PIPE(false, false); break;
      case 1: SCAO_APPLY_PIPE(true, false); break;
      case 2: SCAO_APPLY_PIPE(false, true); break;
      default: SCAO_APPLY_PIPE(true, true); break;
    }
#undef SCAO_APPLY_PIPE
    SCAO_LAUNCH_CHECK("scao_kron_apply");
    return SCAO_OK;
  }
  dim3 g(ntasks), b(256);
#define SCAO_APPLY(GF, LA, FA) \
  hipLaunchKernelGGL((k_apply<GF, LA, FA>), g, b, 0, s, tasks, leaves, params, stat, slots)
  switch (variant) {
    case 0: SCAO_APPLY(false, false, false); break;
    case 1: SCAO_APPLY(true, false, false); break;
    case 2: SCAO_APPLY(false, true, false); break;
    case 3: SCAO_APPLY(true, true, false); break;
    case 4: SCAO_APPLY(false, false, true); break;
    case 5: SCAO_APPLY(true, false, true); break;
    case 6: SCAO_APPLY(false, true, true); break;
    default: SCAO_APPLY(true, true, true); break;
  }
#undef SCAO_APPLY
  SCAO_LAUNCH_CHECK("scao_kron_apply");
  return SCAO_OK;
}

extern "C" int64_t scao_fused_kronecker_workspace(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return (k * n + k * k + m * k) * (int64_t)sizeof(float);
}

namespace {

// The four launches of the reference operator over one block, with the
// block's T, Delta and W in the k*n + k*k + m*k floats at ws.
int launch_fused_kronecker(const float* U_l, const float* s_l_inv4, const float* U_r,
                           const float* s_r_inv4, const float* G, int64_t ldG, float* out,
                           int64_t m, int64_t n, int64_t k, float* ws, hipStream_t s) {
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

// Scratch of the no-allocation entry point: one copy per GPU, alive until the
// process ends.  Host code never uses the array's name as an address (on the
// host it is only a stand-in for the symbol): each device's address comes
// from hipGetSymbolAddress, fetched once with that device current.
static __device__ __align__(256) float scratch[SCAO_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The array of the current device, which must be the device of `stream` (a
// non-null stream of another GPU is rejected: its kernels would be handed an
// address in the wrong GPU's copy).
int scratch_for_current_device(hipStream_t stream, float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    scao_set_error("scao_fused_kronecker_precond_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return SCAO_ERR_HIP;
  }
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) {
      scao_set_error("scao_fused_kronecker_precond_noalloc: hipStreamGetDevice: %s",
                     hipGetErrorString(e));
      return SCAO_ERR_HIP;
    }
    if ((int)sdev != dev) {
      scao_set_error("scao_fused_kronecker_precond_noalloc: stream of device %d while device %d "
                     "is current (make the stream's device current)", (int)sdev, dev);
      return SCAO_ERR_INVALID;
    }
  }
  if (dev < 0 || dev >= kMaxDevices) {
    scao_set_error("scao_fused_kronecker_precond_noalloc: device %d out of range", dev);
    return SCAO_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      scao_set_error("scao_fused_kronecker_precond_noalloc: hipGetSymbolAddress: %s",
                     hipGetErrorString(e));
      return SCAO_ERR_HIP;
    }
    g_scratch_ptr[dev] = (float*)p;
  }
  *out = g_scratch_ptr[dev];
  return SCAO_OK;
}

}  // namespace

#define SCAO_FUSED_ARGS_CHECK(name)                                                          \
  SCAO_CHECK_ARG(U_l && s_l_inv4 && U_r && s_r_inv4 && G && out, name ": null pointer");   \
  SCAO_CHECK_ARG(m > 0 && n > 0 && k > 0 && ldG >= n,                                      \
                 name ": bad shape m=%lld n=%lld k=%lld ldG=%lld", (long long)m,           \
                 (long long)n, (long long)k, (long long)ldG);                              \
  SCAO_CHECK_ARG(m < (1LL << 31) && n < (1LL << 31) && k <= 4096, name ": dimension too large")

extern "C" int scao_fused_kronecker_precond(const float* U_l, const float* s_l_inv4,
                                            const float* U_r, const float* s_r_inv4,
                                            const float* G, int64_t ldG, float* out, int64_t m,
                                            int64_t n, int64_t k, void* workspace,
                                            void* stream) {
  SCAO_CHECK_ARG(workspace, "scao_fused_kronecker_precond: null pointer");
  SCAO_FUSED_ARGS_CHECK("scao_fused_kronecker_precond");
  return launch_fused_kronecker(U_l, s_l_inv4, U_r, s_r_inv4, G, ldG, out, m, n, k,
                                (float*)workspace, (hipStream_t)stream);
}

extern "C" int scao_fused_kronecker_precond_noalloc(const float* U_l, const float* s_l_inv4,
                                                    const float* U_r, const float* s_r_inv4,
                                                    const float* G, int64_t ldG, float* out,
                                                    int64_t m, int64_t n, int64_t k,
                                                    void* stream) {
  SCAO_FUSED_ARGS_CHECK("scao_fused_kronecker_precond_noalloc");
  const int64_t need = scao_fused_kronecker_workspace(m, n, k);
  SCAO_CHECK_ARG(need <= (int64_t)SCAO_NOALLOC_SCRATCH_BYTES,
                 "scao_fused_kronecker_precond_noalloc: m=%lld n=%lld k=%lld needs %lld bytes "
                 "of scratch, above the %lld-byte maximum (use scao_fused_kronecker_precond "
                 "with a workspace)",
                 (long long)m, (long long)n, (long long)k, (long long)need,
                 (long long)SCAO_NOALLOC_SCRATCH_BYTES);
  float* ws = nullptr;
  const int rc = scratch_for_current_device((hipStream_t)stream, &ws);
  if (rc != SCAO_OK) return rc;
  return launch_fused_kronecker(U_l, s_l_inv4, U_r, s_r_inv4, G, ldG, out, m, n, k, ws,
                                (hipStream_t)stream);
}
