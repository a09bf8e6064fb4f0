/*
 * scao_amd.h -- C ABI of the MI355X (gfx950) SCAO optimizer-step library.
 *
 * Plain C: device pointers, sizes and a hipStream_t passed as void*.  No
 * torch types cross this boundary.  Every entry point launches on the stream
 * it is given, allocates nothing, never synchronises the host, and returns
 * SCAO_OK or an error code; scao_last_error() gives the message of the last
 * failure on the calling thread.  Callers own every buffer (inputs, outputs,
 * scratch).  All floating-point state is float32 unless noted.
 *
 * Reference interfaces replaced (whispering3/scao):
 *   scao_fused_kronecker_precond  <- scao.cuda.fused_kronecker_precond
 *                                    (scao/cuda/__init__.py:149-187; fallback :78-99;
 *                                     pybind scao/cuda/low_rank_ops.cu:388-398)
 *   scao_int8_ema_update          <- scao.cuda.int8_ema_update
 *                                    (scao/cuda/__init__.py:231-266; fallback :122-142)
 *   scao_kron_project/delta/lift/apply, scao_step_finalize, scao_lars_write,
 *   scao_adam_step, scao_diag_reduce/apply
 *                                 <- the per-parameter Python loop of
 *                                    SCAO._step_group (scao/optimizer.py:509-645)
 *                                    with SparsePreconditioner.precondition and
 *                                    natural_grad_norm (scao/preconditioner.py:457-564)
 *                                    and SCAO._lars_scale/_curvature_clip
 *                                    (scao/optimizer.py:371-377, 667-678), batched
 *                                    over every parameter and Kronecker block
 *   scao_gram_ema / scao_requant / scao_eig_prep / scao_diag_ema
 *                                 <- SparsePreconditioner.update_curvature
 *                                    (scao/preconditioner.py:297-361, int8 core :342-350)
 *                                    and the dequantise/debias/Tikhonov part of
 *                                    _update_eigenfactors (:381-406)
 */
#ifndef SCAO_AMD_H
#define SCAO_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SCAO_ABI_VERSION 12

enum scao_status { SCAO_OK = 0, SCAO_ERR_INVALID = 1, SCAO_ERR_HIP = 2 };
enum scao_dtype { SCAO_F32 = 0, SCAO_BF16 = 1, SCAO_F16 = 2 };

/* scao_param_desc.flags */
#define SCAO_PF_DECAY 1  /* multiply the parameter by `decay` (weight_decay != 0)   */
#define SCAO_PF_LARS  2  /* LARS trust ratio (lars_coeff > 0): stage the update     */
#define SCAO_PF_CLIP  4  /* curvature clip against `tau` (tau is not None)          */
#define SCAO_PF_GSNR  8  /* gSNR mask on the update                                 */
#define SCAO_PF_DIAG  16 /* diagonal-mode preconditioner (1-D or degenerate 2-D)    */
#define SCAO_PF_NORM  32 /* accumulate ||g||^2 for the global grad-norm EMA         */
#define SCAO_PF_GF32  64 /* the moments see another gradient than `graw`: the fp32
                            buffer `g`, or with FMASK/FNOISE one formed in-kernel   */
#define SCAO_PF_ALIGNED 128 /* every pointer of the param is 16-byte aligned       */
#define SCAO_PF_FMASK 256   /* moment grad = fp32(graw) * (fema >= *fthr): the sparse
                               filter's mask (scao_sparse_filter with out == NULL)  */
#define SCAO_PF_FNOISE 512  /* moment grad += fp32(fnoise * z), z ~ N(0,1) drawn as
                               scao_sparse_filter draws it from *fseed              */

/* One parameter of a batched step.  Scalars arrive already rounded the way
 * the reference rounds a Python float meeting a float32 tensor. */
typedef struct scao_param_desc {
  void* p;                  /* parameter storage (dtype), contiguous             */
  const void* g;            /* gradient for the moments (dtype, or fp32 with      */
                            /* SCAO_PF_GF32), contiguous                         */
  const void* graw;         /* raw p.grad (dtype): preconditioner, norms         */
  float* exp_avg;           /* numel                                             */
  float* exp_avg_sq;
  float* exp_avg_diff;
  float* prev_grad;
  float* upd;               /* LARS staging of the update (numel) or NULL        */
  const float* diag_ema;    /* diagonal-mode curvature (numel) or NULL           */
  const float* fema;        /* SCAO_PF_FMASK: the filter's magnitude EMA (numel) */
  const float* fthr;        /* SCAO_PF_FMASK: device threshold of this step      */
  const uint64_t* fseed;    /* SCAO_PF_FNOISE: device noise key of this step     */
  int64_t numel;
  int64_t cols;             /* row stride of the 2-D view                        */
  double lr;
  float decay;              /* fp32(1 - lr*weight_decay)                         */
  float beta1, omb1;        /* fp32(beta1), fp32(1 - beta1)                      */
  float beta2, omb2;
  float beta3, omb3;
  float bc1, bc2, bc3;      /* fp32(1 - beta_i ** step)                          */
  float blend, omblend;     /* fp32(b), fp32(1 - b)                              */
  float eps, tau, lars, wd, gsnr;
  float diag_bias;          /* fp32(diagonal EMA bias factor)                    */
  float adam_sqrt_bc2;      /* fp32(sqrt(1 - beta2 ** step))                     */
  float adam_alpha;         /* fp32(-(lr / (1 - beta1 ** step)))                 */
  int32_t dtype;            /* enum scao_dtype                                   */
  int32_t flags;            /* SCAO_PF_*                                         */
  int32_t pre_begin, pre_end;   /* reduction slots written before finalize 0     */
  int32_t post_begin, post_end; /* reduction slots written before finalize 1     */
  int32_t norm_index;       /* position in the global grad-norm average, or -1   */
  float fnoise;             /* SCAO_PF_FNOISE: fp32(noise_std)                   */
} scao_param_desc;

/* One Kronecker block (a whole 2-D parameter or one block-diagonal piece). */
typedef struct scao_leaf_desc {
  const float* Ul;          /* m x k row-major (left eigenvectors)               */
  const float* Ur;          /* n x k row-major                                   */
  const float* Sl;          /* k: eigenvalues, or s^-1/4 with SCAO_LF_SINV4      */
  const float* Sr;
  float* T;                 /* scratch k x n  : U_l^T G                          */
  float* Delta;             /* scratch k x k  : (s_l s_r^T - 1) * (U_l^T G U_r)  */
  float* W;                 /* scratch m x k  : U_l Delta                        */
  int64_t off;              /* element offset of the block origin in the param   */
  int64_t ld;               /* row stride of the parameter's 2-D view            */
  int32_t param;            /* index into the scao_param_desc table              */
  int32_t m, n, k;
  int32_t flags;            /* SCAO_LF_*                                         */
  float dbias;              /* SCAO_LF_DIAG: fp32(diagonal EMA bias factor)      */
  uint16_t* Wb;             /* NULL, or 3 x m x k bf16: W split exactly as
                               W = h + m + l (planes h, m, l, each m x k
                               row-major); scao_kron_lift writes it beside W,
                               the strip apply (variant bit 16) reads it   */
} scao_leaf_desc;

#define SCAO_LF_SINV4 1     /* Sl/Sr already hold clamp(S,1e-8)^-1/4             */
#define SCAO_LF_VEC4  2     /* off, ld, n multiples of 4 and 16-byte aligned     */
#define SCAO_LF_DIAG  4     /* a diagonal sub-block (1 x n or m x 1 remainder of a
                               block-diagonal split): Sl is its m*n diag EMA, no
                               U/S/T/Delta/W, k = 0; it takes delta tasks (its
                               norm partials) and masked apply tasks only      */

/* A unit of work: (leaf or param, two tile coordinates, reduction slot). */
typedef struct scao_task {
  int32_t idx;              /* leaf index (tile kernels) or param index (flat)   */
  int32_t a, b;             /* tile origin (rows/cols) or chunk number           */
  int32_t slot;             /* reduction slot, or -1                             */
} scao_task;

/* Per-parameter results of the step's reductions (written by the library). */
typedef struct scao_param_stat {
  double g2, p2, nu2, u2;   /* ||g||^2, ||p_decayed||^2, natural-norm^2, ||u||^2 */
  float gnorm, pnorm, nu, clip;
  float unorm, trust, alpha, pad0;
} scao_param_stat;

/* Number of doubles per reduction slot: [||g||^2, ||p||^2, nu^2 or ||u||^2]. */
#define SCAO_SLOT_WIDTH 3
/* Elements per flat task (chunk of one parameter). */
#define SCAO_FLAT_CHUNK 4096
/* Tile sizes of the Kronecker kernels. */
#define SCAO_PROJ_COLS 256   /* columns of G per projection task (c-chunk of 64) */
#define SCAO_APPLY_TILE 64   /* rows x cols per masked apply task                 */
#define SCAO_APPLY_WIDE_ROWS 16   /* rows of a fast (variant bit 4) apply task    */
#define SCAO_APPLY_WIDE_COLS 256  /* columns of a fast apply task                  */
#define SCAO_APPLY_GROUP 8    /* consecutive fast tasks per block of the pipelined
                                 variant (bit 8)                                 */
#define SCAO_GRAM_TILE 128   /* Gram output tile                                  */

/* ---- library --------------------------------------------------------- */
int scao_abi_version(void);
const char* scao_last_error(void);
/* sizeof and field offsets of the descriptor structs, for binding checks:
 * which = 0 param_desc, 1 leaf_desc, 2 task, 3 param_stat; out[0]=sizeof,
 * out[1..] = offsets in declaration order.  Returns the number written. */
int scao_struct_layout(int which, int64_t* out, int cap);

/* ---- reference operator surface ------------------------------------- */
/* out = G + U_l ((s_l s_r^T - 1) * (U_l^T G U_r)) U_r^T   (m x n, k <= 256).
 * G has row stride ldG; out is dense m x n.  workspace: k*n + k*k + m*k
 * floats + 4 leaf/task descriptors worth of bytes given by
 * scao_fused_kronecker_workspace(). */
/* <- scao.cuda.low_rank_precond_mm (scao/cuda/__init__.py:190-228; kernels
 * scao/cuda/low_rank_ops.cu:239-296).  left != 0: out = (U*s) (U^T G) with U
 * m x k; left == 0: out = (G (U*s)) U^T with U n x k; G and out m x n, all
 * contiguous fp32 on the device, s of length k.  The products run in that
 * order, U*s rounded to fp32 (the reference's fallback, :102-119, which is the
 * path the reference runs).  ws: scao_low_rank_precond_mm_workspace bytes
 * (the k x n or m x k intermediate). */
int64_t scao_low_rank_precond_mm_workspace(int64_t m, int64_t n, int64_t k, int left);
int scao_low_rank_precond_mm(const float* U, const float* s, const float* G, float* out,
                             int64_t m, int64_t n, int64_t k, int left, float* ws, void* stream);
int64_t scao_fused_kronecker_workspace(int64_t m, int64_t n, int64_t k);
int scao_fused_kronecker_precond(const float* U_l, const float* s_l_inv4, const float* U_r,
                                 const float* s_r_inv4, const float* G, int64_t ldG, float* out,
                                 int64_t m, int64_t n, int64_t k, void* workspace,
                                 void* stream);
/* The same operator with no workspace argument and no allocation of any kind.
 * It has no counterpart in the reference.  It exists for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Its scratch is a static device array of
 * SCAO_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, so
 * k*n + k*k + m*k floats must fit in it (m = n = 4096 at k = 256 does); larger
 * sizes are rejected with SCAO_ERR_INVALID.  Every call on one GPU shares that
 * GPU's array: calls on one stream are ordered, but calls that overlap on one
 * GPU (two streams, two threads) race.  The array used is the current
 * device's; a non-null stream must belong to that device (else
 * SCAO_ERR_INVALID).  Results are identical to scao_fused_kronecker_precond's. */
#define SCAO_NOALLOC_SCRATCH_BYTES (16u << 20)
int scao_fused_kronecker_precond_noalloc(const float* U_l, const float* s_l_inv4,
                                         const float* U_r, const float* s_r_inv4,
                                         const float* G, int64_t ldG, float* out, int64_t m,
                                         int64_t n, int64_t k, void* stream);
/* x = fp32(q)*fp32(scale) * fp32(rho) + new_val; scale' = max|x|/127 (double)
 * or 1.0; q' = clamp(rint(x * fp32(1/scale')), +-127).  Updates q in place,
 * writes scale' to *scale_out (device double).  scratch: n floats +
 * scao_reduce_scratch_bytes(n). */
int64_t scao_int8_ema_scratch_bytes(int64_t n);
int scao_int8_ema_update(int8_t* q, double scale_in, const float* new_val, double rho,
                         int64_t n, double* scale_out, void* scratch, void* stream);

/* ---- batched step: Phase 2 (preconditioned Adan) ---------------------- */
/* A1  T = U_l^T G for (leaf, 256-column strip, 64-row chunk of T); also
 *     ||g||^2 (chunk 0) and ||p*decay||^2 (chunk 0 of LARS params) into slots.
 *     variant = (fast ? 1 : 0) | (p norm ? 2 : 0) | (tall ? 4 : 0)
 *     | (wide ? 8 : 0): "fast" tasks promise fp32 data, SCAO_LF_VEC4, a full
 *     256-column strip, a full 64-row chunk of T and m % 32 == 0, and run on
 *     the bf16 matrix cores with fp32 products (three-way bf16 splits); "p
 *     norm" tasks are the chunk-0 tasks of LARS params; "tall" tasks (fast
 *     only) cover 128 rows of T from b = c0, a multiple of 128, with
 *     c0 + 128 <= k; "wide" tasks (fast only, not tall) cover 256 rows of T
 *     from b = c0, a multiple of 256, with c0 + 256 <= k. */
int scao_kron_project(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                      const scao_param_desc* params, double* slots, int variant, void* stream);
/* A2  P = T U_r, Delta = (s_l s_r^T - 1) P and nu^2 partial per 64x64 tile of P. */
int scao_kron_delta(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                    const scao_param_desc* params, double* slots, void* stream);
/* A3  W = U_l Delta per 64-row strip. */
int scao_kron_lift(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                   void* stream);
/* Diagonal-mode params: ||g||^2, ||p*decay||^2 and sum g^2/(sqrt(diag)+eps). */
int scao_diag_reduce(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                     double* slots, void* stream);
/* phase 0: per param ||g||, ||p||, nu, clip; global grad-norm EMA in runtime[0]
 *          (runtime[1] receives the average) when update_norm_ema != 0.
 * phase 1: per param ||u||, LARS trust and the fp32 step multiplier. */
int scao_step_finalize(const scao_param_desc* params, int nparams, const double* slots,
                       scao_param_stat* stat, double* runtime, int phase,
                       int update_norm_ema, int norm_count, void* stream);
/* B   G + W U_r^T -> clip -> blend -> Adan moments -> update; writes the
 *     update to upd (LARS params, ||u||^2 into slots) or the parameter.
 *     variant = (SCAO_PF_GF32 set ? 1 : 0) | (SCAO_PF_LARS set ? 2 : 0) |
 *     (fast ? 4 : 0); every task of a launch must belong to a parameter of
 *     that variant.  "fast" tasks promise fp32 data, SCAO_LF_VEC4,
 *     SCAO_PF_ALIGNED, k % 16 == 0 and a whole 16x256 tile at (a, b)
 *     (SCAO_APPLY_WIDE_ROWS x SCAO_APPLY_WIDE_COLS); other tasks are masked
 *     64x64 tiles (SCAO_APPLY_TILE) at (a, b), clipped to the block.
 *     variant | 8 (with 4): the same fast tasks through a two-role pipeline,
 *     SCAO_APPLY_GROUP consecutive tasks per block (the engine's choice for
 *     k >= 128 other than 128 and 256).
 *     variant | 16 (with 4): strip runs for k = 256 (| 32: k = 128): a task
 *     (leaf, a, b, slot) covers min(SCAO_APPLY_GROUP, (mw - a) / TR) tiles
 *     of TR rows x SW columns going down from row a in the column strip at
 *     b (SW = 64, TR = 128 for k = 256; SW = 128, TR = 64 for k = 128; mw =
 *     m - m % TR), with reduction slots slot, slot + 1, ...; b + SW <= n.
 *     Without SCAO_PF_GF32 the leaf needs Wb (written by scao_kron_lift).
 *     A leaf of another k, or one lacking Wb, gets NaN in its run's slots. */
int scao_kron_apply(const scao_task* tasks, int ntasks, const scao_leaf_desc* leaves,
                    const scao_param_desc* params, const scao_param_stat* stat,
                    double* slots, int variant, void* stream);
int scao_diag_apply(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                    const scao_param_stat* stat, double* slots, void* stream);
/* C   p = fma(upd, alpha, p*decay) for LARS params. */
int scao_lars_write(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                    const scao_param_stat* stat, void* stream);

/* ---- batched step: Phase 1 (Adam(W)) --------------------------------- */
int scao_adam_step(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                   double* slots, void* stream);

/* ---- curvature refresh ------------------------------------------------ */
typedef struct scao_gram_desc {
  const void* g;            /* gradient storage of the param (dtype)             */
  int64_t off, ld;          /* block origin and row stride                       */
  int8_t* q;                /* int8 EMA codes (dim x dim), or NULL for fp32 EMA  */
  const double* scale;      /* current dequantisation scale (device double)      */
  float* ema;               /* fp32 EMA: updated in place; int8: dim x dim scratch */
  float* amax;              /* per-tile |EMA| maxima (int8 mode)                 */
  int32_t rows, cols;       /* block shape m x n                                 */
  int32_t side;             /* 0: L = G G^T (dim m), 1: R = G^T G (dim n)        */
  int32_t dtype;
  int32_t ntiles;           /* amax entries: (tiles per side)^2                  */
  int32_t flags;            /* SCAO_GRAM_SYM                                     */
  float rho, alpha;         /* fp32(rho), fp32(1 - rho)                          */
} scao_gram_desc;
/* The factor is symmetric: the launch's tasks for this desc cover the output
 * tiles (a, b) with a >= b only, and a task with a > b also writes tile
 * (b, a) (EMA update of its own old values with the transposed product) and
 * amax entry b * nt + a.  Both tiles' products are the same sums of the same
 * products in the same order as when computed separately. */
#define SCAO_GRAM_SYM 1
int scao_gram_ema(const scao_task* tasks, int ntasks, const scao_gram_desc* descs,
                  void* stream);
/* requantise every int8 factor of a gram_ema launch; writes the new scale to
 * scale_out[i] (device doubles, may alias the scale inputs). */
int scao_requant(const scao_task* tasks, int ntasks, const scao_gram_desc* descs,
                 double* const* scale_out, void* stream);
/* eigh input: X = (deq or ema) / fp32(bias); X_ii += fp32(max(1e-8, 1e-4*tr(X)/dim)). */
typedef struct scao_prep_desc {
  const int8_t* q;          /* codes or NULL                                     */
  const double* scale;      /* device scale (int8)                               */
  const float* ema;         /* fp32 EMA (when q is NULL)                         */
  float* out;               /* dim x dim                                         */
  float* shift;             /* one float of device scratch: the diagonal shift   */
  int32_t dim;
  float bias;               /* fp32(max(bias_factor, 1e-8))                      */
} scao_prep_desc;
int scao_eig_prep(const scao_task* tasks, int ntasks, const scao_prep_desc* descs,
                  int ndescs, void* stream);
/* Exactly diagonal eigh inputs (scao/preconditioner.py:413-426).  On a matrix
 * whose off-diagonal entries are all zero, LAPACK's syevd (torch's CPU eigh)
 * returns the diagonal values, ordered by its divide-and-conquer selection
 * sort (for i = 0..n-2: k = first position of the minimum of d[i..n-1], ties
 * keeping i; swap d[i], d[k] and columns i, k of the identity), and the
 * eigenvectors +e_j in that order.  With many tied values (an int8 EMA that
 * kept only its diagonal codes) that order decides which unit vectors are the
 * top k, so these two entry points reproduce it instead of solving.
 *
 * scao_eig_offdiag: flags[i] = 1 if descriptor i's EMA (int8 codes when q is
 * set, else the fp32 ema) has a non-zero off-diagonal entry, else 0.  Only q,
 * ema and dim are read; max_dim >= every dim (a larger one is flagged 1);
 * codes = 1 when every descriptor has codes (sizes the grid for 4 codes per
 * load).  flags: ndescs device ints, cleared by the call. */
int scao_eig_offdiag(const scao_prep_desc* descs, int ndescs, int max_dim, int codes, int* flags,
                     void* stream);
/* scao_eig_diag: the kq largest eigenpairs of each descriptor's eigh input X
 * (as scao_eig_prep forms it, shift written to *shift), all of dimension n
 * (1 <= n <= 4096 + SCAO_EIG_BAND, kq <= n), for inputs scao_eig_offdiag
 * flagged 0: w[i*kq + j] (double, descending: the reference's flip), U + i *
 * ustride (n x kq row-major, column j a unit vector) and total[i] = sum of
 * max(X_jj, 0) (double).  The out field is not used. */
int scao_eig_diag(const scao_prep_desc* descs, int ndescs, int n, int kq, double* w, float* U,
                  int64_t ustride, double* total, void* stream);
/* ---- eigen stage: top-k eigenpairs of a batch of symmetric matrices -----
 * Replaces the torch.linalg.eigh calls of _update_eigenfactors
 * (scao/preconditioner.py:413-426), which need every eigenvalue (for
 * utils.adaptive_rank, scao/utils.py:121-151) but only the top-k_max
 * eigenvectors.  Two-stage: the dense matrix is reduced to a band of
 * SCAO_EIG_BAND sub-diagonals by block Householder transformations (panel QR,
 * panel correction and lower-triangle trailing updates here; the first panel
 * product and the last panel's in-band update are batched GEMMs by the
 * caller), the band to tridiagonal by bulge chasing, eigenvalues by bisection
 * on the tridiagonal (float64 Sturm counts), eigenvectors by float64 inverse
 * iteration on the band matrix, back-transformed with the stored block
 * reflectors (scao_eig_back_transform).  Matrix i of a batch starts at base +
 * i * stride (elements); every matrix of one call has the same dim n.  Every
 * scao_eig_* entry point below takes 1 <= n <= 4096 + SCAO_EIG_BAND (and
 * sy2sb_update mr in that range) and returns SCAO_ERR_INVALID otherwise; the
 * refresh sends larger factors to the library solver. */
#define SCAO_EIG_BAND 16
#define SCAO_EIG_BANDW (2 * SCAO_EIG_BAND + 1)  /* band row pitch: diagonals 0..2b */
/* Householder QR of the panel A[c0+b:n, c0:c0+b] of every matrix (A row-major,
 * leading dim n, float32; c0 a multiple of b, c0 + b < n <= 4096 + b),
 * LAPACK geqr2/larft semantics.  The panel of A is overwritten by the
 * reflectors V (explicit: unit lower trapezoidal, n-c0-b x b), the upper
 * triangular factor T (b x b) goes to T + i*b*b and R into the band storage
 * (rows c0+b.., band + i*bstride, pitch SCAO_EIG_BANDW). */
int scao_eig_panel_qr(float* A, int64_t stride, int n, int c0, int batch, float* T, float* band,
                      int64_t bstride, void* stream);
/* One panel step of the trailing update on the lower triangle of the region
 * R (mr x mr, at A + i*sA, leading dim ldA; every matrix): with the panel's
 * reflectors V and correction W (mr x b rows at V + i*sV / W + i*sW, leading
 * dims ldV / ldW), A <- A - V W^T - W V^T for the elements with row >=
 * column (the elements above the diagonal are never read; those of the
 * 64 x 64 diagonal tiles may be overwritten with meaningless values when
 * every leading dimension and mr are multiples of 4); with Vn (the next
 * panel's reflectors, mr x b), also Y = A_new Vn for the symmetric A_new into
 * Y + i*sY (mr x b, row-major), using `work` (scao_eig_sy2sb_work(mr, batch)
 * bytes) for fixed-order partial sums.  Replaces, per panel, the two-sided
 * update A22 - V W^T - W V^T and the next panel's A22 V product of the full
 * matrix (the reference's eigh works on the whole matrix). */
int64_t scao_eig_sy2sb_work(int mr, int batch);
/* The panel at column c0 (its reflectors V in A, rows c0+b.., m = n-c0-b of
 * them): from Y = A22 V (m x b per matrix, row-major, at Y + i*m*b) and T,
 * W = Y T - V (T^T V^T Y T) / 2 into W (m x b per matrix); with strip != 0
 * also the next panel's columns: A[c0+b+i][c0+b+j] -= V_i.W_j + W_i.V_j for
 * j < b (needs c0 + 2b <= n). */
int scao_eig_sy2sb_panel_w(float* A, int64_t sA, int n, int c0, int batch, const float* Y,
                           const float* T, float* W, int strip, void* stream);
int scao_eig_sy2sb_update(float* A, int64_t sA, int ldA, int mr, int batch, const float* V,
                          int64_t sV, int ldV, const float* W, int64_t sW, int ldW,
                          const float* Vn, int64_t sVn, int ldVn, float* Y, int64_t sY,
                          void* work, void* stream);
/* The band matrix: diagonals 0..b of every row, from the final diagonal
 * blocks of A and the R factors in band, into orig (float32, pitch b+1: kept
 * for the eigenvector stage) and into band64 (float64, n x SCAO_EIG_BANDW per
 * matrix, bulge diagonals b+1..2b zeroed: the bulge-chasing work array). */
int scao_eig_band_finish(const float* A, int64_t stride, int n, int batch, const float* band,
                         int64_t bstride, float* orig, int64_t ostride, double* band64,
                         void* stream);
/* Band -> tridiagonal by bulge chasing in float64 (one workgroup per
 * matrix) on band64; writes the diagonal d (n) and sub-diagonal e (n-1) at
 * d + i*n, e + i*n (float64). */
int scao_eig_sb2st(double* band64, int n, int batch, double* d, double* e, void* stream);
/* Eigenvalues of the tridiagonals by bisection: the kq largest, descending,
 * into w + i*kq (float64), and sum over all eigenvalues of max(lambda, 0) into
 * total[i] (float64: the trace minus the negative eigenvalues).  work:
 * scao_eig_bisect_work(n, batch) bytes. */
int64_t scao_eig_bisect_work(int n, int batch);
int scao_eig_bisect(const double* d, const double* e, int n, int batch, int kq, double* w,
                    double* total, void* work, void* stream);
/* Eigenvectors of the band matrices (orig, pitch b+1) for the eigenvalues w
 * (kq per matrix): float64 inverse iteration with band LU and partial
 * pivoting (one solve from a pseudo-random start, a second when the solution
 * did not grow enough to have converged), then Gram-Schmidt inside
 * clusters of eigenvalues closer than 1e-10 of the largest |B| entry (whose
 * members get shifts offset by 1e-13 |B| steps).  Output Z (n x kq row-major,
 * float32) at Z + i*zstride; w is replaced by the vectors' Rayleigh
 * quotients.  work: scao_eig_vectors_work(n, batch, kq) bytes. */
int64_t scao_eig_vectors_work(int n, int batch, int kq);
int scao_eig_vectors(const float* orig, int64_t ostride, int n, int batch, int kq, double* w,
                     float* Z, int64_t zstride, void* work, void* stream);
/* Back-transformation Z <- Q_0 (Q_1 (... Q_last Z)) of the eigenvectors with
 * the stage-1 reflectors: panel p (c0 = 16p < n - 16) holds V_p explicitly in
 * A[c0+16:n, c0:c0+16] of each matrix (as scao_eig_panel_qr leaves it) and
 * T_p at T + (p*batch + i)*256; Q_p = I - V_p T_p V_p^T acts on rows c0+16..
 * of Z (n x kq row-major float32 at Z + i*zstride), in place. */
int scao_eig_back_transform(const float* A, int64_t stride, int n, int batch, const float* T,
                            float* Z, int64_t zstride, int kq, void* stream);

/* diag_ema = fp32(diag*rho) + fp32(alpha * g*g)  (1-D preconditioners). */
int scao_diag_ema(const scao_task* tasks, int ntasks, const scao_param_desc* params,
                  const float* rho_alpha, void* stream);

/* ---- the gradient the moments see -----------------------------------------
 * Replaces the prologue of SCAO._step_group (scao/optimizer.py:533-545) for a
 * batch of parameters: with SCAO_FILTER_MASK, _SparseGradFilter.__call__
 * (:49-57): ema = |g| (SCAO_FILTER_FIRST) or fp32(fp32(ema*decay) +
 * fp32(omd*|g|)); t = torch.quantile(ema, q) (linear interpolation, exact
 * order statistics by radix select); out = fp32(g) * (ema >= t).  Without it
 * out = fp32(g).  With noise > 0, out += fp32(noise * z), z ~ N(0,1) from
 * Philox4x32-10 keyed by *seed, counter = element index / 4 (Box-Muller).
 * With out == NULL the last pass is skipped: the step kernels form the same
 * values themselves (SCAO_PF_FMASK / SCAO_PF_FNOISE; the threshold is the
 * float at work + SCAO_FILTER_THR_WORD).
 * torch.quantile refuses more than 2^24 elements; this entry point has no such
 * limit.  Tasks are (desc index, chunk of SCAO_FLAT_CHUNK elements, 0, -1).
 * After its first call a desc's EMA pass assumes the threshold stays in the
 * previous call's top-digit bin; when it does, one select resolves two
 * digits, and with a candidate buffer (cand, cap >= ceil(numel /
 * SCAO_FLAT_CHUNK) * (SCAO_FILTER_REGION + 4) floats) that receives the
 * bin's values, the last refinement pass reads only those.  Tasks must list
 * each desc's chunks in order for the buffer to be used.  Results do not
 * depend on either. */
#define SCAO_FILTER_BINS 2048
#define SCAO_FILTER_REGION (SCAO_FLAT_CHUNK / 2)
#define SCAO_FILTER_WORK_WORDS (2 * SCAO_FILTER_BINS + 16)
#define SCAO_FILTER_THR_WORD (2 * SCAO_FILTER_BINS + 7)
#define SCAO_FILTER_MASK 1
#define SCAO_FILTER_FIRST 2
typedef struct scao_filter_desc {
  const void* g;            /* gradient (dtype), numel elements                  */
  float* ema;               /* magnitude EMA, updated in place (MASK)            */
  float* out;               /* the moment gradient, fp32                         */
  uint32_t* work;           /* SCAO_FILTER_WORK_WORDS words of device scratch per
                               desc (MASK): zero before its first call; every
                               call leaves it ready for the next                 */
  const uint64_t* seed;     /* device noise key (noise > 0)                      */
  int64_t numel;
  float decay, omd;         /* fp32(ema), fp32(1 - ema)                          */
  float q;                  /* fp32(sparsity)                                    */
  float noise;              /* fp32(noise_std), 0 for none                       */
  int32_t dtype;
  int32_t flags;            /* SCAO_FILTER_MASK | SCAO_FILTER_FIRST              */
  float* cand;              /* optional candidate buffer of cap floats (MASK),
                               NULL for none; kept with work between calls, no
                               initial contents needed                          */
  int64_t cap;
} scao_filter_desc;
int scao_sparse_filter(const scao_task* tasks, int ntasks, const scao_filter_desc* descs,
                       int ndescs, void* stream);

/* ---- lookahead ------------------------------------------------------------
 * Replaces SCAO._lookahead_sync (scao/optimizer.py:356-365) for a batch of
 * parameters: slow = slow + fp32(alpha * (p - slow)); p = slow, with the
 * reference's three roundings in the parameter dtype.  Tasks are (desc index,
 * chunk of SCAO_FLAT_CHUNK elements, 0, -1). */
typedef struct scao_lookahead_desc {
  void* p;                  /* parameter (dtype)                                 */
  void* slow;               /* slow weights, same dtype and layout               */
  int64_t numel;
  int32_t dtype;
  int32_t pad0;
} scao_lookahead_desc;
int scao_lookahead(const scao_task* tasks, int ntasks, const scao_lookahead_desc* descs,
                   float alpha, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SCAO_AMD_H */
