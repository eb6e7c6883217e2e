/*
 * rnrqr.h -- C ABI of the MI355X (gfx950) reflector-free batched QR library, librnrqr.so.
 *
 * The library factors a batch of square fp32 matrices A (row-major, A[b][i][j] at
 * A + b*batch_stride + i*n + j) into the compact LAPACK / torch.geqrf layout (H, tau)
 * without forming or applying a Householder reflector:
 *
 *   I.   frame:   A = P L U (partial pivoting), then CholeskyQR2 on the unit-lower L,
 *                 Q = P * (L Ra^-1 Rb^-1), each Cholesky on G + 1e-7*mean(diag G)*I;
 *   II.  closure: R = triu(Q^T A);
 *   III. chart:   sign-ruled unpivoted LU of I - Q S; its multipliers are the
 *                 reflector tails Y, tau_k = 2 / (1 + ||Y[k+1:,k]||^2),
 *                 H = triu(diag(s) R) + tril(Y, -1).
 *
 * Every entry point is asynchronous on the caller's HIP stream, never throws, keeps no
 * global mutable state, and returns an rnr_status code.  Device pointers only.  The
 * input is never written.  Calls that share one workspace must be ordered on one stream.
 *
 * Reference interfaces replaced (paths relative to the johnzfitch/qr-contest tree):
 *   rnr_qr_f32      custom_kernel(data) -> (H, tau)      reflection_no_reflectors.py:181-196
 *   rnr_frame_f32   _frame(A) -> Q                       reflection_no_reflectors.py:55-81
 *   rnr_lu_f32      torch.linalg.lu(A) (P, L; U dropped) reflection_no_reflectors.py:66
 *   rnr_cholqr_f32  _cholqr(M) -> M R^-1                 reflection_no_reflectors.py:68-77
 *   rnr_chart_f32   _chart(Q) -> (Y, s), tau recompute   reflection_no_reflectors.py:86-176,192
 *   rnr_generate_f32  make_batch / gen_* (the input step)   common/oracle.py:43-146
 *   rnr_orgqr_f32   torch.linalg.householder_product    README.md:122-128 (the consumer)
 *   rnr_ormqr_f32   torch.ormqr (left)                  README.md:122-128
 *   rnr_check_f64   check / check_percol (fp64 gates)    common/oracle.py:152-195
 *   rnr_hh_geqrf_f32  blocked Householder (comparator only)  householder/submission_routed_v3.py:225-281
 */
#ifndef RNRQR_H
#define RNRQR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* rnr_stream_t; /* hipStream_t; NULL = the legacy default stream */

enum rnr_status {
  RNR_OK = 0,
  RNR_ERR_INVALID_ARG = 1,    /* null pointer, negative size, stride < n*n */
  RNR_ERR_UNSUPPORTED_N = 2,  /* n outside [1, RNR_MAX_N] */
  RNR_ERR_WORKSPACE = 3,      /* workspace pointer null or smaller than the query result */
  RNR_ERR_HIP = 4,            /* a HIP launch or attribute call failed */
  RNR_ERR_MISALIGNED = 5,     /* a pointer is not 4-byte aligned (workspace: 256-byte) */
  RNR_ERR_SCRATCH_LIMIT = 6   /* rnr_qr_f32_noalloc: the problem needs more than its scratch */
};

#define RNR_MAX_N 2048

/* Human-readable text of a status code (static storage, never NULL). */
const char* rnr_status_string(int status);

/* Library version, "major.minor.patch". */
const char* rnr_version(void);

/* ---- whole path: custom_kernel (reflection_no_reflectors.py:181-196) ------------------
 * Bytes of device workspace rnr_qr_f32 needs for (batch, n).  0 for batch == 0, and 0 for
 * n <= 64, where the whole path is one fused launch with everything on chip (ws may then
 * be NULL). */
int rnr_qr_f32_workspace(int64_t batch, int64_t n, size_t* bytes);

/* H (batch x n x n, contiguous) and tau (batch x n, contiguous) from A.
 * batch_stride is the element distance between consecutive input matrices (>= n*n).
 * info (optional, batch ints, may be NULL): 0 on success; k > 0 when a Cholesky of
 * matrix b met a non-positive or non-finite pivot at column k (the reference raises
 * from torch.linalg.cholesky in that case, reflection_no_reflectors.py:76).
 * ws: device workspace of at least rnr_qr_f32_workspace bytes, 256-byte aligned. */
int rnr_qr_f32(const float* A, int64_t batch, int64_t n, int64_t batch_stride,
               float* H, float* tau, int32_t* info,
               void* ws, size_t ws_bytes, rnr_stream_t stream);

/* rnr_qr_f32 for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Takes no workspace and calls no allocating routine: the workspace lives in a device array
 * of RNR_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on until the
 * process ends.  Problems whose workspace (rnr_qr_f32_workspace) exceeds it return
 * RNR_ERR_SCRATCH_LIMIT before any launch: at n = 512 up to 31 matrices per call, at
 * n = 1024 up to 7, at n = 2048 one; n <= 64 needs none.  All calls on one GPU share its
 * array, so calls that overlap on one GPU (other streams, other host threads) race and must
 * be ordered by the caller.  Nothing in it needs to start at zero.  Results equal
 * rnr_qr_f32's bit for bit. */
#define RNR_NOALLOC_SCRATCH_BYTES (128u << 20)
int rnr_qr_f32_noalloc(const float* A, int64_t batch, int64_t n, int64_t batch_stride,
                       float* H, float* tau, int32_t* info, rnr_stream_t stream);

/* Same as rnr_qr_f32, and records events[i] (hipEvent_t handles created by the caller) on
 * the stream before stage i of the sequence and events[11] after the last, for per-kernel
 * timing of the live path: 0 LU, 1 Gram(L), 2 Cholesky, 3 the solve's off-diagonal operand
 * (W blocks), 4 solve L R^-1, 5 Gram(Q1), 6 Cholesky, 7 W blocks, 8 solve Q1 R^-1 with the
 * row gather, 9 chart, 10 closure.  A stage is one launch, except in the split form (n > 512
 * with fewer than 128 matrices), where the LU, Cholesky and chart stages are one launch per
 * panel or block.  For n <= 64 the path is one launch: events[0] before it and
 * events[1..11] after it.  Stands in for the reference's event timers around its stages
 * (common/bench.py:12-21). */
#define RNR_QR_TIMED_EVENTS 12
int rnr_qr_f32_timed(const float* A, int64_t batch, int64_t n, int64_t batch_stride,
                     float* H, float* tau, int32_t* info, void* ws, size_t ws_bytes,
                     rnr_stream_t stream, void* const* events, int n_events);

/* ---- stage entry points (the reference's internal stages, for stage-level parity) ---- */

/* Partial-pivot LU (torch.linalg.lu, reflection_no_reflectors.py:66): perm[b][i] is the
 * row of A that lands in position i (A[perm] = L U, first-maximum pivot rule) and L
 * (batch x n x n) is unit lower-triangular with exact zeros above the diagonal.  U is
 * not returned: the reference discards it. */
int rnr_lu_f32_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_lu_f32(const float* A, int64_t batch, int64_t n, int64_t batch_stride,
               float* L, int32_t* perm, void* ws, size_t ws_bytes, rnr_stream_t stream);

/* One CholeskyQR pass (_cholqr, reflection_no_reflectors.py:68-77): G = M^T M,
 * G += 1e-7*mean(diag G)*I, R = chol(G) upper, Q = M R^-1.  R (optional, may be NULL)
 * receives R in its upper triangle (the strict lower triangle is left unspecified). */
int rnr_cholqr_f32_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_cholqr_f32(const float* M, int64_t batch, int64_t n, int64_t batch_stride,
                   float* Q, float* R, int32_t* info,
                   void* ws, size_t ws_bytes, rnr_stream_t stream);

/* The orthogonal frame (_frame, reflection_no_reflectors.py:55-81): Q = P CholQR2(L). */
int rnr_frame_f32_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_frame_f32(const float* A, int64_t batch, int64_t n, int64_t batch_stride,
                  float* Q, int32_t* info, void* ws, size_t ws_bytes, rnr_stream_t stream);

/* The chart (_chart, reflection_no_reflectors.py:86-176, and the tau recompute at :192),
 * in place: on entry Y holds Q (batch x n x n, contiguous); on return its strict lower
 * triangle holds the reflector tails (the upper triangle is left unspecified), s the
 * signs (+1/-1) and tau = 2 / (1 + sum_{i>k} Y[i][k]^2).  No workspace. */
int rnr_chart_f32(float* Y, int64_t batch, int64_t n, float* s, float* tau,
                  rnr_stream_t stream);

/* ---- the input step: device-side seeded generators (common/oracle.py:43-146) ------------
 * The batch of benchmark configuration `config` (1..5; classes as in qr-contest_amd/workloads.py)
 * with its own Philox4x32-10 streams keyed by `seed`: matrix i depends only on (config, n, seed,
 * i), not on the batch size.  A is batch x n x n float32, contiguous.  The workspace (float64
 * Haar factors) is 0 bytes when the configuration has no Haar-class matrix in the batch. */
int rnr_generate_workspace(int config, int64_t batch, int64_t n, size_t* bytes);
int rnr_generate_f32(int config, int64_t batch, int64_t n, uint64_t seed, float* A, void* workspace,
                     size_t workspace_bytes, rnr_stream_t stream);

/* ---- consumers of the path's output (README.md:122-128) ------------------------------
 * Q = householder_product(H, tau) (torch.linalg.householder_product), batch x n x n, all
 * contiguous.  The workspace holds every panel's T (batch * ceil(n/32) * 4 KiB), 256-byte
 * aligned. */
int rnr_orgqr_f32_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_orgqr_f32(const float* H, const float* tau, int64_t batch, int64_t n, float* Q, void* workspace,
                  size_t workspace_bytes, rnr_stream_t stream);

/* C <- Q C (transpose == 0) or Q^T C (transpose != 0) in place (torch.ormqr, left side):
 * C is batch x n x ncol with row stride ldc >= ncol and batch stride >= n * ldc.  Same
 * workspace as rnr_orgqr_f32. */
int rnr_ormqr_f32_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_ormqr_f32(const float* H, const float* tau, int64_t batch, int64_t n, float* C, int64_t ncol,
                  int64_t ldc, int64_t batch_stride_c, int transpose, void* workspace, size_t workspace_bytes,
                  rnr_stream_t stream);

/* ---- benchmark comparator (NOT on the reflector-free path) --------------------------------
 * Householder blocked-WY QR in torch.geqrf layout, in place on H (A in, H out), float32: the
 * classical route the reference measures its kernels against
 * (householder/submission_routed_v3.py:225-281).  custom_kernel never calls it. */
int rnr_hh_geqrf_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_hh_geqrf_f32(float* H, int64_t batch, int64_t n, float* tau, void* workspace, size_t workspace_bytes,
                     rnr_stream_t stream);

/* ---- consumer of the path's output: the contest gates, evaluated on the GPU -------------
 * fp64 restatement of the reference checker (common/oracle.py:152-195, check and
 * check_percol): Q = householder_product(H, tau) in float64, then per matrix
 *   factor[b]   = ||triu(H) - Q^T A||_1 / ||A||_1                               (gate 20 n eps32)
 *   ortho[b]    = ||Q^T Q - I||_1                                              (gate 100 n eps32)
 *   colratio[b] = max_j ||(triu(H) - Q^T A)[:, j]||_1 / (20 n eps32 ||A[:, j]||_1)   (gate 1)
 * with the matrix 1-norm (largest absolute column sum).  A has batch stride batch_stride;
 * H (batch x n x n) and tau (batch x n) are contiguous; colratio may be NULL.  The result is
 * the same on every run (no atomics).  Workspace: rnr_check_f64_workspace bytes, 256-byte
 * aligned. */
int rnr_check_f64_workspace(int64_t batch, int64_t n, size_t* bytes);
int rnr_check_f64(const float* A, int64_t batch_stride, const float* H, const float* tau,
                  int64_t batch, int64_t n, double* factor, double* ortho, double* colratio,
                  void* ws, size_t ws_bytes, rnr_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RNRQR_H */
