// fp64 contest gates of a batched (H, tau) factorization on the GPU -- the checker of
// common/oracle.py:152-195, which consumes the path's output:
//
//   Q        = householder_product(H, tau)            (float64)
//   factor   = ||triu(H) - Q^T A||_1 / ||A||_1         (:163,166)
//   ortho    = ||Q^T Q - I||_1                         (:165-166)
//   colratio = max_j ||(triu(H) - Q^T A)[:, j]||_1 / (20 n eps32 ||A[:, j]||_1)   (:171-195)
//
// with the matrix 1-norm (largest absolute column sum).  Three kernels, all float64:
//   k_apply_q Q = H_0 H_1 ... H_{n-1} I in float64 by blocked WY accumulation (applyq.hpp);
//   k_chk_tn  C = Q^T X for X = A (widened) or Q, 64 x 64 tiles, K staged through LDS; the
//             epilogue reduces |C - ref| (ref = triu(H) or I) over the tile's 64 rows into
//             per-(row tile, column) partial sums -- no atomics, so the result is repeatable;
//   k_chk_red per matrix: column sums of the partials and of |A|, then the three maxima.
#include "../../include/rnrqr.h"
#include "applyq.hpp"

namespace rnr {
namespace {

struct TnArgs64 {
  const double* Q;     // [batch][n][n]
  const float* Xf;     // X = A (widened) when non-null
  const double* Xd;    // X = Q otherwise
  int64_t sx;          // batch stride of Xf
  const float* H;      // reference triu(H) when non-null, else the identity
  double* part;        // [batch][ntile][n] column partial sums of |Q^T X - ref|
  int n, nt, total;
};

// 64 x 64 tile of C = Q^T X per 256-thread workgroup (each thread 4 x 4 outputs), K in
// chunks of 16 through LDS.
__global__ __launch_bounds__(256) void k_chk_tn(TnArgs64 a) {
  __shared__ double Qs[16][64 + 2];
  __shared__ double Xs[16][64 + 2];
  __shared__ double red[16][64 + 2];
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int pid = blockIdx.x;
  const int b = pid / (a.nt * a.nt), t = pid - b * a.nt * a.nt, ti = t / a.nt, tj = t - ti * a.nt;
  const int n = a.n, i0 = ti * 64, j0 = tj * 64;
  const double* Q = a.Q + (int64_t)b * n * n;
  double acc[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[u][v] = 0.0;
  for (int k0 = 0; k0 < n; k0 += 16) {
    for (int idx = tid; idx < 16 * 64; idx += 256) {
      const int k = idx >> 6, c = idx & 63, kr = k0 + k;
      Qs[k][c] = (kr < n && i0 + c < n) ? Q[(int64_t)kr * n + i0 + c] : 0.0;
      double x = 0.0;
      if (kr < n && j0 + c < n)
        x = a.Xf ? (double)a.Xf[b * a.sx + (int64_t)kr * n + j0 + c] : a.Xd[(int64_t)b * n * n + (int64_t)kr * n + j0 + c];
      Xs[k][c] = x;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      double qa[4], xb[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        qa[u] = Qs[k][ty * 4 + u];
        xb[u] = Xs[k][tx * 4 + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] += qa[u] * xb[v];
    }
    __syncthreads();
  }
  // |C - ref| summed over this thread's 4 rows, then over the 16 row groups
  double cs[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = i0 + ty * 4 + u;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int j = j0 + tx * 4 + v;
      if (i < n && j < n) {
        double ref;
        if (a.H) ref = (j >= i) ? (double)a.H[(int64_t)b * n * n + (int64_t)i * n + j] : 0.0;
        else ref = (i == j) ? 1.0 : 0.0;
        cs[v] += fabs(acc[u][v] - ref);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) red[ty][tx * 4 + v] = cs[v];
  __syncthreads();
  if (tid < 64 && j0 + tid < n) {
    double s = 0.0;
    for (int y = 0; y < 16; ++y) s += red[y][tid];
    a.part[((int64_t)b * a.nt + ti) * n + j0 + tid] = s;
  }
}

struct RedArgs {
  const float* A;
  int64_t sa;
  const double* pe;   // [batch][nt][n] partials of |triu(H) - Q^T A|
  const double* po;   // [batch][nt][n] partials of |Q^T Q - I|
  double* factor;
  double* ortho;
  double* colratio;
  int n, nt;
};

// Maximum that keeps NaN (fmax drops it): a NaN residual must fail the gates, as it does in
// the reference checker, whose comparisons with the gate are false for NaN.
__device__ __forceinline__ double max_nan(double x, double y) { return (x > y || x != x) ? x : y; }

__global__ __launch_bounds__(256) void k_chk_red(RedArgs a) {
  __shared__ double r_e[256], r_a[256], r_o[256], r_c[256];
  const int b = blockIdx.x, tid = threadIdx.x, n = a.n;
  const double ftol = 20.0 * n * 1.1920928955078125e-07;
  double me = 0.0, ma = 0.0, mo = 0.0, mc = 0.0;
  for (int j = tid; j < n; j += 256) {
    double e = 0.0, o = 0.0, s = 0.0;
    for (int t = 0; t < a.nt; ++t) {
      e += a.pe[((int64_t)b * a.nt + t) * n + j];
      o += a.po[((int64_t)b * a.nt + t) * n + j];
    }
    for (int i = 0; i < n; ++i) s += fabs((double)a.A[b * a.sa + (int64_t)i * n + j]);
    me = max_nan(me, e);
    ma = max_nan(ma, s);
    mo = max_nan(mo, o);
    mc = max_nan(mc, e / (ftol * fmax(s, 1e-300)));
  }
  r_e[tid] = me; r_a[tid] = ma; r_o[tid] = mo; r_c[tid] = mc;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (tid < off) {
      r_e[tid] = max_nan(r_e[tid], r_e[tid + off]);
      r_a[tid] = max_nan(r_a[tid], r_a[tid + off]);
      r_o[tid] = max_nan(r_o[tid], r_o[tid + off]);
      r_c[tid] = max_nan(r_c[tid], r_c[tid + off]);
    }
    __syncthreads();
  }
  if (tid == 0) {
    a.factor[b] = r_e[0] / r_a[0];
    a.ortho[b] = r_o[0];
    if (a.colratio) a.colratio[b] = r_c[0];
  }
}

inline size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

size_t check_ws(int64_t batch, int64_t n) {
  const int64_t nt = (n + 63) / 64;
  return up256((size_t)batch * n * n * sizeof(double)) + 2 * up256((size_t)batch * nt * n * sizeof(double));
}

}  // namespace
}  // namespace rnr

using namespace rnr;

extern "C" {

int rnr_check_f64_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  *bytes = batch == 0 ? 0 : check_ws(batch, n);
  return RNR_OK;
}

int rnr_check_f64(const float* A, int64_t batch_stride, const float* H, const float* tau, int64_t batch,
                  int64_t n, double* factor, double* ortho, double* colratio, void* ws, size_t ws_bytes,
                  rnr_stream_t stream) {
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  if (batch == 0) return RNR_OK;
  if (batch > INT32_MAX / 4096) return RNR_ERR_INVALID_ARG;
  if (!A || !H || !tau || !factor || !ortho || batch_stride < n * n) return RNR_ERR_INVALID_ARG;
  const size_t need = check_ws(batch, n);
  if (!ws || ws_bytes < need) return RNR_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return RNR_ERR_MISALIGNED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int ni = (int)n, nt = (ni + 63) / 64;
  char* base = static_cast<char*>(ws);
  double* Q = reinterpret_cast<double*>(base);
  double* pe = reinterpret_cast<double*>(base + up256((size_t)batch * n * n * sizeof(double)));
  double* po = reinterpret_cast<double*>(reinterpret_cast<char*>(pe) + up256((size_t)batch * nt * n * sizeof(double)));

  ApplyQArgs<double> fq{H, tau, Q, (int64_t)n * n, ni, ni, ni};
  if (ni <= 1024) {
    const size_t lds = applyq_lds<double, 16>(ni);
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_apply_q<double, 16, false, true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return RNR_ERR_HIP;
    k_apply_q<double, 16, false, true><<<applyq_grid(batch, ni), dim3(kApplyQThreads), lds, st>>>(fq);
  } else {
    const size_t lds = applyq_lds<double, 8>(ni);
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_apply_q<double, 8, false, true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return RNR_ERR_HIP;
    k_apply_q<double, 8, false, true><<<applyq_grid(batch, ni), dim3(kApplyQThreads), lds, st>>>(fq);
  }
  if (hipGetLastError() != hipSuccess) return RNR_ERR_HIP;

  const int64_t tiles = batch * nt * nt;
  if (tiles > INT32_MAX) return RNR_ERR_INVALID_ARG;
  TnArgs64 ta{Q, A, nullptr, batch_stride, H, pe, ni, nt, (int)tiles};
  k_chk_tn<<<dim3((unsigned)tiles), dim3(256), 0, st>>>(ta);
  TnArgs64 tb{Q, nullptr, Q, 0, nullptr, po, ni, nt, (int)tiles};
  k_chk_tn<<<dim3((unsigned)tiles), dim3(256), 0, st>>>(tb);
  RedArgs ra{A, batch_stride, pe, po, factor, ortho, colratio, ni, nt};
  k_chk_red<<<dim3((unsigned)batch), dim3(256), 0, st>>>(ra);
  return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP;
}

}  // extern "C"
