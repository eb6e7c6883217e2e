// Jittered upper Cholesky of one Gram matrix per 512-thread workgroup, in place:
//
//   mu = 1e-7 * mean(diag G);  G += mu I;  G = R^T R        -- reflection_no_reflectors.py:74-76
//
// Blocked right-looking with 64-column blocks.  For block k the diagonal block is
// factored in LDS (two barriers per column), its inverse Dinv_kk = R_kk^-1 is formed in
// LDS (8 lanes per column, back substitution, no workgroup barriers), the block row
// R_k,> = Dinv_kk^T G_k,> and the trailing update G_>,> -= R_k,>^T R_k,> (upper tiles
// only) run on MFMA, each wave owning whole output tiles.  When the block row fits it
// is also kept in LDS for the trailing update (n <= 576), otherwise it is read back
// from G.  The diagonal-block inverses go to Dinv ([n][64] per matrix) for the
// triangular solve that follows.  info records the first column whose pivot was not
// positive (1-based; NaN counts as not positive).
#pragma once
#include "common.hpp"

namespace rnr {

struct CholArgs {
  float* G;
  int64_t sg;
  float* Dinv;   // [batch][n][64]
  int* info;     // [batch]
  int n;
  int strip_lds;
  int keep_info;  // 1: leave an earlier non-zero info in place
};

constexpr int kCholThreads = 512;
constexpr int kCholNb = 64;

inline size_t chol_lds_bytes(int n, bool strip) {
  const size_t w = n > kCholNb ? (size_t)(n - kCholNb) : 1;
  return sizeof(float) * (64 * 65 + 64 + 32 + (strip ? 64 * w : 0));
}

__global__ __launch_bounds__(kCholThreads) void k_chol(CholArgs a) {
  extern __shared__ float smem[];
  float* D = smem;                 // [64][65]: upper = R_kk, strict lower = (R_kk^-1)^T
  float* xd = D + 64 * 65;         // diagonal of R_kk^-1
  float* red = xd + 64;            // [16]
  int* ffail = reinterpret_cast<int*>(red + 16);
  float* S = red + 32;             // block row [64][n-64] when strip_lds

  const int n = a.n, b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int lds_w = n > kCholNb ? n - kCholNb : 1;
  float* G = a.G + b * a.sg;
  float* Dv = a.Dinv + (int64_t)b * n * 64;

  // jitter
  float part = 0.f;
  for (int i = tid; i < n; i += kCholThreads) part += G[(int64_t)i * n + i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) red[wid] = part;
  if (tid == 0) *ffail = INT_MAX;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kCholThreads / 64; ++w) tot += red[w];
  const float mu = 1e-7f * (tot / (float)n);
  for (int i = tid; i < n; i += kCholThreads) G[(int64_t)i * n + i] += mu;
  __syncthreads();

  for (int k0 = 0; k0 < n; k0 += kCholNb) {
    const int kb = min(kCholNb, n - k0), k1 = k0 + kb, w = n - k1;

    for (int idx = tid; idx < 64 * 64; idx += kCholThreads) {
      const int i = idx >> 6, c = idx & 63;
      D[i * 65 + c] = (i < kb && c < kb && c >= i) ? G[(int64_t)(k0 + i) * n + k0 + c] : 0.f;
    }
    __syncthreads();

    // unblocked upper Cholesky of the diagonal block
    for (int j = 0; j < kb; ++j) {
      const float d = D[j * 65 + j];
      if (tid == 0 && !(d > 0.f) && *ffail == INT_MAX) *ffail = k0 + j + 1;
      const float r = sqrtf(d);
      const float rinv = 1.f / r;
      for (int c = j + 1 + tid; c < kb; c += kCholThreads) D[j * 65 + c] *= rinv;
      __syncthreads();
      const int t = kb - j - 1;
      for (int idx = tid; idx < t * t; idx += kCholThreads) {
        const int ra = idx / t, rc = idx - ra * t;
        if (rc >= ra) {
          const int ia = j + 1 + ra, ic = j + 1 + rc;
          D[ia * 65 + ic] -= D[j * 65 + ia] * D[j * 65 + ic];
        }
      }
      if (tid == 0) D[j * 65 + j] = r;
      __syncthreads();
    }

    // Dinv_kk = R_kk^-1 (upper), column j by the 8 lanes of group j; X[i][j] (i < j)
    // is kept as D[j][i] and X[j][j] as xd[j].
    {
      const int j = tid >> 3, sub = tid & 7;
      if (j < kb) {
        const float xjj = 1.f / D[j * 65 + j];
        if (sub == 0) xd[j] = xjj;
        for (int i = j - 1; i >= 0; --i) {
          float s = 0.f;
          for (int q = i + 1 + sub; q <= j; q += 8) {
            const float xq = (q == j) ? xjj : D[j * 65 + q];
            s += D[i * 65 + q] * xq;
          }
          s = group8_sum(s);
          if (sub == 0) D[j * 65 + i] = -s / D[i * 65 + i];
          wave_lds_order();
        }
      }
    }
    __syncthreads();

    for (int idx = tid; idx < kb * 64; idx += kCholThreads) {
      const int i = idx >> 6, c = idx & 63;
      if (c < kb && c >= i) G[(int64_t)(k0 + i) * n + k0 + c] = D[i * 65 + c];
      Dv[(int64_t)(k0 + i) * 64 + c] = (c < kb) ? (c > i ? D[c * 65 + i] : (c == i ? xd[i] : 0.f)) : 0.f;
    }
    if (w <= 0) break;  // uniform; kb == 64 below this line

    // block row R_k,> = Dinv_kk^T G_k,>: each wave owns 32 columns (both 32-row halves),
    // so it can overwrite them in G without racing other waves' reads.
    {
      const int nch = (w + 31) >> 5;
      for (int job = wid; job < nch; job += kCholThreads / 64) {
        const int colr = job * 32 + l32, col = k1 + colr;
        f32x16 acc0 = zero16(), acc1 = zero16();
        for (int kk = 0; kk < kCholNb; kk += 2) {
          const int k = kk + h;
          const float bv = (col < n) ? G[(int64_t)(k0 + k) * n + col] : 0.f;
          const int ia = l32, ib = 32 + l32;
          const float a0 = (k < ia) ? D[ia * 65 + k] : (k == ia ? xd[ia] : 0.f);
          const float a1 = (k < ib) ? D[ib * 65 + k] : (k == ib ? xd[ib] : 0.f);
          acc0 = mfma(a0, bv, acc0);
          acc1 = mfma(a1, bv, acc1);
        }
        if (col < n) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int i0 = acc_row(r, lane), i1 = 32 + acc_row(r, lane);
            G[(int64_t)(k0 + i0) * n + col] = acc0[r];
            G[(int64_t)(k0 + i1) * n + col] = acc1[r];
            if (a.strip_lds) {
              S[i0 * lds_w + colr] = acc0[r];
              S[i1 * lds_w + colr] = acc1[r];
            }
          }
        }
      }
    }
    __syncthreads();

    // trailing G_>,> -= R_k,>^T R_k,> over upper 64x64 tiles, one tile per wave at a time
    {
      const int nt = (w + 63) >> 6, npairs = nt * (nt + 1) / 2;
      for (int pr = wid; pr < npairs; pr += kCholThreads / 64) {
        int I, J;
        upper_tile(pr, nt, I, J);
        f32x16 acc[2][2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int nj = 0; nj < 2; ++nj)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int row = k1 + I * 64 + mi * 32 + acc_row(r, lane);
              const int col = k1 + J * 64 + nj * 32 + l32;
              acc[mi][nj][r] = (row < n && col < n) ? G[(int64_t)row * n + col] : 0.f;
            }
        for (int kk = 0; kk < kCholNb; kk += 2) {
          const int k = kk + h;
          float av[2], bv[2];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const int ci = I * 64 + q * 32 + l32, cj = J * 64 + q * 32 + l32;
            if (a.strip_lds) {
              av[q] = (ci < w) ? -S[k * lds_w + ci] : 0.f;
              bv[q] = (cj < w) ? S[k * lds_w + cj] : 0.f;
            } else {
              av[q] = (ci < w) ? -G[(int64_t)(k0 + k) * n + k1 + ci] : 0.f;
              bv[q] = (cj < w) ? G[(int64_t)(k0 + k) * n + k1 + cj] : 0.f;
            }
          }
#pragma unroll
          for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nj = 0; nj < 2; ++nj) acc[mi][nj] = mfma(av[mi], bv[nj], acc[mi][nj]);
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int nj = 0; nj < 2; ++nj)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int row = k1 + I * 64 + mi * 32 + acc_row(r, lane);
              const int col = k1 + J * 64 + nj * 32 + l32;
              if (row < n && col < n) G[(int64_t)row * n + col] = acc[mi][nj][r];
            }
      }
    }
    __syncthreads();
  }
  __syncthreads();
  if (tid == 0) {
    const int f = (*ffail == INT_MAX) ? 0 : *ffail;
    if (!a.keep_info || a.info[b] == 0) a.info[b] = f;
  }
}

}  // namespace rnr
