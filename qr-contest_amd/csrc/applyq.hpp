// Y <- op(Q) Y for the Q of a compact (H, tau) factorization (LAPACK / torch.geqrf layout):
// Q = H_0 H_1 ... H_{n-1}, H_k = I - tau_k v_k v_k^T with v_k = e_k + H[k+1:, k].  The
// consumer of the path's output (README.md:122-128: Q = householder_product(H, tau)).
//
// Blocked WY: panels of PB reflectors, each P = H_{k0} ... H_{k0+PB-1} = I - V T V^T with T
// from the compact-WY recurrence (LAPACK dlarft, forward / columnwise):
// T[j][j] = tau_j, T[0:j, j] = -tau_j T[0:j, 0:j] (V^T v_j)[0:j].  op = Q applies the panels
// last first (Y <- P Y), op = Q^T first to last (Y <- P^T Y = Y - V T^T V^T Y).  One matrix per
// 512-thread workgroup and 512-column chunk (grid (batch, ceil(nc / 512))), one column of Y per
// thread, V / T in LDS; only rows >= k0 change.  Columns are independent, so the chunks of one
// matrix need no communication (each rebuilds the panel's T).
// IDENT: Y starts as the identity (orgqr), and then a panel leaves the columns left of k0
// untouched (they are still unit vectors).
// T is the arithmetic type, TH the storage type of the reflectors (float for this library's
// output, double for the generator's Haar factors).
#pragma once
#include "common.hpp"

namespace rnr {

constexpr int kApplyQThreads = 512;

template <typename T, typename TH = float>
struct ApplyQArgs {
  const TH* H;       // [batch][n][n]
  const TH* tau;     // [batch][n]
  T* Y;              // [batch] x n rows x nc columns, row stride ldy, batch stride sy
  int64_t sy;
  int ldy;
  int n, nc;
};

template <typename T, int PB>
inline size_t applyq_lds(int n) { return sizeof(T) * ((size_t)n * PB + 2 * PB * PB); }

inline dim3 applyq_grid(int64_t batch, int nc) {
  return dim3((unsigned)batch, (unsigned)((nc + kApplyQThreads - 1) / kApplyQThreads));
}

template <typename T, int PB, bool TRANS, bool IDENT, typename TH = float>
__global__ __launch_bounds__(kApplyQThreads) void k_apply_q(ApplyQArgs<T, TH> a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smraw[];
  T* V = reinterpret_cast<T*>(smraw);  // [m][PB]: row k0 + r of reflector k0 + j
  const int n = a.n, nc = a.nc, b = blockIdx.x, tid = threadIdx.x;
  T* Tm = V + (size_t)n * PB;          // [PB][PB] upper triangular
  T* S = Tm + PB * PB;                 // [PB][PB] V^T V (strict upper part)
  const TH* H = a.H + (int64_t)b * n * n;
  const TH* tau = a.tau + (int64_t)b * n;
  T* Y = a.Y + b * a.sy;
  const int ld = a.ldy;
  const int c = blockIdx.y * kApplyQThreads + tid;  // this thread's column

  if (IDENT && c < nc)
    for (int i = 0; i < n; ++i) Y[(int64_t)i * ld + c] = (i == c) ? T(1) : T(0);

  const int np = (n + PB - 1) / PB;
  for (int s = 0; s < np; ++s) {
    const int p = TRANS ? s : np - 1 - s;
    const int k0 = p * PB, kb = min(PB, n - k0), m = n - k0;
    for (int idx = tid; idx < m * PB; idx += kApplyQThreads) {
      const int r = idx / PB, j = idx - r * PB;
      T v = T(0);
      if (j < kb) v = (r < j) ? T(0) : (r == j ? T(1) : (T)H[(int64_t)(k0 + r) * n + k0 + j]);
      V[idx] = v;
    }
    __syncthreads();
    if (tid < PB * PB) {
      const int i = tid / PB, j = tid - i * PB;
      T acc = T(0);
      if (i < j && j < kb)
        for (int r = j; r < m; ++r) acc += V[r * PB + i] * V[r * PB + j];
      S[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
      for (int j = 0; j < PB; ++j) {
        const T tj = (j < kb) ? (T)tau[k0 + j] : T(0);
        for (int i = 0; i < j; ++i) {
          T acc = T(0);
          for (int l = i; l < j; ++l) acc += Tm[i * PB + l] * S[l * PB + j];
          Tm[i * PB + j] = -tj * acc;
        }
        Tm[j * PB + j] = tj;
        for (int i = j + 1; i < PB; ++i) Tm[i * PB + j] = T(0);
      }
    }
    __syncthreads();
    if (c < nc && (!IDENT || c >= k0)) {
      T z[PB];
#pragma unroll
      for (int j = 0; j < PB; ++j) z[j] = T(0);
      for (int r = 0; r < m; ++r) {
        const T y = Y[(int64_t)(k0 + r) * ld + c];
#pragma unroll
        for (int j = 0; j < PB; ++j) z[j] += V[r * PB + j] * y;
      }
      T w[PB];
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        T acc = T(0);
        if (TRANS) {
#pragma unroll
          for (int j = 0; j <= i; ++j) acc += Tm[j * PB + i] * z[j];
        } else {
#pragma unroll
          for (int j = i; j < PB; ++j) acc += Tm[i * PB + j] * z[j];
        }
        w[i] = acc;
      }
      for (int r = 0; r < m; ++r) {
        T y = Y[(int64_t)(k0 + r) * ld + c];
#pragma unroll
        for (int j = 0; j < PB; ++j) y -= V[r * PB + j] * w[j];
        Y[(int64_t)(k0 + r) * ld + c] = y;
      }
    }
    __syncthreads();
  }
}

}  // namespace rnr
