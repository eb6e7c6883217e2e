// Blocked right-looking elimination of one matrix per 512-thread workgroup.
//
// PIVOT = true : partial-pivot LU, A[perm] = L U (torch.linalg.lu / LAPACK getrf
//                semantics, first maximum of |a_ij| wins) -- reflection_no_reflectors.py:66.
//                Rows are never moved: a logical->physical row map (perm) is kept in LDS and
//                every access goes through it, so the finished factor sits in A's own row
//                order and one gather at the end writes L in pivoted order with a unit
//                diagonal and exact zeros above it.  U is not kept: the reference drops it.
// PIVOT = false: the chart, the sign-ruled unpivoted LU of I - Q S run on the Q copy
//                (reflection_no_reflectors.py:139-174): s_k = +1 iff |1-d| >= |1+d|
//                (:150-155), multipliers (-s_k M[i,k]) / pivot (:157-158), then
//                tau_k = 2 / (1 + sum_{i>k} Y[i,k]^2) (:192).  Runs in place on H.
//
// Per panel of nb columns: the panel (rows k0..n) is factored in LDS; it is written back;
// the unit-lower L11 is inverted in LDS; then, chunk by chunk of 64 trailing columns,
// U12 = L11^-1 A12 and A22 -= L21 U12 run on MFMA.  Both trailing products read their
// operands from LDS; only A22 itself streams through HBM/L2, once per panel.
#pragma once
#include "common.hpp"

namespace rnr {

struct LuArgs {
  const float* src;  // data read by the first panel step (A for the LU, H for the chart)
  int64_t ss;
  float* dst;        // working matrix (LU: workspace W; chart: H itself)
  int64_t sd;
  int n, nb;
  int* perm;         // PIVOT: logical -> original row, [batch][n]
  float* L;          // PIVOT: unit-lower factor, [batch][n][n]
  int64_t sl;
  float* s;          // chart: signs, [batch][n]
  float* tau;        // chart: tau, [batch][n]
};

constexpr int kLuThreads = 512;

inline size_t lu_lds_bytes(int n, int nb) {
  return sizeof(float) * ((size_t)n * (nb + 1) + (size_t)nb * 64 + (size_t)n + 32);
}

template <bool PIVOT>
__global__ __launch_bounds__(kLuThreads) void k_lu(LuArgs a) {
  extern __shared__ float smem[];
  const int n = a.n, nb = a.nb, ldp = nb + 1;
  float* P = smem;                                     // panel, n x (nb+1)
  float* U = P + (size_t)n * ldp;                      // -U12 chunk [nb][64]; L11^-1 scratch
  int* pl = reinterpret_cast<int*>(U + nb * 64);       // logical -> physical row
  float* redv = reinterpret_cast<float*>(pl + n);      // pivot search, one entry per wave
  int* redi = reinterpret_cast<int*>(redv + 8);

  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const float* src = a.src + b * a.ss;
  float* dst = a.dst + b * a.sd;

  if (PIVOT)
    for (int i = tid; i < n; i += kLuThreads) pl[i] = i;
  __syncthreads();

  for (int k0 = 0; k0 < n; k0 += nb) {
    const int kb = min(nb, n - k0), m = n - k0, k1 = k0 + kb;
    const float* cur = (k0 == 0) ? src : dst;

    // ---- load the panel: logical rows k0..n-1, columns k0..k0+nb (zero padded)
    for (int idx = tid; idx < m * nb; idx += kLuThreads) {
      const int r = idx / nb, c = idx - r * nb;
      const int pr = PIVOT ? pl[k0 + r] : k0 + r;
      P[r * ldp + c] = (c < kb) ? cur[(int64_t)pr * n + k0 + c] : 0.f;
    }
    __syncthreads();

    // ---- factor the panel column by column
    for (int j = 0; j < kb; ++j) {
      if constexpr (PIVOT) {
        // first maximum of |P[r][j]| over r in [j, m): per thread rows ascend, ties across
        // threads and waves go to the smaller row index
        float bv = 0.f, babs = -1.f;
        int bi = INT_MAX;
        for (int r = j + tid; r < m; r += kLuThreads) {
          const float v = P[r * ldp + j];
          const float av = fabsf(v);
          if (av > babs) { babs = av; bv = v; bi = r; }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
          const float ob = __shfl_xor(babs, off);
          const float ov = __shfl_xor(bv, off);
          const int oi = __shfl_xor(bi, off);
          if (ob > babs || (ob == babs && oi < bi)) { babs = ob; bv = ov; bi = oi; }
        }
        if (lane == 0) { redv[wid] = bv; redi[wid] = bi; }
        __syncthreads();
        float pv = 0.f, pabs = -1.f;
        int p = INT_MAX;
#pragma unroll
        for (int w = 0; w < kLuThreads / 64; ++w) {
          const float v = redv[w];
          const int i = redi[w];
          const float av = fabsf(v);
          if (i != INT_MAX && (av > pabs || (av == pabs && i < p))) { pabs = av; pv = v; p = i; }
        }
        if (p == INT_MAX) { p = j; pv = P[j * ldp + j]; }   // only non-finite columns get here
        if (p != j) {
          for (int c = tid; c < nb; c += kLuThreads) {
            const float t = P[j * ldp + c];
            P[j * ldp + c] = P[p * ldp + c];
            P[p * ldp + c] = t;
          }
          if (tid == 0) {
            const int t = pl[k0 + j];
            pl[k0 + j] = pl[k0 + p];
            pl[k0 + p] = t;
          }
        }
        __syncthreads();
        // LAPACK xGETRF2: scale by the reciprocal unless the pivot is subnormal; a zero
        // pivot leaves the column as it is (the update below is then a no-op).
        const bool nz = pv != 0.f;
        const bool recip = fabsf(pv) >= 1.17549435e-38f;
        const float inv = 1.f / pv;
        for (int r = j + 1 + tid; r < m; r += kLuThreads) {
          float l = P[r * ldp + j];
          if (nz) {
            l = recip ? l * inv : l / pv;
            P[r * ldp + j] = l;
          }
          for (int c = j + 1; c < kb; ++c) P[r * ldp + c] -= l * P[j * ldp + c];
        }
        __syncthreads();
      } else {
        const float d = P[j * ldp + j];
        const float pp = 1.f - d, pm = 1.f + d;
        const bool plus = fabsf(pp) >= fabsf(pm);
        const float sk = plus ? 1.f : -1.f;
        const float piv = plus ? pp : pm;
        if (tid == 0) a.s[(int64_t)b * n + k0 + j] = sk;
        for (int r = j + 1 + tid; r < m; r += kLuThreads) {
          const float mult = (-sk * P[r * ldp + j]) / piv;
          P[r * ldp + j] = mult;
          for (int c = j + 1; c < kb; ++c) P[r * ldp + c] -= mult * P[j * ldp + c];
        }
        __syncthreads();
      }
    }

    if constexpr (!PIVOT) {
      // tau of the panel's columns from the finished multipliers (rows below the diagonal)
      const int c = tid >> 3, sub = tid & 7;
      if (c < kb) {
        float acc = 0.f;
        for (int r = c + 1 + sub; r < m; r += 8) {
          const float y = P[r * ldp + c];
          acc += y * y;
        }
        acc = group8_sum(acc);
        if (sub == 0) a.tau[(int64_t)b * n + k0 + c] = 2.f / (acc + 1.f);
      }
    }

    // ---- write the factored panel back (same physical rows it came from)
    for (int idx = tid; idx < m * kb; idx += kLuThreads) {
      const int r = idx / kb, c = idx - r * kb;
      const int pr = PIVOT ? pl[k0 + r] : k0 + r;
      dst[(int64_t)pr * n + k0 + c] = P[r * ldp + c];
    }
    if (k1 >= n) break;  // uniform: no trailing matrix (and kb == nb below this line)

    // ---- X = L11^-1 (unit lower): 8 lanes per column, forward substitution down the
    //      column, into U[i*nb + j]; then copied over L11/U11 in the panel (unit diagonal,
    //      zeros above) so that rows 0..nb of P hold X for the MFMA below.
    {
      const int j = tid >> 3, sub = tid & 7;
      if (j < nb) {
        for (int i = j + 1; i < nb; ++i) {
          float part = 0.f;
          for (int q = j + sub; q < i; q += 8) {
            const float xq = (q == j) ? 1.f : U[q * nb + j];
            part += P[i * ldp + q] * xq;
          }
          part = group8_sum(part);
          if (sub == 0) U[i * nb + j] = -part;
          wave_lds_order();
        }
      }
    }
    __syncthreads();
    for (int idx = tid; idx < nb * nb; idx += kLuThreads) {
      const int i = idx / nb, c = idx - i * nb;
      P[i * ldp + c] = (c < i) ? U[i * nb + c] : (c == i ? 1.f : 0.f);
    }
    __syncthreads();

    // ---- trailing update in chunks of 64 columns
    for (int c0 = k1; c0 < n; c0 += 64) {
      // -U12 chunk = -(X * A12[:, c0:c0+64]) into U[k][j], waves 0 .. 2*ceil(nb/32)-1
      const int nqm = (nb + 31) >> 5;
      if (wid < 2 * nqm) {
        const int mi = wid >> 1, nj = wid & 1;
        const int i = mi * 32 + l32;
        const int col = c0 + nj * 32 + l32;
        f32x16 acc = zero16();
        for (int kk = 0; kk < nb; kk += 2) {
          const int k = kk + h;
          const float av = (i < nb) ? P[i * ldp + k] : 0.f;
          const int pr = PIVOT ? pl[k0 + k] : k0 + k;
          const float bv = (col < n) ? cur[(int64_t)pr * n + col] : 0.f;
          acc = mfma(av, bv, acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ii = mi * 32 + acc_row(r, lane);
          if (ii < nb) U[ii * 64 + nj * 32 + l32] = -acc[r];
        }
      }
      __syncthreads();

      // A22[:, chunk] += L21 * (-U12): one 32-row tile per wave at a time
      const int ntr = (n - k1 + 31) >> 5;
      for (int tr = wid; tr < ntr; tr += kLuThreads / 64) {
        const int r0 = k1 + tr * 32;
        f32x16 acc[2];
#pragma unroll
        for (int nj = 0; nj < 2; ++nj)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = r0 + acc_row(r, lane), col = c0 + nj * 32 + l32;
            float v = 0.f;
            if (row < n && col < n) {
              const int pr = PIVOT ? pl[row] : row;
              v = cur[(int64_t)pr * n + col];
            }
            acc[nj][r] = v;
          }
        const int lr = r0 - k0 + l32;
        for (int kk = 0; kk < nb; kk += 2) {
          const int k = kk + h;
          const float av = (lr < m) ? P[lr * ldp + k] : 0.f;
          acc[0] = mfma(av, U[k * 64 + l32], acc[0]);
          acc[1] = mfma(av, U[k * 64 + 32 + l32], acc[1]);
        }
#pragma unroll
        for (int nj = 0; nj < 2; ++nj)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = r0 + acc_row(r, lane), col = c0 + nj * 32 + l32;
            if (row < n && col < n) {
              const int pr = PIVOT ? pl[row] : row;
              dst[(int64_t)pr * n + col] = acc[nj][r];
            }
          }
      }
      __syncthreads();
    }
  }
  __syncthreads();

  if constexpr (PIVOT) {
    for (int i = tid; i < n; i += kLuThreads) a.perm[(int64_t)b * n + i] = pl[i];
    float* L = a.L + b * a.sl;
    for (int idx = tid; idx < n * n; idx += kLuThreads) {
      const int i = idx / n, j = idx - i * n;
      L[idx] = (j < i) ? dst[(int64_t)pl[i] * n + j] : (j == i ? 1.f : 0.f);
    }
  }
}

}  // namespace rnr
