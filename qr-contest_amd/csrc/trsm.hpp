// Right triangular solve Q = M R^-1 (R upper), batched, one 64-row block of one matrix per
// 256-thread workgroup -- the solve_triangular of reflection_no_reflectors.py:77.
//
// Left-looking over 64-column blocks c:  T = M[:, c] - Q[:, <c] R[<c, c];  Q[:, c] = T Dinv_c,
// where Dinv_c is the inverse of R's diagonal block (written by the Cholesky kernel).  Row
// blocks are independent, so the whole solve is one launch with batch * n/64 workgroups.
// The product with Q[:, <c] re-reads this workgroup's own earlier output (L2-resident)
// through double-buffered LDS chunks of 32 columns.
//
// Optional row scatter: output row i goes to row perm[i] (the frame's Q = P Q2,
// reflection_no_reflectors.py:81, done as a gather instead of a dense product), optionally
// to a second buffer too (the chart then runs in place on that copy).
#pragma once
#include "common.hpp"

namespace rnr {

struct TrsmArgs {
  const float* M;
  int64_t sm;
  const float* R;
  int64_t sr;
  const float* Dinv;  // [batch][n][64]
  float* Q;
  int64_t sq;
  float* Q2;          // optional copy (nullptr: none), batch stride sq2
  int64_t sq2;
  const int* perm;    // optional row scatter [batch][n] (nullptr: identity)
  const int* mperm;   // non-null: M is the unit-lower L stored in A's row order (the LU's
                      // in-place factor); logical row r is physical row mperm[b][r]
  int n, nrb, total;
};

template <bool VEC4>
__global__ __launch_bounds__(256) void k_trsm(TrsmArgs a) {
  __shared__ float As[2][64][33];                             // -Q[rows][k-chunk]
  __shared__ __attribute__((aligned(16))) float Bs[2][32][64];  // R[k-chunk][c-block]
  __shared__ float Ts[64][65];
  __shared__ float Ds[64][64];
  __shared__ int prow[64];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5, mi = wid >> 1, nj = wid & 1;
  const int pid = xcd_remap(blockIdx.x, a.total);
  const int b = pid / a.nrb, r0 = (pid - b * a.nrb) * 64, n = a.n;
  const float* M = a.M + b * a.sm;
  const float* R = a.R + b * a.sr;
  const float* Dv = a.Dinv + (int64_t)b * n * 64;
  float* Q = a.Q + b * a.sq;
  float* Q2 = a.Q2 ? a.Q2 + b * a.sq2 : nullptr;

  if (tid < 64) {
    const int row = r0 + tid;
    prow[tid] = (row < n) ? (a.perm ? a.perm[(int64_t)b * n + row] : row) : 0;
  }
  __syncthreads();

  float ra[8], rb[8];
  auto gload = [&](int kc, int c0) {
    if constexpr (VEC4) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int idx = tid + 256 * p;
        const int i = idx >> 3, ca = 4 * (idx & 7);
        float4 va = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r0 + i < n) va = *reinterpret_cast<const float4*>(Q + (int64_t)prow[i] * n + kc + ca);
        const int k = idx >> 4, cb = c0 + 4 * (idx & 15);
        float4 vb = make_float4(0.f, 0.f, 0.f, 0.f);
        if (cb < n) vb = *reinterpret_cast<const float4*>(R + (int64_t)(kc + k) * n + cb);
        ra[4 * p] = va.x; ra[4 * p + 1] = va.y; ra[4 * p + 2] = va.z; ra[4 * p + 3] = va.w;
        rb[4 * p] = vb.x; rb[4 * p + 1] = vb.y; rb[4 * p + 2] = vb.z; rb[4 * p + 3] = vb.w;
      }
    } else {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int idx = tid + 256 * p;
        const int i = idx >> 5, ca = idx & 31;
        ra[p] = (r0 + i < n) ? Q[(int64_t)prow[i] * n + kc + ca] : 0.f;
        const int k = idx >> 6, cb = c0 + (idx & 63);
        rb[p] = (cb < n) ? R[(int64_t)(kc + k) * n + cb] : 0.f;
      }
    }
  };
  auto lstore = [&](int buf) {
    if constexpr (VEC4) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int idx = tid + 256 * p;
        const int i = idx >> 3, ca = 4 * (idx & 7);
#pragma unroll
        for (int q = 0; q < 4; ++q) As[buf][i][ca + q] = -ra[4 * p + q];
        const int k = idx >> 4, cb = 4 * (idx & 15);
        *reinterpret_cast<float4*>(&Bs[buf][k][cb]) =
            make_float4(rb[4 * p], rb[4 * p + 1], rb[4 * p + 2], rb[4 * p + 3]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int idx = tid + 256 * p;
        As[buf][idx >> 5][idx & 31] = -ra[p];
        Bs[buf][idx >> 6][idx & 63] = rb[p];
      }
    }
  };

  for (int c0 = 0; c0 < n; c0 += 64) {
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = r0 + mi * 32 + acc_row(r, lane), col = c0 + nj * 32 + l32;
      if (a.mperm)
        acc[r] = (row < n && col < row) ? M[(int64_t)a.mperm[(int64_t)b * n + row] * n + col]
                                        : (row < n && col == row ? 1.f : 0.f);
      else
        acc[r] = (row < n && col < n) ? M[(int64_t)row * n + col] : 0.f;
    }
    if (c0 > 0) {
      int buf = 0;
      gload(0, c0);
      lstore(0);
      __syncthreads();
      for (int kc = 0; kc < c0; kc += 32) {
        const bool more = kc + 32 < c0;
        if (more) gload(kc + 32, c0);
#pragma unroll
        for (int kk = 0; kk < 32; kk += 2) {
          const int k = kk + h;
          acc = mfma(As[buf][mi * 32 + l32][k], Bs[buf][k][nj * 32 + l32], acc);
        }
        if (more) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Ts[mi * 32 + acc_row(r, lane)][nj * 32 + l32] = acc[r];
    for (int idx = tid; idx < 64 * 64; idx += 256) {
      const int k = idx >> 6, j = idx & 63;
      Ds[k][j] = (c0 + k < n) ? Dv[(int64_t)(c0 + k) * 64 + j] : 0.f;
    }
    __syncthreads();
    acc = zero16();
#pragma unroll 8
    for (int kk = 0; kk < 64; kk += 2) {
      const int k = kk + h;
      acc = mfma(Ts[mi * 32 + l32][k], Ds[k][nj * 32 + l32], acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lrow = mi * 32 + acc_row(r, lane), col = c0 + nj * 32 + l32;
      if (r0 + lrow < n && col < n) {
        const int64_t off = (int64_t)prow[lrow] * n + col;
        Q[off] = acc[r];
        if (Q2) Q2[off] = acc[r];
      }
    }
    __syncthreads();
  }
}

}  // namespace rnr
