// Right triangular solve Q = M R^-1 (R upper), batched, one 128-row block of one matrix per
// 256-thread workgroup -- the solve_triangular of reflection_no_reflectors.py:77.
//
// Left-looking over 64-column blocks c:  T = M[:, c] - Q[:, <c] R[<c, c];  Q[:, c] = T Dinv_c,
// where Dinv_c is the inverse of R's diagonal block (written by the Cholesky kernel).  Row
// blocks are independent, so the whole solve is one launch with batch * n/128 workgroups.
// Each wave owns 32 rows x 64 columns (two 32x32 MFMA accumulators).  The product with
// Q[:, <c] re-reads this workgroup's own earlier output (L2-resident) through double-
// buffered LDS chunks of 32 columns; T and Dinv_c reuse the chunk buffers.
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

constexpr int kTrsmRows = 128;

template <bool VEC4>
__global__ __launch_bounds__(256) void k_trsm(TrsmArgs a) {
  constexpr int RB = kTrsmRows, LDA = 33;
  // K-loop buffers: As[2][RB][33] (-Q rows x 32-column chunk), Bs[2][32][64] (R chunk).
  // After the loop the same memory holds Ts[RB][65] (over As) and Ds[64][64] (over Bs).
  __shared__ __attribute__((aligned(16))) float smA[2 * RB * LDA];
  __shared__ __attribute__((aligned(16))) float smB[2 * 32 * 64];
  __shared__ int prow[RB];
  __shared__ int mrow[RB];
  float* Ts = smA;
  float* Ds = smB;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5, wr = wid * 32;
  const int pid = xcd_remap(blockIdx.x, a.total);
  const int b = pid / a.nrb, r0 = (pid - b * a.nrb) * RB, n = a.n;
  const float* M = a.M + b * a.sm;
  const float* R = a.R + b * a.sr;
  const float* Dv = a.Dinv + (int64_t)b * n * 64;
  float* Q = a.Q + b * a.sq;
  float* Q2 = a.Q2 ? a.Q2 + b * a.sq2 : nullptr;

  if (tid < RB) {
    const int row = r0 + tid;
    prow[tid] = (row < n) ? (a.perm ? a.perm[(int64_t)b * n + row] : row) : 0;
    mrow[tid] = (row < n) ? (a.mperm ? a.mperm[(int64_t)b * n + row] : row) : 0;
  }
  __syncthreads();

  // staging: A chunk = RB x 32 floats (RB*8 float4), B chunk = 32 x 64 floats (512 float4)
  constexpr int AF4 = RB * 8 / 256, BF4 = 512 / 256;
  float ra[4 * AF4], rb[4 * BF4];
  auto gload = [&](int kc, int c0) {
    if constexpr (VEC4) {
#pragma unroll
      for (int p = 0; p < AF4; ++p) {
        const int idx = tid + 256 * p;
        const int i = idx >> 3, ca = 4 * (idx & 7);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r0 + i < n) v = *reinterpret_cast<const float4*>(Q + (int64_t)prow[i] * n + kc + ca);
        ra[4 * p] = v.x; ra[4 * p + 1] = v.y; ra[4 * p + 2] = v.z; ra[4 * p + 3] = v.w;
      }
#pragma unroll
      for (int p = 0; p < BF4; ++p) {
        const int idx = tid + 256 * p;
        const int k = idx >> 4, cb = c0 + 4 * (idx & 15);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (cb < n) v = *reinterpret_cast<const float4*>(R + (int64_t)(kc + k) * n + cb);
        rb[4 * p] = v.x; rb[4 * p + 1] = v.y; rb[4 * p + 2] = v.z; rb[4 * p + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int p = 0; p < 4 * AF4; ++p) {
        const int idx = tid + 256 * p;
        const int i = idx >> 5, ca = idx & 31;
        ra[p] = (r0 + i < n) ? Q[(int64_t)prow[i] * n + kc + ca] : 0.f;
      }
#pragma unroll
      for (int p = 0; p < 4 * BF4; ++p) {
        const int idx = tid + 256 * p;
        const int k = idx >> 6, cb = c0 + (idx & 63);
        rb[p] = (cb < n) ? R[(int64_t)(kc + k) * n + cb] : 0.f;
      }
    }
  };
  auto lstore = [&](int buf) {
    float* As = smA + buf * RB * LDA;
    float* Bs = smB + buf * 32 * 64;
    if constexpr (VEC4) {
#pragma unroll
      for (int p = 0; p < AF4; ++p) {
        const int idx = tid + 256 * p;
        const int i = idx >> 3, ca = 4 * (idx & 7);
#pragma unroll
        for (int q = 0; q < 4; ++q) As[i * LDA + ca + q] = -ra[4 * p + q];
      }
#pragma unroll
      for (int p = 0; p < BF4; ++p) {
        const int idx = tid + 256 * p;
        const int k = idx >> 4, cb = 4 * (idx & 15);
        *reinterpret_cast<float4*>(&Bs[k * 64 + cb]) =
            make_float4(rb[4 * p], rb[4 * p + 1], rb[4 * p + 2], rb[4 * p + 3]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < 4 * AF4; ++p) {
        const int idx = tid + 256 * p;
        As[(idx >> 5) * LDA + (idx & 31)] = -ra[p];
      }
#pragma unroll
      for (int p = 0; p < 4 * BF4; ++p) {
        const int idx = tid + 256 * p;
        Bs[(idx >> 6) * 64 + (idx & 63)] = rb[p];
      }
    }
  };

  for (int c0 = 0; c0 < n; c0 += 64) {
    f32x16 acc[2];
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = wr + acc_row(r, lane), row = r0 + lrow, col = c0 + nj * 32 + l32;
        float v = 0.f;
        if (row < n && col < n) {
          if (a.mperm)
            v = (col < row) ? M[(int64_t)mrow[lrow] * n + col] : (col == row ? 1.f : 0.f);
          else
            v = M[(int64_t)row * n + col];
        }
        acc[nj][r] = v;
      }
    if (c0 > 0) {
      int buf = 0;
      gload(0, c0);
      lstore(0);
      __syncthreads();
      for (int kc = 0; kc < c0; kc += 32) {
        const bool more = kc + 32 < c0;
        if (more) gload(kc + 32, c0);
        const float* As = smA + buf * RB * LDA;
        const float* Bs = smB + buf * 32 * 64;
#pragma unroll
        for (int kk = 0; kk < 32; kk += 2) {
          const int k = kk + h;
          const float av = As[(wr + l32) * LDA + k];
          acc[0] = mfma(av, Bs[k * 64 + l32], acc[0]);
          acc[1] = mfma(av, Bs[k * 64 + 32 + l32], acc[1]);
        }
        if (more) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
      }
    }
    // T -> LDS (over the A buffers), Dinv_c -> LDS (over the B buffers)
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int r = 0; r < 16; ++r) Ts[(wr + acc_row(r, lane)) * 65 + nj * 32 + l32] = acc[nj][r];
    for (int idx = tid; idx < 64 * 64; idx += 256) {
      const int k = idx >> 6, j = idx & 63;
      Ds[k * 64 + j] = (c0 + k < n) ? Dv[(int64_t)(c0 + k) * 64 + j] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) acc[nj] = zero16();
#pragma unroll 8
    for (int kk = 0; kk < 64; kk += 2) {
      const int k = kk + h;
      const float av = Ts[(wr + l32) * 65 + k];
      acc[0] = mfma(av, Ds[k * 64 + l32], acc[0]);
      acc[1] = mfma(av, Ds[k * 64 + 32 + l32], acc[1]);
    }
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = wr + acc_row(r, lane), col = c0 + nj * 32 + l32;
        if (r0 + lrow < n && col < n) {
          const int64_t off = (int64_t)prow[lrow] * n + col;
          Q[off] = acc[nj][r];
          if (Q2) Q2[off] = acc[nj][r];
        }
      }
    __syncthreads();
  }
}

}  // namespace rnr
