// Right triangular solve Q = M R^-1 (R upper), batched, one 128-row block of one matrix per
// 256-thread workgroup -- the solve_triangular of reflection_no_reflectors.py:77.
//
// With 64-column blocks, Dinv_c = R_cc^-1 and W[k][c] = R[k][c] Dinv_c (k < c; both written
// by the Cholesky kernel), block column c of the solution is
//
//     Q[:, c] = M[:, c] Dinv_c - sum_{k < c} Q[:, k] W[k][c],
//
// one MFMA product over K = 64 (c + 1): the chunks k < c take -Q (this workgroup's own
// earlier output, L2-resident) against W, the last chunk takes M against Dinv_c.  The result
// leaves the accumulators straight for HBM -- no per-block transpose or second product.  Row
// blocks are independent, so the whole solve is one launch with batch * n/128 workgroups.
// Each wave owns 32 rows x 64 columns (two 32x32 MFMA accumulators); K is staged through
// double-buffered LDS chunks of 16 (26 KB of LDS: several workgroups per CU).
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
  const float* Wm;    // W[k][c] blocks at their R positions (rows k < c of block column c)
  int64_t sw;
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

struct WblkArgs {
  const float* R;     // upper factor, stride sr (only the blocks above the diagonal are read)
  int64_t sr;
  const float* Dinv;  // [batch][n][64]
  float* Wm;          // out: W blocks at their R positions, stride sw
  int64_t sw;
  int n, ncol, total;
  int vec4;           // n % 4 == 0 and R 16-byte aligned (batch stride too)
};

// W[:c, c] = R[:c, c] Dinv_c for block column c >= 1 (64-wide blocks): one block column of
// one matrix per 256-thread workgroup.  Dinv_c is staged in LDS once; each wave takes 32-row
// strips of the rows above the diagonal block: the strip is read row-contiguously (16 lanes
// per 64-float row, float4 each) into the wave's own LDS tile, then multiplied on
// v_mfma_f32_32x32x2f32 (two 32x32 accumulators over the 64 columns, K = 64), so every R entry
// is read from HBM once and coalesced.
__global__ __launch_bounds__(256) void k_wblocks(WblkArgs a) {
  constexpr int LDR = 65;  // odd stride: the MFMA operand reads (32 rows, one column) are conflict-free
  __shared__ __attribute__((aligned(16))) float Ds[64 * 64];
  __shared__ float Rs[4][32 * LDR];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int pid = xcd_remap(blockIdx.x, a.total);
  const int b = pid / a.ncol, c = 1 + pid - b * a.ncol, n = a.n, c0 = 64 * c;
  const float* R = a.R + b * a.sr;
  const float* Dv = a.Dinv + (int64_t)b * n * 64;
  float* W = a.Wm + b * a.sw;
  float* Rw = Rs[wid];
  for (int idx = tid; idx < 64 * 16; idx += 256) {
    const int k = idx >> 4, j4 = idx & 15;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c0 + k < n) v = reinterpret_cast<const float4*>(Dv + (int64_t)(c0 + k) * 64)[j4];  // zero past the block
    reinterpret_cast<float4*>(Ds + k * 64)[j4] = v;
  }
  __syncthreads();
  for (int strip = wid; strip < 2 * c; strip += 4) {
    // strip rows 32 strip .. +31 (< c0 <= n), columns c0 .. c0 + 63: 4 rows per instruction
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int rr = 4 * u + (lane >> 4), col = c0 + 4 * (lane & 15);
      const float* src = R + (int64_t)(32 * strip + rr) * n + col;
      float4 v;
      if (a.vec4 && col + 3 < n) {
        v = *reinterpret_cast<const float4*>(src);
      } else {
        v.x = (col < n) ? src[0] : 0.f;
        v.y = (col + 1 < n) ? src[1] : 0.f;
        v.z = (col + 2 < n) ? src[2] : 0.f;
        v.w = (col + 3 < n) ? src[3] : 0.f;
      }
      float* d = Rw + rr * LDR + 4 * (lane & 15);
      d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    }
    wave_lds_order();
    f32x16 acc0 = zero16(), acc1 = zero16();
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      const int k = 2 * t + h;
      const float x = Rw[l32 * LDR + k];
      acc0 = mfma(x, Ds[k * 64 + l32], acc0);
      acc1 = mfma(x, Ds[k * 64 + 32 + l32], acc1);
    }
    wave_lds_order();  // the next strip's tile stores stay behind these reads
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t o = (int64_t)(32 * strip + acc_row(r, lane)) * n + c0 + l32;
      if (c0 + l32 < n) W[o] = acc0[r];
      if (c0 + 32 + l32 < n) W[o + 32] = acc1[r];
    }
  }
}

template <bool VEC4>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_trsm(TrsmArgs a) {
  constexpr int RB = kTrsmRows, BK = 16, LDA = BK + 1;
  __shared__ __attribute__((aligned(16))) float smA[2 * RB * LDA];  // A chunk: RB rows x BK
  __shared__ __attribute__((aligned(16))) float smB[2 * BK * 64];   // B chunk: BK x 64
  __shared__ int prow[RB];
  __shared__ int mrow[RB];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5, wr = wid * 32;
  const int pid = xcd_remap(blockIdx.x, a.total);
  const int b = pid / a.nrb, r0 = (pid - b * a.nrb) * RB, n = a.n;
  const float* M = a.M + b * a.sm;
  const float* Wm = a.Wm + b * a.sw;
  const float* Dv = a.Dinv + (int64_t)b * n * 64;
  float* Q = a.Q + b * a.sq;
  float* Q2 = a.Q2 ? a.Q2 + b * a.sq2 : nullptr;

  if (tid < RB) {
    const int row = r0 + tid;
    prow[tid] = (row < n) ? (a.perm ? a.perm[(int64_t)b * n + row] : row) : 0;
    mrow[tid] = (row < n) ? (a.mperm ? a.mperm[(int64_t)b * n + row] : row) : 0;
  }
  __syncthreads();

  // staging: A chunk = RB x BK floats (2 float4 per thread), B chunk = BK x 64 floats (1)
  float ra[8], rb[4];
  // element (i, k) of the A operand of chunk column k: -Q (k < c0) or M (k >= c0)
  auto a_elem = [&](int i, int k, int c0) -> float {
    const int row = r0 + i;
    if (row >= n || k >= n) return 0.f;
    if (k < c0) return -Q[(int64_t)prow[i] * n + k];
    if (a.mperm) return (k < row) ? M[(int64_t)mrow[i] * n + k] : (k == row ? 1.f : 0.f);
    return M[(int64_t)row * n + k];
  };
  auto gload = [&](int kc, int c0) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int idx = tid + 256 * p;
      const int i = idx >> 2, ca = 4 * (idx & 3), k = kc + ca;
      const int row = r0 + i;
      if (VEC4 && row < n && k + 3 < n && (k < c0 ? k + 3 < c0 : !a.mperm)) {
        const float* src = (k < c0) ? Q + (int64_t)prow[i] * n + k : M + (int64_t)row * n + k;
        const float4 v = *reinterpret_cast<const float4*>(src);
        const float s = (k < c0) ? -1.f : 1.f;
        ra[4 * p] = s * v.x; ra[4 * p + 1] = s * v.y; ra[4 * p + 2] = s * v.z; ra[4 * p + 3] = s * v.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[4 * p + q] = a_elem(i, k + q, c0);
      }
    }
    {
      const int kr = tid >> 4, cb = 4 * (tid & 15), k = kc + kr, col = c0 + cb;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (k < n) {
        if (k < c0) {
          if (VEC4 && col + 3 < n) {
            v = *reinterpret_cast<const float4*>(Wm + (int64_t)k * n + col);
          } else {
            v.x = (col < n) ? Wm[(int64_t)k * n + col] : 0.f;
            v.y = (col + 1 < n) ? Wm[(int64_t)k * n + col + 1] : 0.f;
            v.z = (col + 2 < n) ? Wm[(int64_t)k * n + col + 2] : 0.f;
            v.w = (col + 3 < n) ? Wm[(int64_t)k * n + col + 3] : 0.f;
          }
        } else {
          v = *reinterpret_cast<const float4*>(Dv + (int64_t)k * 64 + cb);  // zero past the block
        }
      }
      rb[0] = v.x; rb[1] = v.y; rb[2] = v.z; rb[3] = v.w;
    }
  };
  auto lstore = [&](int buf) {
    float* As = smA + buf * RB * LDA;
    float* Bs = smB + buf * BK * 64;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int idx = tid + 256 * p;
      const int i = idx >> 2, ca = 4 * (idx & 3);
#pragma unroll
      for (int q = 0; q < 4; ++q) As[i * LDA + ca + q] = ra[4 * p + q];
    }
    *reinterpret_cast<float4*>(&Bs[(tid >> 4) * 64 + 4 * (tid & 15)]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
  };

  for (int c0 = 0; c0 < n; c0 += 64) {
    const int kend = min(c0 + 64, n);
    f32x16 acc[2] = {zero16(), zero16()};
    int buf = 0;
    gload(0, c0);
    lstore(0);
    __syncthreads();
    for (int kc = 0; kc < kend; kc += BK) {
      const bool more = kc + BK < kend;
      if (more) gload(kc + BK, c0);
      const float* As = smA + buf * RB * LDA;
      const float* Bs = smB + buf * BK * 64;
#pragma unroll
      for (int kk = 0; kk < BK; kk += 2) {
        const int k = kk + h;
        const float av = As[(wr + l32) * LDA + k];
        acc[0] = mfma(av, Bs[k * 64 + l32], acc[0]);
        acc[1] = mfma(av, Bs[k * 64 + 32 + l32], acc[1]);
      }
      if (more) lstore(buf ^ 1);
      __syncthreads();
      buf ^= 1;
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
    // the next block column reads these outputs back (other threads of this workgroup)
    __syncthreads();
  }
}

}  // namespace rnr
