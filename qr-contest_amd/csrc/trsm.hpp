// Right triangular solve Q = M R^-1 (R upper), batched, one 128-row block of one matrix per
// 256-thread workgroup -- the solve_triangular of reflection_no_reflectors.py:77.
//
// With 64-column blocks, Dinv_c = R_cc^-1 and the negated W[k][c] = -R[k][c] Dinv_c (k < c;
// both written after the Cholesky factor), block column c of the solution is
//
//     Q[:, c] = M[:, c] Dinv_c + sum_{k < c} Q[:, k] (-W[k][c]),
//
// one MFMA product over K = 64 (c + 1): the chunks k < c take Q (this workgroup's own
// earlier output, L2-resident) against -W, the last chunk takes M against Dinv_c.  The result
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
  const float* Wm;    // -W[k][c] blocks at their R positions (rows k < c of block column c)
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
  float* Wm;          // out: -W blocks at their R positions, stride sw
  int64_t sw;
  int n, ncol, total;
  int vec4;           // n % 4 == 0 and R 16-byte aligned (batch stride too)
  int lpt;            // total % 8 == 0 and ncol | total / 8: largest block columns first
};

// -W[:c, c] = -R[:c, c] Dinv_c for block column c >= 1 (64-wide blocks): one block column of
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
  // block column c has 2c strips: each XCD's matrices are dispatched block column by block
  // column, largest first, so the small ones fill the tail (same matrices per XCD as xcd_remap)
  int b, c;
  if (a.lpt) {
    const int mpx = a.total / 8 / a.ncol, q = blockIdx.x >> 3, cr = q / mpx;
    b = (blockIdx.x & 7) * mpx + (q - cr * mpx);
    c = a.ncol - cr;
  } else {
    const int pid = xcd_remap(blockIdx.x, a.total);
    b = pid / a.ncol;
    c = 1 + pid - b * a.ncol;
  }
  const int n = a.n, c0 = 64 * c;
  const float* R = a.R + b * a.sr;
  const float* Dv = a.Dinv + (int64_t)b * n * 64;
  float* W = a.Wm + b * a.sw;
  float* Rw = Rs[wid];
  // strip rows 32 strip .. +31 (< c0 <= n), columns c0 .. c0 + 63: 4 rows per instruction.
  // The first strip's loads issue before Dinv_c is staged, and each next strip's
  // as soon as the current one is in LDS, under its MFMAs.
  const int rq = lane >> 4, cq = 4 * (lane & 15), col = c0 + cq;
  float4 v[8];
  auto load_strip = [&](int strip) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float* src = R + (int64_t)(32 * strip + 4 * u + rq) * n + col;
      if (a.vec4 && col + 3 < n) {
        v[u] = *reinterpret_cast<const float4*>(src);
      } else {
        v[u].x = (col < n) ? src[0] : 0.f;
        v[u].y = (col + 1 < n) ? src[1] : 0.f;
        v[u].z = (col + 2 < n) ? src[2] : 0.f;
        v[u].w = (col + 3 < n) ? src[3] : 0.f;
      }
    }
  };
  if (wid < 2 * c) load_strip(wid);
  for (int idx = tid; idx < 64 * 16; idx += 256) {
    const int k = idx >> 4, j4 = idx & 15;
    float4 dv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c0 + k < n) dv = reinterpret_cast<const float4*>(Dv + (int64_t)(c0 + k) * 64)[j4];  // zero past the block
    reinterpret_cast<float4*>(Ds + k * 64)[j4] = dv;
  }
  __syncthreads();
  for (int strip = wid; strip < 2 * c; strip += 4) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float* d = Rw + (4 * u + rq) * LDR + cq;
      d[0] = v[u].x; d[1] = v[u].y; d[2] = v[u].z; d[3] = v[u].w;
    }
    wave_lds_order();
    if (strip + 4 < 2 * c) load_strip(strip + 4);
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
      if (c0 + l32 < n) W[o] = -acc0[r];
      if (c0 + 32 + l32 < n) W[o + 32] = -acc1[r];
    }
  }
}

// RB = 128: each wave owns 32 rows x 64 columns (two 32x32 accumulators); RB = 64 (small
// batches at large n, twice the workgroups): 2 x 2 waves of 32 x 32.
// SK = 2 (small batches at large n, where one 256-thread workgroup per row block leaves two
// waves per SIMD): 512 threads, two groups of four waves splitting each block column's K
// chunks between them (group g takes chunks g, g + 2, ...), group 1's sums added into group
// 0's through LDS before group 0 stores -- twice the waves for the same row blocks.
template <bool VEC4, int RB = kTrsmRows, int SK = 1>
__global__ __launch_bounds__(256 * SK) __attribute__((amdgpu_waves_per_eu(4))) void k_trsm(TrsmArgs a) {
  constexpr int BK = 16, LDA = BK + 1;
  constexpr int NP = RB / 64;    // A-chunk float4 slots per thread
  constexpr int WN = 128 / RB;   // waves side by side across the 64 columns
  constexpr int NACC = 2 / WN;   // 32x32 accumulators per wave
  __shared__ __attribute__((aligned(16))) float smA[2 * SK * RB * LDA];  // A chunks: RB rows x BK
  __shared__ __attribute__((aligned(16))) float smB[2 * SK * BK * 64];   // B chunks: BK x 64
  __shared__ __attribute__((aligned(16))) int prow[RB];
  __shared__ int mrow[RB];
  __shared__ float red[SK == 2 ? 4 * NACC * 16 * 64 : 1];  // group 1's accumulators (SK = 2)

  const int ttid = threadIdx.x, grp = SK == 2 ? ttid >> 8 : 0;
  const int tid = ttid & 255, lane = tid & 63, wid = tid >> 6;  // within the group
  const int l32 = lane & 31, h = lane >> 5, wr = (wid / WN) * 32, wc = (wid % WN) * 32 * NACC;
  const int pid = xcd_remap(blockIdx.x, a.total);
  const int b = pid / a.nrb, r0 = (pid - b * a.nrb) * RB, n = a.n;
  const float* M = a.M + b * a.sm;
  const float* Wm = a.Wm + b * a.sw;
  const float* Dv = a.Dinv + (int64_t)b * n * 64;
  float* Q = a.Q + b * a.sq;
  float* Q2 = a.Q2 ? a.Q2 + b * a.sq2 : nullptr;

  if (ttid < RB) {
    const int row = r0 + tid;
    prow[tid] = (row < n) ? (a.perm ? a.perm[(int64_t)b * n + row] : row) : 0;
    mrow[tid] = (row < n) ? (a.mperm ? a.mperm[(int64_t)b * n + row] : row) : 0;
  }
  __syncthreads();

  // staging: A chunk = RB x BK floats (2 float4 per thread), B chunk = BK x 64 floats (1).
  // A chunk never straddles c0 (BK divides 64), so the -Q / M choice is uniform per chunk, and
  // the loads are branch-free: rows past n read row 0 (prow / mrow hold 0 there) and columns
  // past n read clamped ones -- such entries only reach rows or columns of the accumulators
  // that are never stored -- except the K rows past n of the diagonal chunk, which meet B rows
  // set to zero.  Each thread's two A rows are fixed, so their offsets stay in registers.
  // The loads are used only by the LDS stores after the chunk's MFMAs, so nothing touches the
  // loaded registers before then: the diagonal chunk's masks are applied in lstore.
  float ra[4 * NP], rb[4];
  const int ca = 4 * (tid & 3);
  int ia[NP], qo[NP], mo[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    ia[p] = (tid >> 2) + 64 * p;
    qo[p] = prow[ia[p]] * n;
    mo[p] = mrow[ia[p]] * n;
  }
  const int kr = tid >> 4, cb = 4 * (tid & 15);
  auto gload = [&](int kc, int c0) {
    const int k = kc + ca;
    if (kc < c0) {  // Q (this workgroup's earlier output) against -W
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const float* src = Q + qo[p] + k;  // k + 3 < c0 <= n
        float4 v;
        if (VEC4) {
          v = *reinterpret_cast<const float4*>(src);
        } else {
          v = make_float4(src[0], src[1], src[2], src[3]);
        }
        ra[4 * p] = v.x; ra[4 * p + 1] = v.y; ra[4 * p + 2] = v.z; ra[4 * p + 3] = v.w;
      }
      const float* wrow = Wm + (kc + kr) * n;  // kc + kr < c0
      const int col = c0 + cb;
      float4 v;
      if (VEC4) {
        v = *reinterpret_cast<const float4*>(wrow + min(col, n - 4));
      } else {
        v = make_float4(wrow[min(col, n - 1)], wrow[min(col + 1, n - 1)], wrow[min(col + 2, n - 1)],
                        wrow[min(col + 3, n - 1)]);
      }
      rb[0] = v.x; rb[1] = v.y; rb[2] = v.z; rb[3] = v.w;
    } else {  // the diagonal chunk: M (or the unit-lower view of L) against Dinv_c
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const float* mr = M + mo[p];
        float4 v;
        if (VEC4) {
          v = *reinterpret_cast<const float4*>(mr + min(k, n - 4));
        } else {
          v = make_float4(mr[min(k, n - 1)], mr[min(k + 1, n - 1)], mr[min(k + 2, n - 1)], mr[min(k + 3, n - 1)]);
        }
        ra[4 * p] = v.x; ra[4 * p + 1] = v.y; ra[4 * p + 2] = v.z; ra[4 * p + 3] = v.w;
      }
      const float4 v = *reinterpret_cast<const float4*>(Dv + min(kc + kr, n - 1) * 64 + cb);  // zero past the block
      rb[0] = v.x; rb[1] = v.y; rb[2] = v.z; rb[3] = v.w;
    }
  };
  auto lstore = [&](int buf, int kc, int c0) {
    float* As = smA + (buf * SK + grp) * RB * LDA;
    float* Bs = smB + (buf * SK + grp) * BK * 64;
    if (kc >= c0) {  // uniform: the diagonal chunk
      if (a.mperm) {  // L[row][k]: stored below the diagonal, 1 on it, 0 above
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          int d = r0 + ia[p] - (kc + ca);  // row - k
          asm volatile("" : "+v"(d));  // keeps the selects here instead of hoisted out of the loops
#pragma unroll
          for (int q = 0; q < 4; ++q) ra[4 * p + q] = (q < d) ? ra[4 * p + q] : (q == d ? 1.f : 0.f);
        }
      }
      if (kc + kr >= n) rb[0] = rb[1] = rb[2] = rb[3] = 0.f;  // K rows past n
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int q = 0; q < 4; ++q) As[ia[p] * LDA + ca + q] = ra[4 * p + q];
    }
    *reinterpret_cast<float4*>(&Bs[(tid >> 4) * 64 + 4 * (tid & 15)]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
  };

  for (int c0 = 0; c0 < n; c0 += 64) {
    const int kend = min(c0 + 64, n);
    f32x16 acc[NACC];
#pragma unroll
    for (int j = 0; j < NACC; ++j) acc[j] = zero16();
    int buf = 0;
    // this group's chunks: K = kc0, kc0 + SK BK, ... (uniform per group)
    const int kc0 = grp * BK;
    if (kc0 < kend) {
      gload(kc0, c0);
      lstore(0, kc0, c0);
    }
    __syncthreads();
    for (int kb = 0; kb < kend; kb += SK * BK) {
      const int kc = kb + kc0;
      const bool more = kc + SK * BK < kend;
      if (more) gload(kc + SK * BK, c0);
      if (kc < kend) {
        const float* As = smA + (buf * SK + grp) * RB * LDA;
        const float* Bs = smB + (buf * SK + grp) * BK * 64;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
          const int k = kk + h;
          const float av = As[(wr + l32) * LDA + k];
#pragma unroll
          for (int j = 0; j < NACC; ++j) acc[j] = mfma(av, Bs[k * 64 + wc + 32 * j + l32], acc[j]);
        }
      }
      if (more) lstore(buf ^ 1, kc + SK * BK, c0);
      __syncthreads();
      buf ^= 1;
    }
    if constexpr (SK == 2) {
      if (grp == 1) {
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[((wid * NACC + j) * 16 + r) * 64 + lane] = acc[j][r];
      }
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[j][r] += red[((wid * NACC + j) * 16 + r) * 64 + lane];
      }
    }
    // accumulator registers 4g .. 4g + 3 hold the consecutive rows wr + 8g + 4h + (0..3):
    // their targets come from one 16-byte LDS read; full tiles store without masks
    int ln = lane;
    asm volatile("" : "+v"(ln));
    auto store_tile = [&](float* dst, auto masked) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int lb = wr + 8 * g + 4 * (ln >> 5);
        const int4 pr = *reinterpret_cast<const int4*>(&prow[lb]);
        const int prr[4] = {pr.x, pr.y, pr.z, pr.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int nj = 0; nj < NACC; ++nj) {
            const int col = c0 + wc + nj * 32 + (ln & 31);
            if (!decltype(masked)::value || (r0 + lb + q < n && col < n)) dst[prr[q] * n + col] = acc[nj][4 * g + q];
          }
      }
    };
    if (grp == 0) {
      if (r0 + RB <= n && c0 + 64 <= n) {  // uniform
        store_tile(Q, std::false_type{});
        if (Q2) store_tile(Q2, std::false_type{});
      } else {
        store_tile(Q, std::true_type{});
        if (Q2) store_tile(Q2, std::true_type{});
      }
    }
    // the next block column reads these outputs back (other threads of this workgroup)
    __syncthreads();
  }
}

}  // namespace rnr
