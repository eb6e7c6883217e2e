// Batched "transpose-A" fp32 MFMA product restricted to upper-triangular tiles:
//
//   C[b][i][j] = rs[b][i] * sum_{r = klo}^{n-1} X[b][r][i] * Y[b][r][j]     (tile ti <= tj)
//
// It serves the three contractions of the path whose outputs are (block-)upper:
//   * Gram of the unit-lower L, G = L^T L (klo = first column of the tile: the rows above
//     it are exact zeros of L)        -- reflection_no_reflectors.py:73 (first pass)
//   * Gram of Q1, G = Q1^T Q1         -- reflection_no_reflectors.py:73 (second pass)
//   * closure, H_upper = diag(s) triu(Q^T A), written only on and above the diagonal so
//     the reflector tails below it survive -- reflection_no_reflectors.py:186,195
//
// Tile BM x BM per 256-thread workgroup (2 x 2 waves, each BM/2 x BM/2 from 32x32 MFMA
// blocks); the K dimension (rows of X and Y) is staged through double-buffered LDS in
// chunks of BK rows, so every operand element is read from HBM/L2 once per tile.
#pragma once
#include "common.hpp"

namespace rnr {

struct TnArgs {
  const float* X;
  int64_t sx;
  const float* Y;
  int64_t sy;
  float* C;
  int64_t sc;
  const float* rs;  // row scale, batch stride n (ROW_SCALE only)
  const int* lperm; // non-null: X = Y = unit-lower L stored in A's row order (the LU's
                    // in-place factor); logical row r is physical row lperm[b][r]
  int n;
  int nt;       // tiles per matrix edge
  int ntiles;   // upper tiles per matrix
  int total;    // grid size
  int klo_from_j;
  int lpt;      // klo_from_j with total % 8 == 0 and ntiles | total / 8: longest tiles first
};

// LV: the kernel may be given the unit-lower L view (a.lperm); without it the row map's LDS is
// not allocated, which leaves room for more workgroups per CU.
template <int BM, bool MASK_LOWER, bool ROW_SCALE, bool VEC4, int BK = 32, bool LV = true>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_tn_upper(TnArgs a) {
  constexpr int WM = BM / 2;
  constexpr int NB = WM / 32;
  constexpr int PER = BK * BM / 256;  // elements per thread per operand per chunk
  __shared__ __attribute__((aligned(16))) float Xs[2][BK][BM];
  __shared__ __attribute__((aligned(16))) float Ys[2][BK][BM];
  __shared__ int lps[LV ? RNR_MAX_N : 1];  // the row map of L (L view only)
  __shared__ __attribute__((aligned(16))) float rss[ROW_SCALE ? BM : 1];  // the tile's row scales (ROW_SCALE only)

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  int b, ti, tj;
  if (a.lpt) {
    // the Gram of L: a tile's K range is n - j0, so each XCD's matrices are dispatched tile by
    // tile in column-major order (decreasing K) -- the short tiles fill the tail -- while the
    // XCD keeps the same matrices (and their L2 sharing) as below
    const int per = a.total / 8, mpx = per / a.ntiles, q = blockIdx.x >> 3;
    const int tr = q / mpx;
    b = (blockIdx.x & 7) * mpx + (q - tr * mpx);
    int t = tr, j = 0;
    while (t > j) {
      t -= j + 1;
      ++j;
    }
    ti = t;
    tj = j;
  } else {
    const int pid = xcd_remap(blockIdx.x, a.total);
    b = pid / a.ntiles;
    upper_tile(pid - b * a.ntiles, a.nt, ti, tj);
  }
  const int n = a.n, i0 = ti * BM, j0 = tj * BM;
  const float* X = a.X + b * a.sx;
  const float* Y = a.Y + b * a.sy;
  // On a diagonal tile the 32x32 blocks strictly below the diagonal are never used (the closure
  // masks them; the Cholesky reads only the upper triangle of G), so only the ten upper blocks
  // are computed, spread 3/3/2/2 over the waves when BM = 128: waves 0 and 3 take the upper
  // three blocks of their diagonal 64x64 quadrants, waves 1 and 2 one 32-row strip each of the
  // off-diagonal quadrant (rows 0..31 and 32..63, columns 64..127).  With BM = 64 the wave below
  // the diagonal has nothing to do.
  const bool diag = ti == tj;
  int wi0 = (wid >> 1) * WM, wj0 = (wid & 1) * WM;
  if (NB == 2 && diag && wid == 2) {  // the strip of rows 32..63, columns 64..127
    wi0 = 32;
    wj0 = 64;
  }
  // blocks this wave computes: 0 every block, 1 those with mi <= nj, 2 none, 3 the mi = 0 strip
  const int low = !diag ? 0 : (wid == 0 || wid == 3) ? 1 : (NB == 2 ? 3 : (wid == 1 ? 0 : 2));

  f32x16 acc[NB][NB];
#pragma unroll
  for (int mi = 0; mi < NB; ++mi)
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) acc[mi][nj] = zero16();

  float rx[PER], ry[PER];
  // the row map is staged in LDS once: every K chunk then looks its rows up there instead of
  // waiting on a dependent global load before the data load
  const int* lp = nullptr;
  if (LV && a.lperm) {
    const int* g = a.lperm + (int64_t)b * n;
    for (int i = (a.klo_from_j ? j0 : 0) + tid; i < n; i += 256) lps[i] = g[i];
    __syncthreads();
    lp = lps;
  }
  // row scales staged once, made visible by the barrier after the first chunk's LDS store (read
  // per element in the epilogue they were a chain of dependent global loads)
  if constexpr (ROW_SCALE) {
    for (int i = tid; i < BM; i += 256) rss[i] = (i0 + i < n) ? a.rs[(int64_t)b * n + i0 + i] : 0.f;
  }
  // element (r, c) of the unit-lower view: below the diagonal from row lp[r], 1 on it, 0 above
  auto lview1 = [&](int gr, int c) -> float {
    return (c < gr) ? X[(int64_t)lp[gr] * n + c] : (c == gr ? 1.f : 0.f);
  };
  // float4 slots (VEC4): a thread's column is the same in every slot, since 256 is a multiple
  // of BM / 4.  The loads are branch-free -- rows past n read row n - 1 and columns past n read
  // clamped ones (those only reach accumulator entries that are never stored) -- and nothing
  // touches the loaded registers before the LDS store after the chunk's MFMAs, which applies
  // the unit-lower view's masks and zeroes the K rows past n, both under uniform conditions.
  constexpr int RQ = 256 / (BM / 4);  // rows between a thread's slots
  const int c4 = 4 * (tid % (BM / 4)), rq = tid / (BM / 4);
  const int cx = min(i0 + c4, n - 4), cy = min(j0 + c4, n - 4);
  auto gload = [&](int k) {
    if constexpr (VEC4) {
#pragma unroll
      for (int p = 0; p < PER / 4; ++p) {
        const int gr = min(k + rq + RQ * p, n - 1);
        const int ro = (lp ? lp[gr] : gr) * n;
        const float4 vx = *reinterpret_cast<const float4*>(X + ro + cx);
        const float4 vy = *reinterpret_cast<const float4*>((lp ? X : Y) + ro + cy);
        rx[4 * p + 0] = vx.x; rx[4 * p + 1] = vx.y; rx[4 * p + 2] = vx.z; rx[4 * p + 3] = vx.w;
        ry[4 * p + 0] = vy.x; ry[4 * p + 1] = vy.y; ry[4 * p + 2] = vy.z; ry[4 * p + 3] = vy.w;
      }
      return;
    }
    if (lp) {
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int idx = tid + 256 * p;
        const int row = idx / BM, c = idx % BM;
        const int gr = k + row;
        rx[p] = (gr < n && i0 + c < n) ? lview1(gr, i0 + c) : 0.f;
        ry[p] = (gr < n && j0 + c < n) ? lview1(gr, j0 + c) : 0.f;
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + 256 * p;
      const int row = idx / BM, c = idx % BM;
      const int gr = k + row;
      rx[p] = (gr < n && i0 + c < n) ? X[(int64_t)gr * n + i0 + c] : 0.f;
      ry[p] = (gr < n && j0 + c < n) ? Y[(int64_t)gr * n + j0 + c] : 0.f;
    }
  };
  auto lstore = [&](int buf, int k) {
    if constexpr (VEC4) {
      if (lp) {
        // L[gr][col]: stored below the diagonal, 1 on it, 0 above (only chunks that reach the
        // tile's columns have entries on or above the diagonal)
        auto lmask = [&](float* r, int col0) {
#pragma unroll
          for (int p = 0; p < PER / 4; ++p) {
            int d = k + rq + RQ * p - col0;  // gr - col
            asm volatile("" : "+v"(d));
#pragma unroll
            for (int e = 0; e < 4; ++e) r[4 * p + e] = (e < d) ? r[4 * p + e] : (e == d ? 1.f : 0.f);
          }
        };
        if (k < i0 + BM) lmask(rx, i0 + c4);
        if (k < j0 + BM) lmask(ry, j0 + c4);
      }
      if (k + BK > n) {
#pragma unroll
        for (int p = 0; p < PER / 4; ++p)
          if (k + rq + RQ * p >= n)
#pragma unroll
            for (int e = 0; e < 4; ++e) rx[4 * p + e] = ry[4 * p + e] = 0.f;
      }
#pragma unroll
      for (int p = 0; p < PER / 4; ++p) {
        const int row = rq + RQ * p;
        *reinterpret_cast<float4*>(&Xs[buf][row][c4]) =
            make_float4(rx[4 * p], rx[4 * p + 1], rx[4 * p + 2], rx[4 * p + 3]);
        *reinterpret_cast<float4*>(&Ys[buf][row][c4]) =
            make_float4(ry[4 * p], ry[4 * p + 1], ry[4 * p + 2], ry[4 * p + 3]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int idx = tid + 256 * p;
        Xs[buf][idx / BM][idx % BM] = rx[p];
        Ys[buf][idx / BM][idx % BM] = ry[p];
      }
    }
  };

  const int klo = a.klo_from_j ? j0 : 0;
  // the unit-lower L is zero above its diagonal: this wave's operand columns start at i0 + wi0
  // and j0 + wj0, so its chunks below both multiply zeros only and their MFMAs are skipped
  // (the chunk is still staged: the other waves of the tile read it)
  const int kz = a.klo_from_j ? max(i0 + wi0, j0 + wj0) : 0;
  int buf = 0;
  gload(klo);
  lstore(0, klo);
  __syncthreads();
  auto kloop = [&](auto lowc) {
    constexpr int LOW = decltype(lowc)::value;
    for (int kc = klo; kc < n; kc += BK) {
      const bool more = kc + BK < n;
      if (more) gload(kc + BK);
      if (LOW != 2 && kc + BK > kz) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
          const int k = kk + h;
          float av[NB], bv[NB];
#pragma unroll
          for (int mi = 0; mi < NB; ++mi) av[mi] = Xs[buf][k][wi0 + mi * 32 + l32];
#pragma unroll
          for (int nj = 0; nj < NB; ++nj) bv[nj] = Ys[buf][k][wj0 + nj * 32 + l32];
#pragma unroll
          for (int mi = 0; mi < NB; ++mi)
#pragma unroll
            for (int nj = 0; nj < NB; ++nj)
              if (LOW == 0 || (LOW == 1 && mi <= nj) || (LOW == 3 && mi == 0))
                acc[mi][nj] = mfma(av[mi], bv[nj], acc[mi][nj]);
        }
      }
      if (more) lstore(buf ^ 1, kc + BK);
      __syncthreads();
      buf ^= 1;
    }
  };
  if (low == 0) kloop(std::integral_constant<int, 0>{});
  else if (low == 1) kloop(std::integral_constant<int, 1>{});
  else if (low == 3) kloop(std::integral_constant<int, 3>{});
  else kloop(std::integral_constant<int, 2>{});

  float* C = a.C + b * a.sc;
  // accumulator registers 4g .. 4g + 3 hold the consecutive rows wr + 8g + 4h + (0..3): their
  // row scales are one float4 LDS read
  const int mlim = low == 3 ? 1 : NB;  // a strip wave's other row block overlaps wave 3's blocks
#pragma unroll
  for (int mi = 0; mi < NB; ++mi)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (mi >= mlim) continue;
      const int lr0 = wi0 + mi * 32 + 8 * g + 4 * h;
      float sc[4] = {1.f, 1.f, 1.f, 1.f};
      if constexpr (ROW_SCALE) {
        const float4 s4 = *reinterpret_cast<const float4*>(&rss[lr0]);
        sc[0] = s4.x; sc[1] = s4.y; sc[2] = s4.z; sc[3] = s4.w;
      }
#pragma unroll
      for (int nj = 0; nj < NB; ++nj)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = i0 + lr0 + e, col = j0 + wj0 + nj * 32 + l32;
          if (row < n && col < n && (!MASK_LOWER || col >= row)) {
            float v = acc[mi][nj][4 * g + e];
            if (ROW_SCALE) v *= sc[e];
            C[(int64_t)row * n + col] = v;
          }
        }
    }
}

}  // namespace rnr
