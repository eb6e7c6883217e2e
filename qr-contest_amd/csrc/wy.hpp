// Blocked-WY application of the compact (H, tau) factor on MFMA, float32:
//   Y <- Q Y   (TRANS = false; orgqr when Y starts as the identity)
//   Y <- Q^T Y (TRANS = true)
// with Q = H_0 ... H_{n-1} grouped into panels of 32 reflectors, P_p = I - V_p T_p V_p^T
// (LAPACK slarft, forward / columnwise).  Two kernels:
//   k_wy_tmat   all panels' T at once, one 256-thread workgroup per (matrix, panel):
//               S = V^T V on v_mfma_f32_32x32x2f32 (rows split over the waves, V read
//               straight from H), then T row-parallel, T[i][j] = -tau_j sum_{l=i}^{j-1}
//               T[i][l] S[l][j] (thread i needs only its own row);
//   k_wy_apply  one launch per panel, one workgroup per column tile of Y (rows >= k0 of the
//               panel): the tile stays in the MFMA accumulators for the whole update --
//               loaded once, W = V^T C with the accumulator registers used directly as the B
//               operand (register r of a 32x32 accumulator holds rows 8(r/4) + r%4 and that
//               + 4 in its two half-waves: a K = 2 pair), the waves' W summed in LDS, W' =
//               op(T) W formed by every wave in registers, C -= V W' with W' again straight
//               from the accumulators, one store.
// NW waves each own NS strips of 32 rows; a tile is NC (32 or 64) columns wide.
#pragma once
#include "common.hpp"

namespace rnr {

constexpr int kWyPb = 32;

struct WyArgs {
  const float* H;    // [batch][n][n] reflectors below the diagonal
  const float* tau;  // [batch][n]
  float* T;          // [batch][np][32][32]
  float* Y;          // batch stride sy, row stride ldy
  int64_t sy;
  int ldy, n, nc, np;
  int p;             // k_wy_apply: the panel
  int c_lo;          // k_wy_apply: first column of Y that changes
  int ntile;         // k_wy_apply: column tiles per matrix
};

__global__ __launch_bounds__(256) void k_wy_tmat(WyArgs a) {
  __shared__ float Sp[4][32][33];
  __shared__ float Tm[32][33];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, l32 = lane & 31, h = lane >> 5;
  const int64_t pid = blockIdx.x;
  const int64_t b = pid / a.np;
  const int p = (int)(pid - b * a.np), n = a.n, k0 = p * kWyPb, kb = min(kWyPb, n - k0), m = n - k0;
  const float* H = a.H + b * n * n;
  const float* tau = a.tau + b * n;
  {
    const int chunk = ((m + 7) / 8) * 2;  // rows per wave, even
    const int r0 = wid * chunk, r1 = min(m, r0 + chunk);
    f32x16 acc = zero16();
    for (int r = r0 + h; r < r0 + chunk; r += 2) {
      float v = 0.f;
      if (r < r1 && l32 < kb) v = (r < l32) ? 0.f : (r == l32 ? 1.f : H[(k0 + r) * n + k0 + l32]);
      acc = mfma(v, v, acc);
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) Sp[wid][acc_row(q, lane)][l32] = acc[q];
  }
  __syncthreads();
  if (tid < 32) {
    const int i = tid;
    for (int j = 0; j < 32; ++j) Tm[i][j] = 0.f;
    if (i < kb) {
      Tm[i][i] = tau[k0 + i];
      for (int j = i + 1; j < kb; ++j) {
        float acc = 0.f;
        for (int l = i; l < j; ++l)
          acc += Tm[i][l] * (Sp[0][l][j] + Sp[1][l][j] + Sp[2][l][j] + Sp[3][l][j]);
        Tm[i][j] = -tau[k0 + j] * acc;
      }
    }
    float* T = a.T + (b * a.np + p) * 32 * 32;
    for (int j = 0; j < 32; ++j) T[i * 32 + j] = Tm[i][j];
  }
}

template <bool TRANS, int NW, int NS, int NC>
__global__ __launch_bounds__(NW * 64) void k_wy_apply(WyArgs a) {
  constexpr int NJ = NC / 32;  // accumulators per strip
  constexpr int LW = NC + 1;
  // per wave: V staging [32][33] and, after the wave's own W = V^T C, its W partial
  // [32][NC + 1] (the same words: a wave writes its partial only after its last staged read)
  __shared__ float Sw[NW][32 * LW];
  __shared__ float Ts[32][33];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, l32 = lane & 31, h = lane >> 5;
  auto Vs = [&](int r, int j) -> float& { return Sw[wid][r * 33 + j]; };
  auto Wp = [&](int q, int k, int col) -> float& { return Sw[q][k * LW + col]; };
  const int64_t pid = blockIdx.x;
  const int64_t b = pid / a.ntile;
  const int tile = (int)(pid - b * a.ntile);
  const int n = a.n, k0 = a.p * kWyPb, kb = min(kWyPb, n - k0), m = n - k0;
  const int c0 = a.c_lo + NC * tile;
  const float* H = a.H + b * n * n;
  float* Y = a.Y + b * a.sy;
  const int ld = a.ldy;
  const float* T = a.T + (b * a.np + a.p) * 32 * 32;
  for (int idx = tid; idx < 32 * 32; idx += NW * 64) Ts[idx >> 5][idx & 31] = T[idx];

  // the tile rows k0 + 32 (NW s + wid) + (0..31), in accumulator layout
  // (the lane id is laundered per strip: the row offsets of all strips, hoisted together,
  // would not fit in registers next to the tile)
  f32x16 c[NS][NJ];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * (NW * s + wid) + acc_row(r, ln), col = c0 + 32 * j + (ln & 31);
        c[s][j][r] = (row < m && col < a.nc) ? Y[(int64_t)(k0 + row) * ld + col] : 0.f;
      }
  }

  // stage V rows rs .. rs + 31 of the panel (row-major, reflectors along the row)
  auto stage_v = [&](int rs) {
    for (int idx = lane; idx < 32 * 32; idx += 64) {
      const int rr = idx >> 5, j = idx & 31, r = rs + rr;
      float v = 0.f;
      if (r < m && j < kb) v = (r < j) ? 0.f : (r == j ? 1.f : H[(k0 + r) * n + k0 + j]);
      Vs(rr, j) = v;
    }
    wave_lds_order();
  };

  // W = V^T C over this wave's rows
  f32x16 w[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) w[j] = zero16();
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int rs = 32 * (NW * s + wid);
    if (rs < m) {  // uniform per wave
      stage_v(rs);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = Vs(acc_row(r, lane), l32);  // A[i = reflector][k = row of register r]
#pragma unroll
        for (int j = 0; j < NJ; ++j) w[j] = mfma(v, c[s][j][r], w[j]);
      }
      wave_lds_order();
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) Wp(wid, acc_row(r, lane), 32 * j + l32) = w[j][r];
  __syncthreads();

  // W' = op(T) W (every wave, in registers): op(T)[i][k] = T[i][k] or T[k][i]
  f32x16 wt[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) wt[j] = zero16();
#pragma unroll
  for (int kk = 0; kk < 32; kk += 2) {
    const int k = kk + h;
    const float t = TRANS ? Ts[k][l32] : Ts[l32][k];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float wk = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) wk += Wp(q, k, 32 * j + l32);
      wt[j] = mfma(t, wk, wt[j]);
    }
  }
  __syncthreads();  // every wave has read all partials before V is staged over them again

  // C -= V W', K over the reflectors in the accumulator's row pairs
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int rs = 32 * (NW * s + wid);
    if (rs < m) {
      stage_v(rs);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = -Vs(l32, acc_row(r, lane));  // A[i = row][k = reflector of register r]
#pragma unroll
        for (int j = 0; j < NJ; ++j) c[s][j] = mfma(v, wt[j][r], c[s][j]);
      }
      wave_lds_order();
    }
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * (NW * s + wid) + acc_row(r, ln), col = c0 + 32 * j + (ln & 31);
        if (row < m && col < a.nc) Y[(int64_t)(k0 + row) * ld + col] = c[s][j][r];
      }
  }
}

// Y = I (batch x n x n, row stride ld): workgroup g covers chunk g % nchunk of matrix g / nchunk.
__global__ __launch_bounds__(256) void k_wy_identity(float* Y, int64_t sy, int ld, int n, int nchunk) {
  const int64_t g = blockIdx.x, b = g / nchunk;
  const int chunk = (int)(g - b * nchunk);
  float* y = Y + b * sy;
  const int nn = n * n;
  for (int idx = chunk * 256 + threadIdx.x; idx < nn; idx += nchunk * 256) {
    const int i = idx / n, c = idx - i * n;
    y[(int64_t)i * ld + c] = (i == c) ? 1.f : 0.f;
  }
}

}  // namespace rnr
