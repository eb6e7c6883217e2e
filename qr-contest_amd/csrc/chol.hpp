// Jittered upper Cholesky of one Gram matrix per 512-thread workgroup, in place:
//
//   mu = 1e-7 * mean(diag G);  G += mu I;  G = R^T R        -- reflection_no_reflectors.py:74-76
//
// Blocked right-looking with 64-column blocks.  For block k:
//   * wave 0 factors the diagonal block with one symmetric row per lane in registers and
//     the scaled pivot row broadcast through LDS inside the wave (no barriers or fences);
//   * every wave then forms 8 columns of Dinv_kk = R_kk^-1 by back substitution, one row
//     per lane in registers, readlane broadcasts; Dinv_kk^T is staged in LDS;
//   * the block row R_k,> = Dinv_kk^T G_k,> and the trailing update G_>,> -= R_k,>^T R_k,>
//     (upper 64x64 tiles only) run on MFMA, each wave owning whole output tiles.  When the
//     block row fits it is also kept in LDS for the trailing update (n <= 576), otherwise
//     it is read back from G.
// The diagonal-block inverses go to Dinv ([n][64] per matrix) for the triangular solve
// that follows.  info records the first column whose pivot was not positive (1-based; NaN
// counts as not positive).
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
  return sizeof(float) * (2 * 64 * 65 + 64 + 32 + (strip ? 64 * w : 0));
}

__global__ __launch_bounds__(kCholThreads) void k_chol(CholArgs a) {
  constexpr int NW = kCholThreads / 64, CPW = 64 / NW;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* D = smem;                 // [64][65] diagonal block, then R_kk (upper, zero below)
  float* XT = D + 64 * 65;         // [64][65] (R_kk^-1)^T: XT[i][k] = Dinv_kk[k][i]
  float* SB = XT + 64 * 65;        // [64] scaled pivot row broadcast (wave 0)
  float* red = SB + 64;            // [16]
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
  for (int w = 0; w < NW; ++w) tot += red[w];
  const float mu = 1e-7f * (tot / (float)n);
  for (int i = tid; i < n; i += kCholThreads) G[(int64_t)i * n + i] += mu;
  __syncthreads();

  for (int k0 = 0; k0 < n; k0 += kCholNb) {
    const int kb = min(kCholNb, n - k0), k1 = k0 + kb, w = n - k1;

    // diagonal block (upper part as stored); outside kb an identity pads it
    for (int idx = tid; idx < 64 * 64; idx += kCholThreads) {
      const int i = idx >> 6, c = idx & 63;
      float v = (i == c) ? 1.f : 0.f;
      if (i < kb && c < kb && c >= i) v = G[(int64_t)(k0 + i) * n + k0 + c];
      D[i * 65 + c] = v;
    }
    __syncthreads();

    if (wid == 0) {
      // lane i holds symmetric row i of the block; step j broadcasts the scaled pivot row
      // R[j][c] = G'[j][c] / r (held by lane c) through LDS inside the wave.  A wave issues
      // its LDS operations in order and the store/load addresses may alias, so neither the
      // hardware nor the compiler reorders them: no fence or barrier sits on the chain.
      // the row is four named 16-wide vectors (element access with compile-time indices), so
      // it stays in VGPRs whatever the unrolled code around it looks like
      f32x16 v0, v1, v2, v3;
      auto V = [&](auto qc) -> f32x16& {
        constexpr int q = decltype(qc)::value;
        if constexpr (q == 0) return v0;
        else if constexpr (q == 1) return v1;
        else if constexpr (q == 2) return v2;
        else return v3;
      };
      static_for<0, 4>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        f32x16& v = V(qc);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int c = 16 * q + e;
          v[e] = D[(c >= lane) ? lane * 65 + c : c * 65 + lane];
        }
      });
      int fail = INT_MAX;
      static_for<0, 64>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const float rjj = V(std::integral_constant<int, j / 16>{})[j % 16];
        const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rjj), j));
        if (!(d > 0.f) && fail == INT_MAX) fail = j;
        const float r = sqrtf(d), rinv = 1.f / r;
        const float si = (ln == j) ? r : rjj * rinv;  // lane c > j: R[j][c]
        const float sm = (ln > j) ? si : 0.f;          // rows below j take the update
        SB[ln] = si;
        // 16 broadcast values at a time (scheduling barriers keep the reads from all being
        // hoisted at once)
        static_for<(j + 1) / 16, 4>([&](auto qc) {
          constexpr int q = decltype(qc)::value;
          f32x16& v = V(qc);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            if (16 * q + e > j) v[e] -= sm * SB[16 * q + e];
          }
          __builtin_amdgcn_sched_barrier(0);
        });
        D[j * 65 + ln] = (ln >= j) ? si : 0.f;  // row j of R
        __builtin_amdgcn_sched_barrier(0);
      });
      if (lane == 0 && fail != INT_MAX && fail < kb && *ffail == INT_MAX) *ffail = k0 + fail + 1;
    }
    __syncthreads();

    // Dinv_kk = R_kk^-1 by back substitution: wave w solves columns w*CPW.., lane i holding
    // row i of R and entry i of the running right-hand side
    {
      float rr[64];
#pragma unroll
      for (int c = 0; c < 64; ++c) rr[c] = D[lane * 65 + c];  // R_kk is zero below the diagonal
      const float rd = 1.f / D[lane * 65 + lane];  // 1 / R[i][i] in lane i
      float x[CPW];
      const int cw = __builtin_amdgcn_readfirstlane(wid * CPW);
#pragma unroll
      for (int u = 0; u < CPW; ++u) x[u] = (lane == cw + u) ? 1.f : 0.f;
      static_for<0, 64>([&](auto kc) {
        constexpr int k = 63 - decltype(kc)::value;  // k = 63 .. 0
        int ln = lane, c0w = cw;
        asm volatile("" : "+v"(ln), "+s"(c0w));
        const float rk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rd), k));
        const float mr = (ln < k) ? rr[k] : 0.f;  // rows above k take the update
#pragma unroll
        for (int u = 0; u < CPW; ++u) {
          if (k <= c0w + u) {
            const float xk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[u]), k)) * rk;
            x[u] = (ln == k) ? xk : x[u] - mr * xk;
          }
        }
      });
      // column cw+u of the inverse -> XT[cw+u][i]
#pragma unroll
      for (int u = 0; u < CPW; ++u) XT[(cw + u) * 65 + lane] = (lane <= cw + u) ? x[u] : 0.f;
    }
    __syncthreads();

    // R_kk (upper) and Dinv_kk (row-major, zero below the diagonal) to HBM
    for (int idx = tid; idx < kb * 64; idx += kCholThreads) {
      const int i = idx >> 6, c = idx & 63;
      if (c < kb && c >= i) G[(int64_t)(k0 + i) * n + k0 + c] = D[i * 65 + c];
      Dv[(int64_t)(k0 + i) * 64 + c] = (c < kb) ? XT[c * 65 + i] : 0.f;
    }
    if (w <= 0) break;  // uniform; kb == 64 below this line

    // block row R_k,> = Dinv_kk^T G_k,>: each wave owns 32 columns (both 32-row halves),
    // so it can overwrite them in G without racing other waves' reads.
    {
      const int nch = (w + 31) >> 5;
      for (int job = wid; job < nch; job += NW) {
        const int colr = job * 32 + l32, col = k1 + colr;
        float bv[32];
#pragma unroll
        for (int t = 0; t < 32; ++t)
          bv[t] = (col < n) ? G[(int64_t)(k0 + 2 * t + h) * n + col] : 0.f;
        f32x16 acc0 = zero16(), acc1 = zero16();
#pragma unroll
        for (int t = 0; t < 32; ++t) {
          const int k = 2 * t + h;
          acc0 = mfma(XT[l32 * 65 + k], bv[t], acc0);
          acc1 = mfma(XT[(32 + l32) * 65 + k], bv[t], acc1);
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
      for (int pr = wid; pr < npairs; pr += NW) {
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
#pragma unroll 4
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
