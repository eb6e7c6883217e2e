// Jittered upper Cholesky of one Gram matrix per 512-thread workgroup, in place:
//
//   mu = 1e-7 * mean(diag G);  G += mu I;  G = R^T R        -- reflection_no_reflectors.py:74-76
//
// Blocked right-looking with 64-column blocks and a look-ahead of one diagonal block.  For
// block k:
//   * R_kk and Dinv_kk = R_kk^-1 (already in LDS) go to HBM;
//   * all waves form the block row R_k,> = Dinv_kk^T G_k,> on MFMA, each wave owning whole
//     32-column strips; when it fits it is also kept in LDS for the trailing update
//     (n <= 576), otherwise it is read back from G;
//   * the trailing update G_>,> -= R_k,>^T R_k,> (upper 64x64 tiles, MFMA) is split: the
//     first diagonal tile -- the next diagonal block -- is updated into LDS by quadrants on
//     waves 0, 1 and 3 (three SIMDs; its lower-left quadrant is never read), then, after a
//     workgroup barrier, wave 0 factors it (rank-1 updates on MFMA with the block held in
//     accumulators, no barriers) and forms its inverse blocked by 32, while waves 1..7 update
//     the other tiles.  The sequential diagonal work thus runs under the
//     trailing update.
// The diagonal-block inverses go to Dinv ([n][64] per matrix) for the triangular solve that
// follows.  info records the first column whose pivot was not positive (1-based; NaN
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
  float* Wm;      // non-null: also form the solve's operand -W[k][c] = -R[k][c] Dinv_c (k < c) here,
  int64_t sw;     // at the R positions of a [batch][n][n] buffer (batch stride sw)
};

constexpr int kCholThreads = 512;
constexpr int kCholNb = 64;

inline size_t chol_lds_bytes(int n, bool strip) {
  const size_t w = n > kCholNb ? (size_t)(n - kCholNb) : 1;
  return sizeof(float) * (64 * 65 + 64 * 68 + 64 + 32 + (strip ? 64 * w + 64 : 0));
}

// Wave 0: factor the 64x64 diagonal block held in D (symmetric; the upper part is read) in
// place into R (upper, zeros below), with R also written column-major into RT (RT[c][k] =
// R[k][c], row stride 68) and 1 / R[j][j] into RI; returns the first non-positive pivot
// (column index, or INT_MAX).  The block lives in MFMA accumulators -- the diagonal 32x32
// blocks (0,0) and (1,1) as the two blocks of one v_mfma_f32_32x32x1_2b_f32 result, the
// upper off-diagonal block (0,1) as one 32x32x2 result (the lower one is never read) -- and
// each step's rank-1 update G -= u u^T is two MFMAs:
//   * the pivot G[j][j] is read from its accumulator lane (readlane), r = sqrt, 1 / r;
//   * row j of G sits in one accumulator register per block, in the lanes of one half-wave:
//     v_permlane32_swap gathers it as lane c -> G[j][c] (c = 0..63) and it is scaled to the row
//     of R (r at c = j, zero below);
//   * u (the row past j) is the A and B operand of the 2-block product for (0,0) and (1,1), and
//     with its halves swapped the B operand of the 32x32x2 product for (0,1).
// So a step is a chain of MFMA -> readlane -> sqrt / rcp -> swap -> MFMA with no LDS round trip
// and no per-lane loop over the row; rows of R go to LDS as they finish.
// The pivot's square root and reciprocal are the hardware's (1 ulp).
__device__ __forceinline__ int chol_diag_wave(float* D, float* RT, float* RI, int lane) {
  asm volatile("" : "+v"(lane));  // lane-derived values stay here, not hoisted out of the caller's loop
  f32x32 dg;  // (0,0) in registers 0..15, (1,1) in 16..31
  f32x16 od;  // (0,1)
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int bb = r >> 4, i = 32 * bb + acc_row(r & 15, lane), c = 32 * bb + (lane & 31);
    dg[r] = D[(i <= c) ? i * 65 + c : c * 65 + i];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) od[r] = D[acc_row(r, lane) * 65 + 32 + (lane & 31)];
  int fail = INT_MAX;
  static_for<0, 64>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    constexpr int B = j / 32, I = j % 32, HJ = (I / 4) % 2, RR = 4 * (I / 8) + I % 4;
    int ln = lane;
    asm volatile("" : "+v"(ln));  // the step's lane masks are formed here, not hoisted
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dg[16 * B + RR]), I + 32 * HJ));
    if (!(d > 0.f) && fail == INT_MAX) fail = j;
    const float r = __builtin_amdgcn_sqrtf(d);
    const float rinv = __builtin_amdgcn_rcpf(r);
    // lane c: G[j][c] (columns below j are masked out below)
    float v;
    if constexpr (B == 0) {
      const float2 p = lane_halves(dg[RR], od[RR]);
      v = HJ == 0 ? p.x : p.y;
    } else if constexpr (HJ == 1) {
      v = dg[16 + RR];
    } else {
      v = lane_halves(0.f, dg[16 + RR]).x;
    }
    const float rv = (ln == j) ? r : v * rinv;
    const float rj = (ln >= j) ? rv : 0.f;  // row j of R
    if constexpr (j < 63) {
      const float u = (ln > j) ? rv : 0.f;
      dg = mfma_2b(-u, u, dg);
      if constexpr (j < 31) {  // rows of block row 0 below j remain
        const float2 q = lane_halves(u, u);  // .y: u[32 + (l % 32)]
        od = mfma((ln < 32) ? -u : 0.f, q.y, od);
      }
    }
    D[j * 65 + ln] = rj;   // row j of R
    RT[ln * 68 + j] = rj;  // column ln of R
    RI[j] = rinv;          // same value from every lane
  });
  wave_lds_order();
  return fail;
}

// Wave 0: XT = (R^-1)^T (XT[i][k] = Dinv[k][i], row stride 65) for the upper R given column-
// major in RT (row stride 68) and row-major in D (row stride 65, zeros below the diagonal),
// with 1 / R[c][c] in RI.  Blocked by 32 (LAPACK strtri's block form):
//   * X11 = R11^-1 and X22 = R22^-1 at once, lane 32 d + i forming row i of block d from
//     X R = I column by column, X[i][c] = (delta_ic - sum_{k<c} X[i][k] R[k][c]) / R[c][c]
//     (the columns of R are float4 LDS reads; rows below the diagonal come out as exact zeros);
//   * X12 = -X11 (R12 X22) on v_mfma_f32_32x32x2f32, R12 X22 staying in the accumulators and
//     used from there as the B operand of the second product (register r of a 32x32
//     accumulator holds rows 8(r/4) + r%4 and that + 4 in its two half-waves: a K = 2 pair).
// XT aliases RT: the diagonal blocks are written only after the last read of RT, and the
// products read R12 from D.
__device__ __forceinline__ void chol_inverse_wave(const float* RT, const float* RI, const float* D, float* XT,
                                                  int lane) {
  asm volatile("" : "+v"(lane));  // lane-derived values stay here, not hoisted out of the caller's loop
  const int l32 = lane & 31, h = lane >> 5, o = 32 * h;  // block h, row l32 within it
  float x[32];
  static_for<0, 32>([&](auto cc) {
    constexpr int c = decltype(cc)::value;
    float acc = (l32 == c) ? 1.f : 0.f;
    // the column's reads depend on x[c - 2]: they issue one column ahead, not all at the start
    // (hoisted together they would not fit in registers)
    int off = (o + c) * 68 + o, ri = o + c;
    if constexpr (c >= 2) asm volatile("" : "+v"(off), "+v"(ri) : "v"(x[c - 2]));
    const lds_f4* rtc = lds_base(RT + off);
#pragma unroll
    for (int k4 = 0; k4 < (c + 3) / 4; ++k4) {
      const float4 rv = lds_get(rtc, k4);
      const float rvv[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * k4 + e < c) acc -= x[4 * k4 + e] * rvv[e];
    }
    x[c] = acc * RI[ri];
  });
  wave_lds_order();
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    XT[(o + c) * 65 + o + l32] = x[c];
    if (h) XT[c * 65 + 32 + l32] = 0.f;  // X21
  }
  wave_lds_order();
  f32x16 u = zero16();  // R12 X22
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int k = 2 * t + h;
    u = mfma(D[l32 * 65 + 32 + k], XT[(32 + l32) * 65 + 32 + k], u);
  }
  f32x16 x12 = zero16();  // -X11 (R12 X22)
#pragma unroll
  for (int r = 0; r < 16; ++r) x12 = mfma(-XT[acc_row(r, lane) * 65 + l32], u[r], x12);
#pragma unroll
  for (int r = 0; r < 16; ++r) XT[(32 + l32) * 65 + acc_row(r, lane)] = x12[r];
}

// T: threads per workgroup (512; 256 for n <= 256, where more waves would mostly idle; the
// next diagonal tile's quadrants need waves 0, 1 and 3).
template <int T = kCholThreads>
__global__ __launch_bounds__(T) __attribute__((amdgpu_waves_per_eu(2))) void k_chol(CholArgs a) {
  static_assert(T >= 256, "the diagonal-tile quadrants run on waves 0, 1 and 3");
  constexpr int NW = T / 64;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* D = smem;                 // [64][65] diagonal block, then R_kk (upper, zero below)
  float* XT = D + 64 * 65;         // [64][65] (R_kk^-1)^T: XT[i][k] = Dinv_kk[k][i] ...
  float* RT = XT;                  // ... over [64][68] R_kk column-major while it is factored
  float* RI = XT + 64 * 68;        // [64] 1 / R[j][j] of the diagonal block
  float* red = RI + 64;            // [16]
  int* ffail = reinterpret_cast<int*>(red + 16);
  float* S = red + 32;             // block row [64][n-64] when strip_lds

  const int n = a.n, b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int lds_w = n > kCholNb ? n - kCholNb : 1;
  // offsets inside one matrix are 32-bit (n * n < 2^31): one VGPR per address, not two
  float* G = a.G + b * a.sg;
  float* Dv = a.Dinv + (int64_t)b * n * 64;

  // jitter
  float part = 0.f;
  for (int i = tid; i < n; i += T) part += G[(int64_t)i * n + i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) red[wid] = part;
  if (tid == 0) *ffail = INT_MAX;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) tot += red[w];
  const float mu = 1e-7f * (tot / (float)n);
  for (int i = tid; i < n; i += T) G[(int64_t)i * n + i] += mu;
  __syncthreads();

  // Iteration k0 = -64 has no block of its own: its "trailing update" is wave 0 taking the
  // first diagonal block from G (so the factor and the inverse exist once in the code).
  // -W[:k, k] = -R[:k, k] Dinv_kk for block k at k0 (kb columns), strip m = rows 32 m .. + 31:
  // A = R[row][k0 + kk] (lane: row l32, kk = 2 t + h), B = Dinv_kk[kk][j] -- from its transposed
  // LDS copy XT, or (while the next factor overwrites XT) from HBM.  Columns of the block past n
  // meet zero rows of Dinv.
  auto w_strip = [&](int m, int k0, int kb, bool lds) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int l32 = ln & 31, h = ln >> 5;
    const float* rr = G + (32 * m + l32) * n;
    float av[32];
#pragma unroll
    for (int t = 0; t < 32; ++t) av[t] = rr[min(k0 + 2 * t + h, n - 1)];
    float* W = a.Wm + b * a.sw;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int j = 32 * half + l32;
      f32x16 acc = zero16();
      if (lds) {
        issue_loads_first();
#pragma unroll
        for (int t = 0; t < 32; ++t) acc = mfma(av[t], XT[j * 65 + 2 * t + h], acc);
      } else {
        float bw[32];
#pragma unroll
        for (int t = 0; t < 32; ++t) bw[t] = Dv[(k0 + 2 * t + h) * 64 + j];
        issue_loads_first();
#pragma unroll
        for (int t = 0; t < 32; ++t) acc = mfma(av[t], bw[t], acc);
      }
      if (j < kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) W[(32 * m + acc_row(r, ln)) * n + k0 + j] = -acc[r];
      }
    }
  };

  for (int k0 = -kCholNb; k0 < n; k0 += kCholNb) {
    const bool first = k0 < 0;
    const int kb = first ? 0 : min(kCholNb, n - k0), k1 = first ? 0 : k0 + kb, w = n - k1;

    if (!first) {
      // R_kk (upper) and Dinv_kk (row-major, zero below the diagonal) to HBM
      for (int idx = tid; idx < kb * 64; idx += T) {
        const int i = idx >> 6, c = idx & 63;
        if (c < kb && c >= i) G[(k0 + i) * n + k0 + c] = D[i * 65 + c];
        Dv[(k0 + i) * 64 + c] = (c < kb) ? XT[c * 65 + i] : 0.f;
      }
      // block row R_k,> = Dinv_kk^T G_k,>: each wave owns 32 columns (both 32-row halves),
      // so it can overwrite them in G without racing other waves' reads.  After the last
      // block (no trailing phase) the same loop forms that block's W strips (see w_strip).
      const int nch = w > 0 ? (w + 31) >> 5 : 0, nwj = (a.Wm && w <= 0) ? k0 >> 5 : 0;
      for (int job = wid; job < nch + nwj; job += NW) {
        if (job >= nch) {
          w_strip(job - nch, k0, kb, true);
          continue;
        }
        // lane-derived offsets are laundered per job: hoisted out of the block loop they
        // would stay live across it (32+ VGPRs) and spill
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int l32 = ln & 31, h = ln >> 5;
        const int colr = job * 32 + l32, col = k1 + colr;
        const int base = (k0 + h) * n + min(col, n - 1);  // columns past n: computed, not stored
        float bv[32];
#pragma unroll
        for (int t = 0; t < 32; ++t) bv[t] = G[base + 2 * t * n];
        issue_loads_first();
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
            const int i0 = acc_row(r, ln), i1 = 32 + acc_row(r, ln);
            G[(k0 + i0) * n + col] = acc0[r];
            G[(k0 + i1) * n + col] = acc1[r];
            if (a.strip_lds) {
              S[i0 * lds_w + colr] = acc0[r];
              S[i1 * lds_w + colr] = acc1[r];
            }
          }
        }
      }
      if (w <= 0) break;  // uniform; kb == 64 below this line
      __syncthreads();
    }

    // trailing G_>,> -= R_k,>^T R_k,> over upper 64x64 tiles.  Tile 0 is the next diagonal
    // block: wave 0 keeps it in LDS and factors and inverts it; waves 1..7 take the other
    // tiles and write them back to G.
    {
      const int nt = (w + 63) >> 6, npairs = first ? 1 : nt * (nt + 1) / 2;
      const int t0 = wid == 0 ? 0 : wid, tstep = wid == 0 ? npairs : NW - 1;
      const int kbn = min(kCholNb, w);
      // one 32x32 quadrant (qi, qj) of the next diagonal tile, updated and written into D
      // (identity past n)
      auto diag_quadrant = [&](int qi, int qj) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int l32 = ln & 31, h = ln >> 5;
        f32x16 q;
#pragma unroll
        for (int r = 0; r < 16; ++r) {  // rows / columns past n clamped: never stored
          const int row = min(k1 + 32 * qi + acc_row(r, ln), n - 1);
          const int col = min(k1 + 32 * qj + l32, n - 1);
          q[r] = G[row * n + col];
        }
        issue_loads_first();
        const int ci = 32 * qi + l32, cj = 32 * qj + l32;
        if (a.strip_lds) {
#pragma unroll 8
          for (int kk = 0; kk < kCholNb; kk += 2) {
            const float* sk = S + (kk + h) * lds_w;
            q = mfma(-sk[ci], sk[cj], q);
          }
        } else {
#pragma unroll 8
          for (int kk = 0; kk < kCholNb; kk += 2) {
            const float* gk = G + (k0 + kk + h) * n + k1;
            q = mfma(-gk[ci], gk[cj], q);
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 32 * qi + acc_row(r, ln), c = 32 * qj + l32;
          D[i * 65 + c] = (i < kbn && c < kbn) ? q[r] : (i == c ? 1.f : 0.f);
        }
      };
      // the next diagonal tile is updated by quadrants on three SIMDs at once -- (0,0) on wave
      // 0, (0,1) and (1,1) on waves 1 and 3; its quadrant (1,0) lies below the diagonal, which
      // the factor never reads -- and one barrier later wave 0 factors it while the other
      // waves take the remaining tiles
      if (!first) {
        if (wid == 0 || wid == 1 || wid == 3) diag_quadrant(wid == 3 ? 1 : 0, wid == 0 ? 0 : 1);
        __syncthreads();
      }
      auto diag_factor = [&]() {
        wave_lds_order();
        const int fail = chol_diag_wave(D, RT, RI, lane);
        if (lane == 0 && fail != INT_MAX && fail < kbn && *ffail == INT_MAX) *ffail = k1 + fail + 1;
        wave_lds_order();
        chol_inverse_wave(RT, RI, D, XT, lane);
      };
      for (int pr = t0; pr < npairs; pr += tstep) {
        if (pr == 0 && !first) {  // wave 0: the next diagonal tile, complete in D since the barrier
          diag_factor();
          continue;
        }
        int I, J;
        upper_tile(pr, nt, I, J);
        int ln = lane;  // laundered per tile, as above
        asm volatile("" : "+v"(ln));
        const int l32 = ln & 31, h = ln >> 5;
        f32x16 acc[2][2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int nj = 0; nj < 2; ++nj)
#pragma unroll
            for (int r = 0; r < 16; ++r) {  // rows / columns past n clamped: never stored
              const int row = min(k1 + I * 64 + mi * 32 + acc_row(r, ln), n - 1);
              const int col = min(k1 + J * 64 + nj * 32 + l32, n - 1);
              acc[mi][nj][r] = G[row * n + col];
            }
        issue_loads_first();
        if (!first) {
          // Operand reads are unconditional: a row ci >= w of R_k,> only meets accumulator
          // rows (or columns) >= w of this tile, which are never stored.  The strip has 64
          // floats of padding for that, and in G such reads stay inside the matrix (k1 < n).
          const int ci0 = I * 64 + l32, cj0 = J * 64 + l32;
          if (a.strip_lds) {
#pragma unroll 8
            for (int kk = 0; kk < kCholNb; kk += 2) {
              const float* sk = S + (kk + h) * lds_w;
              const float av[2] = {-sk[ci0], -sk[ci0 + 32]}, bv[2] = {sk[cj0], sk[cj0 + 32]};
#pragma unroll
              for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int nj = 0; nj < 2; ++nj) acc[mi][nj] = mfma(av[mi], bv[nj], acc[mi][nj]);
            }
          } else {
#pragma unroll 8
            for (int kk = 0; kk < kCholNb; kk += 2) {
              const float* gk = G + (k0 + kk + h) * n + k1;
              const float av[2] = {-gk[ci0], -gk[ci0 + 32]}, bv[2] = {gk[cj0], gk[cj0 + 32]};
#pragma unroll
              for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int nj = 0; nj < 2; ++nj) acc[mi][nj] = mfma(av[mi], bv[nj], acc[mi][nj]);
            }
          }
        }
        if (pr == 0) {
          // the first diagonal block (iteration k0 = -64: no update) -> D, then factor and invert it
#pragma unroll
          for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nj = 0; nj < 2; ++nj)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int i = mi * 32 + acc_row(r, ln), c = nj * 32 + l32;
                D[i * 65 + c] = (i < kbn && c < kbn) ? acc[mi][nj][r] : (i == c ? 1.f : 0.f);
              }
          diag_factor();
        } else {
#pragma unroll
          for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nj = 0; nj < 2; ++nj)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int row = k1 + I * 64 + mi * 32 + acc_row(r, ln);
                const int col = k1 + J * 64 + nj * 32 + l32;
                if (row < n && col < n) G[row * n + col] = acc[mi][nj][r];
              }
        }
      }
      // this block's W strips on the waves past their tiles (wave 0's factor is the longer
      // chain); Dinv_kk went to HBM before the block row's barrier
      if (!first && a.Wm && wid > 0)
        for (int m = wid - 1; m < (k0 >> 5); m += NW - 1) w_strip(m, k0, kb, false);
    }
    __syncthreads();
  }
  __syncthreads();
  if (tid == 0) {
    const int f = (*ffail == INT_MAX) ? 0 : *ffail;
    if (!a.keep_info || a.info[b] == 0) a.info[b] = f;
  }
}

// ---- split form: batches too small to fill the GPU with one workgroup per matrix ----------
// The same arithmetic as k_chol, operation for operation, in four kinds of launches per
// matrix batch: the jitter once, then per 64-column block the diagonal factor and inverse
// (one wave per matrix), the block row (one wave per 32 columns) and the trailing update (one
// wave per upper 64x64 tile).  The diagonal tile goes through G instead of staying in LDS.
constexpr int kCholSplitThreads = 256;

struct CholSplitArgs {
  float* G;
  int64_t sg;
  float* Dinv;
  int* info;
  int n, k0, keep_info, njob;
  int nb;  // k_chol_step: the batch (its first nb workgroups factor the next diagonal block)
};

__global__ __launch_bounds__(kCholThreads) void k_chol_jitter(CholSplitArgs a) {
  __shared__ float red[kCholThreads / 64];
  constexpr int NW = kCholThreads / 64;
  const int n = a.n, b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float* G = a.G + b * a.sg;
  float part = 0.f;
  for (int i = tid; i < n; i += kCholThreads) part += G[(int64_t)i * n + i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) red[wid] = part;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) tot += red[w];
  const float mu = 1e-7f * (tot / (float)n);
  for (int i = tid; i < n; i += kCholThreads) G[(int64_t)i * n + i] += mu;
  if (tid == 0 && (!a.keep_info || a.info[b] == 0)) a.info[b] = 0;
}

// Wave 0 of a split-form launch: factor and invert the diagonal block at k0 held in D (upper
// part; the identity past n), write R_kk (upper) and Dinv_kk, record a failed pivot in info.
__device__ __forceinline__ void chol_split_factor(const CholSplitArgs& a, int b, int k0, float* D, float* XT,
                                                  float* RI, int lane) {
  const int n = a.n, kb = min(kCholNb, n - k0);
  float* G = a.G + b * a.sg;
  float* Dv = a.Dinv + (int64_t)b * n * 64;
  wave_lds_order();
  const int fail = chol_diag_wave(D, XT, RI, lane);
  if (lane == 0 && fail != INT_MAX && fail < kb && a.info[b] == 0) a.info[b] = k0 + fail + 1;
  wave_lds_order();
  chol_inverse_wave(XT, RI, D, XT, lane);
  wave_lds_order();
#pragma unroll 16
  for (int i = 0; i < kb; ++i) {
    const int c = lane;
    if (c < kb && c >= i) G[(k0 + i) * n + k0 + c] = D[i * 65 + c];
    Dv[(k0 + i) * 64 + c] = (c < kb) ? XT[c * 65 + i] : 0.f;
  }
}

__global__ __launch_bounds__(64) void k_chol_diag(CholSplitArgs a) {
  __shared__ float D[64 * 65];
  __shared__ __attribute__((aligned(16))) float XT[64 * 68];  // RT while factoring, then XT
  __shared__ float RI[64];
  const int n = a.n, k0 = a.k0, b = blockIdx.x, lane = threadIdx.x;
  const int kb = min(kCholNb, n - k0);
  const float* G = a.G + b * a.sg;
  {
    // the block row by row, the lanes along each row: all 64 loads in flight together
    // (addresses clamped past n, the identity written there)
    const int cl = min(lane, kb - 1);
    float v[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = G[(k0 + min(i, kb - 1)) * n + k0 + cl];
#pragma unroll
    for (int i = 0; i < 64; ++i) D[i * 65 + lane] = (i < kb && lane < kb) ? v[i] : (i == lane ? 1.f : 0.f);
  }
  chol_split_factor(a, b, k0, D, XT, RI, lane);
}

// R_k,> = Dinv_kk^T G_k,>: wave w of workgroup g takes the 32 columns starting at
// k1 + 32 (4 g + w).
__global__ __launch_bounds__(kCholSplitThreads) void k_chol_row(CholSplitArgs a) {
  __shared__ float XT[64 * 65];
  const int n = a.n, k0 = a.k0, k1 = k0 + kCholNb, w = n - k1;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, l32 = lane & 31, h = lane >> 5;
  const int64_t pid = blockIdx.x;
  const int64_t b = pid / a.njob;
  const int job = 4 * (int)(pid - b * a.njob) + wid;
  float* G = a.G + b * a.sg;
  const float* Dv = a.Dinv + b * n * 64;
  // the job's block-row operand is loaded first (clamped for jobs past the end, which only
  // stage Dinv), then Dinv_kk with all its loads in flight together
  const int colr = job * 32 + l32, col = k1 + colr;
  const int base = (k0 + h) * n + min(col, n - 1);  // columns past n: computed, not stored
  float bv[32];
#pragma unroll
  for (int t = 0; t < 32; ++t) bv[t] = G[base + 2 * t * n];
  issue_loads_first();
  constexpr int DPT = 64 * 64 / kCholSplitThreads;
  float dv[DPT];
#pragma unroll
  for (int u = 0; u < DPT; ++u) {
    const int idx = tid + kCholSplitThreads * u, i = idx >> 6, c = idx & 63;
    dv[u] = Dv[(k0 + i) * 64 + c];
  }
#pragma unroll
  for (int u = 0; u < DPT; ++u) {
    const int idx = tid + kCholSplitThreads * u, i = idx >> 6, c = idx & 63;  // XT[c][i] = Dinv_kk[i][c]
    XT[c * 65 + i] = dv[u];
  }
  __syncthreads();
  if (32 * job >= w) return;
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
      G[(k0 + i0) * n + col] = acc0[r];
      G[(k0 + i1) * n + col] = acc1[r];
    }
  }
}

// One upper 64x64 tile pair pr of G_>,> -= R_k,>^T R_k,> (the trailing matrix right of block k0).
__device__ __forceinline__ void chol_trail_pair(const CholSplitArgs& a, int64_t b, int pr, int lane) {
  const int n = a.n, k0 = a.k0, k1 = k0 + kCholNb, w = n - k1;
  const int l32 = lane & 31, h = lane >> 5;
  const int nt = (w + 63) >> 6;
  float* G = a.G + b * a.sg;
  int I, J;
  upper_tile(pr, nt, I, J);
  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int r = 0; r < 16; ++r) {  // rows / columns past n clamped: never stored
        const int row = min(k1 + I * 64 + mi * 32 + acc_row(r, lane), n - 1);
        const int col = min(k1 + J * 64 + nj * 32 + l32, n - 1);
        acc[mi][nj][r] = G[row * n + col];
      }
  issue_loads_first();
  const int ci0 = I * 64 + l32, cj0 = J * 64 + l32;  // reads past w reach unstored entries only
#pragma unroll
  for (int kk = 0; kk < kCholNb; kk += 2) {
    const float* gk = G + (k0 + kk + h) * n + k1;
    const float av[2] = {-gk[ci0], -gk[ci0 + 32]}, bv[2] = {gk[cj0], gk[cj0 + 32]};
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
        if (row < n && col < n) G[row * n + col] = acc[mi][nj][r];
      }
}

// The trailing update of block k0 and the factor of the next diagonal block, in one launch so
// the two run side by side.  Workgroups [0, batch) take matrix b's next diagonal tile (tile pair
// 0): its upper 32x32 quadrants updated by the block row on waves 0-2 straight into LDS (the
// lower-left one is never read by the factor), then wave 0 factors and inverts it as
// k_chol_diag does.  The others take tile pairs 1 .. npairs - 1, one per wave (a.njob
// workgroups per matrix).
__global__ __launch_bounds__(kCholSplitThreads) void k_chol_step(CholSplitArgs a) {
  __shared__ float D[64 * 65];
  __shared__ __attribute__((aligned(16))) float XT[64 * 68];  // RT while factoring, then XT
  __shared__ float RI[64];
  const int n = a.n, k0 = a.k0, k1 = k0 + kCholNb, w = n - k1;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t pid = blockIdx.x;
  if (pid < a.nb) {
    const int b = (int)pid, kbn = min(kCholNb, w);
    const float* G = a.G + b * a.sg;
    if (wid < 3) {
      const int qi = wid == 2 ? 1 : 0, qj = wid == 0 ? 0 : 1;
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int l32 = ln & 31, h = ln >> 5;
      f32x16 q;
#pragma unroll
      for (int r = 0; r < 16; ++r) {  // rows / columns past n clamped: never stored
        const int row = min(k1 + 32 * qi + acc_row(r, ln), n - 1);
        const int col = min(k1 + 32 * qj + l32, n - 1);
        q[r] = G[row * n + col];
      }
      issue_loads_first();
      const int ci = 32 * qi + l32, cj = 32 * qj + l32;
#pragma unroll 8
      for (int kk = 0; kk < kCholNb; kk += 2) {
        const float* gk = G + (k0 + kk + h) * n + k1;
        q = mfma(-gk[ci], gk[cj], q);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * qi + acc_row(r, ln), c = 32 * qj + l32;
        D[i * 65 + c] = (i < kbn && c < kbn) ? q[r] : (i == c ? 1.f : 0.f);
      }
    }
    __syncthreads();
    if (wid == 0) chol_split_factor(a, b, k1, D, XT, RI, lane);
    return;
  }
  const int64_t q = pid - a.nb, b = q / a.njob;
  const int nt = (w + 63) >> 6, npairs = nt * (nt + 1) / 2;
  const int pr = 1 + 4 * (int)(q - b * a.njob) + wid;
  if (pr < npairs) chol_trail_pair(a, b, pr, lane);
}


}  // namespace rnr
