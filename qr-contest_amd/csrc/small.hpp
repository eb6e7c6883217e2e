// The whole reflector-free QR of small matrices (n <= NP <= 64) in one launch, one matrix
// per group of NP lanes of a wave (64 / NP matrices per wave), lane r of a group holding
// row r of the working matrix in registers -- reflection_no_reflectors.py:181-196 end to end:
//
//   LU (:66)      partial pivoting with LAPACK's first-maximum rule over the current row
//                 order; rows never move: each lane keeps its row's logical position, so
//                 the factor stays in A's row order and the frame's Q = P Q2 (:81) is the
//                 row order the lanes already hold;
//   CholeskyQR2 (:68-80)  G = M^T M on 16x16x4 MFMA from an LDS copy of M (upper blocks);
//                 mu = 1e-7 mean(diag G) added to the diagonal; the Cholesky runs on
//                 the rows of G held by the lanes (pivot row broadcast through LDS); the
//                 solve M R^-1 is a forward substitution inside each lane with the
//                 columns of R read as LDS broadcasts;
//   closure (:186) R = triu(Q^T A) on MFMA, A kept in LDS from the load;
//   chart (:139-174, :192)  the sign-ruled unpivoted elimination of the Q rows, then
//                 tau_k = 2 / (1 + sum_{i>k} Y[i][k]^2);
//   pack (:195)   H = triu(diag(s) R) + tril(Y, -1), staged in LDS and stored coalesced.
//
// Rows and columns past n are zero and every step runs only for column indices < n, so the
// padding never takes part.  All LDS traffic of a group stays inside its wave (a wave issues
// its LDS operations in order; wave_lds_order keeps the compiler from reordering them), so
// the kernel has no workgroup barrier and idle waves may leave early.
#pragma once
#include "common.hpp"

namespace rnr {

struct SmallArgs {
  const float* A;
  int64_t sa;
  float* H;
  float* tau;
  int* info;  // may be null
  int n;
  int batch;
  int vec4;   // n % 4 == 0, A / H 16-byte aligned, sa % 4 == 0
};

constexpr int kSmallWaves = 4;  // waves per workgroup (each works alone)
constexpr int kSmallMaxN = 64;

template <int NP>
struct SmallLayout {
  static constexpr int G = 64 / NP;    // matrices per wave
  static constexpr int LD = NP + 4;    // LDS row stride: row-per-lane float4 access is conflict-free
  static constexpr int MAT = NP * LD;  // one matrix buffer
  static constexpr int SLOT = NP + 4;  // broadcast row
  // per wave: As[G][MAT] (A, later Y), Ws[G][MAT] (MFMA staging, G, R^T, R, H),
  // Sl[G][SLOT] (broadcast row), Dv[G][NP] (1 / R[c][c])
  static constexpr int PER_WAVE = 2 * G * MAT + G * SLOT + G * NP;
};

inline int small_np(int n) { return n <= 16 ? 16 : (n <= 32 ? 32 : 64); }

inline size_t small_lds_bytes(int np) {
  const int per = np == 16 ? SmallLayout<16>::PER_WAVE
                           : (np == 32 ? SmallLayout<32>::PER_WAVE : SmallLayout<64>::PER_WAVE);
  return sizeof(float) * (size_t)per * kSmallWaves;
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4v mfma16x4(float a, float b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The value of lane l ^ 16 (v_permlane16_swap of v with itself: .x holds rows 0, 0, 2, 2 of
// 16 lanes, .y rows 1, 1, 3, 3) and of lane l ^ 32 (v_permlane32_swap: .x the low half twice,
// .y the high half twice) -- VALU lane exchanges, no LDS round trip.
__device__ __forceinline__ uint32_t lane_xor16(uint32_t v) {
  const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (__lane_id() & 16) ? p[0] : p[1];
}
__device__ __forceinline__ uint32_t lane_xor32(uint32_t v) {
  const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (__lane_id() & 32) ? p[0] : p[1];
}
__device__ __forceinline__ float lane_xor16(float v) { return __uint_as_float(lane_xor16(__float_as_uint(v))); }
__device__ __forceinline__ float lane_xor32(float v) { return __uint_as_float(lane_xor32(__float_as_uint(v))); }
__device__ __forceinline__ int lane_xor16(int v) { return (int)lane_xor16((uint32_t)v); }
__device__ __forceinline__ int lane_xor32(int v) { return (int)lane_xor32((uint32_t)v); }

// First-maximum argmax of (|v|, position) over aligned groups of GL lanes; every lane of a
// group ends with the group's winner.  Butterfly steps: four DPP exchanges inside rows of 16
// lanes, then lane-xor 16 and 32 by permlane swaps.
template <int GL>
__device__ __forceinline__ void group_argmax(float& babs, float& bv, int& bi) {
  argmax_dpp_step<kDppQuad1032>(babs, bv, bi);
  argmax_dpp_step<kDppQuad2301>(babs, bv, bi);
  argmax_dpp_step<kDppRowHalfMirror>(babs, bv, bi);
  argmax_dpp_step<kDppRowMirror>(babs, bv, bi);
  if constexpr (GL >= 32)
    argmax_take(babs, bv, bi, lane_xor16(babs), lane_xor16(bv), lane_xor16(bi));
  if constexpr (GL >= 64)
    argmax_take(babs, bv, bi, lane_xor32(babs), lane_xor32(bv), lane_xor32(bi));
}

// Sum over aligned groups of GL lanes, the same value in every lane of the group.
template <int GL>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<kDppQuad1032>(v);
  v += dpp_f<kDppQuad2301>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  if constexpr (GL >= 32) v += lane_xor16(v);
  if constexpr (GL >= 64) v += lane_xor32(v);
  return v;
}

template <int GL>
__device__ __forceinline__ int group_min(int v) {
  v = min(v, dpp_i<kDppQuad1032>(v));
  v = min(v, dpp_i<kDppQuad2301>(v));
  v = min(v, dpp_i<kDppRowHalfMirror>(v));
  v = min(v, dpp_i<kDppRowMirror>(v));
  if constexpr (GL >= 32) v = min(v, lane_xor16(v));
  if constexpr (GL >= 64) v = min(v, lane_xor32(v));
  return v;
}

// row <-> LDS, float4 at a time
template <int NP>
__device__ __forceinline__ void lds_load_row(float (&x)[NP], const float* p) {
#pragma unroll
  for (int c4 = 0; c4 < NP / 4; ++c4) {
    const float4 v = reinterpret_cast<const float4*>(p)[c4];
    x[4 * c4] = v.x; x[4 * c4 + 1] = v.y; x[4 * c4 + 2] = v.z; x[4 * c4 + 3] = v.w;
  }
}
// columns from chunk C0 on
template <int NP, int C0 = 0>
__device__ __forceinline__ void lds_store_row(float* p, const float (&x)[NP]) {
#pragma unroll
  for (int c4 = C0; c4 < NP / 4; ++c4)
    reinterpret_cast<float4*>(p)[c4] = make_float4(x[4 * c4], x[4 * c4 + 1], x[4 * c4 + 2], x[4 * c4 + 3]);
}

// x[c] -= l * S[c] for compile-time c > J: S is the group's broadcast row in LDS.  Columns
// past n are zero in S and in x, so they are updated too (no runtime test between the LDS
// reads: they issue back to back and complete under one wait).
template <int NP, int J>
__device__ __forceinline__ void rank1_from_slot(float (&x)[NP], float l, const float* S) {
  constexpr int C0 = (J + 1) / 4;
  float4 p[NP / 4 - C0 > 0 ? NP / 4 - C0 : 1];
#pragma unroll
  for (int c4 = C0; c4 < NP / 4; ++c4) p[c4 - C0] = reinterpret_cast<const float4*>(S)[c4];
#pragma unroll
  for (int c4 = C0; c4 < NP / 4; ++c4) {
    const float pv[4] = {p[c4 - C0].x, p[c4 - C0].y, p[c4 - C0].z, p[c4 - C0].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (4 * c4 + e > J) x[4 * c4 + e] -= l * pv[e];
  }
}

// Broadcast within each group of NP lanes from the group's lane p[g] (uniform lane indices, one
// per group): readlane into scalar registers, no LDS (whose instructions cost their full width
// even for one storing lane, on a pipe every wave of the CU shares).  For 1 or 2 groups per wave.
template <int G>
__device__ __forceinline__ float group_bcast(float v, const int (&p)[G], bool upper) {
  const float u0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), p[0]));
  if constexpr (G == 1) {
    return u0;
  } else {
    const float u1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), p[1]));
    return upper ? u1 : u0;
  }
}

// x[c] -= l * (x[c] of the group's lane p) for compile-time c > J
template <int NP, int G, int J>
__device__ __forceinline__ void rank1_from_lanes(float (&x)[NP], float l, const int (&p)[G], bool upper) {
#pragma unroll
  for (int c = J + 1; c < NP; ++c) x[c] -= l * group_bcast<G>(x[c], p, upper);
}

// acc[g][u] = upper 16x16 blocks (bi <= bj, row-major order u) of X_g^T Y_g for the G
// matrices of this wave: X_g, Y_g are NP x NP (row stride LD) at X + g*MAT, Y + g*MAT,
// zero past row and column n.
template <int NP>
__device__ __forceinline__ void wave_upper_tn(const float* X, const float* Y, bool same, int lane,
                                              f32x4v (&acc)[SmallLayout<NP>::G][(NP / 16) * (NP / 16 + 1) / 2]) {
  using Lay = SmallLayout<NP>;
  constexpr int NB = NP / 16;
  const int l16 = lane & 15, q4 = lane >> 4;
#pragma unroll
  for (int g = 0; g < Lay::G; ++g)
#pragma unroll
    for (int u = 0; u < NB * (NB + 1) / 2; ++u) acc[g][u] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < Lay::G; ++g) {
    const float* Xg = X + g * Lay::MAT;
    const float* Yg = Y + g * Lay::MAT;
#pragma unroll
    for (int t = 0; t < NP / 4; ++t) {
      float xa[NB], yb[NB];
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        xa[bb] = Xg[(4 * t + q4) * Lay::LD + 16 * bb + l16];
        yb[bb] = same ? xa[bb] : Yg[(4 * t + q4) * Lay::LD + 16 * bb + l16];
      }
      int u = 0;
#pragma unroll
      for (int bi = 0; bi < NB; ++bi)
#pragma unroll
        for (int bj = bi; bj < NB; ++bj) {
          acc[g][u] = mfma16x4(xa[bi], yb[bj], acc[g][u]);
          ++u;
        }
    }
  }
}

// D[row][col] of a 16x16x4 result sits in lane col + 16 * (row / 4), register row % 4.
// SYM: the blocks below the diagonal too, as the transposes (a symmetric product).
template <int NP, bool SYM = false>
__device__ __forceinline__ void wave_store_upper(float* W, int lane,
                                                 const f32x4v (&acc)[SmallLayout<NP>::G][(NP / 16) * (NP / 16 + 1) / 2]) {
  using Lay = SmallLayout<NP>;
  constexpr int NB = NP / 16;
  const int l16 = lane & 15, q4 = lane >> 4;
#pragma unroll
  for (int g = 0; g < Lay::G; ++g) {
    int u = 0;
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
#pragma unroll
      for (int bj = bi; bj < NB; ++bj) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          W[g * Lay::MAT + (16 * bi + 4 * q4 + e) * Lay::LD + 16 * bj + l16] = acc[g][u][e];
          if (SYM && bj > bi) W[g * Lay::MAT + (16 * bj + l16) * Lay::LD + 16 * bi + 4 * q4 + e] = acc[g][u][e];
        }
        ++u;
      }
  }
}

template <int NP>
__global__ __launch_bounds__(64 * kSmallWaves) void k_small(SmallArgs a) {
  using Lay = SmallLayout<NP>;
  constexpr int G = Lay::G, LD = Lay::LD, MAT = Lay::MAT, NP4 = NP / 4;
  constexpr int NBU = (NP / 16) * (NP / 16 + 1) / 2;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int g = lane / NP, r = lane - g * NP;
  const int mat0 = (blockIdx.x * kSmallWaves + wid) * G;
  if (mat0 >= a.batch) return;  // the whole wave is idle; the kernel has no workgroup barrier
  const int n = a.n, mat = mat0 + g;
  const bool live = r < n;
  // one matrix per wave: row broadcasts by readlane (RL); two or four: through LDS slots (with
  // two groups the readlanes and selects cost more than the LDS round trips they replace:
  // 4096 x 32, 85 -> 102 us)
  constexpr bool RL = G == 1;
  const bool gup = g == 1;  // RL with two groups: this lane's group is the upper one
  float* As = smem + wid * Lay::PER_WAVE;
  float* Ws = As + G * MAT;
  float* Sl = Ws + G * MAT;
  float* Dv = Sl + G * Lay::SLOT;
  float* myA = As + g * MAT;
  float* myW = Ws + g * MAT;
  float* myS = Sl + g * Lay::SLOT;
  float* myD = Dv + g * NP;

  // ---- A of the wave's G matrices -> As (zero padded), coalesced
  if (a.vec4) {
    constexpr int TOT4 = G * NP * NP / 4;
#pragma unroll
    for (int i = 0; i < TOT4 / 64; ++i) {
      const int idx = lane + 64 * i;
      const int gg = idx / (NP * NP4), rem = idx - gg * NP * NP4, row = rem / NP4, c = 4 * (rem - row * NP4);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (mat0 + gg < a.batch && row < n && c < n)
        v = *reinterpret_cast<const float4*>(a.A + (int64_t)(mat0 + gg) * a.sa + (int64_t)row * n + c);
      *reinterpret_cast<float4*>(As + gg * MAT + row * LD + c) = v;
    }
  } else {
    constexpr int TOT = G * NP * NP;
#pragma unroll 4
    for (int i = 0; i < TOT / 64; ++i) {
      const int idx = lane + 64 * i;
      const int gg = idx / (NP * NP), rem = idx - gg * NP * NP, row = rem / NP, c = rem - row * NP;
      float v = 0.f;
      if (mat0 + gg < a.batch && row < n && c < n) v = a.A[(int64_t)(mat0 + gg) * a.sa + (int64_t)row * n + c];
      As[gg * MAT + row * LD + c] = v;
    }
  }
  myD[r] = 1.f;  // 1 / R[c][c]; stays 1 for the padded columns
  wave_lds_order();
  float x[NP];
  lds_load_row<NP>(x, myA + r * LD);

  // ---- LU with partial pivoting (lane r keeps row r; pos = its row's logical position)
  int pos = r;
  static_for<0, NP>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j < n) {
      int rr = r;
      asm volatile("" : "+v"(rr));  // keeps the per-column lane masks local to this column
      const bool cand = (rr < n) && (pos >= j);
      const float v = x[j];
      float babs = cand ? (v != v ? -0.5f : fabsf(v)) : -1.f;  // NaN ranks below any number
      float bv = cand ? v : 0.f;
      int bi = cand ? pos : INT_MAX;
      group_argmax<NP>(babs, bv, bi);
      const bool win = cand && pos == bi;
      int pw[RL ? G : 1];  // RL: the winning lane of each group (one per group), uniform
      if constexpr (RL) {
        const uint64_t wm = __ballot(win);
        pw[0] = __builtin_amdgcn_readfirstlane(__ffsll((long long)(G == 1 ? wm : (wm & 0xffffffffull))) - 1);
        if constexpr (G == 2) pw[G - 1] = __builtin_amdgcn_readfirstlane(__ffsll((long long)(wm >> 32)) + 31);
      } else {
        if (win) lds_store_row<NP, (j + 1) / 4>(myS, x);
        wave_lds_order();
      }
      // LAPACK xGETRF2: scale by the reciprocal unless the pivot is subnormal; a zero pivot
      // (all-zero column) leaves the column as it is
      const float pv = bv;
      const bool nz = pv != 0.f, recip = fabsf(pv) >= 1.17549435e-38f;
      const float inv = 1.f / pv;
      float l = 0.f;
      if (cand && !win) {
        l = x[j];
        if (nz) {
          l = recip ? l * inv : l / pv;
          x[j] = l;
        }
      }
      pos = win ? j : (pos == j ? bi : pos);
      if constexpr (RL) {
        rank1_from_lanes<NP, G, j>(x, l, pw, gup);  // the winner's own l is 0
      } else {
        rank1_from_slot<NP, j>(x, l, myS);
        wave_lds_order();  // the next column's slot store stays behind these reads
      }
    }
  });
  // unit-lower L in A's row order: row r of the factor sits at logical position pos
  static_for<0, NP>([&](auto cc) {
    constexpr int c = decltype(cc)::value;
    x[c] = live ? (c < pos ? x[c] : (c == pos ? 1.f : 0.f)) : 0.f;
  });

  // ---- CholeskyQR, twice: x <- x R^-1 with R = chol(x^T x + mu I)
  int fail0 = INT_MAX, fail1 = INT_MAX;
#pragma nounroll
  for (int pass = 0; pass < 2; ++pass) {
    lds_store_row<NP>(myW + r * LD, x);
    wave_lds_order();
    {
      f32x4v acc[G][NBU];
      wave_upper_tn<NP>(Ws, Ws, true, lane, acc);
      wave_lds_order();
      wave_store_upper<NP, RL>(Ws, lane, acc);  // RL: whole (symmetric), the Cholesky reads both halves
    }
    wave_lds_order();
    // jitter: mu = 1e-7 * mean(diag G), added to the diagonal (reflection_no_reflectors.py:74-75)
    const float dg = live ? myW[r * LD + r] : 0.f;
    const float mu = 1e-7f * (group_sum<NP>(dg) / (float)n);
    if (live) myW[r * LD + r] = dg + mu;
    int f = INT_MAX;
    if constexpr (G == 2) {
      // two matrices per wave: their G' are the two blocks of one v_mfma_f32_32x32x1_2b_f32
      // accumulator (block g from lanes 32 g ..), and each step's rank-1 update G' -= u u^T of
      // both is one MFMA: the pivots are read from their accumulator lanes, row j of each
      // block (one register, one half-wave) is gathered into lane order with a permlane32
      // swap and scaled into row j of R, which goes straight to R^T in Ws
      wave_lds_order();  // the jitter's diagonal stores before these reads of other lanes' rows
      f32x32 acc;
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const int i = acc_row(q & 15, lane), c = lane & 31;
        acc[q] = Ws[(q >> 4) * MAT + ((i <= c) ? i * LD + c : c * LD + i)];  // upper part of G'
      }
      wave_lds_order();  // the R^T stores below stay behind these reads
      static_for<0, NP>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        constexpr int HJ = (j / 4) % 2, RR = 4 * (j / 8) + j % 4;
        if (j < n) {
          int rr = r;
          asm volatile("" : "+v"(rr));  // the step's lane masks are formed here, not hoisted
          const float d0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc[RR]), j + 32 * HJ));
          const float d1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc[16 + RR]), j + 32 * HJ));
          const float d = gup ? d1 : d0;
          if (!(d > 0.f) && f == INT_MAX) f = j;
          const float rjj = sqrtf(d), rinv = 1.f / rjj;
          const float2 p = lane_halves(acc[RR], acc[16 + RR]);
          const float v = HJ == 0 ? p.x : p.y;  // lane c of group g: G'_g[j][c]
          const float rv = (rr == j) ? rjj : v * rinv;
          if (j + 1 < n) {
            const float u = (rr > j) ? rv : 0.f;
            acc = mfma_2b(-u, u, acc);
          }
          myW[rr * LD + j] = (rr >= j) ? rv : 0.f;  // R^T[c][j] = R[j][c]
          if (rr == j) myD[j] = rinv;
        }
      });
    } else {
    float gr[NP];
    lds_load_row<NP>(gr, myW + r * LD);  // upper part of row r of G (+ mu I)
    wave_lds_order();

    // upper Cholesky on the rows: step j broadcasts row j of R = G'[j][j:] / sqrt(G'[j][j])
    static_for<0, NP>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if (j < n) {
        int rr = r;
        asm volatile("" : "+v"(rr));
        if constexpr (RL) {
          // G' is held whole (symmetric): lane r's G'[r][j] is G'[j][r], so R[j][r] / R[j][j] =
          // G'[r][j] / G'[j][j] is lane-local and only row j's raw values are broadcast (read
          // before lane j scales its row)
          int pj[G];
          pj[0] = j;
          if constexpr (G == 2) pj[G - 1] = NP + j;
          const float d = group_bcast<G>(gr[j], pj, gup);
          const float rjj = sqrtf(d), rinv = 1.f / rjj;
          if (rr > j && rr < n) rank1_from_lanes<NP, G, j>(gr, (gr[j] * rinv) * rinv, pj, gup);
          if (rr == j) {
            if (!(d > 0.f)) f = j;
            gr[j] = rjj;
#pragma unroll
            for (int c = j + 1; c < NP; ++c) gr[c] *= rinv;
            myD[j] = rinv;
          }
        } else {
          if (rr == j) {
            const float d = gr[j];
            if (!(d > 0.f)) f = j;
            const float rjj = sqrtf(d), rinv = 1.f / rjj;
            gr[j] = rjj;
#pragma unroll
            for (int c = j + 1; c < NP; ++c) gr[c] *= rinv;
            lds_store_row<NP, j / 4>(myS, gr);
            myD[j] = rinv;
          }
          wave_lds_order();
          if (rr > j && rr < n) {
            const float rj = myS[rr];  // R[j][r]
            rank1_from_slot<NP, j>(gr, rj, myS);
          }
          wave_lds_order();
        }
      }
    });
    // R^T -> Ws (column c of R contiguous), then x <- x R^-1 by forward substitution.  Rows
    // of G past n are zero, so R^T is zero there; 1 / R[c][c] is 1 past n: the padded
    // columns of x stay zero and need no test.
#pragma unroll
    for (int c = 0; c < NP; ++c) myW[c * LD + r] = gr[c];
    }
    f = group_min<NP>(f);
    if (pass == 0) fail0 = f; else fail1 = f;
    wave_lds_order();
    static_for<0, NP>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      float acc = x[c];
#pragma unroll
      for (int k4 = 0; k4 < (c + 3) / 4; ++k4) {
        const float4 rv = reinterpret_cast<const float4*>(myW + c * LD)[k4];
        const float rvv[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * k4 + e < c) acc -= x[4 * k4 + e] * rvv[e];
      }
      x[c] = acc * myD[c];
    });
    wave_lds_order();
  }

  // ---- closure: Rc = triu(Q^T A) -> Ws (x holds row r of Q)
  lds_store_row<NP>(myW + r * LD, x);
  wave_lds_order();
  {
    f32x4v acc[G][NBU];
    wave_upper_tn<NP>(Ws, As, false, lane, acc);
    wave_lds_order();
    wave_store_upper<NP>(Ws, lane, acc);
  }
  wave_lds_order();

  // ---- chart: sign-ruled unpivoted elimination of the Q rows
  float my_s = 1.f;
  if constexpr (G == 2) {
    // two matrices per wave, no pivoting: each Q is held twice in v_mfma_f32_32x32x1_2b_f32
    // accumulators, as itself (D1[i][c] = x[i][c]) and transposed (D2[c][i] = x[i][c]), block g
    // for matrix g.  Step k reads its pivot row from D1 and its column (the multipliers' source)
    // from D2 -- each one register of one half-wave, gathered into lane order by a permlane32
    // swap -- and the rank-1 update x -= mult pivot_row^T is one 2-block MFMA per copy.  The
    // multipliers (the reflector tails Y) go to As as they are formed.
    lds_store_row<NP>(myA + r * LD, x);
    wave_lds_order();
    f32x32 d1, d2;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      const int i = acc_row(q & 15, lane), c = lane & 31;
      d1[q] = As[(q >> 4) * MAT + i * LD + c];
      d2[q] = As[(q >> 4) * MAT + c * LD + i];
    }
    wave_lds_order();  // the Y stores below stay behind these reads
    static_for<0, NP>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      constexpr int HK = (k / 4) % 2, RK = 4 * (k / 8) + k % 4;
      if (k < n) {
        int rr = r;
        asm volatile("" : "+v"(rr));  // the step's lane masks are formed here, not hoisted
        const float e0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(d1[RK]), k + 32 * HK));
        const float e1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(d1[16 + RK]), k + 32 * HK));
        const float d = gup ? e1 : e0;
        const float pp = 1.f - d, pm = 1.f + d;
        const bool plus = fabsf(pp) >= fabsf(pm);  // |1-d| >= |1+d|, the tie d = 0 takes +1
        const float sk = plus ? 1.f : -1.f;
        const float piv = plus ? pp : pm;
        if (rr == k) my_s = sk;
        const float2 pr = lane_halves(d1[RK], d1[16 + RK]);  // lane c: x[k][c]
        const float2 pc = lane_halves(d2[RK], d2[16 + RK]);  // lane i: x[i][k]
        const float prow = HK == 0 ? pr.x : pr.y, pcol = HK == 0 ? pc.x : pc.y;
        const float mult = (rr > k && rr < n) ? (-sk * pcol) / piv : 0.f;
        if (rr > k) myA[rr * LD + k] = mult;  // Y[i][k]
        if (k + 1 < n) {
          const float u = (rr > k) ? prow : 0.f;
          d1 = mfma_2b(-mult, u, d1);
          d2 = mfma_2b(-u, mult, d2);
        }
      }
    });
    wave_lds_order();
    lds_load_row<NP>(x, myA + r * LD);  // row r of Y (below the diagonal) for the packing below
  } else {
  static_for<0, NP>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    if (k < n) {
      int rr = r;
      asm volatile("" : "+v"(rr));
      int pk[G];
      pk[0] = k;
      if constexpr (G > 1) pk[1] = NP + k;
      float d;
      if constexpr (RL) {
        d = group_bcast<G>(x[k], pk, gup);
      } else {
        if (rr == k) lds_store_row<NP, k / 4>(myS, x);
        wave_lds_order();
        d = myS[k];
      }
      const float pp = 1.f - d, pm = 1.f + d;
      const bool plus = fabsf(pp) >= fabsf(pm);  // |1-d| >= |1+d|, the tie d = 0 takes +1
      const float sk = plus ? 1.f : -1.f;
      const float piv = plus ? pp : pm;
      if (rr == k) my_s = sk;
      if (rr > k && rr < n) {
        const float mult = (-sk * x[k]) / piv;
        x[k] = mult;
        if constexpr (RL) rank1_from_lanes<NP, G, k>(x, mult, pk, gup);
        else rank1_from_slot<NP, k>(x, mult, myS);
      }
      if constexpr (!RL) wave_lds_order();
    }
  });

  // ---- tau_k = 2 / (1 + sum_{i>k} Y[i][k]^2): Y rows -> As, lane k sums column k
  lds_store_row<NP>(myA + r * LD, x);
  }
  wave_lds_order();
  if (live && mat < a.batch) {
    float ss = 0.f;
#pragma unroll
    for (int i = 1; i < NP; ++i) {
      const float y = myA[i * LD + r];
      ss += (i > r && i < n) ? y * y : 0.f;
    }
    a.tau[(int64_t)mat * n + r] = 2.f / (1.f + ss);
  }

  // ---- H = triu(diag(s) Rc) + tril(Y, -1), row r by lane r, staged in Ws
  {
    float rc[NP];
    lds_load_row<NP>(rc, myW + r * LD);
    static_for<0, NP>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      rc[c] = (c < r) ? x[c] : my_s * rc[c];
    });
    lds_store_row<NP>(myW + r * LD, rc);
  }
  wave_lds_order();
  if (a.vec4) {
    constexpr int TOT4 = G * NP * NP / 4;
#pragma unroll
    for (int i = 0; i < TOT4 / 64; ++i) {
      const int idx = lane + 64 * i;
      const int gg = idx / (NP * NP4), rem = idx - gg * NP * NP4, row = rem / NP4, c = 4 * (rem - row * NP4);
      if (mat0 + gg < a.batch && row < n && c < n)
        *reinterpret_cast<float4*>(a.H + (int64_t)(mat0 + gg) * n * n + (int64_t)row * n + c) =
            *reinterpret_cast<const float4*>(Ws + gg * MAT + row * LD + c);
    }
  } else {
    constexpr int TOT = G * NP * NP;
#pragma unroll 4
    for (int i = 0; i < TOT / 64; ++i) {
      const int idx = lane + 64 * i;
      const int gg = idx / (NP * NP), rem = idx - gg * NP * NP, row = rem / NP, c = rem - row * NP;
      if (mat0 + gg < a.batch && row < n && c < n)
        a.H[(int64_t)(mat0 + gg) * n * n + (int64_t)row * n + c] = Ws[gg * MAT + row * LD + c];
    }
  }
  if (a.info && r == 0 && mat < a.batch) {
    a.info[mat] = fail0 != INT_MAX ? fail0 + 1 : (fail1 != INT_MAX ? fail1 + 1 : 0);
  }
}

}  // namespace rnr
