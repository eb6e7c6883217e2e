// Blocked right-looking elimination of one matrix per 512-thread workgroup.
//
// PIVOT = true : partial-pivot LU, A[perm] = L U (torch.linalg.lu / LAPACK getrf
//                semantics, first maximum of |a_ij| wins) -- reflection_no_reflectors.py:66.
//                Rows are never moved: a logical->physical row map (perm) is kept in LDS and
//                every access goes through it, so the factor sits in A's own row order;
//                consumers read L through perm (or one optional gather writes it out in
//                pivoted order).  U is not kept: the reference drops it.
// PIVOT = false: the chart, the sign-ruled unpivoted LU of I - Q S run on the Q copy
//                (reflection_no_reflectors.py:139-174): s_k = +1 iff |1-d| >= |1+d|
//                (:150-155), multipliers (-s_k M[i,k]) / pivot (:157-158), then
//                tau_k = 2 / (1 + sum_{i>k} Y[i,k]^2) (:192).  Runs in place on H.
//
// Per panel of NB columns (NB = 64 / 32 / 16 for n <= 512 / 1024 / 2048):
//   * the panel's rows live in registers, RPT rows per thread (one row per thread up to
//     n = 512).  A column step of the LU is a DPP argmax per wave, one barrier, the pivot
//     row broadcast through LDS, a second barrier and a register rank-1 update; the chart
//     needs only the broadcast and one barrier;
//   * the factored panel goes to LDS (row stride NB+1: conflict-free column reads, and a
//     thread addresses its own row with one base register) and back to HBM;
//   * X = L11^-1: for 64-wide panels blocked by 32 in one wave (lu_inverse_wave), otherwise
//     swept column by column inside each wave (readlane broadcasts, no barriers); per chunk
//     of 64 trailing columns -U12 = -X A12 runs on 16x16x4 MFMA over all waves and
//     A22 += L21 (-U12) on 32x32x2 MFMA, one 32-row tile per wave at a time.  Only A22
//     streams through HBM/L2; with 64-wide panels the chunk of the next panel's columns is
//     updated last and written straight into the LDS panel.
#pragma once
#include "common.hpp"

namespace rnr {

struct LuArgs {
  const float* src;  // data read by the first panel step (A for the LU, Q for the chart)
  int64_t ss;
  float* dst;        // working matrix (LU: workspace W; chart: H)
  int64_t sd;
  int n;
  int vec4;          // n % 4 == 0 and src, dst 16-byte aligned (batch strides too)
  int* perm;         // PIVOT: logical -> original row, [batch][n]
  float* L;          // PIVOT: optional unit-lower factor in pivoted order, [batch][n][n]
  int64_t sl;
  float* s;          // chart: signs, [batch][n]
  float* tau;        // chart: tau, [batch][n]
  int k0;            // SPLIT: the panel this launch factors
  float* X;          // SPLIT: out, L11^-1 of that panel, [batch][NB][NB]
};

constexpr int kLuThreads = 512;

// 32 wide at n <= 128: the smaller LDS panel (26 KB instead of 51 KB) fits six 128-thread
// workgroups per CU instead of three (1024 x 128: LU 0.246 -> 0.168 ms, chart 0.167 -> 0.134).
inline int lu_panel_nb(int n) { return n <= 128 ? 32 : (n <= 512 ? 64 : (n <= 1024 ? 32 : 16)); }

// direct (split) panels: 1024-thread workgroups, each wave with a row-staging area of 32 rows
constexpr int kLuDirectWaves = 16;
constexpr int kLuStageLd = 36;  // staging row stride (floats): 16 lanes' rows cover the 64 banks
constexpr int kLuStageFloats = 32 * kLuStageLd + 32;  // per wave: 32 rows + their target rows (int)

// panel [n][nb+1] | -U12 chunk [nb][64] | row map [n] | pivot keys [3] (u64) | pivot row
// slots [2][nb+4] | (direct) row staging [waves][kLuStageFloats]
inline size_t lu_lds_bytes(int n, int nb, bool direct = false) {
  const size_t p = ((size_t)(direct ? nb : n) * (nb + 1) + 3) & ~(size_t)3;
  const size_t pl = ((size_t)n + 3) & ~(size_t)3;
  const size_t stage = direct ? (size_t)kLuDirectWaves * kLuStageFloats : 0;
  return sizeof(float) * (p + (size_t)nb * 64 + pl + 8 + 2 * (size_t)(nb + 4) + stage);
}

// SPLIT = true: one launch factors only panel a.k0 and stops before its trailing update,
// which k_lu_trail_g runs over many workgroups (for batches too small to fill the GPU with one
// workgroup per matrix).  The row map then lives in a.perm between launches and L11^-1 goes
// to a.X.
// One wave: X = L^-1 for the 64 x 64 unit-lower L11 of a panel, written over the panel's top
// 64 rows P (row stride 65), with the strict lower part of L given transposed in LT
// (LT[c][k] = L[k][c], row stride 64, zero for k <= c).  Blocked by 32:
//   * X11 = L11^-1 and X22 = L22^-1 at once, lane 32 d + i forming row i of block d from
//     X L = I column by column, last column first: X[i][c] = delta_ic - sum_{k>c} X[i][k] L[k][c]
//     (the columns of L are float4 LDS reads; entries above the diagonal come out as exact
//     zeros);
//   * X21 = -X22 (L21 X11) on v_mfma_f32_32x32x2f32, L21 X11 staying in the accumulators and
//     used from there as the B operand of the second product (register r of a 32x32
//     accumulator holds rows 8(r/4) + r%4 and that + 4 in its two half-waves: a K = 2 pair).
__device__ __forceinline__ void lu_inverse_wave(float* P, const float* LT, int lane) {
  constexpr int LDP = 65;
  asm volatile("" : "+v"(lane));  // lane-derived values stay here, not hoisted out of the caller's loop
  const int l32 = lane & 31, h = lane >> 5, o = 32 * h;  // block h, row l32 within it
  float x[32];
  static_for<0, 32>([&](auto cc) {
    constexpr int c = 31 - decltype(cc)::value;
    float acc = (l32 == c) ? 1.f : 0.f;
    if constexpr (c < 31) {
      // the column's reads depend on x[c + 2]: they issue one column ahead, not all at the
      // start (hoisted together they would not fit in registers)
      int off = (o + c) * 64 + o;
      if constexpr (c <= 29) asm volatile("" : "+v"(off) : "v"(x[c + 2]));
      const lds_f4* lc = lds_base(LT + off);
#pragma unroll
      for (int k4 = (c + 1) / 4; k4 < 8; ++k4) {
        const float4 lv = lds_get(lc, k4);
        const float lvv[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * k4 + e > c) acc -= x[4 * k4 + e] * lvv[e];
      }
    }
    x[c] = acc;
  });
  wave_lds_order();
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    P[(o + l32) * LDP + o + c] = x[c];
    if (!h) P[l32 * LDP + 32 + c] = 0.f;  // X12
  }
  wave_lds_order();
  f32x16 v = zero16();  // L21 X11
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int k = 2 * t + h;
    v = mfma(LT[k * 64 + 32 + l32], P[k * LDP + l32], v);
  }
  f32x16 x21 = zero16();  // -X22 (L21 X11)
#pragma unroll
  for (int r = 0; r < 16; ++r) x21 = mfma(-P[(32 + l32) * LDP + 32 + acc_row(r, lane)], v[r], x21);
#pragma unroll
  for (int r = 0; r < 16; ++r) P[(32 + acc_row(r, lane)) * LDP + l32] = x21[r];
}

// T: threads per workgroup (512; 128 or 256 for n <= 128 / 256 with 64-wide panels, so that
// small matrices do not hold idle waves and several workgroups share a CU).
template <bool PIVOT, int NB, int RPT, bool SPLIT = false, int T = kLuThreads>
__global__ __launch_bounds__(T) __attribute__((amdgpu_waves_per_eu(T > 512 ? 4 : 2))) void k_lu(LuArgs a) {
  constexpr int NW = T / 64;
  constexpr int NB4 = NB / 4;
  constexpr int LDP = NB + 1;
  constexpr int CPW = NB / NW;       // columns of L11^-1 per wave
  static_assert(NB % NW == 0 && NB <= 64, "panel width");
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int n = a.n;
  float* P = smem;                                  // panel [n][NB+1]
  // DIRECT (split launches with 32-wide panels): the panel's rows go between HBM and registers
  // directly and only its first NB logical rows (L11) are kept in P; the chart's tau then comes
  // from k_chart_tau after the last panel
  constexpr bool DIRECT = SPLIT && NB == 32;
  float* U = P + (((size_t)(DIRECT ? NB : n) * LDP + 3) & ~(size_t)3);  // -U12 chunk [NB][64]
  int* pl = reinterpret_cast<int*>(U + NB * 64);    // logical -> physical row
  unsigned long long* pkeys =                       // [3] pivot keys (LU), by step mod 3
      reinterpret_cast<unsigned long long*>(reinterpret_cast<float*>(pl) + ((n + 3) & ~3));
  float* slots = reinterpret_cast<float*>(pkeys) + 8;  // [2][NB+4] pivot rows, by column parity
  // DIRECT: this wave's row staging (32 rows at stride kLuStageLd, then their target rows), so the
  // panel's rows move between HBM and the threads' registers row-contiguously (8 lanes a row)
  // instead of one row per lane (64 rows, 16 bytes each, per memory instruction)
  static_assert(!DIRECT || T / 64 == kLuDirectWaves, "direct panels: staging sized for 16 waves");
  float* const stg = slots + 2 * (NB + 4);

  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, h = lane >> 5, l16 = lane & 15, q4 = lane >> 4;
  const float* src = a.src + b * a.ss;
  float* dst = a.dst + b * a.sd;
  auto sw = [](int r, int c) { return r * LDP + c; };

  if (PIVOT)
    for (int i = tid; i < n; i += T) pl[i] = (SPLIT && a.k0 > 0) ? a.perm[(int64_t)b * n + i] : i;
  if (tid < 3) pkeys[tid] = 0ull;
  int kb3 = 0;  // pivot key buffer of this LU column step: steps so far mod 3 (a rotating counter)
  __syncthreads();

  // 64-wide panels: the trailing update's chunk of the next panel's columns runs last and is
  // written straight into the LDS panel (it never makes the round trip through HBM)
  constexpr bool kNextInLds = NB == 64 && !SPLIT;
  bool preloaded = false;
  for (int k0 = SPLIT ? a.k0 : 0; k0 < n; k0 += NB) {
    const int kb = min(NB, n - k0), m = n - k0, k1 = k0 + kb;
    const float* cur = (k0 == 0) ? src : dst;

    // ---- panel HBM -> LDS, four float4 loads in flight per thread
    if (preloaded || DIRECT) {
      // already in P from the previous panel's trailing update (or loaded into registers below)
    } else if (a.vec4) {
      const int tot = m * NB4;
      for (int f0 = tid; f0 < tot; f0 += 4 * T) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int f = f0 + T * u;
          v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (f < tot) {
            const int r = f / NB4, c = 4 * (f - r * NB4);
            const int pr = PIVOT ? pl[k0 + r] : k0 + r;
            if (c < kb) v[u] = *reinterpret_cast<const float4*>(cur + (int64_t)pr * n + k0 + c);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int f = f0 + T * u;
          if (f < tot) {
            const int r = f / NB4, c = 4 * (f - r * NB4);
            float* d = P + sw(r, c);
            d[0] = v[u].x; d[1] = v[u].y; d[2] = v[u].z; d[3] = v[u].w;
          }
        }
      }
    } else {
      for (int idx = tid; idx < m * NB; idx += T) {
        const int r = idx / NB, c = idx - r * NB;
        const int pr = PIVOT ? pl[k0 + r] : k0 + r;
        P[sw(r, c)] = (c < kb) ? cur[(int64_t)pr * n + k0 + c] : 0.f;
      }
    }
    __syncthreads();
    float row[RPT][NB];
    if constexpr (DIRECT) {
      // per half-wave: its 32 rows loaded row-contiguously into the staging (lane: row
      // it * 8 + lane / 8, float4 lane % 8), then each thread takes its own row from there
      static_assert(NB == 32, "direct panels are 32 wide");
      float* wst = stg + wid * kLuStageFloats;
#pragma unroll
      for (int q = 0; q < RPT; ++q)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int sr = it * 8 + (lane >> 3), c4 = lane & 7;
            const int r = wid * 64 + h2 * 32 + sr + T * q;
            const int pr = (r < m) ? (PIVOT ? pl[k0 + r] : k0 + r) : 0;
            const float* src4 = cur + (int64_t)pr * n + k0 + 4 * c4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (a.vec4) {
              if (r < m && 4 * c4 < kb) v = *reinterpret_cast<const float4*>(src4);
            } else if (r < m) {
              v.x = (4 * c4 < kb) ? src4[0] : 0.f;
              v.y = (4 * c4 + 1 < kb) ? src4[1] : 0.f;
              v.z = (4 * c4 + 2 < kb) ? src4[2] : 0.f;
              v.w = (4 * c4 + 3 < kb) ? src4[3] : 0.f;
            }
            *reinterpret_cast<float4*>(wst + sr * kLuStageLd + 4 * c4) = v;
          }
          wave_lds_order();
          if ((lane >> 5) == h2) {
            const int sr = lane & 31;
#pragma unroll
            for (int c4 = 0; c4 < NB4; ++c4) {
              const float4 v = *reinterpret_cast<const float4*>(wst + sr * kLuStageLd + 4 * c4);
              row[q][4 * c4] = v.x; row[q][4 * c4 + 1] = v.y; row[q][4 * c4 + 2] = v.z; row[q][4 * c4 + 3] = v.w;
            }
          }
          wave_lds_order();  // the next half's staging stores stay behind these reads
        }
    } else {
#pragma unroll
      for (int q = 0; q < RPT; ++q) {
        const int r = tid + T * q;
#pragma unroll
        for (int c = 0; c < NB; ++c) row[q][c] = (r < m) ? P[sw(r, c)] : 0.f;
      }
    }

    // ---- factor the panel column by column (compile-time column index).  Rows stay in
    //      their threads: pos[q] is the logical position (relative to k0) of the row a thread
    //      holds, and a pivot choice only swaps two labels.  LU: each wave publishes its best
    //      candidate key in one LDS atomic maximum; after a barrier the lane holding the
    //      winning key stores its row in the pivot slot (double-buffered by column parity),
    //      and after a second barrier every thread reads it.  Chart: the pivot row's thread
    //      stores it, one barrier.  Waves whose rows all lie at or past m (finished rows)
    //      only take part in the barriers.
    const int nwa = min(NW, (m + 63) >> 6);  // waves holding rows < m
    const bool wact = wid < nwa;
    int pos[RPT], phys[RPT];
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int r = tid + T * q;
      pos[q] = r;
      phys[q] = (PIVOT && r < m) ? pl[k0 + r] : 0;
    }
    constexpr int SLOT4 = NB4 + 1;  // float4 units per slot: one spare + the row
    float4* slot4 = reinterpret_cast<float4*>(slots);
    int buf = 0;
    float my_s = 1.f;
    static_for<0, NB>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int C0 = j / 4;  // first chunk holding a column >= j
      if (j < kb) {  // uniform
        // the row index is laundered through an empty asm each column so that the per-column
        // lane masks are formed here instead of being hoisted for all NB columns to the
        // kernel start (which spills ~1000 SGPRs)
        int rbase = tid;
        asm volatile("" : "+v"(rbase));
        float4* sb = slot4 + buf * SLOT4;
        float4 pr4[NB4 - C0];
        float l[RPT];
        if constexpr (PIVOT) {
          // key: candidates (rows at positions >= j) rank by |v| (NaN lowest), ties by the
          // smaller position (LAPACK's first maximum); the low 4 bits name the wave.  Key
          // buffer = step mod 3; the next step's buffer is cleared now (its last readers
          // finished two barriers ago).
          const int kb3n = kb3 == 2 ? 0 : kb3 + 1;
          unsigned long long* kcur = pkeys + kb3;
          if (tid == 0) pkeys[kb3n] = 0ull;
          kb3 = kb3n;
          uint64_t best = 0;
          int bq = 0;
          if (wact) {
#pragma unroll
            for (int q = 0; q < RPT; ++q) {
              const int r = rbase + T * q;
              const float v = row[q][j];
              const bool cand = r < m && pos[q] >= j;
              const uint32_t kb32 = cand ? (v != v ? 1u : __float_as_uint(fabsf(v)) + 2u) : 0u;
              const uint64_t key = ((uint64_t)kb32 << 32) | (uint32_t)(((2047 - pos[q]) << 4) | wid);
              if (key > best) { best = key; bq = q; }
            }
            const uint64_t wbest = wave_max_key(best);
            if (best == wbest) atomicMax(kcur, (unsigned long long)wbest);  // one lane: keys are distinct
          }
          __syncthreads();
          // only the winning lane publishes its row, between two barriers: LDS instructions cost
          // their full wave width whatever the active lanes, so one wave storing beats every
          // wave storing its own candidate
          const uint64_t pk = *kcur;
          const bool winner = wact && best == pk;
          // one masked store block per row of the thread, only the winner's executing; a
          // compiler memory barrier between the blocks keeps them apart (merged, they would
          // become copies into common registers, or a lane-dependent index into row[] that puts
          // row[] on the stack)
#pragma unroll
          for (int q = 0; q < RPT; ++q) {
            if (winner && (RPT == 1 || bq == q)) {
#pragma unroll
              for (int c4 = C0; c4 < NB4; ++c4)
                sb[1 + c4] = make_float4(row[q][4 * c4], row[q][4 * c4 + 1], row[q][4 * c4 + 2], row[q][4 * c4 + 3]);
            }
            if (RPT > 1) asm volatile("" ::: "memory");
          }
          __syncthreads();
          if (wact) {
            const int p = 2047 - (int)((uint32_t)pk >> 4);
            // one base register per column, the reads at immediate offsets from it (otherwise the
            // compiler forms one address per read, hoisted out of the panel loop and parked in
            // spilled registers)
            const lds_f4* prow = lds_base(sb + 1);
#pragma unroll
            for (int c4 = C0; c4 < NB4; ++c4) pr4[c4 - C0] = lds_get(prow, c4);
            const float pv = f4get<j % 4>(pr4[0]);
            // LAPACK xGETRF2: scale by the reciprocal unless the pivot is subnormal; a zero
            // pivot leaves the column as it is (then every candidate is zero: no update)
            const bool nz = pv != 0.f;
            const bool recip = fabsf(pv) >= 1.17549435e-38f;
            const float inv = 1.f / pv;
#pragma unroll
            for (int q = 0; q < RPT; ++q) {
              const int r = rbase + T * q;
              const bool below = r < m && pos[q] >= j && pos[q] != p;
              l[q] = 0.f;
              if (below) {
                l[q] = row[q][j];
                if (nz) {
                  l[q] = recip ? l[q] * inv : l[q] / pv;
                  row[q][j] = l[q];
                }
              }
              pos[q] = (pos[q] == p) ? j : ((pos[q] == j) ? p : pos[q]);
            }
          }
        } else {
          // chart: the pivot row is row j (held by thread j, j < NB <= T)
          if (tid == j) {
#pragma unroll
            for (int c4 = C0; c4 < NB4; ++c4)
              sb[1 + c4] = make_float4(row[0][4 * c4], row[0][4 * c4 + 1], row[0][4 * c4 + 2],
                                       row[0][4 * c4 + 3]);
          }
          __syncthreads();
          if (wact) {
            const lds_f4* prow = lds_base(sb + 1);  // one base register per column, as in the LU branch
#pragma unroll
            for (int c4 = C0; c4 < NB4; ++c4) pr4[c4 - C0] = lds_get(prow, c4);
            const float d = f4get<j % 4>(pr4[0]);
            const float pp = 1.f - d, pm = 1.f + d;
            const bool plus = fabsf(pp) >= fabsf(pm);  // |1-d| >= |1+d|: the tie d = 0 takes +1
            const float sk = plus ? 1.f : -1.f;
            const float piv = plus ? pp : pm;
            if (tid == j) my_s = sk;
#pragma unroll
            for (int q = 0; q < RPT; ++q) {
              const int r = rbase + T * q;
              l[q] = 0.f;
              if (r > j && r < m) {
                l[q] = (-sk * row[q][j]) / piv;
                row[q][j] = l[q];
              }
            }
          }
        }
        if (wact) {
          // rank-1 update of the columns right of j
#pragma unroll
          for (int c4 = C0; c4 < NB4; ++c4) {
            const float pcv[4] = {pr4[c4 - C0].x, pr4[c4 - C0].y, pr4[c4 - C0].z, pr4[c4 - C0].w};
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              if (4 * c4 + e2 > j) {
#pragma unroll
                for (int q = 0; q < RPT; ++q) row[q][4 * c4 + e2] -= l[q] * pcv[e2];
              }
            }
          }
        }
        buf ^= 1;
      }
    });

    // ---- registers -> LDS panel, each row at its logical position; the row map follows
    //      (DIRECT: only L11's rows go to P, every row straight back to its row of HBM)
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int r = tid + T * q;
      if (r < m) {
        if (!DIRECT || pos[q] < NB) {
#pragma unroll
          for (int c = 0; c < NB; ++c) P[sw(pos[q], c)] = row[q][c];
        }
        if (PIVOT) pl[k0 + pos[q]] = phys[q];
      }
    }
    if constexpr (DIRECT) {
      // every row straight back to its row of HBM, through the staging: per half-wave, the
      // threads' rows and target rows in, then 8 lanes a row out
      float* wst = stg + wid * kLuStageFloats;
      int* wdst = reinterpret_cast<int*>(wst + 32 * kLuStageLd);
#pragma unroll
      for (int q = 0; q < RPT; ++q)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          if ((lane >> 5) == h2) {
            const int sr = lane & 31, r = tid + T * q;
#pragma unroll
            for (int c4 = 0; c4 < NB4; ++c4)
              *reinterpret_cast<float4*>(wst + sr * kLuStageLd + 4 * c4) =
                  make_float4(row[q][4 * c4], row[q][4 * c4 + 1], row[q][4 * c4 + 2], row[q][4 * c4 + 3]);
            wdst[sr] = (r < m) ? (PIVOT ? phys[q] : k0 + r) : -1;
          }
          wave_lds_order();
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int sr = it * 8 + (lane >> 3), c4 = lane & 7;
            const int dr = wdst[sr];
            const float4 v = *reinterpret_cast<const float4*>(wst + sr * kLuStageLd + 4 * c4);
            float* d4 = dst + (int64_t)max(dr, 0) * n + k0 + 4 * c4;
            if (dr >= 0) {
              if (a.vec4) {
                if (4 * c4 < kb) *reinterpret_cast<float4*>(d4) = v;
              } else {
                if (4 * c4 < kb) d4[0] = v.x;
                if (4 * c4 + 1 < kb) d4[1] = v.y;
                if (4 * c4 + 2 < kb) d4[2] = v.z;
                if (4 * c4 + 3 < kb) d4[3] = v.w;
              }
            }
          }
          wave_lds_order();  // the next half's staging stores stay behind these reads
        }
    }
    if (!PIVOT && tid < kb) a.s[(int64_t)b * n + k0 + tid] = my_s;
    __syncthreads();

    if constexpr (!PIVOT && !DIRECT) {
      // tau of the panel's columns from the finished multipliers (rows below the diagonal)
      for (int c = tid >> 3; c < kb; c += T / 8) {
        const int sub = tid & 7;
        float acc = 0.f;
        for (int r = c + 1 + sub; r < m; r += 8) {
          const float y = P[sw(r, c)];
          acc += y * y;
        }
        acc = group8_sum(acc);
        if (sub == 0) a.tau[(int64_t)b * n + k0 + c] = 2.f / (acc + 1.f);
      }
    }

    // ---- factored panel -> HBM (same physical rows it came from; DIRECT: done above)
    if (DIRECT) {
    } else if (a.vec4) {
      const int tot = m * NB4;
      for (int f = tid; f < tot; f += T) {
        const int r = f / NB4, c = 4 * (f - r * NB4);
        if (c < kb) {
          const int pr = PIVOT ? pl[k0 + r] : k0 + r;
          *reinterpret_cast<float4*>(dst + (int64_t)pr * n + k0 + c) =
              make_float4(P[sw(r, c)], P[sw(r, c + 1)], P[sw(r, c + 2)], P[sw(r, c + 3)]);
        }
      }
    } else {
      for (int idx = tid; idx < m * kb; idx += T) {
        const int r = idx / kb, c = idx - r * kb;
        const int pr = PIVOT ? pl[k0 + r] : k0 + r;
        dst[(int64_t)pr * n + k0 + c] = P[sw(r, c)];
      }
    }
    if (k1 >= n) break;  // uniform: no trailing matrix (and kb == NB below this line)

    // ---- X = L11^-1 (unit lower) into panel rows 0..NB
    if constexpr (NB == 64) {
      // L11^T (strict lower part) staged in the -U12 buffer, which is free until the trailing
      // update; then one wave forms X by 32 x 32 blocks (lu_inverse_wave)
      for (int idx = tid; idx < 64 * 64; idx += T) {
        const int c = idx >> 6, k = idx & 63;
        U[idx] = (k > c) ? P[sw(k, c)] : 0.f;
      }
      __syncthreads();
      if (wid == 0) lu_inverse_wave(P, U, lane);
      __syncthreads();
    } else {
      // wave w sweeps columns w*CPW .. w*CPW+CPW-1, lane i holding row i;
      // x_i -= L[i][k] x_k for i > k >= c
      float Lr[NB];
#pragma unroll
      for (int k = 0; k < NB; ++k) Lr[k] = (lane < NB && k < lane) ? P[sw(lane, k)] : 0.f;
      __syncthreads();
      float x[CPW];
#pragma unroll
      for (int u = 0; u < CPW; ++u) x[u] = (lane == wid * CPW + u) ? 1.f : 0.f;
      static_for<0, NB - 1>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        int ln = lane, c0w = __builtin_amdgcn_readfirstlane(wid * CPW);  // laundered: masks stay local
        asm volatile("" : "+v"(ln), "+s"(c0w));
#pragma unroll
        for (int u = 0; u < CPW; ++u) {
          const float xk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[u]), k));
          if (k >= c0w + u && ln > k) x[u] -= Lr[k] * xk;
        }
      });
      if (lane < NB) {
#pragma unroll
        for (int u = 0; u < CPW; ++u) P[sw(lane, wid * CPW + u)] = x[u];
      }
      __syncthreads();
    }
    if constexpr (SPLIT) {
      // hand the row map and L11^-1 to the trailing-update launch
      if (PIVOT)
        for (int i = k0 + tid; i < n; i += T) a.perm[(int64_t)b * n + i] = pl[i];
      for (int idx = tid; idx < NB * NB; idx += T) a.X[(int64_t)b * NB * NB + idx] = P[sw(idx / NB, idx % NB)];
      return;
    }

    // ---- trailing update, 64 columns at a time (the next panel's chunk last when it is kept)
    const int nch = (n - k1 + 63) >> 6;
    f32x16 kt0[2], kt1[2];  // the kept chunk's tiles (at most two per wave: n <= 512)
    for (int it = 0; it < nch; ++it) {
      const int c0 = k1 + 64 * (kNextInLds ? (it + 1) % nch : it);
      const bool keep = kNextInLds && it == nch - 1;
      // -U12 = -(X A12[:, c0:c0+64]) as (NB/16) x 4 blocks of 16x16 spread over the waves
      {
        // a wave's jobs load their A12 columns first, then multiply: one load latency per
        // chunk instead of one per job
        // (in rounds of at most two jobs per wave: few waves would otherwise hold many rows)
        constexpr int NBI = NB / 16, NJOB = NBI * 4, JPW = (NJOB + NW - 1) / NW, JPR = JPW < 2 ? JPW : 2;
#pragma unroll
        for (int u0 = 0; u0 < JPW; u0 += JPR) {
          float bv[JPR][NB4];
#pragma unroll
          for (int u = 0; u < JPR; ++u) {
            const int job = wid + (u0 + u) * NW, bj = job & 3;
            const int col = c0 + bj * 16 + l16;
#pragma unroll
            for (int t = 0; t < NB4; ++t) {
              const int k = 4 * t + q4;
              const int pr = PIVOT ? pl[k0 + k] : k0 + k;
              bv[u][t] = (job < NJOB) ? cur[(int64_t)pr * n + min(col, n - 1)] : 0.f;  // columns past n: unstored
            }
          }
#pragma unroll
          for (int u = 0; u < JPR; ++u) {
            const int job = wid + (u0 + u) * NW;
            if (job < NJOB) {
              const int bi = job >> 2, bj = job & 3;
              const int i = bi * 16 + l16;
              f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int t = 0; t < NB4; ++t) acc = mfma16(P[sw(i, 4 * t + q4)], bv[u][t], acc);
#pragma unroll
              for (int r = 0; r < 4; ++r) U[(bi * 16 + 4 * q4 + r) * 64 + bj * 16 + l16] = -acc[r];
            }
          }
        }
      }
      __syncthreads();

      // A22[:, chunk] += L21 (-U12): one 32-row tile per wave at a time.  The loads are
      // branch-free: rows / columns past n are clamped (their accumulator entries are not
      // stored), so the row-map reads and the loads issue as one batch; panel rows past m
      // are read as they are (stale rows inside the LDS allocation, again only reaching
      // unstored accumulator rows).
      const int ntr = (n - k1 + 31) >> 5;
      for (int tr = wid, slot = 0; tr < ntr; tr += NW, ++slot) {
        const int r0 = k1 + tr * 32;
        int ln = lane;  // laundered per tile: the row offsets are formed here, not kept live
        asm volatile("" : "+v"(ln));
        const int l32 = ln & 31, h = ln >> 5;
        int prw[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rw = min(r0 + acc_row(r, ln), n - 1);
          prw[r] = PIVOT ? pl[rw] : rw;
        }
        const int colc0 = min(c0 + l32, n - 1), colc1 = min(c0 + 32 + l32, n - 1);
        f32x16 c[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          c[0][r] = cur[(int64_t)prw[r] * n + colc0];
          c[1][r] = cur[(int64_t)prw[r] * n + colc1];
        }
        const int lr = r0 - k0 + l32;
#pragma unroll
        for (int kk = 0; kk < NB; kk += 2) {
          const int k = kk + h;
          const float av = P[sw(lr, k)];
          c[0] = mfma(av, U[k * 64 + l32], c[0]);
          c[1] = mfma(av, U[k * 64 + 32 + l32], c[1]);
        }
        if (keep) {
          if (slot == 0) { kt0[0] = c[0]; kt0[1] = c[1]; }
          else { kt1[0] = c[0]; kt1[1] = c[1]; }
          continue;
        }
#pragma unroll
        for (int nj = 0; nj < 2; ++nj)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rw = r0 + acc_row(r, ln), col = c0 + nj * 32 + l32;
            if (rw < n && col < n) dst[(int64_t)prw[r] * n + col] = c[nj][r];
          }
      }
      __syncthreads();
      if (keep) {
        // every wave is past its reads of this panel: the kept tiles become the next panel,
        // row at logical position k1 + r in P row r (columns past n zero, as the load writes)
        for (int tr = wid, slot = 0; tr < ntr; tr += NW, ++slot) {
          const int r0 = k1 + tr * 32;
          int ln = lane;
          asm volatile("" : "+v"(ln));
          const int l32 = ln & 31;
#pragma unroll
          for (int nj = 0; nj < 2; ++nj)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int rw = r0 + acc_row(r, ln), cc = nj * 32 + l32;
              const float v = slot == 0 ? kt0[nj][r] : kt1[nj][r];
              if (rw < n) P[sw(rw - k1, cc)] = (k1 + cc < n) ? v : 0.f;
            }
        }
      }
    }
    preloaded = kNextInLds;  // uniform; the next panel's load is skipped
  }
  __syncthreads();

  if constexpr (PIVOT) {
    for (int i = tid; i < n; i += T) a.perm[(int64_t)b * n + i] = pl[i];
    if (a.L) {
      float* L = a.L + b * a.sl;
      for (int idx = tid; idx < n * n; idx += T) {
        const int i = idx / n, j = idx - i * n;
        L[idx] = (j < i) ? dst[(int64_t)pl[i] * n + j] : (j == i ? 1.f : 0.f);
      }
    }
  }
}

// tau of the finished chart for the split form, tau_c = 2 / (1 + sum_{r > c} Y[r][c]^2)
// (reflection_no_reflectors.py:192), summed in k_lu's in-panel order -- rows c + 1 + sub in
// steps of 8, then the 8 lanes of a group -- so the values equal the fused kernel's bit for bit.
// One 256-thread workgroup per 32 columns of one matrix.
__global__ __launch_bounds__(256) void k_chart_tau(const float* H, int64_t sh, float* tau, int n, int ncb) {
  const int64_t g = blockIdx.x, b = g / ncb;
  const int c = (int)(g - b * ncb) * 32 + (threadIdx.x >> 3), sub = threadIdx.x & 7;
  const float* Hb = H + b * sh;
  float acc = 0.f;
  if (c < n)
    for (int r = c + 1 + sub; r < n; r += 8) {
      const float y = Hb[(int64_t)r * n + c];
      acc += y * y;
    }
  acc = group8_sum(acc);
  if (sub == 0 && c < n) tau[b * n + c] = 2.f / (acc + 1.f);
}

constexpr int kLuTrailThreads = 256;

constexpr int kLuTrailRows = 256;  // rows per workgroup (eight 32-row tiles)

// Grouped trailing update for SPLIT launches (32-wide panels): apply the S <= 4 consecutive
// panels starting at column kg, already factored, to the columns [cb, ce) of the rows whose
// logical position is >= kg + 32 S:
//
//     U = L11^-1 A[pivot rows kg .. kg + 32 S, cb:ce]      (L11: the panels' unit-lower block)
//     A[rows, cb:ce] -= L[rows, kg .. kg + 32 S] U
//
// -- the blocked LU's rank-32S update, with U formed by block forward substitution over the
// panels (U_s = X_s (A_s - sum_{t<s} L_st U_t), X_s = L_ss^-1 from the panel launch s, slot s of
// a.X).  The split LU calls it twice per group of four panels: before panel s is factored, to
// bring its 32 columns up to date with panels 0 .. s-1 of the group (S = s), and after the
// group, for everything right of it (S = 4) -- one pass over the trailing matrix per 128
// columns instead of one per 32.  The pivot rows' own columns are read as the earlier groups
// left them: within a group no pass writes them (U is not kept; the reference drops it).
// One 256-thread workgroup per (64-column chunk, group of rpw rows): each forms its chunk's U
// itself, so a workgroup takes as many rows as still leaves the GPU a few workgroups per CU
// (the launch picks rpw), which spreads that work over more row tiles.  U is formed in LDS on
// 16x16x4 MFMA (stored negated), each wave on its own 16 columns, so the substitution needs no
// workgroup barrier; the row tiles run on 32x32x2 MFMA with L's rows loaded straight into
// registers: the two half-waves take the two halves of K, so each lane's 16 S values of its row
// are contiguous (float4 loads).
template <bool PIVOT, int S>
__global__ __launch_bounds__(kLuTrailThreads) void k_lu_trail_g(LuArgs a, int kg, int cb, int ce, int nchunk,
                                                               int nrg, int rpw, int64_t xslot) {
  constexpr int NW = kLuTrailThreads / 64, K = 32 * S, HK = K / 2;
  __shared__ float Xs[S][32][33];
  __shared__ __attribute__((aligned(16))) float U[K][64];  // rows 32 s + i: A_s, then -U_s
  __shared__ int pls[RNR_MAX_N];
  const int n = a.n, rb = kg + K;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l16 = lane & 15, q4 = lane >> 4;
  const int64_t pid = blockIdx.x;
  const int64_t b = pid / ((int64_t)nchunk * nrg);
  const int rem = (int)(pid - b * nchunk * nrg), rg = rem / nchunk;
  const int c0 = cb + 64 * (rem - rg * nchunk);
  const float* cur = ((kg == 0) ? a.src + b * a.ss : a.dst + b * a.sd);
  float* dst = a.dst + b * a.sd;
#pragma unroll
  for (int u = 0; u < RNR_MAX_N / kLuTrailThreads; ++u) {
    const int i = kg + tid + kLuTrailThreads * u;
    if (i < n) pls[i] = PIVOT ? a.perm[b * n + i] : i;
  }
#pragma unroll
  for (int u = 0; u < S * 1024 / kLuTrailThreads; ++u) {
    const int idx = tid + kLuTrailThreads * u, sp = idx >> 10, e = idx & 1023;
    Xs[sp][e >> 5][e & 31] = a.X[sp * xslot + b * 1024 + e];
  }
  __syncthreads();
  // the pivot rows' values of this chunk (columns past n clamped: never stored)
#pragma unroll
  for (int u = 0; u < K * 64 / kLuTrailThreads; ++u) {
    const int idx = tid + kLuTrailThreads * u, i = idx >> 6, j = idx & 63;
    U[i][j] = cur[pls[kg + i] * n + min(c0 + j, n - 1)];
  }
  __syncthreads();

  // block forward substitution, wave w on the chunk's columns 16 w .. 16 w + 15, both 16-row
  // halves of each 32-row block (D[i][j] of a 16x16x4 result: lane j + 16 (i / 4), register i % 4)
  const int wc = 16 * wid + l16;
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
    f32x4 acc[2];
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[ti][r] = U[32 * sp + 16 * ti + 4 * q4 + r][wc];
    // T = A_s + sum_{t < s} L_st (-U_t)
#pragma unroll
    for (int t = 0; t < sp; ++t) {
      float av[2][8];
#pragma unroll
      for (int ti = 0; ti < 2; ++ti) {
        const float* lr = dst + pls[kg + 32 * sp + 16 * ti + l16] * n + kg + 32 * t + q4;
#pragma unroll
        for (int k4 = 0; k4 < 8; ++k4) av[ti][k4] = lr[4 * k4];
      }
#pragma unroll
      for (int k4 = 0; k4 < 8; ++k4) {
        const float bv = U[32 * t + 4 * k4 + q4][wc];
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) acc[ti] = mfma16(av[ti][k4], bv, acc[ti]);
      }
    }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) U[32 * sp + 16 * ti + 4 * q4 + r][wc] = acc[ti][r];
    wave_lds_order();
    // -U_s = -X_s T, over T in place (the wave's own columns: every read precedes the stores)
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) acc[ti] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k4 = 0; k4 < 8; ++k4) {
      const float bv = U[32 * sp + 4 * k4 + q4][wc];
#pragma unroll
      for (int ti = 0; ti < 2; ++ti) acc[ti] = mfma16(Xs[sp][16 * ti + l16][4 * k4 + q4], bv, acc[ti]);
    }
    wave_lds_order();
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) U[32 * sp + 16 * ti + 4 * q4 + r][wc] = -acc[ti][r];
    wave_lds_order();
  }
  __syncthreads();

  // the row tiles: C[32 x 64] += L[32 x K] (-U)[K x 64], half-wave h on k in [h K/2, (h+1) K/2)
  const int tpw = rpw >> 5;  // row tiles per workgroup
  const int ntr = min((n - rb + 31) >> 5, (rg + 1) * tpw);
  for (int tr = rg * tpw + wid; tr < ntr; tr += NW) {
    const int r0 = rb + tr * 32;
    int ln = lane;  // laundered per tile: the row offsets are formed here, not kept live
    asm volatile("" : "+v"(ln));
    const int l32 = ln & 31, h = ln >> 5;
    const float* lrow = dst + pls[min(r0 + l32, n - 1)] * n + kg + h * HK;  // rows past n clamped: never stored
    float lv[HK];
    if (a.vec4) {
#pragma unroll
      for (int u = 0; u < HK / 4; ++u) {
        const float4 v = *reinterpret_cast<const float4*>(lrow + 4 * u);
        lv[4 * u] = v.x; lv[4 * u + 1] = v.y; lv[4 * u + 2] = v.z; lv[4 * u + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int t = 0; t < HK; ++t) lv[t] = lrow[t];
    }
    f32x16 c[2];
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rw = min(r0 + acc_row(r, ln), n - 1), col = min(c0 + nj * 32 + l32, n - 1);
        c[nj][r] = cur[pls[rw] * n + col];  // clamped rows / columns are not stored
      }
    issue_loads_first();
#pragma unroll
    for (int t = 0; t < HK; ++t) {
      const int k = h * HK + t;
      c[0] = mfma(lv[t], U[k][l32], c[0]);
      c[1] = mfma(lv[t], U[k][32 + l32], c[1]);
    }
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rw = r0 + acc_row(r, ln), col = c0 + nj * 32 + l32;
        if (rw < n && col < ce) dst[pls[rw] * n + col] = c[nj][r];
      }
  }
}

}  // namespace rnr
