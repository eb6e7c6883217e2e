// Householder blocked-WY QR in torch.geqrf layout -- a BENCHMARK COMPARATOR, not part of the
// reflector-free path (custom_kernel never calls it).  It is the classical algorithm the
// reference measures its route against (householder/submission_routed_v3.py:225-281: a panel
// kernel per NB columns, then the trailing update C <- (I - V T^T V^T) C by three products),
// built here for gfx950:
//
//   k_hh_panel   one 256-thread workgroup per matrix: the panel (rows p0.., NB columns) in LDS,
//                column-major; per column the norm (one barrier), the LAPACK slarfg reflector
//                (beta = -sign(alpha) ||x||, tau = (beta - alpha) / beta, v = x / (alpha - beta)),
//                then the dot products with the later panel columns (one barrier) and the rank-1
//                update of the rows each thread owns.  Then S = V^T V on v_mfma_f32_32x32x2f32
//                (rows split over the four waves) and T row-parallel from the compact-WY
//                recurrence T[i][j] = -tau_j sum_{l=i}^{j-1} T[i][l] S[l][j] (LAPACK slarft,
//                forward / columnwise; thread i needs only row i).
//   k_hh_update  one 256-thread workgroup per 64-column tile of the trailing matrix:
//                W = V^T C (MFMA, K = the panel's rows split over the waves), W' = T^T W,
//                C -= V W' (MFMA, 32-row strips, V staged row-contiguously through LDS).
//
// The slot width in the update is always 32 reflectors (a 16-wide panel leaves zeros).  LAPACK's
// rescaling of tiny beta (slarfg's safmin loop) is not reproduced: inputs whose column norms
// underflow float32 are outside what this comparator handles.
#include "../../include/rnrqr.h"
#include "common.hpp"

namespace rnr {
namespace {

constexpr int kHhThreads = 256;

struct HhArgs {
  float* H;       // [batch][n][n] in place: A in, geqrf's H out
  float* tau;     // [batch][n]
  float* T;       // [batch][32][32] the current panel's T (workspace)
  int n, p0, kb, ntile;
};

__host__ __device__ inline int hh_ldp(int m) { return m | 1; }  // odd column stride: conflict-free row-indexed reads

template <int NB>
size_t hh_panel_lds(int n) {
  const int ldp = hh_ldp(n);
  return sizeof(float) * ((size_t)NB * ldp + 4 * 32 * 33 + 32 * 33 + 32 * 33 + 4 * (NB + 1) + NB);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int NB>
__global__ __launch_bounds__(kHhThreads) void k_hh_panel(HhArgs a) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int n = a.n, p0 = a.p0, kb = a.kb, m = n - p0, ldp = hh_ldp(m);
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float* P = sm;                             // [NB][ldp]: P[c * ldp + r] = panel(r, c)
  float* Sp = P + (size_t)NB * ldp;          // [4][32][33] per-wave partial V^T V
  float* S = Sp + 4 * 32 * 33;               // [32][33]
  float* Tm = S + 32 * 33;                   // [32][33]
  float* red = Tm + 32 * 33;                 // [4][NB + 1]
  float* tl = red + 4 * (NB + 1);            // [NB] the panel's taus
  const int64_t b = blockIdx.x;
  float* H = a.H + b * n * n;
  float* tau = a.tau + b * n;

  for (int idx = tid; idx < m * NB; idx += kHhThreads) {
    const int r = idx / NB, c = idx - r * NB;
    P[c * ldp + r] = (c < kb) ? H[(int64_t)(p0 + r) * n + p0 + c] : 0.f;
  }
  __syncthreads();

  // Thread tid owns rows r = tid (mod 256) for the whole panel: the rank-1 update of a column
  // and the next column's norm touch only owned rows, so they need no barrier between them.
  for (int j = 0; j < kb; ++j) {
    // ||x[j+1:]||^2 over the rows this thread owns
    float ss = 0.f;
    for (int r = tid; r < m; r += kHhThreads) {
      const float x = P[j * ldp + r];
      if (r > j) ss += x * x;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wid * (NB + 1) + NB] = ss;
    __syncthreads();
    const float alpha = P[j * ldp + j];
    const float xn = sqrtf(red[NB] + red[(NB + 1) + NB] + red[2 * (NB + 1) + NB] + red[3 * (NB + 1) + NB]);
    float t = 0.f, beta = alpha, scale = 0.f;
    if (xn > 0.f) {
      beta = -copysignf(hypotf(alpha, xn), alpha);
      t = (beta - alpha) / beta;
      scale = 1.f / (alpha - beta);
    }
    // v over the owned rows (row j: 1), partial dots with the later panel columns
    float pd[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) pd[c] = 0.f;
    for (int r = tid; r < m; r += kHhThreads) {
      if (r < j) continue;
      float v = 1.f;
      if (r > j) {
        v = P[j * ldp + r] * scale;
        P[j * ldp + r] = v;
      }
#pragma unroll
      for (int c = 0; c < NB; ++c)
        if (c > j) pd[c] += v * P[c * ldp + r];
    }
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      if (c > j) {
        const float s = wave_sum(pd[c]);
        if (lane == 0) red[wid * (NB + 1) + c] = s;
      }
    }
    __syncthreads();  // also orders this column's alpha / red[NB] reads before the next writes
    if (tid == 0) {
      P[j * ldp + j] = beta;
      tau[p0 + j] = t;
      tl[j] = t;
    }
    for (int r = tid; r < m; r += kHhThreads) {
      if (r < j) continue;
      const float v = (r == j) ? 1.f : P[j * ldp + r];
#pragma unroll
      for (int c = 0; c < NB; ++c) {
        if (c > j) {
          const float w = t * (red[c] + red[(NB + 1) + c] + red[2 * (NB + 1) + c] + red[3 * (NB + 1) + c]);
          P[c * ldp + r] -= v * w;
        }
      }
    }
    // the next column's norm reads only rows this thread updated itself; its alpha and the
    // partial sums are read after the next barrier
  }
  __syncthreads();

  // write the panel back (R part, beta, v) and rebuild V(r, j) for S = V^T V
  for (int idx = tid; idx < m * kb; idx += kHhThreads) {
    const int r = idx / kb, c = idx - r * kb;
    H[(int64_t)(p0 + r) * n + p0 + c] = P[c * ldp + r];
  }
  {
    const int l32 = lane & 31, h = lane >> 5;
    const int chunk = ((m + 7) / 8) * 2;  // rows per wave, even
    const int r0 = wid * chunk, r1 = min(m, r0 + chunk);
    f32x16 acc = zero16();
    for (int r = r0 + h; r < r0 + chunk; r += 2) {
      float v = 0.f;
      if (r < r1 && l32 < kb) v = (r < l32) ? 0.f : (r == l32 ? 1.f : P[l32 * ldp + r]);
      acc = mfma(v, v, acc);
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) Sp[wid * 32 * 33 + acc_row(q, lane) * 33 + l32] = acc[q];
  }
  __syncthreads();
  for (int idx = tid; idx < 32 * 32; idx += kHhThreads) {
    const int i = idx >> 5, j = idx & 31;
    S[i * 33 + j] = Sp[i * 33 + j] + Sp[32 * 33 + i * 33 + j] + Sp[2 * 32 * 33 + i * 33 + j] +
                    Sp[3 * 32 * 33 + i * 33 + j];
  }
  __syncthreads();
  if (tid < 32) {
    const int i = tid;
    for (int j = 0; j < 32; ++j) Tm[i * 33 + j] = 0.f;
    if (i < kb) {
      Tm[i * 33 + i] = tl[i];
      for (int j = i + 1; j < kb; ++j) {
        float acc = 0.f;
        for (int l = i; l < j; ++l) acc += Tm[i * 33 + l] * S[l * 33 + j];
        Tm[i * 33 + j] = -tl[j] * acc;
      }
    }
    float* T = a.T + b * 32 * 32;
    for (int j = 0; j < 32; ++j) T[i * 32 + j] = Tm[i * 33 + j];
  }
}

// C = H[p0:, pe + 64 tile : +64] <- C - V T^T V^T C for the panel's reflectors.
__global__ __launch_bounds__(kHhThreads) void k_hh_update(HhArgs a) {
  __shared__ float Wp[4][32][65];
  __shared__ float Ws[32][65];
  __shared__ float Ts[32][33];
  __shared__ float Vs[4][32][33];
  const int n = a.n, p0 = a.p0, kb = a.kb, m = n - p0, pe = p0 + kb;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, l32 = lane & 31, h = lane >> 5;
  const int64_t pid = blockIdx.x;
  const int64_t b = pid / a.ntile;
  const int tile = (int)(pid - b * a.ntile), c0 = pe + 64 * tile;
  float* H = a.H + b * n * n;
  const float* T = a.T + b * 32 * 32;
  const bool ok0 = c0 + l32 < n, ok1 = c0 + 32 + l32 < n;
  auto V = [&](int r, int j) -> float {  // reflector j of the panel at panel row r
    if (j >= kb || r < j) return 0.f;
    return r == j ? 1.f : H[(int64_t)(p0 + r) * n + p0 + j];
  };

  for (int idx = tid; idx < 32 * 32; idx += kHhThreads) Ts[idx >> 5][idx & 31] = T[idx];
  // W = V^T C, rows split over the waves
  {
    const int chunk = ((m + 7) / 8) * 2;
    const int r0 = wid * chunk, r1 = min(m, r0 + chunk);
    f32x16 acc0 = zero16(), acc1 = zero16();
    for (int r = r0 + h; r < r0 + chunk; r += 2) {
      float v = 0.f, x0 = 0.f, x1 = 0.f;
      if (r < r1) {
        v = V(r, l32);
        const float* row = H + (int64_t)(p0 + r) * n + c0;
        if (ok0) x0 = row[l32];
        if (ok1) x1 = row[32 + l32];
      }
      acc0 = mfma(v, x0, acc0);
      acc1 = mfma(v, x1, acc1);
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      Wp[wid][acc_row(q, lane)][l32] = acc0[q];
      Wp[wid][acc_row(q, lane)][32 + l32] = acc1[q];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < 32 * 64; idx += kHhThreads) {
    const int i = idx >> 6, c = idx & 63;
    Ws[i][c] = Wp[0][i][c] + Wp[1][i][c] + Wp[2][i][c] + Wp[3][i][c];
  }
  __syncthreads();
  // W' = T^T W (wave 0: columns 0..31, wave 1: 32..63), into Wp[0]
  if (wid < 2) {
    f32x16 acc = zero16();
#pragma unroll
    for (int k = 0; k < 32; k += 2) acc = mfma(Ts[k + h][l32], Ws[k + h][32 * wid + l32], acc);
#pragma unroll
    for (int q = 0; q < 16; ++q) Wp[0][acc_row(q, lane)][32 * wid + l32] = acc[q];
  }
  __syncthreads();
  // C -= V W', 32-row strips
  for (int s = wid; 32 * s < m; s += 4) {
    const int rs = 32 * s;
    // stage the strip's V rows (32 x 32) row-contiguously
    for (int idx = lane; idx < 32 * 32; idx += 64) {
      const int rr = idx >> 5, j = idx & 31;
      Vs[wid][rr][j] = (rs + rr < m) ? V(rs + rr, j) : 0.f;
    }
    wave_lds_order();
    f32x16 acc0, acc1;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = rs + acc_row(q, lane);
      const float* row = H + (int64_t)(p0 + r) * n + c0;
      acc0[q] = (r < m && ok0) ? row[l32] : 0.f;
      acc1[q] = (r < m && ok1) ? row[32 + l32] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 32; k += 2) {
      const float v = -Vs[wid][l32][k + h];
      acc0 = mfma(v, Wp[0][k + h][l32], acc0);
      acc1 = mfma(v, Wp[0][k + h][32 + l32], acc1);
    }
    wave_lds_order();
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = rs + acc_row(q, lane);
      if (r < m) {
        float* row = H + (int64_t)(p0 + r) * n + c0;
        if (ok0) row[l32] = acc0[q];
        if (ok1) row[32 + l32] = acc1[q];
      }
    }
  }
}

template <int NB>
int hh_run(float* H, float* tau, float* T, int64_t batch, int n, hipStream_t st) {
  const size_t lds = hh_panel_lds<NB>(n);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_hh_panel<NB>), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return RNR_ERR_HIP;
  for (int p0 = 0; p0 < n; p0 += NB) {
    const int kb = std::min(NB, n - p0), pe = p0 + kb;
    const int ntile = (n - pe + 63) / 64;
    HhArgs a{H, tau, T, n, p0, kb, ntile};
    k_hh_panel<NB><<<dim3((unsigned)batch), dim3(kHhThreads), lds, st>>>(a);
    if (ntile > 0) k_hh_update<<<dim3((unsigned)(batch * ntile)), dim3(kHhThreads), 0, st>>>(a);
  }
  return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP;
}

}  // namespace
}  // namespace rnr

using namespace rnr;

extern "C" {

int rnr_hh_geqrf_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  *bytes = (size_t)batch * 32 * 32 * sizeof(float);
  return RNR_OK;
}

int rnr_hh_geqrf_f32(float* H, int64_t batch, int64_t n, float* tau, void* ws, size_t ws_bytes,
                     rnr_stream_t stream) {
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  if (batch == 0) return RNR_OK;
  if (!H || !tau) return RNR_ERR_INVALID_ARG;
  if (batch * ((n + 63) / 64) > INT32_MAX) return RNR_ERR_INVALID_ARG;
  if (!ws || ws_bytes < (size_t)batch * 32 * 32 * sizeof(float)) return RNR_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return RNR_ERR_MISALIGNED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* T = static_cast<float*>(ws);
  return n <= 1024 ? hh_run<32>(H, tau, T, batch, (int)n, st) : hh_run<16>(H, tau, T, batch, (int)n, st);
}

}  // extern "C"
