// Device-side seeded generators for the five benchmark configurations (the input step of the
// path; the reference builds its batches with torch's generator in common/oracle.py:43-146).
//
// Random streams: Philox4x32-10 (Salmon et al., SC 2011), key = seed, counter = (t low,
// t high, purpose, matrix index), so matrix i of a batch does not depend on the batch size.
// Each draw gives two 53-bit uniforms and, by Box-Muller, two N(0, 1) values in float64.
//
// Classes: dense N(0, 1); rowscaled (row r times 10^u_r, u_r ~ U(-6, 6)); uppertri;
// haar(sigma) = U diag(sigma) W with independent Haar U, W built by Stewart's construction
// (SIAM J. Numer. Anal. 17, 1980): reflector k is the Householder vector (LAPACK dlarfg
// convention) of an independent N(0, I_{n-k}) vector, and U = H_0 ... H_{n-1} diag(sign beta_k),
// which has the distribution of the Q factor of a Gaussian matrix with the signs of diag(R)
// folded in.  Kernels:
//   k_gen_direct      non-Haar matrices, one Philox draw (two entries) per thread, into A;
//   k_gen_reflectors  one workgroup per (factor, Haar matrix, reflector k): the normal vector,
//                     its norm, v_k / tau_k / sign(beta_k), float64 into the workspace;
//   k_apply_q         (applyq.hpp, float64) Y = W_H, then Y <- U_H Y;
//   k_gen_scale       between the two: Y[r][c] *= sigma_r dU_r dW_c;
//   k_gen_store       A[i] = float32(Y[h]).
#include "../../include/rnrqr.h"
#include "applyq.hpp"

namespace rnr {
namespace {

constexpr int P_DENSE = 0, P_U = 1, P_W = 2, P_ROW = 3;   // counter word 2
constexpr int C_DENSE = 0, C_HAAR = 1, C_ROWSCALED = 2, C_UPPERTRI = 3;
constexpr int S_NONE = 0, S_LOG = 1, S_HEADTAIL = 2;

struct Recipe {
  int cls, sk;
  double p;
};

// Class of matrix i of configuration `config` (the table of qr-contest_amd/workloads.py).
__host__ __device__ inline Recipe recipe(int config, int64_t i) {
  switch (config) {
    case 3: return {C_HAAR, S_LOG, 6.0};
    case 4:
      switch ((int)(i % 6)) {
        case 0: return {C_DENSE, S_NONE, 0.0};
        case 1: return {C_HAAR, S_LOG, 12.0};
        case 2: return {C_HAAR, S_HEADTAIL, 0.0};
        case 3: return {C_ROWSCALED, S_NONE, 0.0};
        case 4: return {C_HAAR, S_HEADTAIL, 1e-10};
        default: return {C_UPPERTRI, S_NONE, 0.0};
      }
    case 5: return (i % 2 == 0) ? Recipe{C_DENSE, S_NONE, 0.0} : Recipe{C_HAAR, S_LOG, 8.0};
    default: return {C_DENSE, S_NONE, 0.0};
  }
}

// Matrix index of the h-th Haar-class matrix of the batch.
__host__ __device__ inline int64_t haar_matrix(int config, int64_t h) {
  switch (config) {
    case 3: return h;
    case 4: return 6 * (h / 3) + (h % 3 == 0 ? 1 : (h % 3 == 1 ? 2 : 4));
    case 5: return 2 * h + 1;
    default: return -1;
  }
}

int64_t haar_count(int config, int64_t batch) {
  switch (config) {
    case 3: return batch;
    case 4: {
      int64_t c = 3 * (batch / 6);
      const int64_t r = batch % 6;  // classes 0..r-1 of the last cycle
      c += (r > 1) + (r > 2) + (r > 4);
      return c;
    }
    case 5: return batch / 2;
    default: return 0;
  }
}

__device__ inline double sigma_at(const Recipe& rc, int k, int n) {
  if (rc.sk == S_LOG) return n == 1 ? 1.0 : pow(10.0, -rc.p * (double)k / (double)(n - 1));
  const int r = n / 2;
  if (k >= r) return rc.p;
  return r == 1 ? 1.0 : pow(10.0, -1.0 * (double)k / (double)(r - 1));
}

// ---- random streams -----------------------------------------------------------------------
__device__ inline void philox4x32_10(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3, uint32_t k0,
                                     uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// Two uniforms in [0, 1) with 53 random bits each: draw t of stream (seed, matrix, purpose).
__device__ inline void draw_uniform2(uint64_t seed, uint32_t matrix, uint32_t purpose, uint64_t t, double& ua,
                                     double& ub) {
  uint32_t c0 = (uint32_t)t, c1 = (uint32_t)(t >> 32), c2 = purpose, c3 = matrix;
  philox4x32_10(c0, c1, c2, c3, (uint32_t)seed, (uint32_t)(seed >> 32));
  const uint64_t a = (((uint64_t)c0 << 32) | c1) >> 11, b = (((uint64_t)c2 << 32) | c3) >> 11;
  ua = (double)a * 0x1.0p-53;
  ub = (double)b * 0x1.0p-53;
}

__device__ inline void draw_normal2(uint64_t seed, uint32_t matrix, uint32_t purpose, uint64_t t, double& z0,
                                    double& z1) {
  double ua, ub;
  draw_uniform2(seed, matrix, purpose, t, ua, ub);
  const double r = sqrt(-2.0 * log1p(-ua));
  double s, c;
  sincospi(2.0 * ub, &s, &c);
  z0 = r * c;
  z1 = r * s;
}

__device__ inline double normal_at(uint64_t seed, uint32_t matrix, uint32_t purpose, uint64_t e) {
  double z0, z1;
  draw_normal2(seed, matrix, purpose, e >> 1, z0, z1);
  return (e & 1) ? z1 : z0;
}

__device__ inline double uniform_at(uint64_t seed, uint32_t matrix, uint32_t purpose, uint64_t e) {
  double ua, ub;
  draw_uniform2(seed, matrix, purpose, e >> 1, ua, ub);
  return (e & 1) ? ub : ua;
}

// ---- kernels ------------------------------------------------------------------------------
struct GenArgs {
  float* A;                 // [batch][n][n]
  double* V;                // [2][nh][n][n] reflector vectors (U factors, then W factors)
  double* tau;              // [2][nh][n]
  double* dsg;              // [2][nh][n] sign(beta_k)
  double* Y;                // [nh][n][n]
  uint64_t seed;
  int64_t batch, nh, chunks;
  int config, n;
};

constexpr int kGenThreads = 256;

__global__ __launch_bounds__(kGenThreads) void k_gen_direct(GenArgs g) {
  const int64_t blk = blockIdx.x, i = blk / g.chunks, ch = blk - i * g.chunks;
  const Recipe rc = recipe(g.config, i);
  if (rc.cls == C_HAAR) return;
  const int n = g.n;
  const int64_t nn = (int64_t)n * n, t = ch * kGenThreads + threadIdx.x;
  if (2 * t >= nn) return;
  double z[2];
  draw_normal2(g.seed, (uint32_t)i, P_DENSE, (uint64_t)t, z[0], z[1]);
  float* A = g.A + i * nn;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int64_t e = 2 * t + q;
    if (e >= nn) break;
    const int r = (int)(e / n), c = (int)(e - (int64_t)r * n);
    double v = z[q];
    if (rc.cls == C_ROWSCALED) v *= pow(10.0, uniform_at(g.seed, (uint32_t)i, P_ROW, (uint64_t)r) * 12.0 - 6.0);
    if (rc.cls == C_UPPERTRI && c < r) v = 0.0;
    A[e] = (float)v;
  }
}

constexpr int kRefPer = RNR_MAX_N / kGenThreads;  // vector entries per thread

__global__ __launch_bounds__(kGenThreads) void k_gen_reflectors(GenArgs g) {
  __shared__ double red[kGenThreads / 64];
  __shared__ double alpha_s;
  const int n = g.n, tid = threadIdx.x;
  const int64_t blk = blockIdx.x, fh = blk / n;        // factor-major: fh = q * nh + h
  const int k = (int)(blk - fh * n);
  const int q = (int)(fh / g.nh);
  const int64_t h = fh - (int64_t)q * g.nh;
  const int64_t i = haar_matrix(g.config, h);
  const uint32_t purpose = q == 0 ? P_U : P_W;
  const int L = n - k;
  double x[kRefPer];
  double ss = 0.0;
#pragma unroll
  for (int s = 0; s < kRefPer; ++s) {
    const int j = tid + s * kGenThreads;
    x[s] = 0.0;
    if (j < L) {
      x[s] = normal_at(g.seed, (uint32_t)i, purpose, (uint64_t)k * n + j);
      if (j > 0) ss += x[s] * x[s];
    }
  }
  if (tid == 0) alpha_s = x[0];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int w = 0; w < kGenThreads / 64; ++w) tot += red[w];
  const double alpha = alpha_s, xn = sqrt(tot);
  double* V = g.V + fh * n * (int64_t)n;
  if (xn == 0.0) {
    if (tid == 0) {
      g.tau[fh * n + k] = 0.0;
      g.dsg[fh * n + k] = alpha >= 0.0 ? 1.0 : -1.0;
    }
#pragma unroll
    for (int s = 0; s < kRefPer; ++s) {
      const int j = tid + s * kGenThreads;
      if (j > 0 && j < L) V[(int64_t)(k + j) * n + k] = 0.0;
    }
    return;
  }
  const double beta = -copysign(hypot(alpha, xn), alpha), den = alpha - beta;
  if (tid == 0) {
    g.tau[fh * n + k] = (beta - alpha) / beta;
    g.dsg[fh * n + k] = beta > 0.0 ? 1.0 : -1.0;
  }
#pragma unroll
  for (int s = 0; s < kRefPer; ++s) {
    const int j = tid + s * kGenThreads;
    if (j > 0 && j < L) V[(int64_t)(k + j) * n + k] = x[s] / den;
  }
}

__global__ __launch_bounds__(kGenThreads) void k_gen_scale(GenArgs g) {
  const int n = g.n;
  const int64_t nn = (int64_t)n * n, total = g.nh * nn;
  for (int64_t e = (int64_t)blockIdx.x * kGenThreads + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kGenThreads) {
    const int64_t h = e / nn, w = e - h * nn;
    const int r = (int)(w / n), c = (int)(w - (int64_t)r * n);
    const Recipe rc = recipe(g.config, haar_matrix(g.config, h));
    const double du = g.dsg[h * n + r], dw = g.dsg[(g.nh + h) * n + c];
    g.Y[e] *= sigma_at(rc, r, n) * du * dw;
  }
}

__global__ __launch_bounds__(kGenThreads) void k_gen_store(GenArgs g) {
  const int n = g.n;
  const int64_t nn = (int64_t)n * n, total = g.nh * nn;
  for (int64_t e = (int64_t)blockIdx.x * kGenThreads + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * kGenThreads) {
    const int64_t h = e / nn, w = e - h * nn;
    g.A[haar_matrix(g.config, h) * nn + w] = (float)g.Y[e];
  }
}

inline size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

struct GenLayout {
  size_t v, tau, dsg, y, total;
};

GenLayout gen_layout(int64_t nh, int64_t n) {
  GenLayout l;
  l.v = 0;
  l.tau = l.v + up256((size_t)2 * nh * n * n * sizeof(double));
  l.dsg = l.tau + up256((size_t)2 * nh * n * sizeof(double));
  l.y = l.dsg + up256((size_t)2 * nh * n * sizeof(double));
  l.total = nh == 0 ? 0 : l.y + up256((size_t)nh * n * n * sizeof(double));
  return l;
}

template <bool IDENT>
int launch_apply_f64(const ApplyQArgs<double, double>& a, int64_t batch, hipStream_t st) {
  if (a.n <= 1024) {
    const size_t lds = applyq_lds<double, 16>(a.n);
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_apply_q<double, 16, false, IDENT, double>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return RNR_ERR_HIP;
    k_apply_q<double, 16, false, IDENT, double><<<applyq_grid(batch, a.nc), dim3(kApplyQThreads), lds, st>>>(a);
  } else {
    const size_t lds = applyq_lds<double, 8>(a.n);
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_apply_q<double, 8, false, IDENT, double>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return RNR_ERR_HIP;
    k_apply_q<double, 8, false, IDENT, double><<<applyq_grid(batch, a.nc), dim3(kApplyQThreads), lds, st>>>(a);
  }
  return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP;
}

int check_gen_args(int config, int64_t batch, int64_t n) {
  if (config < 1 || config > 5 || batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  if (batch > INT32_MAX) return RNR_ERR_INVALID_ARG;  // matrix index is counter word 3
  return RNR_OK;
}

}  // namespace
}  // namespace rnr

using namespace rnr;

extern "C" {

int rnr_generate_workspace(int config, int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (int e = check_gen_args(config, batch, n)) return e;
  *bytes = gen_layout(haar_count(config, batch), n).total;
  return RNR_OK;
}

int rnr_generate_f32(int config, int64_t batch, int64_t n, uint64_t seed, float* A, void* ws, size_t ws_bytes,
                     rnr_stream_t stream) {
  if (int e = check_gen_args(config, batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!A) return RNR_ERR_INVALID_ARG;
  const int64_t nh = haar_count(config, batch);
  const GenLayout l = gen_layout(nh, n);
  if (l.total > 0) {
    if (!ws || ws_bytes < l.total) return RNR_ERR_WORKSPACE;
    if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return RNR_ERR_MISALIGNED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(ws);
  GenArgs g{};
  g.A = A;
  g.seed = seed;
  g.batch = batch;
  g.nh = nh;
  g.config = config;
  g.n = (int)n;
  const int64_t nn = n * n, pairs = (nn + 1) / 2;
  g.chunks = (pairs + kGenThreads - 1) / kGenThreads;
  if (batch * g.chunks > INT32_MAX) return RNR_ERR_INVALID_ARG;
  k_gen_direct<<<dim3((unsigned)(batch * g.chunks)), dim3(kGenThreads), 0, st>>>(g);
  if (hipGetLastError() != hipSuccess) return RNR_ERR_HIP;
  if (nh == 0) return RNR_OK;

  g.V = reinterpret_cast<double*>(base + l.v);
  g.tau = reinterpret_cast<double*>(base + l.tau);
  g.dsg = reinterpret_cast<double*>(base + l.dsg);
  g.Y = reinterpret_cast<double*>(base + l.y);
  if (2 * nh * n > INT32_MAX) return RNR_ERR_INVALID_ARG;
  k_gen_reflectors<<<dim3((unsigned)(2 * nh * n)), dim3(kGenThreads), 0, st>>>(g);
  if (hipGetLastError() != hipSuccess) return RNR_ERR_HIP;
  const int ni = (int)n;
  // Y = W_H (the identity times the W reflectors), then the diagonal, then Y <- U_H Y
  ApplyQArgs<double, double> aw{g.V + nh * nn, g.tau + nh * n, g.Y, nn, ni, ni, ni};
  if (int e = launch_apply_f64<true>(aw, nh, st)) return e;
  const unsigned eb = (unsigned)std::min<int64_t>((nh * nn + kGenThreads - 1) / kGenThreads, 65536);
  k_gen_scale<<<dim3(eb), dim3(kGenThreads), 0, st>>>(g);
  if (hipGetLastError() != hipSuccess) return RNR_ERR_HIP;
  ApplyQArgs<double, double> au{g.V, g.tau, g.Y, nn, ni, ni, ni};
  if (int e = launch_apply_f64<false>(au, nh, st)) return e;
  k_gen_store<<<dim3(eb), dim3(kGenThreads), 0, st>>>(g);
  return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP;
}

}  // extern "C"
