// fp32 consumers of the compact (H, tau) output on the GPU (README.md:122-128):
//   rnr_orgqr_f32  Q = householder_product(H, tau)  (torch.linalg.householder_product)
//   rnr_ormqr_f32  C <- Q C or Q^T C                 (torch.ormqr, left side)
// Both run the MFMA blocked-WY kernels of wy.hpp: every panel's T in one launch, then one
// launch per 32-reflector panel that updates the target's column tiles held in registers.
// Q applies the panels last to first (orgqr: from the identity, and panel p leaves the
// columns left of its first reflector alone -- they are still unit vectors); Q^T first to last.
#include "../../include/rnrqr.h"
#include "wy.hpp"

using namespace rnr;

namespace {

inline size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

size_t wy_ws(int64_t batch, int64_t n) {
  const int64_t np = (n + kWyPb - 1) / kWyPb;
  return up256((size_t)batch * np * 32 * 32 * sizeof(float));
}

int check_sizes(int64_t batch, int64_t n) {
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  if (batch > INT32_MAX / 64) return RNR_ERR_INVALID_ARG;  // grids of batch x tiles
  return RNR_OK;
}

template <bool TRANS, int NW, int NS, int NC>
int wy_run(WyArgs a, int64_t batch, bool ident, hipStream_t st) {
  k_wy_tmat<<<dim3((unsigned)(batch * a.np)), dim3(256), 0, st>>>(a);
  if (ident) {
    const int nchunk = (a.n * a.n + 255) / 256 < 64 ? (a.n * a.n + 255) / 256 : 64;
    k_wy_identity<<<dim3((unsigned)(batch * nchunk)), dim3(256), 0, st>>>(a.Y, a.sy, a.ldy, a.n, nchunk);
  }
  for (int s = 0; s < a.np; ++s) {
    a.p = TRANS ? s : a.np - 1 - s;
    a.c_lo = ident ? a.p * kWyPb : 0;
    a.ntile = (a.nc - a.c_lo + NC - 1) / NC;
    if (a.ntile <= 0) continue;
    k_wy_apply<TRANS, NW, NS, NC><<<dim3((unsigned)(batch * a.ntile)), dim3(NW * 64), 0, st>>>(a);
  }
  return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP;
}

// rows per tile = 32 NW NS >= n
template <bool TRANS>
int wy_dispatch(const WyArgs& a, int64_t batch, bool ident, hipStream_t st) {
  if (a.n <= 512) return wy_run<TRANS, 4, 4, 32>(a, batch, ident, st);
  if (a.n <= 1024) return wy_run<TRANS, 8, 4, 32>(a, batch, ident, st);
  return wy_run<TRANS, 8, 8, 32>(a, batch, ident, st);
}

int check_ws(void* ws, size_t ws_bytes, size_t need) {
  if (!ws || ws_bytes < need) return RNR_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return RNR_ERR_MISALIGNED;
  return RNR_OK;
}

}  // namespace

extern "C" {

int rnr_orgqr_f32_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (int e = check_sizes(batch, n)) return e;
  *bytes = batch == 0 ? 0 : wy_ws(batch, n);
  return RNR_OK;
}

int rnr_ormqr_f32_workspace(int64_t batch, int64_t n, size_t* bytes) {
  return rnr_orgqr_f32_workspace(batch, n, bytes);
}

int rnr_orgqr_f32(const float* H, const float* tau, int64_t batch, int64_t n, float* Q, void* ws,
                  size_t ws_bytes, rnr_stream_t stream) {
  if (int e = check_sizes(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!H || !tau || !Q) return RNR_ERR_INVALID_ARG;
  if (int e = check_ws(ws, ws_bytes, wy_ws(batch, n))) return e;
  const int ni = (int)n;
  WyArgs a{H, tau, static_cast<float*>(ws), Q, n * n, ni, ni, ni, (ni + kWyPb - 1) / kWyPb, 0, 0, 0};
  return wy_dispatch<false>(a, batch, true, reinterpret_cast<hipStream_t>(stream));
}

int rnr_ormqr_f32(const float* H, const float* tau, int64_t batch, int64_t n, float* C, int64_t ncol,
                  int64_t ldc, int64_t batch_stride_c, int transpose, void* ws, size_t ws_bytes,
                  rnr_stream_t stream) {
  if (int e = check_sizes(batch, n)) return e;
  if (batch == 0 || ncol == 0) return RNR_OK;
  if (!H || !tau || !C || ncol < 0 || ncol > INT32_MAX / 2 || ldc < ncol || ldc > INT32_MAX ||
      batch_stride_c < n * ldc)
    return RNR_ERR_INVALID_ARG;
  if (batch * ((ncol + 31) / 32) > INT32_MAX) return RNR_ERR_INVALID_ARG;
  if (int e = check_ws(ws, ws_bytes, wy_ws(batch, n))) return e;
  const int ni = (int)n;
  WyArgs a{H, tau, static_cast<float*>(ws), C, batch_stride_c, (int)ldc, ni, (int)ncol,
           (ni + kWyPb - 1) / kWyPb, 0, 0, 0};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return transpose ? wy_dispatch<true>(a, batch, false, st) : wy_dispatch<false>(a, batch, false, st);
}

}  // extern "C"
