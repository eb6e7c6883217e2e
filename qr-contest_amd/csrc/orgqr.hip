// fp32 consumers of the compact (H, tau) output on the GPU (README.md:122-128):
//   rnr_orgqr_f32  Q = householder_product(H, tau)  (torch.linalg.householder_product)
//   rnr_ormqr_f32  C <- Q C or Q^T C                 (torch.ormqr, left side)
// Both run the blocked-WY kernel of applyq.hpp in float32.
#include "../../include/rnrqr.h"
#include "applyq.hpp"

using namespace rnr;

namespace {

template <bool TRANS, bool IDENT>
int launch_apply(const ApplyQArgs<float>& a, int64_t batch, hipStream_t st) {
  const size_t lds = applyq_lds<float, 16>(a.n);
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_apply_q<float, 16, TRANS, IDENT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return RNR_ERR_HIP;
  k_apply_q<float, 16, TRANS, IDENT><<<applyq_grid(batch, a.nc), dim3(kApplyQThreads), lds, st>>>(a);
  return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP;
}

int check_sizes(int64_t batch, int64_t n) {
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  if (batch > INT32_MAX) return RNR_ERR_INVALID_ARG;
  return RNR_OK;
}

}  // namespace

extern "C" {

int rnr_orgqr_f32(const float* H, const float* tau, int64_t batch, int64_t n, float* Q, rnr_stream_t stream) {
  if (int e = check_sizes(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!H || !tau || !Q) return RNR_ERR_INVALID_ARG;
  ApplyQArgs<float> a{H, tau, Q, n * n, (int)n, (int)n, (int)n};
  return launch_apply<false, true>(a, batch, reinterpret_cast<hipStream_t>(stream));
}

int rnr_ormqr_f32(const float* H, const float* tau, int64_t batch, int64_t n, float* C, int64_t ncol,
                  int64_t ldc, int64_t batch_stride_c, int transpose, rnr_stream_t stream) {
  if (int e = check_sizes(batch, n)) return e;
  if (batch == 0 || ncol == 0) return RNR_OK;
  if (!H || !tau || !C || ncol < 0 || ncol > INT32_MAX || ldc < ncol || ldc > INT32_MAX ||
      batch_stride_c < n * ldc)
    return RNR_ERR_INVALID_ARG;
  ApplyQArgs<float> a{H, tau, C, batch_stride_c, (int)ldc, (int)n, (int)ncol};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return transpose ? launch_apply<true, false>(a, batch, st) : launch_apply<false, false>(a, batch, st);
}

}  // extern "C"
