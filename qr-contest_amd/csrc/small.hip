// Launcher of the fused small-n kernel (own translation unit: it compiles in parallel with
// the blocked path).
#include "small.hpp"

namespace rnr {

namespace {
template <int NP>
int launch_np(const SmallArgs& a, hipStream_t st) {
  const size_t lds = small_lds_bytes(NP);
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k_small<NP>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return 1;
  const int per_wg = kSmallWaves * SmallLayout<NP>::G;
  const unsigned grid = (unsigned)((a.batch + per_wg - 1) / per_wg);
  k_small<NP><<<dim3(grid), dim3(64 * kSmallWaves), lds, st>>>(a);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
}  // namespace

// 0 on success, 1 on a HIP error.  Requires 1 <= n <= kSmallMaxN and batch >= 1.
int launch_small(const SmallArgs& a, hipStream_t st) {
  const int np = small_np(a.n);
  if (np == 16) return launch_np<16>(a, st);
  if (np == 32) return launch_np<32>(a, st);
  return launch_np<64>(a, st);
}

}  // namespace rnr
