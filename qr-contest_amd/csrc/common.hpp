// Shared device helpers for the gfx950 (CDNA4) kernels of librnrqr.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <limits.h>

namespace rnr {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x2_f32 on one wave64: D(32x32) = A(32x2) * B(2x32) + C.
// Operand lanes: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32].
// Result lanes:  D[row][col] sits in lane col + 32 * ((row / 4) % 2), register
//                4 * (row / 8) + row % 4  (acc_row inverts this for a given register).
__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int r, int lane) {
  return ((r >> 2) << 3) + ((lane >> 5) << 2) + (r & 3);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X.  Regroup the
// logical ids so that consecutive ones (the tiles of one matrix) land on one XCD and
// share its L2; the remainder after the last full round keeps its order.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  constexpr int kXcd = 8;
  const int per = total / kXcd;
  if (pid >= per * kXcd) return pid;
  return (pid % kXcd) * per + pid / kXcd;
}

// Orders LDS traffic between lanes of one wave (a wave executes its LDS operations in
// program order; this keeps the compiler from moving loads above earlier stores).
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum over the 8 consecutive lanes of an aligned lane group.
__device__ __forceinline__ float group8_sum(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  return v;
}

// Upper-triangular tile enumeration: t -> (ti, tj), ti <= tj < nt, row by row.
__device__ __forceinline__ void upper_tile(int t, int nt, int& ti, int& tj) {
  int i = 0;
  while (t >= nt - i) {
    t -= nt - i;
    ++i;
  }
  ti = i;
  tj = i + t;
}

}  // namespace rnr
