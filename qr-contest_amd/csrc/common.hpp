// Shared device helpers for the gfx950 (CDNA4) kernels of librnrqr.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <limits.h>
#include <type_traits>

namespace rnr {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x2_f32 on one wave64: D(32x32) = A(32x2) * B(2x32) + C.
// Operand lanes: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32].
// Result lanes:  D[row][col] sits in lane col + 32 * ((row / 4) % 2), register
//                4 * (row / 8) + row % 4  (acc_row inverts this for a given register).
__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

typedef float f32x32 __attribute__((ext_vector_type(32)));

// v_mfma_f32_32x32x1_2b_f32: two independent 32x32 outer products, D_b = A_b B_b + C_b.
// Block b takes A_b[i] from lane 32 b + i and B_b[j] from lane 32 b + j; its result sits in
// registers 16 b .. 16 b + 15 with the layout of mfma above (D_b[row][col] in lane
// col + 32 * ((row / 4) % 2), register 16 b + 4 * (row / 8) + row % 4).
__device__ __forceinline__ f32x32 mfma_2b(float a, float b, f32x32 c) {
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
}

// v_permlane32_swap of (x, y): returns [x lanes 0-31, y lanes 0-31] in .x and
// [x lanes 32-63, y lanes 32-63] in .y (lane l < 32 of the result's upper half reading l + 32).
__device__ __forceinline__ float2 lane_halves(float x, float y) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return make_float2(__uint_as_float(p[0]), __uint_as_float(p[1]));
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

typedef float f32x4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16];
// D[row][col] sits in lane col + 16 * (row / 4), register row % 4.
__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Keeps the loads issued above this point ahead of everything below it.  Left alone, the
// scheduler interleaves a block of independent loads with their consumers (MFMAs), so each
// consumer waits on a load issued just before it instead of all loads sharing one latency.
__device__ __forceinline__ void issue_loads_first() { __builtin_amdgcn_sched_barrier(0); }

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

// DPP lane permutations within rows of 16 lanes (VALU, no LDS round trip).
constexpr int kDppQuad1032 = 0xB1;      // lane ^ 1
constexpr int kDppQuad2301 = 0x4E;      // lane ^ 2
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15 - i within 16

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// One combine step of the first-maximum argmax: larger |value| wins, equal |value| goes to
// the smaller index.
__device__ __forceinline__ void argmax_take(float& babs, float& bv, int& bi, float oabs, float ov, int oi) {
  const bool take = (oabs > babs) | ((oabs == babs) & (oi < bi));  // branch-free
  babs = take ? oabs : babs;
  bv = take ? ov : bv;
  bi = take ? oi : bi;
}

template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float& babs, float& bv, int& bi) {
  argmax_take(babs, bv, bi, dpp_f<CTRL>(babs), dpp_f<CTRL>(bv), dpp_i<CTRL>(bi));
}

// Wave-wide first-maximum argmax of (|v|, index); every lane gets the wave's winner.
// Four DPP steps reduce each row of 16 lanes, the four rows are combined by readlane.
__device__ __forceinline__ void wave_argmax(float& babs, float& bv, int& bi) {
  argmax_dpp_step<kDppQuad1032>(babs, bv, bi);
  argmax_dpp_step<kDppQuad2301>(babs, bv, bi);
  argmax_dpp_step<kDppRowHalfMirror>(babs, bv, bi);
  argmax_dpp_step<kDppRowMirror>(babs, bv, bi);
  float ra = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(babs), 0));
  float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
  int ri = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
  for (int row = 1; row < 4; ++row) {
    const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(babs), 16 * row));
    const float tv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 16 * row));
    const int ti = __builtin_amdgcn_readlane(bi, 16 * row);
    argmax_take(ra, rv, ri, t, tv, ti);
  }
  babs = ra;
  bv = rv;
  bi = ri;
}

// Wave-wide maximum of an unsigned 32-bit value (all 64 lanes active); the result is uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp_i<kDppQuad1032>((int)v));
  v = max(v, (uint32_t)dpp_i<kDppQuad2301>((int)v));
  v = max(v, (uint32_t)dpp_i<kDppRowHalfMirror>((int)v));
  v = max(v, (uint32_t)dpp_i<kDppRowMirror>((int)v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// Wave-wide maximum of a 64-bit key as two 32-bit reductions: the largest high word, then the
// largest low word among the lanes that hold it (lexicographic order = unsigned 64-bit order).
// When one lane alone holds the largest high word (the usual case), its low word is read
// directly; only ties run the second reduction.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t key) {
  const uint32_t hi = (uint32_t)(key >> 32), lo = (uint32_t)key;
  const uint32_t mh = wave_max_u32(hi);
  const uint64_t holders = __ballot(hi == mh);  // uniform
  uint32_t ml;
  if (__popcll(holders) == 1)
    ml = (uint32_t)__builtin_amdgcn_readlane((int)lo, __ffsll((long long)holders) - 1);
  else
    ml = wave_max_u32(hi == mh ? lo : 0u);
  return ((uint64_t)mh << 32) | ml;
}

// An LDS float4 pointer in a register the compiler cannot see through: reads from it use
// immediate offsets from that one register instead of one materialised (and hoisted) address
// per read.
typedef float lds_v4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const lds_v4_t lds_f4;
__device__ __forceinline__ const lds_f4* lds_base(const float* p) {
  const lds_f4* q = (const lds_f4*)p;
  asm volatile("" : "+v"(q));
  return q;
}
__device__ __forceinline__ const lds_f4* lds_base(const float4* p) {
  return lds_base(reinterpret_cast<const float*>(p));
}
__device__ __forceinline__ float4 lds_get(const lds_f4* p, int i) {
  const lds_v4_t v = p[i];
  return make_float4(v[0], v[1], v[2], v[3]);
}

// Component I of a float4 (compile-time I).
template <int I>
__device__ __forceinline__ float f4get(const float4& v) {
  if constexpr (I == 0) return v.x;
  else if constexpr (I == 1) return v.y;
  else if constexpr (I == 2) return v.z;
  else return v.w;
}

// Calls f(std::integral_constant<int, I>) for I = B .. E-1, fully unrolled at compile time
// (register arrays indexed by I then stay in registers).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
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
