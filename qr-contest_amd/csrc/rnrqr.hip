// librnrqr: C ABI and launch sequence of the reflector-free batched QR for gfx950.
//
// Launch sequence of rnr_qr_f32 on the caller's stream (reflection_no_reflectors.py:181-196):
//   1. k_lu<true>        A -> W (in-place factor, A's row order), perm, L      (:66)
//   2. k_tn_upper        G = L^T L, upper tiles, zero rows of L skipped         (:73)
//   3. k_chol            G -> R_a (upper, jittered), Dinv, info, and W = the off-diagonal
//                        blocks of R_a times Dinv -> Qb (the solve's operand)      (:74-76)
//                        (n > 512 with fewer than 128 matrices: k_chol_jitter, k_chol_diag, then
//                        per 64-column block k_chol_row / k_chol_step, and W from k_wblocks)
//   4. k_trsm            Q1 = L R_a^-1 -> L buffer                              (:77)
//   5. k_tn_upper        G = Q1^T Q1                                            (:73)
//   6. k_chol            G -> R_b, Dinv, info; W for R_b -> the (now dead) LU buffer (:74-76)
//   7. k_trsm            Q = P (Q1 R_b^-1) -> Qb (row scatter)                   (:77,81)
//   8. k_lu<false>       chart of Q, read from Qb, worked in H: tails Y, signs  (:139-174,192)
//                        s, tau (Qb stays intact for the closure)
//   9. k_tn_upper        H_upper = diag(s) triu(Q^T A), masked to j >= i         (:186,195)
// rnr_qr_f32_timed records one caller event before each launch and one after the last.
//
// For n <= kSmallMaxN (64) the whole path is instead one launch of k_small (small.hpp), one
// matrix per group of lanes of a wave; it needs no workspace.
#include <mutex>

#include "../../include/rnrqr.h"
#include "common.hpp"
#include "gemm_tn.hpp"
#include "lu.hpp"
#include "chol.hpp"
#include "trsm.hpp"
#include "small.hpp"

namespace rnr {
int launch_small(const SmallArgs& a, hipStream_t st);  // small.hip
}

using namespace rnr;

namespace {

constexpr size_t kLdsMax = 160 * 1024;

inline size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

struct Ws {
  float* W;
  float* L;
  float* G;
  float* Qb;
  float* Dinv;
  float* s;
  int* perm;
  int* info;
};

enum WsNeed : unsigned {
  kNeedW = 1u, kNeedL = 2u, kNeedG = 4u, kNeedQb = 8u, kNeedDinv = 16u,
  kNeedS = 32u, kNeedPerm = 64u, kNeedInfo = 128u
};

// Carves the workspace; returns the bytes needed.  With base == nullptr only sizes.
size_t carve(int64_t batch, int64_t n, unsigned need, char* base, Ws* ws) {
  const size_t nn = (size_t)batch * n * n * sizeof(float);
  size_t off = 0;
  auto take = [&](unsigned bit, size_t bytes) -> char* {
    if (!(need & bit)) return nullptr;
    char* p = base ? base + off : nullptr;
    off += up256(bytes);
    return p;
  };
  Ws w;
  w.W = reinterpret_cast<float*>(take(kNeedW, nn));
  w.L = reinterpret_cast<float*>(take(kNeedL, nn));
  w.G = reinterpret_cast<float*>(take(kNeedG, nn));
  w.Qb = reinterpret_cast<float*>(take(kNeedQb, nn));
  w.Dinv = reinterpret_cast<float*>(take(kNeedDinv, (size_t)batch * n * 64 * sizeof(float)));
  w.s = reinterpret_cast<float*>(take(kNeedS, (size_t)batch * n * sizeof(float)));
  w.perm = reinterpret_cast<int*>(take(kNeedPerm, (size_t)batch * n * sizeof(int)));
  w.info = reinterpret_cast<int*>(take(kNeedInfo, (size_t)batch * sizeof(int)));
  if (ws) *ws = w;
  return off;
}

constexpr unsigned kQrNeed = kNeedW | kNeedL | kNeedG | kNeedQb | kNeedDinv | kNeedS | kNeedPerm | kNeedInfo;
constexpr unsigned kLuNeed = kNeedW | kNeedDinv;
constexpr unsigned kCholqrNeed = kNeedG | kNeedQb | kNeedDinv | kNeedInfo;
constexpr unsigned kFrameNeed = kNeedW | kNeedL | kNeedG | kNeedQb | kNeedDinv | kNeedPerm | kNeedInfo;

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_common(int64_t batch, int64_t n) {
  if (batch < 0 || n < 0) return RNR_ERR_INVALID_ARG;
  if (n < 1 || n > RNR_MAX_N) return RNR_ERR_UNSUPPORTED_N;
  if (batch > (int64_t)INT32_MAX / 64) return RNR_ERR_INVALID_ARG;
  return RNR_OK;
}

int hip_status() { return hipGetLastError() == hipSuccess ? RNR_OK : RNR_ERR_HIP; }

template <typename K>
int set_lds(K kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return RNR_OK;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess
             ? RNR_OK
             : RNR_ERR_HIP;
}

template <bool PIVOT, int NB, int RPT, int T = kLuThreads>
int launch_lu_nb(const LuArgs& a, int64_t batch, hipStream_t st) {
  const size_t lds = lu_lds_bytes(a.n, NB);
  if (lds > kLdsMax) return RNR_ERR_UNSUPPORTED_N;
  if (int e = set_lds(k_lu<PIVOT, NB, RPT, false, T>, lds)) return e;
  k_lu<PIVOT, NB, RPT, false, T><<<dim3((unsigned)batch), dim3(T), lds, st>>>(a);
  return hip_status();
}

// Batches too small to occupy the GPU with one workgroup per matrix (fewer matrices than
// half the CUs) at n > 512: each LU / chart panel is its own launch, and the trailing updates
// are spread over one workgroup per 64-column chunk (k_lu_trail_g, once per group of four
// panels); the Cholesky likewise runs per block (k_chol_row, then k_chol_step: trailing tiles
// beside the next diagonal factor).
bool lu_split(int64_t batch, int n) { return n > 512 && batch < 128; }
// The Cholesky's per-block form also at n <= 128, where the fused kernel (205 VGPRs: two
// 256-thread workgroups per CU) takes two rounds for a large batch and the per-block kernels
// fit at once (1024 x 128: 0.12 -> 0.09 ms per pass, 0.11 with the W blocks).
bool chol_split(int64_t batch, int n) { return lu_split(batch, n) || n <= 128; }

// Grouped update: panels kg .. kg + 32 S applied to columns [cb, ce) of the rows below them.
template <bool PIVOT>
void launch_lu_trail_g(const LuArgs& a, int S, int kg, int cb, int ce, int64_t batch, hipStream_t st) {
  const int rb = kg + 32 * S, rows = a.n - rb;
  const int nchunk = (ce - cb + 63) / 64;
  // rows per workgroup: each workgroup forms its chunk's U itself, so it takes as many rows as
  // still leaves about one workgroup per two CUs (at least 256; measured at 16 x 2048 against
  // thresholds of 2 to 8 workgroups per CU, which redo the U more often: 20.0 -> 19.5 ms)
  // The catch-up launches (S < 4: one 32-column chunk, a U of a few 32 x 32 blocks that costs
  // little to redo) take 128 rows, one row tile per wave, for more workgroups (16 x 2048:
  // 19.1 -> 18.7 ms against 256 rows and more).
  int rpw = S < 4 ? 128 : kLuTrailRows;
  if (S == 4)
    while (rpw < rows && batch * nchunk * ((rows + 2 * rpw - 1) / (2 * rpw)) >= 128) rpw *= 2;
  const int nrg = (rows + rpw - 1) / rpw;
  const dim3 grid((unsigned)(batch * nchunk * nrg)), block(kLuTrailThreads);
  const int64_t xslot = batch * 1024;
  switch (S) {
    case 1: k_lu_trail_g<PIVOT, 1><<<grid, block, 0, st>>>(a, kg, cb, ce, nchunk, nrg, rpw, xslot); break;
    case 2: k_lu_trail_g<PIVOT, 2><<<grid, block, 0, st>>>(a, kg, cb, ce, nchunk, nrg, rpw, xslot); break;
    case 3: k_lu_trail_g<PIVOT, 3><<<grid, block, 0, st>>>(a, kg, cb, ce, nchunk, nrg, rpw, xslot); break;
    default: k_lu_trail_g<PIVOT, 4><<<grid, block, 0, st>>>(a, kg, cb, ce, nchunk, nrg, rpw, xslot); break;
  }
}

// 32-wide panels in groups of four: panel s of a group is first brought up to date with the
// group's earlier panels (its 32 columns only), then factored (L11^-1 to slot s of the xbuf);
// after the group one rank-128 pass updates everything right of it.  The panel launches run
// 1024 threads (16 waves, RPT rows each): one workgroup per matrix leaves most CUs idle here,
// so each column step's per-thread work is what sets the time.
template <bool PIVOT, int RPT>
int launch_lu_split(LuArgs a, int64_t batch, hipStream_t st) {
  constexpr int NB = 32, G = 4, T = 1024;
  const size_t lds = lu_lds_bytes(a.n, NB, true);  // the panel's rows stay out of LDS (L11 only)
  if (lds > kLdsMax) return RNR_ERR_UNSUPPORTED_N;
  if (int e = set_lds(k_lu<PIVOT, NB, RPT, true, T>, lds)) return e;
  const int n = a.n;
  float* const xbase = a.X;
  for (int kg = 0; kg < n; kg += G * NB) {
    const int np = min(G, (n - kg + NB - 1) / NB);  // panels in this group
    for (int sp = 0; sp < np; ++sp) {
      const int kp = kg + NB * sp;
      a.X = xbase;
      if (sp > 0) launch_lu_trail_g<PIVOT>(a, sp, kg, kp, min(kp + NB, n), batch, st);
      a.k0 = kp;
      a.X = xbase + (int64_t)sp * batch * NB * NB;
      k_lu<PIVOT, NB, RPT, true, T><<<dim3((unsigned)batch), dim3(T), lds, st>>>(a);
    }
    a.X = xbase;
    if (kg + G * NB < n) launch_lu_trail_g<PIVOT>(a, G, kg, kg + G * NB, n, batch, st);
  }
  if (!PIVOT) {  // the chart's tau, from the finished multipliers
    const int ncb = (n + 31) / 32;
    k_chart_tau<<<dim3((unsigned)(batch * ncb)), dim3(256), 0, st>>>(a.dst, a.sd, a.tau, n, ncb);
  }
  return hip_status();
}

// xbuf: batch * 64 * 64 floats of scratch for the split form (the four 32x32 L11^-1 of a panel
// group between launches, slot-major).
int launch_lu(bool pivot, const float* src, int64_t ss, float* dst, int64_t sd, int64_t batch,
              int n, int* perm, float* L, float* s, float* tau, float* xbuf, hipStream_t st) {
  LuArgs a;
  a.src = src; a.ss = ss; a.dst = dst; a.sd = sd; a.n = n;
  a.vec4 = (n % 4 == 0) && (ss % 4 == 0) && (sd % 4 == 0) && aligned(src, 16) && aligned(dst, 16);
  a.perm = perm; a.L = L; a.sl = (int64_t)n * n; a.s = s; a.tau = tau;
  a.k0 = 0; a.X = xbuf;
  const int nb = lu_panel_nb(n);
  if (lu_split(batch, n) && xbuf) {
    // 32-wide panels at every split size: the panel's rows go straight between HBM and registers,
    // so its width is not bound by an n-row LDS copy (rank-32 trailing updates, half the passes)
    if (pivot) return n <= 1024 ? launch_lu_split<true, 1>(a, batch, st) : launch_lu_split<true, 2>(a, batch, st);
    return n <= 1024 ? launch_lu_split<false, 1>(a, batch, st) : launch_lu_split<false, 2>(a, batch, st);
  }
  // rows per thread: n <= T * RPT; one row per thread with 128 or 256 threads at n <= 128 / 256
  if (pivot) {
    if (nb == 64) {
      if (n <= 256) return launch_lu_nb<true, 64, 1, 256>(a, batch, st);
      return launch_lu_nb<true, 64, 1>(a, batch, st);
    }
    if (nb == 32) return n <= 128 ? launch_lu_nb<true, 32, 1, 128>(a, batch, st) : launch_lu_nb<true, 32, 2>(a, batch, st);
    return launch_lu_nb<true, 16, 4>(a, batch, st);
  }
  if (nb == 64) {
    if (n <= 256) return launch_lu_nb<false, 64, 1, 256>(a, batch, st);
    return launch_lu_nb<false, 64, 1>(a, batch, st);
  }
  if (nb == 32) return n <= 128 ? launch_lu_nb<false, 32, 1, 128>(a, batch, st) : launch_lu_nb<false, 32, 2>(a, batch, st);
  return launch_lu_nb<false, 16, 4>(a, batch, st);
}

// C[b] upper tiles of X^T Y (see gemm_tn.hpp); closure = masked + row-scaled.
int launch_tn(bool closure, const float* X, int64_t sx, const float* Y, int64_t sy, float* C,
              int64_t sc, const float* rs, const int* lperm, int64_t batch, int n, bool klo_from_j,
              hipStream_t st) {
  const bool big = n > 256;
  const int BM = big ? 128 : 64;
  TnArgs a;
  a.X = X; a.sx = sx; a.Y = Y; a.sy = sy; a.C = C; a.sc = sc; a.rs = rs; a.lperm = lperm; a.n = n;
  a.nt = (n + BM - 1) / BM;
  a.ntiles = a.nt * (a.nt + 1) / 2;
  a.klo_from_j = klo_from_j ? 1 : 0;
  const int64_t total = batch * a.ntiles;
  if (total > INT32_MAX) return RNR_ERR_INVALID_ARG;
  a.total = (int)total;
  a.lpt = (klo_from_j && total % 8 == 0 && (total / 8) % a.ntiles == 0) ? 1 : 0;
  const bool vec4 = (n % 4 == 0) && (sx % 4 == 0) && (sy % 4 == 0) && aligned(X, 16) && aligned(Y, 16);
  const dim3 grid((unsigned)total), block(256);
#define RNR_TN(BMv, MASK, RS, V, BKv, LVv) k_tn_upper<BMv, MASK, RS, V, BKv, LVv><<<grid, block, 0, st>>>(a)
  if (closure) {  // no L view: the row map's LDS is left out
    if (big) { if (vec4) RNR_TN(128, true, true, true, 16, false); else RNR_TN(128, true, true, false, 32, false); }
    else     { if (vec4) RNR_TN(64, true, true, true, 32, false);  else RNR_TN(64, true, true, false, 32, false); }
  } else if (big && vec4) {
    // the Grams: 16-row K chunks halve the LDS, so more workgroups per CU cover each tile's
    // fixed load / store latency (the short K ranges of the Gram of L gain most); the Gram of
    // Q1 has no L view and leaves the row map out as well
    if (lperm) RNR_TN(128, false, false, true, 16, true); else RNR_TN(128, false, false, true, 16, false);
  } else {
    if (big) { if (vec4) RNR_TN(128, false, false, true, 32, true); else RNR_TN(128, false, false, false, 32, true); }
    else     { if (vec4) RNR_TN(64, false, false, true, 32, true);  else RNR_TN(64, false, false, false, 32, true); }
  }
#undef RNR_TN
  return hip_status();
}

// W[k][c] = R[k][c] Dinv_c for the 64-block pairs k < c (the solve's off-diagonal operand)
int launch_wblocks(const float* R, int64_t sr, const float* Dinv, float* Wm, int64_t batch, int n,
                   hipStream_t st) {
  const int nblk = (n + 63) / 64;
  if (nblk < 2) return RNR_OK;
  WblkArgs a;
  a.R = R; a.sr = sr; a.Dinv = Dinv; a.Wm = Wm; a.sw = (int64_t)n * n; a.n = n;
  a.ncol = nblk - 1;
  a.vec4 = (n % 4 == 0) && (sr % 4 == 0) && aligned(R, 16);
  const int64_t total = batch * a.ncol;
  if (total > INT32_MAX) return RNR_ERR_INVALID_ARG;
  a.total = (int)total;
  a.lpt = (total % 8 == 0 && (total / 8) % a.ncol == 0) ? 1 : 0;
  k_wblocks<<<dim3((unsigned)total), dim3(256), 0, st>>>(a);
  return hip_status();
}

// Wm non-null: the one-workgroup-per-matrix Cholesky also forms the solve's W blocks there
// (the split form leaves them to k_wblocks).
int launch_chol(float* G, int64_t sg, float* Dinv, int* info, int64_t batch, int n, bool keep_info,
                float* Wm, hipStream_t st) {
  CholArgs a;
  a.G = G; a.sg = sg; a.Dinv = Dinv; a.info = info; a.n = n;
  a.keep_info = keep_info ? 1 : 0;
  a.Wm = Wm; a.sw = (int64_t)n * n;
  if (chol_split(batch, n)) {
    // small batch: the first diagonal block, then per 64-column block the block row (one wave
    // per 32 columns) and one launch that runs the trailing tiles (one wave per tile) beside the
    // next diagonal block's update and factor (one workgroup per matrix)
    CholSplitArgs c{G, sg, Dinv, info, n, 0, a.keep_info, 0, (int)batch};
    k_chol_jitter<<<dim3((unsigned)batch), dim3(kCholThreads), 0, st>>>(c);
    k_chol_diag<<<dim3((unsigned)batch), dim3(64), 0, st>>>(c);
    for (int k0 = 0; k0 < n; k0 += kCholNb) {
      const int w = n - k0 - kCholNb;
      if (w <= 0) break;
      c.k0 = k0;
      c.njob = (w + 127) / 128;
      k_chol_row<<<dim3((unsigned)(batch * c.njob)), dim3(kCholSplitThreads), 0, st>>>(c);
      const int nt = (w + 63) / 64;
      c.njob = (nt * (nt + 1) / 2 - 1 + 3) / 4;  // tile pairs 1 .. npairs - 1
      k_chol_step<<<dim3((unsigned)(batch * (1 + c.njob))), dim3(kCholSplitThreads), 0, st>>>(c);
    }
  } else {
    a.strip_lds = chol_lds_bytes(n, true) <= kLdsMax ? 1 : 0;
    const size_t lds = chol_lds_bytes(n, a.strip_lds != 0);
    if (n <= 256) {  // half the waves: the other half would mostly idle
      if (int e = set_lds(k_chol<256>, lds)) return e;
      k_chol<256><<<dim3((unsigned)batch), dim3(256), lds, st>>>(a);
    } else {
      if (int e = set_lds(k_chol<>, lds)) return e;
      k_chol<><<<dim3((unsigned)batch), dim3(kCholThreads), lds, st>>>(a);
    }
  }
  return hip_status();
}

int launch_trsm(const float* M, int64_t sm, const int* mperm, const float* Wm, int64_t sw,
                const float* Dinv, float* Q, int64_t sq, float* Q2, int64_t sq2, const int* perm,
                int64_t batch, int n, hipStream_t st) {
  TrsmArgs a;
  a.M = M; a.sm = sm; a.Wm = Wm; a.sw = sw; a.Dinv = Dinv; a.Q = Q; a.sq = sq; a.Q2 = Q2; a.sq2 = sq2;
  // 64-row blocks when 128-row ones would give fewer than two workgroups per CU (small batches
  // at large n): twice the workgroups for the same work
  const bool half = batch * ((n + kTrsmRows - 1) / kTrsmRows) < 512;
  const int rb = half ? 64 : kTrsmRows;
  a.perm = perm; a.mperm = mperm; a.n = n; a.nrb = (n + rb - 1) / rb;
  const int64_t total = batch * a.nrb;
  if (total > INT32_MAX) return RNR_ERR_INVALID_ARG;
  a.total = (int)total;
  const bool vec4 = (n % 4 == 0) && (sq % 4 == 0) && (sm % 4 == 0) && aligned(Q, 16) && aligned(M, 16) &&
                    aligned(Wm, 16);
  const dim3 grid((unsigned)total), block(256);
  if (half) {  // and each block column's K split over two groups of waves
    if (vec4) k_trsm<true, 64, 2><<<grid, dim3(512), 0, st>>>(a);
    else k_trsm<false, 64, 2><<<grid, dim3(512), 0, st>>>(a);
  } else {
    if (vec4) k_trsm<true, kTrsmRows><<<grid, block, 0, st>>>(a);
    else k_trsm<false, kTrsmRows><<<grid, block, 0, st>>>(a);
  }
  return hip_status();
}

int check_ws(void* ws, size_t ws_bytes, size_t need) {
  if (need == 0) return RNR_OK;
  if (!ws || ws_bytes < need) return RNR_ERR_WORKSPACE;
  if (!aligned(ws, 256)) return RNR_ERR_MISALIGNED;
  return RNR_OK;
}

// Optional per-launch timing: events[i] is recorded on the stream before launch i of the
// sequence and events[last] after it (the hook behind rnr_qr_f32_timed).
struct Marks {
  void* const* ev;
  int n;
  int next;
  int mark(hipStream_t st) {
    if (!ev) return RNR_OK;
    if (next >= n) return RNR_ERR_INVALID_ARG;
    return hipEventRecord(static_cast<hipEvent_t>(ev[next++]), st) == hipSuccess ? RNR_OK : RNR_ERR_HIP;
  }
  // records every event not yet recorded (a path with fewer launches than stages)
  int rest(hipStream_t st) {
    while (ev && next < RNR_QR_TIMED_EVENTS)
      if (int e = mark(st)) return e;
    return RNR_OK;
  }
};

bool small_path(int64_t n) { return n <= kSmallMaxN; }

// One CholeskyQR pass: Q = M chol(M^T M + mu I)^-1, R left in G.  With lperm, M is the unit-
// lower L held in A's row order (the LU's in-place factor) and is read through lperm.
int cholqr_pass(const float* M, int64_t sm, const int* lperm, float* G, float* Dinv, float* Wm, int* info,
                bool keep_info, float* Q, float* Q2, const int* perm, int64_t batch, int n,
                hipStream_t st, Marks& mk) {
  const int64_t nn = (int64_t)n * n;
  if (int e = mk.mark(st)) return e;
  if (int e = launch_tn(false, M, sm, M, sm, G, nn, nullptr, lperm, batch, n, lperm != nullptr, st))
    return e;
  if (int e = mk.mark(st)) return e;
  const bool w_in_chol = !chol_split(batch, n);  // the fused Cholesky forms W itself
  if (int e = launch_chol(G, nn, Dinv, info, batch, n, keep_info, w_in_chol ? Wm : nullptr, st)) return e;
  if (int e = mk.mark(st)) return e;
  if (!w_in_chol)
    if (int e = launch_wblocks(G, nn, Dinv, Wm, batch, n, st)) return e;
  if (int e = mk.mark(st)) return e;
  return launch_trsm(M, sm, lperm, Wm, nn, Dinv, Q, nn, Q2, nn, perm, batch, n, st);
}

// The frame: LU of A in place into ws.W (+ ws.perm), CholeskyQR2 of L read through perm,
// Q = P Q2 -> Q (and Qcopy).  Q1 goes to ws.L.
int frame(const float* A, int64_t sa, const Ws& w, float* Q, float* Qcopy, int* info, int64_t batch,
          int n, hipStream_t st, Marks& mk) {
  const int64_t nn = (int64_t)n * n;
  if (int e = mk.mark(st)) return e;
  if (int e = launch_lu(true, A, sa, w.W, nn, batch, n, w.perm, nullptr, nullptr, nullptr, w.Dinv, st))
    return e;
  // W (the solve's off-diagonal operand) lives in Qb for the first pass and in the then
  // dead LU buffer for the second
  if (int e = cholqr_pass(w.W, nn, w.perm, w.G, w.Dinv, w.Qb, info, false, w.L, nullptr, nullptr, batch, n,
                          st, mk))
    return e;
  return cholqr_pass(w.L, nn, nullptr, w.G, w.Dinv, w.W, info, true, Q, Qcopy, w.perm, batch, n, st, mk);
}

// The whole path (see the launch list at the top of this file).
int qr_path(const float* A, int64_t batch, int64_t n, int64_t batch_stride, float* H, float* tau,
            int32_t* info, void* ws, size_t ws_bytes, hipStream_t st, Marks& mk) {
  if (int e = check_common(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!A || !H || !tau || batch_stride < n * n) return RNR_ERR_INVALID_ARG;
  if (!aligned(A, 4) || !aligned(H, 4) || !aligned(tau, 4)) return RNR_ERR_MISALIGNED;
  if (small_path(n)) {
    if (batch > INT32_MAX) return RNR_ERR_INVALID_ARG;
    SmallArgs sa;
    sa.A = A; sa.sa = batch_stride; sa.H = H; sa.tau = tau; sa.info = info;
    sa.n = (int)n; sa.batch = (int)batch;
    sa.vec4 = (n % 4 == 0) && (batch_stride % 4 == 0) && aligned(A, 16) && aligned(H, 16);
    if (int e = mk.mark(st)) return e;
    if (launch_small(sa, st)) return RNR_ERR_HIP;
    return mk.rest(st);
  }
  const size_t need = carve(batch, n, kQrNeed, nullptr, nullptr);
  if (int e = check_ws(ws, ws_bytes, need)) return e;
  Ws w;
  carve(batch, n, kQrNeed, static_cast<char*>(ws), &w);
  const int ni = (int)n;
  const int64_t nn = n * n;
  int* inf = info ? info : w.info;
  if (int e = frame(A, batch_stride, w, w.Qb, nullptr, inf, batch, ni, st, mk)) return e;
  if (int e = mk.mark(st)) return e;
  // the chart's first panel step reads Q from Qb, everything after works in H (the entries of
  // H it never writes, its U12 blocks, lie above the diagonal, which the closure overwrites)
  if (int e = launch_lu(false, w.Qb, nn, H, nn, batch, ni, nullptr, nullptr, w.s, tau, w.Dinv, st)) return e;
  if (int e = mk.mark(st)) return e;
  if (int e = launch_tn(true, w.Qb, nn, A, batch_stride, H, nn, w.s, nullptr, batch, ni, false, st))
    return e;
  return mk.mark(st);
}

// ---- scratch of the allocation-free entry point (rnr_qr_f32_noalloc) -----------------------
// One file-scope device array per GPU, held from the code object's load to the end of the
// process.  Host code never uses the array's name as an address (in host code it is only a
// stand-in for the symbol): the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and is kept per device.
static __device__ __align__(256) unsigned char scratch[RNR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch address on the stream's device (looked up on the first call there).
int scratch_on(hipStream_t st, void** out) {
  int dev = -1;
  if (hipStreamGetDevice(st, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RNR_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return RNR_ERR_HIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return RNR_ERR_HIP;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return RNR_ERR_HIP;
    if (e != hipSuccess || !p) return RNR_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return RNR_OK;
}

}  // namespace

extern "C" {

const char* rnr_status_string(int status) {
  switch (status) {
    case RNR_OK: return "success";
    case RNR_ERR_INVALID_ARG: return "invalid argument (null pointer, negative size or stride < n*n)";
    case RNR_ERR_UNSUPPORTED_N: return "unsupported matrix size (need 1 <= n <= 2048)";
    case RNR_ERR_WORKSPACE: return "workspace missing or smaller than the size query returned";
    case RNR_ERR_HIP: return "HIP launch or attribute call failed";
    case RNR_ERR_MISALIGNED: return "misaligned pointer (data: 4 bytes, workspace: 256 bytes)";
    case RNR_ERR_SCRATCH_LIMIT:
      return "the problem needs more scratch than rnr_qr_f32_noalloc holds (RNR_NOALLOC_SCRATCH_BYTES, "
             "128 MiB per GPU); use rnr_qr_f32 with a workspace, or a smaller batch";
    default: return "unknown status";
  }
}

const char* rnr_version(void) { return "0.1.0"; }

int rnr_qr_f32_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (int e = check_common(batch, n)) return e;
  *bytes = (batch == 0 || small_path(n)) ? 0 : carve(batch, n, kQrNeed, nullptr, nullptr);
  return RNR_OK;
}

int rnr_qr_f32(const float* A, int64_t batch, int64_t n, int64_t batch_stride, float* H, float* tau,
               int32_t* info, void* ws, size_t ws_bytes, rnr_stream_t stream) {
  Marks mk{nullptr, 0, 0};
  return qr_path(A, batch, n, batch_stride, H, tau, info, ws, ws_bytes,
                 reinterpret_cast<hipStream_t>(stream), mk);
}

int rnr_qr_f32_noalloc(const float* A, int64_t batch, int64_t n, int64_t batch_stride, float* H, float* tau,
                       int32_t* info, rnr_stream_t stream) {
  if (int e = check_common(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  const size_t need = small_path(n) ? 0 : carve(batch, n, kQrNeed, nullptr, nullptr);
  if (need > (size_t)RNR_NOALLOC_SCRATCH_BYTES) return RNR_ERR_SCRATCH_LIMIT;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (need > 0)
    if (int e = scratch_on(st, &ws)) return e;
  Marks mk{nullptr, 0, 0};
  return qr_path(A, batch, n, batch_stride, H, tau, info, ws, need, st, mk);
}

int rnr_qr_f32_timed(const float* A, int64_t batch, int64_t n, int64_t batch_stride, float* H,
                     float* tau, int32_t* info, void* ws, size_t ws_bytes, rnr_stream_t stream,
                     void* const* events, int n_events) {
  if (!events || n_events < RNR_QR_TIMED_EVENTS) return RNR_ERR_INVALID_ARG;
  for (int i = 0; i < RNR_QR_TIMED_EVENTS; ++i)
    if (!events[i]) return RNR_ERR_INVALID_ARG;
  Marks mk{events, n_events, 0};
  return qr_path(A, batch, n, batch_stride, H, tau, info, ws, ws_bytes,
                 reinterpret_cast<hipStream_t>(stream), mk);
}

int rnr_lu_f32_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (int e = check_common(batch, n)) return e;
  *bytes = batch == 0 ? 0 : carve(batch, n, kLuNeed, nullptr, nullptr);
  return RNR_OK;
}

int rnr_lu_f32(const float* A, int64_t batch, int64_t n, int64_t batch_stride, float* L, int32_t* perm,
               void* ws, size_t ws_bytes, rnr_stream_t stream) {
  if (int e = check_common(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!A || !L || !perm || batch_stride < n * n) return RNR_ERR_INVALID_ARG;
  if (!aligned(A, 4) || !aligned(L, 4) || !aligned(perm, 4)) return RNR_ERR_MISALIGNED;
  const size_t need = carve(batch, n, kLuNeed, nullptr, nullptr);
  if (int e = check_ws(ws, ws_bytes, need)) return e;
  Ws w;
  carve(batch, n, kLuNeed, static_cast<char*>(ws), &w);
  return launch_lu(true, A, batch_stride, w.W, n * n, batch, (int)n, perm, L, nullptr, nullptr, w.Dinv,
                   reinterpret_cast<hipStream_t>(stream));
}

int rnr_cholqr_f32_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (int e = check_common(batch, n)) return e;
  *bytes = batch == 0 ? 0 : carve(batch, n, kCholqrNeed, nullptr, nullptr);
  return RNR_OK;
}

int rnr_cholqr_f32(const float* M, int64_t batch, int64_t n, int64_t batch_stride, float* Q, float* R,
                   int32_t* info, void* ws, size_t ws_bytes, rnr_stream_t stream) {
  if (int e = check_common(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!M || !Q || batch_stride < n * n) return RNR_ERR_INVALID_ARG;
  if (!aligned(M, 4) || !aligned(Q, 4) || (R && !aligned(R, 4))) return RNR_ERR_MISALIGNED;
  const size_t need = carve(batch, n, kCholqrNeed, nullptr, nullptr);
  if (int e = check_ws(ws, ws_bytes, need)) return e;
  Ws w;
  carve(batch, n, kCholqrNeed, static_cast<char*>(ws), &w);
  float* G = R ? R : w.G;
  Marks mk{nullptr, 0, 0};
  return cholqr_pass(M, batch_stride, nullptr, G, w.Dinv, w.Qb, info ? info : w.info, false, Q, nullptr,
                     nullptr, batch, (int)n, reinterpret_cast<hipStream_t>(stream), mk);
}

int rnr_frame_f32_workspace(int64_t batch, int64_t n, size_t* bytes) {
  if (!bytes) return RNR_ERR_INVALID_ARG;
  if (int e = check_common(batch, n)) return e;
  *bytes = batch == 0 ? 0 : carve(batch, n, kFrameNeed, nullptr, nullptr);
  return RNR_OK;
}

int rnr_frame_f32(const float* A, int64_t batch, int64_t n, int64_t batch_stride, float* Q, int32_t* info,
                  void* ws, size_t ws_bytes, rnr_stream_t stream) {
  if (int e = check_common(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!A || !Q || batch_stride < n * n) return RNR_ERR_INVALID_ARG;
  if (!aligned(A, 4) || !aligned(Q, 4)) return RNR_ERR_MISALIGNED;
  const size_t need = carve(batch, n, kFrameNeed, nullptr, nullptr);
  if (int e = check_ws(ws, ws_bytes, need)) return e;
  Ws w;
  carve(batch, n, kFrameNeed, static_cast<char*>(ws), &w);
  Marks mk{nullptr, 0, 0};
  return frame(A, batch_stride, w, Q, nullptr, info ? info : w.info, batch, (int)n,
               reinterpret_cast<hipStream_t>(stream), mk);
}

int rnr_chart_f32(float* Y, int64_t batch, int64_t n, float* s, float* tau, rnr_stream_t stream) {
  if (int e = check_common(batch, n)) return e;
  if (batch == 0) return RNR_OK;
  if (!Y || !s || !tau) return RNR_ERR_INVALID_ARG;
  if (!aligned(Y, 4) || !aligned(s, 4) || !aligned(tau, 4)) return RNR_ERR_MISALIGNED;
  const int64_t nn = n * n;
  // no workspace here: the fused one-workgroup-per-matrix form at every batch size
  return launch_lu(false, Y, nn, Y, nn, batch, (int)n, nullptr, nullptr, s, tau, nullptr,
                   reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
