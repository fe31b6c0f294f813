// Local code refinement on gfx950: after GPTQ, sweep the columns again and move each
// code one level up or down when that lowers the row's Hessian error e Hs e^T.
//
// Reference: hi2/refine.py:43-106 (refine_expanded, the torch loop every device runs)
// and its op-by-op spec in hi2/refine_kernel.py:63-91.
//
// Work per row, with e = fp16(lo + c st) - w and g = e Hs:
//   * the residual e (elementwise) and g = e Hs, one fp32 MFMA GEMM of rank K whose every
//     element is the sequential FMA chain over k;
//   * per sweep and 128-column block [b0, b1): the column loop (refine_block_kernel),
//     then g += dw Hs[b0:b1, :] over all K columns (the GPTQ cross-block GEMM with the
//     block's changes negated: g - ((-dw) Hs) is g + (dw Hs) exactly, since negation is
//     exact and round-to-nearest-even is symmetric);
//   * the reference stops after a sweep that moves no code.  Here each sweep adds its
//     moves to a device counter and every launch of the next sweep reads the previous
//     counter and returns at once when it is zero, so no host synchronisation is needed:
//     a sweep after one that moved nothing would repeat the same decisions.
#include <stdio.h>

#include <utility>

#include "common.h"
#include "mfma_gemm.h"

namespace hi2x {
namespace {

constexpr int LMAX = 128;
constexpr int QL = 16;                // lanes per row
constexpr int CPL = LMAX / QL;        // columns per lane
constexpr int RPW = 64 / QL;          // rows per wave
constexpr int WPG = 4;                // waves per workgroup
constexpr int RPG = RPW * WPG;        // rows per workgroup
constexpr int USTR = QL * CPL + 4;    // LDS row stride of the Hessian block (floats)

// Start of lane q's 8 columns in an LDS row: lanes 8..15 are shifted by 4 floats so that
// the 16 lanes' 16-byte reads fall on distinct banks.
__device__ __forceinline__ int lane_off(int q) { return q * CPL + ((q >> 3) << 2); }

template <int S>
// Lane S of each 16-lane row.  Every source lane is valid, so the old value and bound_ctrl
// never apply; written as update_dpp with bound_ctrl so that the compiler folds the
// broadcast into the instruction that uses it (it does not fold a plain DPP move).
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x150 + S, 0xf, 0xf, true));
}

// ---------------------------------------------------------------------------------
// e[r, j] = fp16(lo[r, j / B_r] + c[r, j] st[r, j / B_r]) - w[r, j]   (hi2/refine.py:73)
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void refine_residual_kernel(
    const float* __restrict__ w, const uint8_t* __restrict__ codes, int64_t N, int64_t K,
    const float* __restrict__ lo, const float* __restrict__ st, int64_t ldp,
    const int32_t* __restrict__ block, float* __restrict__ e) {
  // workgroup (x, y): 1024 columns of rows y, y + gridDim.y, ...
  const int64_t j0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  for (int64_t r = blockIdx.y; r < N; r += gridDim.y) {
    const int B = block[r] > 0 ? block[r] : 1;
    const float* lr = lo + r * ldp;
    const float* sr = st + r * ldp;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t j = j0 + 256 * t;
      if (j < K) {
        int64_t b = (int)j / B;
        b = b < ldp ? b : ldp - 1;
        const int64_t i = r * K + j;
        e[i] = f16_round(lr[b] + (float)codes[i] * sr[b]) - w[i];
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// g = e Hs on fp32 MFMA (128 x 128 tiles, rank K from zero in k order: every element is
// the sequential fp32 FMA chain, the rounding of the reference's BLAS product at the
// shapes its tests use).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void refine_gradient_kernel(
    const float* __restrict__ e, const float* __restrict__ hs, float* __restrict__ g,
    int64_t N, int64_t K, int64_t tn, int64_t ntiles) {
  __shared__ MgSmem sm;
  const int64_t tile = xcd_tile(blockIdx.x, ntiles);
  if (tile < 0) return;
  const int64_t r0 = (tile / tn) * MG_T, c0 = (tile % tn) * MG_T;
  RowsLoader<NoMask> al{e, K, N, K, NoMask{}};
  ColsLoader<NoMask> bl{hs, K, K, K, NoMask{}};
  f32x16 acc[2][2];
  mg_zero(acc);
  mg_mainloop(acc, sm, al, bl, r0, c0, 0, K);
  const CTile<> ct(g, K, N, K, r0, c0);
  ct.store(acc, [](int, int, int) { return true; });
}

// ---------------------------------------------------------------------------------
// Column loop of one block (hi2/refine.py:79-98; kernel spec hi2/refine_kernel.py:63-91).
//
// The layout is the GPTQ block kernel's: a row is owned by 16 lanes (a DPP row), lane q
// holds the row's columns c = 16m + q (m = 0..7) of the block in registers (g, code,
// ladder, Hessian diagonal), and Hs[b0:b0+L, b0:b0+L] sits in LDS so that lane q reads
// its 8 columns of a row as two 16-byte vectors; the row of step i+1 is read during
// step i.
//
// Step i (fully unrolled): every lane evaluates the two candidate moves of its own column
// m = i/16 with the reference's arithmetic (every product and sum rounded separately,
// fp16 rounding to nearest even); only lane q = i%16 owns column i.  Its change dw
// (0 when no move is taken) goes to the row's other lanes by DPP row_newbcast, and the
// row applies g[c] += dw * Hs[i][c] to the columns it holds (columns <= i are dead).
// Gains are compared as torch's max over the stacked pair (+1, -1): a NaN propagates and
// is never taken, and ties keep +1.  A wave whose rows keep every gain finite over the
// block (refine_bounded and the workgroup's test of the Hessian block) runs the loop with
// the plain max of the pair and the off-ladder moves folded into their terms (gain
// -inf), four operations fewer on each step's dependent chain; any other wave runs it
// with the NaN-aware comparison.  The owner's new code and dw stay in registers
// (pinned selects, no branch) and are written after the loop: the code in place, dw (or
// -dw with NEG) to dw[r, i].  Moves are counted into *moved (when not null).
// ---------------------------------------------------------------------------------
struct RefRegs {
  float g[CPL], cc[CPL], loc[CPL], stc[CPL], hd[CPL], dw[CPL];
  // per column, from its code before the block's sweep (a column's code changes only at
  // its own step): the changes of the two moves, their gain terms 2 dw and dw^2 Hs[j][j],
  // and whether each move stays on the ladder
  float dwp[CPL], dwm[CPL], ap[CPL], bp[CPL], am[CPL], bm[CPL];
  bool okp[CPL], okm[CPL];
  int nmv;
};

// The parts of a column's two candidate moves that do not depend on its gradient, with
// the step's operations in its order (each product and sum rounded separately).
__device__ __forceinline__ void refine_prepare(RefRegs& R, float tp) {
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const float cj = R.cc[m], lo_j = R.loc[m], st_j = R.stc[m], hd = R.hd[m];
    const float now = f16_round(lo_j + cj * st_j);
    const float cp = cj + 1.0f, cm = cj + -1.0f;
    const float dwp = f16_round(lo_j + cp * st_j) - now;
    const float dwm = f16_round(lo_j + cm * st_j) - now;
    R.okp[m] = (cp >= 0.0f) & (cp <= tp) & (st_j > 0.0f);
    R.okm[m] = (cm >= 0.0f) & (cm <= tp) & (st_j > 0.0f);
    R.dwp[m] = dwp;
    R.dwm[m] = dwm;
    R.ap[m] = 2.0f * dwp;
    R.bp[m] = (dwp * dwp) * hd;
    R.am[m] = 2.0f * dwm;
    R.bm[m] = (dwm * dwm) * hd;
  }
}

template <int I, bool FULL, bool EXACT>
__device__ __forceinline__ void refine_step(RefRegs& R, int L, int q, float tp,
                                            const float* __restrict__ shq, f32x4 (&hb)[2][2]) {
  constexpr int m = I / QL, s = I % QL, cur = I & 1;
  if (!FULL && I >= L) return;
  if (I + 1 < LMAX) {
    hb[cur ^ 1][0] = *reinterpret_cast<const f32x4*>(shq + (I + 1) * USTR);
    hb[cur ^ 1][1] = *reinterpret_cast<const f32x4*>(shq + (I + 1) * USTR + 4);
  }
  // gain of a move: -(2 dw g_j + dw^2 Hs[j][j]) (the gradient-free terms prepared)
  const float gj = R.g[m], cj = R.cc[m];
  bool pick_m, take;
  if constexpr (EXACT) {
    const float gp = R.okp[m] ? -(R.ap[m] * gj + R.bp[m]) : -__builtin_inff();
    const float gm = R.okm[m] ? -(R.am[m] * gj + R.bm[m]) : -__builtin_inff();
    pick_m = (gp == gp) & ((gm != gm) | (gm > gp));
    const float best = pick_m ? gm : gp;
    take = best > 0.0f;  // false for NaN
  } else {
    // every gain is finite, or -inf for a move off the ladder (its terms were set to 0
    // and +inf), so torch's max of the pair is the plain one (ties keep +1)
    const float gp = -(R.ap[m] * gj + R.bp[m]);
    const float gm = -(R.am[m] * gj + R.bm[m]);
    pick_m = gm > gp;
    take = __builtin_fmaxf(gp, gm) > 0.0f;
  }
  const float dw = take ? (pick_m ? R.dwm[m] : R.dwp[m]) : 0.0f;
  const float cn = take ? (pick_m ? cj + -1.0f : cj + 1.0f) : cj;
  const float db = row_bcast<s>(dw);
  const bool own = q == s;
  R.cc[m] = own ? cn : R.cc[m];
  R.dw[m] = own ? dw : R.dw[m];
  R.nmv += (own & take) ? 1 : 0;
  asm volatile("" : "+v"(R.cc[m]), "+v"(R.dw[m]));
#pragma unroll
  for (int mm = (I + 1) / QL; mm < CPL; ++mm) R.g[mm] = R.g[mm] + db * hb[cur][mm >> 2][mm & 3];
}

template <bool FULL, bool EXACT, int... Is>
__device__ __forceinline__ void refine_steps(std::integer_sequence<int, Is...>, RefRegs& R,
                                             int L, int q, float tp,
                                             const float* __restrict__ shq, f32x4 (&hb)[2][2]) {
  (refine_step<Is, FULL, EXACT>(R, L, q, tp, shq, hb), ...);
}

// Whether this lane's columns keep every gain of the block finite: with |g| <= 2^60,
// |dw| <= 2^30 for both moves and every element of the block's Hessian within 2^30 (the
// workgroup's test), a step changes g by at most 2^60, so |g| stays below 2^68 over the
// block's 128 steps, |2 dw g| below 2^99 and dw^2 Hs[j][j] below 2^90: no overflow, no
// NaN.  NaN and infinities fail the comparisons.
__device__ __forceinline__ bool refine_bounded(const RefRegs& R) {
  bool ok = true;
#pragma unroll
  for (int m = 0; m < CPL; ++m)
    ok = ok && __builtin_fabsf(R.g[m]) <= 0x1p60f && __builtin_fabsf(R.dwp[m]) <= 0x1p30f &&
         __builtin_fabsf(R.dwm[m]) <= 0x1p30f;
  return ok;
}

template <bool FULL, bool NEG>
__global__ __launch_bounds__(RPG * QL) void refine_block_kernel(
    const float* __restrict__ g, int64_t ldg, int64_t N, int64_t K, int64_t b0, int L,
    uint8_t* __restrict__ codes, const float* __restrict__ lo, const float* __restrict__ st,
    int64_t ldp, const int32_t* __restrict__ block, const float* __restrict__ top,
    const float* __restrict__ hs, float* __restrict__ dwo, int64_t ldw,
    unsigned long long* __restrict__ moved, const unsigned long long* __restrict__ prev) {
  if (prev != nullptr && *prev == 0ull) return;  // the previous sweep moved nothing
  __shared__ float sh[LMAX * USTR];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int q = lane & (QL - 1);
  const int64_t rbase = (int64_t)blockIdx.x * RPG;
  const int lr = wave * RPW + lane / QL;  // row within the workgroup
  const int64_t r = rbase + lr;
  const bool live = r < N;
  const int nrows = (int)(((rbase + RPG < N) ? rbase + RPG : N) - rbase);

  bool hwide = false;  // an element of the Hessian block beyond 2^30 (or not finite)
  {
    // Hs[b0:b0+L, b0:b0+L]: rows >= L read zero, columns >= L are zeroed here
    const __amdgpu_buffer_rsrc_t hr = mg_rsrc(hs + b0 * K + b0, (int64_t)(L - 1) * K + L);
    constexpr int NV = LMAX * LMAX / 4 / (RPG * QL);  // 16-byte vectors per thread
    f32x4 hv[NV];
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int idx = tid + RPG * QL * t, i = idx / (LMAX / 4), c = 4 * (idx % (LMAX / 4));
      const uint32_t off = i < L ? (uint32_t)(((int64_t)i * K + c) * 4) : MG_OOB;
      hv[t] = mg_load4(hr, off);
    }
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int idx = tid + RPG * QL * t, i = idx / (LMAX / 4), c = 4 * (idx % (LMAX / 4));
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int cc = c + x;
        const float h = (cc < L) ? hv[t][x] : 0.0f;
        sh[i * USTR + lane_off(cc % QL) + cc / QL] = h;
        hwide = hwide || !(__builtin_fabsf(h) <= 0x1p30f);
      }
    }
  }

  RefRegs R;
  R.nmv = 0;
  const float tp = live ? top[r] : 0.0f;
  {
    // this row's columns c = 16m + q: g, code and ladder block (dead rows and columns
    // read zero through the buffer ranges)
    const __amdgpu_buffer_rsrc_t grs = mg_rsrc(g + rbase * ldg, (int64_t)(nrows - 1) * ldg + L);
    const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
        codes + rbase * K + b0, (short)0, (int)((int64_t)(nrows - 1) * K + L), 0x00020000);
    const int B = live ? (block[r] > 0 ? block[r] : 1) : 1;
    int bix[CPL];
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int c = QL * m + q;
      const uint32_t go = c < L ? (uint32_t)(((int64_t)lr * ldg + c) * 4) : MG_OOB;
      const uint32_t co = c < L ? (uint32_t)((int64_t)lr * K + c) : MG_OOB;
      R.g[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(grs, (int)go, 0, 0));
      R.cc[m] = (float)__builtin_amdgcn_raw_buffer_load_b8(crs, (int)co, 0, 0);
      const uint32_t b = (uint32_t)(b0 + c) / (uint32_t)B;  // columns stay below 2^31
      bix[m] = (int)((int64_t)b < ldp ? (int64_t)b : ldp - 1);
    }
    const __amdgpu_buffer_rsrc_t lrs = mg_rsrc(lo + rbase * ldp, (int64_t)nrows * ldp);
    const __amdgpu_buffer_rsrc_t srs = mg_rsrc(st + rbase * ldp, (int64_t)nrows * ldp);
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const uint32_t po = (uint32_t)(((int64_t)lr * ldp + bix[m]) * 4);
      R.loc[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lrs, (int)po, 0, 0));
      R.stc[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srs, (int)po, 0, 0));
      R.dw[m] = 0.0f;
    }
  }
  hwide = __syncthreads_or(hwide);  // the Hessian block is in LDS
#pragma unroll
  for (int m = 0; m < CPL; ++m) R.hd[m] = sh[(QL * m + q) * USTR + lane_off(q) + m];

  refine_prepare(R, tp);
  const float* shq = sh + lane_off(q);
  f32x4 hb[2][2];
  hb[0][0] = *reinterpret_cast<const f32x4*>(shq);
  hb[0][1] = *reinterpret_cast<const f32x4*>(shq + 4);
  if (!hwide && __builtin_amdgcn_ballot_w64(!refine_bounded(R)) == 0) {
    // a move off the ladder gets the terms 0 and +inf: its gain is -inf for finite g
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      R.ap[m] = R.okp[m] ? R.ap[m] : 0.0f;
      R.bp[m] = R.okp[m] ? R.bp[m] : __builtin_inff();
      R.am[m] = R.okm[m] ? R.am[m] : 0.0f;
      R.bm[m] = R.okm[m] ? R.bm[m] : __builtin_inff();
    }
    refine_steps<FULL, false>(std::make_integer_sequence<int, LMAX>{}, R, L, q, tp, shq, hb);
  } else {
    refine_steps<FULL, true>(std::make_integer_sequence<int, LMAX>{}, R, L, q, tp, shq, hb);
  }

  if (live) {
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int c = QL * m + q;
      if (c < L) {
        codes[r * K + b0 + c] = (uint8_t)R.cc[m];
        dwo[r * ldw + c] = NEG ? -R.dw[m] : R.dw[m];
      }
    }
  }
  if (moved != nullptr) {
    int n = R.nmv;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) n += __shfl_xor(n, o, 64);
    if (lane == 0 && n != 0) atomicAdd(moved, (unsigned long long)n);
  }
}

__global__ void refine_init_kernel(int32_t* __restrict__ zeros, int64_t n,
                                   int64_t* __restrict__ u_ptr, const float* hs,
                                   unsigned long long* __restrict__ moved, int passes) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) zeros[i] = 0;
  if (i == 0) u_ptr[0] = (int64_t)(uintptr_t)hs;
  if (i < passes) moved[i] = 0ull;
}

int launch_residual(const float* w, const uint8_t* codes, int64_t n, int64_t k, const float* lo,
                    const float* st, int64_t ldp, const int32_t* block, float* e, hipStream_t s) {
  const dim3 grid((unsigned)((k + 1023) / 1024), (unsigned)(n < 65535 ? n : 65535));
  hipLaunchKernelGGL(refine_residual_kernel, grid, dim3(256), 0, s, w, codes, n, k, lo, st, ldp,
                     block, e);
  return launch_status("refine_residual_kernel");
}

int launch_gradient(const float* e, const float* hs, float* g, int64_t n, int64_t k,
                    hipStream_t s) {
  const int64_t tn = (k + MG_T - 1) / MG_T, tm = (n + MG_T - 1) / MG_T;
  const int64_t ntiles = tn * tm;
  LaunchTimer timer(HI2X_TIME_REFINE_GEMM, 2.0 * n * k * k, s);
  hipLaunchKernelGGL(refine_gradient_kernel, dim3((unsigned)((ntiles + 7) / 8 * 8)), dim3(256),
                     0, s, e, hs, g, n, k, tn, ntiles);
  return launch_status("refine_gradient_kernel");
}

int launch_block(const float* g, int64_t ldg, int64_t n, int64_t k, int64_t b0, int64_t len,
                 uint8_t* codes, const float* lo, const float* st, int64_t ldp,
                 const int32_t* block, const float* top, const float* hs, float* dw, int64_t ldw,
                 bool neg, unsigned long long* moved, const unsigned long long* prev,
                 hipStream_t s) {
  const dim3 grid((unsigned)((n + RPG - 1) / RPG));
  LaunchTimer timer(HI2X_TIME_REFINE_BLOCK, (double)n * len, s);
#define HI2X_REFINE_LAUNCH(F, NG)                                                          \
  hipLaunchKernelGGL((refine_block_kernel<F, NG>), grid, dim3(RPG * QL), 0, s, g, ldg, n, k, \
                     b0, (int)len, codes, lo, st, ldp, block, top, hs, dw, ldw, moved, prev)
  const bool full = len == LMAX;
  if (neg) {
    if (full) HI2X_REFINE_LAUNCH(true, true);
    else HI2X_REFINE_LAUNCH(false, true);
  } else {
    if (full) HI2X_REFINE_LAUNCH(true, false);
    else HI2X_REFINE_LAUNCH(false, false);
  }
#undef HI2X_REFINE_LAUNCH
  return launch_status("refine_block_kernel");
}

constexpr int64_t SB = 4;  // blocks per super-block of the sweep's update schedule

// Workspace layout of hi2x_refine_run (each part 256-byte aligned).
struct RefineWs {
  size_t e, g, dw, zeros, uptr, moved, total;
};
RefineWs refine_ws(int64_t n, int64_t k, int64_t passes) {
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  RefineWs w;
  w.e = 0;
  w.g = up(w.e + (size_t)n * k * 4);
  w.dw = up(w.g + (size_t)n * k * 4);
  w.zeros = up(w.dw + (size_t)n * SB * LMAX * 4);
  w.uptr = up(w.zeros + (size_t)n * 4);
  w.moved = up(w.uptr + 8);
  w.total = up(w.moved + (size_t)(passes > 0 ? passes : 1) * 8);
  return w;
}

bool ladder_args_ok(int64_t n, int64_t k, int64_t ldp) { return n >= 0 && k > 0 && ldp > 0; }

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int64_t hi2x_refine_workspace_bytes(int64_t n, int64_t k, int64_t passes) {
  if (n < 0 || k <= 0 || passes < 0) return -1;
  return (int64_t)refine_ws(n, k, passes).total;
}

extern "C" int hi2x_refine_gradient(const float* w, const uint8_t* codes, int64_t n, int64_t k,
                                    const float* lo, const float* st, int64_t ldp,
                                    const int32_t* block, const float* hs, float* e, float* g,
                                    void* stream) {
  clear_error();
  HI2X_REQUIRE(ladder_args_ok(n, k, ldp), "refine_gradient: bad shape n=%lld k=%lld ldp=%lld",
               (long long)n, (long long)k, (long long)ldp);
  if (n == 0) return HI2X_OK;
  HI2X_REQUIRE(w && codes && lo && st && block && hs && e, "refine_gradient: null buffer");
  hipStream_t s = as_stream(stream);
  int rc = launch_residual(w, codes, n, k, lo, st, ldp, block, e, s);
  if (rc || g == nullptr) return rc;
  return launch_gradient(e, hs, g, n, k, s);
}

extern "C" int hi2x_refine_block(const float* g, int64_t ldg, int64_t n, int64_t k, int64_t b0,
                                 int64_t len, uint8_t* codes, const float* lo, const float* st,
                                 int64_t ldp, const int32_t* block, const float* top,
                                 const float* hs, float* dw, int64_t ldw,
                                 unsigned long long* moved, void* stream) {
  clear_error();
  HI2X_REQUIRE(ladder_args_ok(n, k, ldp), "refine_block: bad shape n=%lld k=%lld ldp=%lld",
               (long long)n, (long long)k, (long long)ldp);
  HI2X_REQUIRE(len > 0 && len <= LMAX && b0 >= 0 && b0 + len <= k,
               "refine_block: block [%lld, +%lld) outside K=%lld", (long long)b0,
               (long long)len, (long long)k);
  HI2X_REQUIRE(ldg >= len && ldw >= len, "refine_block: ldg/ldw < len");
  if (n == 0) return HI2X_OK;
  HI2X_REQUIRE(g && codes && lo && st && block && top && hs && dw, "refine_block: null buffer");
  return launch_block(g, ldg, n, k, b0, len, codes, lo, st, ldp, block, top, hs, dw, ldw, false,
                      moved, nullptr, as_stream(stream));
}

extern "C" int hi2x_refine_run(const float* w, uint8_t* codes, int64_t n, int64_t k,
                               const float* lo, const float* st, int64_t ldp,
                               const int32_t* block, const float* top, const float* hs,
                               int64_t passes, unsigned long long* moved, void* ws,
                               int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(ladder_args_ok(n, k, ldp), "refine_run: bad shape n=%lld k=%lld ldp=%lld",
               (long long)n, (long long)k, (long long)ldp);
  HI2X_REQUIRE(passes >= 0 && passes <= 1000000, "refine_run: passes=%lld", (long long)passes);
  if (n == 0 || passes == 0) return HI2X_OK;
  HI2X_REQUIRE(w && codes && lo && st && block && top && hs, "refine_run: null buffer");
  hipStream_t s = as_stream(stream);
  const RefineWs L = refine_ws(n, k, passes);
  Workspace wsp;
  int rc = take_workspace(wsp, ws, ws_bytes, L.total, s, "refine_run");
  if (rc) return rc;
  float* e = reinterpret_cast<float*>(wsp.p + L.e);
  float* g = reinterpret_cast<float*>(wsp.p + L.g);
  int32_t* zeros = reinterpret_cast<int32_t*>(wsp.p + L.zeros);
  int64_t* uptr = reinterpret_cast<int64_t*>(wsp.p + L.uptr);
  unsigned long long* cnt = moved ? moved : reinterpret_cast<unsigned long long*>(wsp.p + L.moved);
  {
    const int64_t m = n > passes ? n : passes;
    hipLaunchKernelGGL(refine_init_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s,
                       zeros, n, uptr, hs, cnt, (int)passes);
    if ((rc = launch_status("refine_init_kernel"))) return rc;
  }
  if ((rc = launch_residual(w, codes, n, k, lo, st, ldp, block, e, s))) return rc;
  if ((rc = launch_gradient(e, hs, g, n, k, s))) return rc;
  // The sweep in super-blocks of SB blocks.  Every block's product P_b = dw_b Hs[b, :]
  // must reach every column of g that is read later, added in block order.  After block b
  // the columns of the super-block's later blocks get P_b at once (near update); the other
  // columns get the super-block's products at its end, each tile held in registers while
  // the SB products stream through (far update): the columns ahead before the next
  // super-block runs, and the columns behind (with the super-block's own, which still lack
  // the products of their own and later blocks) only when another sweep will read them.
  float* ndw = reinterpret_cast<float*>(wsp.p + L.dw);  // -dw of the super-block's blocks
  const int64_t lde = SB * LMAX;
  const int64_t nblocks = (k + LMAX - 1) / LMAX;
  for (int64_t p = 0; p < passes; ++p) {
    const unsigned long long* prev = p > 0 ? cnt + p - 1 : nullptr;
    const bool last = p + 1 == passes;
    for (int64_t s0 = 0; s0 < nblocks; s0 += SB) {
      const int64_t s1 = (s0 + SB < nblocks) ? s0 + SB : nblocks;
      const int64_t cs0 = s0 * LMAX, cs1 = (s1 * LMAX < k) ? s1 * LMAX : k;
      for (int64_t b = s0; b < s1; ++b) {
        const int64_t b0 = b * LMAX, len = (k - b0 < LMAX) ? k - b0 : LMAX;
        float* db = ndw + (b - s0) * LMAX;
        rc = launch_block(g + b0, k, n, k, b0, len, codes, lo, st, ldp, block, top, hs, db, lde,
                          true, cnt + p, prev, s);
        if (rc) return rc;
        // g - ((-dw) Hs) = g + dw Hs: the near columns of this super-block
        rc = trailing_update(g, n, k, b0, 1, db, lde, b0 + len, cs1, zeros, uptr, s, cnt + p,
                             HI2X_TIME_REFINE_GEMM);
        if (rc) return rc;
      }
      rc = trailing_update(g, n, k, cs0, (int)(s1 - s0), ndw, lde, cs1, k, zeros, uptr, s,
                           cnt + p, HI2X_TIME_REFINE_GEMM);
      if (rc) return rc;
      if (last) continue;  // columns behind are read only by a later sweep
      rc = trailing_update(g, n, k, cs0, (int)(s1 - s0), ndw, lde, 0, cs0, zeros, uptr, s,
                           cnt + p, HI2X_TIME_REFINE_GEMM);
      if (rc) return rc;
      for (int64_t b = s0; b < s1; ++b) {  // block b's own columns: products of blocks >= b
        const int64_t b0 = b * LMAX, b1 = (b0 + LMAX < k) ? b0 + LMAX : k;
        rc = trailing_update(g, n, k, b0, (int)(s1 - b), ndw + (b - s0) * LMAX, lde, b0, b1,
                             zeros, uptr, s, cnt + p, HI2X_TIME_REFINE_GEMM);
        if (rc) return rc;
      }
    }
  }
  return HI2X_OK;
}
