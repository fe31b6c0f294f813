// GPTQ column loop on gfx950: the intra-block rounding kernel, the cross-block
// (trailing) update on fp32 MFMA, and the block schedule that drives them.
//
// Reference: hi2/hessian.py:235-315 (_round_reference / _round_kernel) and the op-by-op
// rounding spec of hi2/gptq_kernel.py:82-100.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <utility>

#include <algorithm>

#include "common.h"
#include "mfma_gemm.h"

namespace hi2x {
namespace {

// Intra-block kernel.
//
// One row is owned by 16 lanes (a DPP row: 4 rows per wave, 16 per workgroup).  Lane q
// holds the row's columns c = 16m + q (m = 0..7) of the 128-column block in registers,
// with the decoded (lo, step) of each column's ladder block.  The factor block
// U[i1:i1+128, i1:i1+128] of the row's group sits in LDS, laid out so that lane q reads
// its 8 columns of a U row as two 16-byte vectors (U[i1+i][i1+16m+q], m = 0..7, from
// lane_off(q)).  The U row of step i+1 is read during step i.
//
// Step i (fully unrolled): every lane runs the rounding chain on its own column m=i/16
// (the two divisions are the bare reciprocal iteration on the lane's precomputed
// reciprocals; the lanes whose operands leave the range where the iteration is exact are
// collected in a wave mask, and the rare wave with any runs the block again with
// div_rcp_code for the code and IEEE division for the error);
// only lane q = i%16 owns column i (its U value of row i is then U[i][i]), so its error e
// is broadcast to the row with DPP row_newbcast, and the row applies
// w[c] -= e * U[i][c] to the columns it holds.  Columns <= i of the other lanes are dead
// (already rounded), so updating them is harmless.  The owner keeps e, the code and the
// rounded-from value of its column in registers (selects, no branch); they are written
// after the loop.  Every product and difference is rounded separately
// (-ffp-contract=off), division is IEEE, rounding to an integer is half-to-even, and
// every column receives its updates in step order: the codes, errors and compensated
// values are bit-identical to the reference loop.
// ---------------------------------------------------------------------------------
constexpr int LMAX = 128;
constexpr int QL = 16;                // lanes per row
constexpr int CPL = LMAX / QL;        // columns per lane
constexpr int RPW = 64 / QL;          // rows per wave
constexpr int WPG = 4;                // waves per workgroup
constexpr int RPG = RPW * WPG;        // rows per workgroup
constexpr int USTR = QL * CPL + 4;    // LDS U row stride (floats)

// Start of lane q's 8 columns in an LDS U row: lanes 8..15 are shifted by 4 floats so
// that the 16 lanes' 16-byte reads fall on distinct banks.
__device__ __forceinline__ int lane_off(int q) { return q * CPL + ((q >> 3) << 2); }

template <int S>
// Lane S of each 16-lane row.  Every source lane is valid, so the old value and bound_ctrl
// never apply; written as update_dpp with bound_ctrl so that the compiler folds the
// broadcast into the instruction that uses it (it does not fold a plain DPP move).
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x150 + S, 0xf, 0xf, true));
}

// Register state of one row (this lane's 8 columns): working values, ladder (lo, step)
// and the reciprocals of the step (ys) and of the factor diagonal U[c][c] (yu) of each.
template <bool COMP>
struct RowRegs {
  float w[CPL], loc[CPL], stc[CPL], ys[CPL], yu[CPL], er[CPL], qc[CPL];
  float cm[COMP ? CPL : 1];  // value each owned column was rounded from
  // lanes of the wave whose error quotient may fall outside the iteration's exact range
  // (wave-uniform: scalar registers)
  uint64_t inexact;
};

// The live part of this lane's U row at p: columns mm >= M (earlier ones are dead at the
// step that uses the row), each element loaded once.  A dead element brought in with its
// 16-byte vector would be reused by the compiler at once, and the load waited for there.
template <int LO>  // first live element of the 4 at p (4: none)
__device__ __forceinline__ void load4_live(float* u, const float* p) {
  if constexpr (LO == 0) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(p);
    u[0] = x[0];
    u[1] = x[1];
    u[2] = x[2];
    u[3] = x[3];
  } else if constexpr (LO == 1 || LO == 2) {
    if constexpr (LO == 1) u[1] = p[1];
    const float2 y = *reinterpret_cast<const float2*>(p + 2);
    u[2] = y.x;
    u[3] = y.y;
  } else if constexpr (LO == 3) {
    u[3] = p[3];
  }
}
template <int M>
__device__ __forceinline__ void load_urow(float (&u)[CPL], const float* p) {
  static_assert(CPL == 8, "two 4-vectors per lane");
  load4_live<(M > 4 ? 4 : M)>(u, p);
  load4_live<(M < 4 ? 0 : (M > 8 ? 4 : M - 4))>(u + 4, p + 4);
}

// Step I of the column loop, I a compile-time constant so that every register index
// below is static (no dynamic VGPR indexing).  ub[I & 1] holds this lane's U row I;
// the step fills ub[(I + 1) & 1] with row I + 1.  With FULL the block has LMAX columns
// (no length test per step).  Both quotients are the bare reciprocal iteration, their
// operand ranges recorded in the scalar mask R.inexact (a branch in the loop would
// serialise it); EXACT uses div_rcp_code for the code and the IEEE division for the
// error instead, for the rare block that has to be run again.
template <int I, bool FULL, bool COMP, bool EXACT>
__device__ __forceinline__ void gptq_step(RowRegs<COMP>& R, int L, int q, float nm,
                                          const float* __restrict__ suq, float (&ub)[2][CPL]) {
  constexpr int m = I / QL, s = I % QL, cur = I & 1;
  if (!FULL && I >= L) return;
  if constexpr (I + 1 < LMAX) load_urow<(I + 1) / QL>(ub[cur ^ 1], suq + (I + 1) * USTR);
  const float col = R.w[m];
  const float lo_j = R.loc[m], st_j = R.stc[m];
  const float safe = (st_j == 0.0f) ? 1.0f : st_j;
  const float dq = col - lo_j;
  float qv;
  if constexpr (EXACT) {
    qv = clamp_code(__builtin_rintf(div_rcp_code(dq, safe, R.ys[m])), nm);
  } else {
    // div_rcp_code without its select: the iteration's quotient, whose code is the IEEE
    // quotient's while |q0| = |dq ys| <= 2^100.  That holds in every lane the wave keeps:
    // load_row_c marks the wave unless |ys| <= 2^40, |lo| <= 2^40 and |step| <= 2^32, and
    // the error test below marks it unless |num| <= 2^50 with wq finite in fp16, so that
    // |dq| <= |num| + |wq| + |lo| < 2^51 (NaN and infinities fail those tests).  Every
    // lane kept has a finite quotient, so the clamp is one median (clamp_code's NaN
    // propagation only matters in the waves the rerun redoes).  A zero step's column has
    // ys = 0 (load_row_c): its quotient is +0 for every finite dq, the code 0 the
    // reference gives it, without a select in the chain.
    qv = __builtin_amdgcn_fmed3f(__builtin_rintf(div_rcp_fast(dq, safe, R.ys[m])), 0.0f, nm);
  }
  if constexpr (EXACT) {
    if (st_j == 0.0f) qv = 0.0f;
  }
  const float wq = f16_round(lo_j + qv * st_j);
  const float ujj = ub[cur][m];  // U[I][I] in the owner lane
  const bool own = q == s;
  const float num = col - wq;
  float e;
  if constexpr (EXACT) {
    e = num / ujj;
  } else {
    e = div_rcp_fast(num, ujj, R.yu[m]);
    // div_rcp_ok(num, num yu) holds when |num| is in [2^-50, 2^50] (every column's yu is
    // in [2^-50, 2^50], checked once per block) or num is +0: tested in every lane, owner
    // or not (a false alarm only costs a rerun), the lanes that fail OR-ed into a wave
    // mask in scalar registers
    // (one ballot per comparison, each the comparison's own lane mask: no vector select)
    const float an = __builtin_fabsf(num);
    const uint64_t small = __builtin_amdgcn_ballot_w64(!(an >= 0x1p-50f));  // NaN too
    const uint64_t large = __builtin_amdgcn_ballot_w64(!(an <= 0x1p50f));
    // +0 passes (the iteration gives +0 there); -0 does not (it would give +0)
    const uint64_t zero = __builtin_amdgcn_ballot_w64(num == 0.0f);
    const uint64_t neg = __builtin_amdgcn_ballot_w64(__builtin_bit_cast(int32_t, num) < 0);
    R.inexact |= (small | large) & ~(zero & ~neg);
  }
  const float eb = row_bcast<s>(e);
  // the selects are pinned here (empty asm): left free, the compiler keeps every step's
  // e and code in its own register until the end of the loop, which costs occupancy
  R.er[m] = own ? e : R.er[m];
  R.qc[m] = own ? qv : R.qc[m];
  asm volatile("" : "+v"(R.er[m]), "+v"(R.qc[m]));
  if constexpr (COMP) {
    R.cm[m] = own ? col : R.cm[m];
    asm volatile("" : "+v"(R.cm[m]));
  }
#pragma unroll
  for (int mm = (I + 1) / QL; mm < CPL; ++mm) R.w[mm] = R.w[mm] - eb * ub[cur][mm];
}

template <bool FULL, bool COMP, bool EXACT, int... Is>
__device__ __forceinline__ void gptq_steps(std::integer_sequence<int, Is...>, RowRegs<COMP>& R,
                                           int L, int q, float nm, const float* __restrict__ suq,
                                           float (&ub)[2][CPL]) {
  (gptq_step<Is, FULL, COMP, EXACT>(R, L, q, nm, suq, ub), ...);
}

// The state of this lane's 8 columns of row lr of the workgroup, in three parts so that
// the kernel can overlap their loads with the U block's: (a) the working copy and each
// column's ladder block index (blk: the group's column -> block map at column i1),
// (b) the decoded (lo, step) of those blocks (a second, dependent round trip), (c) the
// reciprocals of the steps and of the factor diagonal (su: the U block in LDS).
template <bool COMP>
__device__ __forceinline__ void load_row_a(RowRegs<COMP>& R, int (&bix)[CPL],
                                           const float* __restrict__ wc, int64_t K,
                                           int64_t i1, int L, int64_t rbase, int nrows, int lr,
                                           const int32_t* __restrict__ blk, int gspan, int gsel,
                                           int q) {
  // this row's columns c = 16m + q: the working copy and each column's ladder block, the
  // latter from map gsel of the gspan + 1 block maps at blk (a run of groups sharing one
  // factor, factor_run_end: gspan * K + L < 2^29, so the byte offsets fit in 32 bits)
  const __amdgpu_buffer_rsrc_t wrs = mg_rsrc(wc + rbase * K + i1, (int64_t)(nrows - 1) * K + L);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(blk + i1), (short)0, (int)(((int64_t)gspan * K + L) * 4), 0x00020000);
  const uint32_t boff = (uint32_t)gsel * (uint32_t)K;
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const int c = QL * m + q;
    const uint32_t wo = c < L ? (uint32_t)(((int64_t)lr * K + c) * 4) : MG_OOB;
    R.w[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (int)wo, 0, 0));
    bix[m] = (int)__builtin_amdgcn_raw_buffer_load_b32(
        brs, (int)(c < L ? (boff + (uint32_t)c) * 4u : MG_OOB), 0, 0);
  }
}
template <bool COMP>
__device__ __forceinline__ void load_row_b(RowRegs<COMP>& R, const int (&bix)[CPL],
                                           int64_t rbase, int nrows, int lr,
                                           const float* __restrict__ lo,
                                           const float* __restrict__ st, int64_t ldp) {
  // decoded (lo, step) of those blocks (block 0 for the dead columns c >= L)
  const __amdgpu_buffer_rsrc_t lrs = mg_rsrc(lo + rbase * ldp, (int64_t)nrows * ldp);
  const __amdgpu_buffer_rsrc_t srs = mg_rsrc(st + rbase * ldp, (int64_t)nrows * ldp);
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const uint32_t po = (uint32_t)(((int64_t)lr * ldp + bix[m]) * 4);
    R.loc[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lrs, (int)po, 0, 0));
    R.stc[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srs, (int)po, 0, 0));
    R.er[m] = 0.0f;
    R.qc[m] = 0.0f;
    if constexpr (COMP) R.cm[m] = 0.0f;
  }
}
template <bool COMP>
__device__ __forceinline__ void load_row_c(RowRegs<COMP>& R, int L, const float* su, int q) {
  // IEEE reciprocals (correctly rounded) of each column's step and factor diagonal;
  // dead columns (c >= L) get 1.  A reciprocal of the diagonal outside [2^-50, 2^50], of
  // the step above 2^40, a ladder origin above 2^40 or a step above 2^32 in magnitude (or
  // any of them not finite) marks the wave for the exact rerun: the per-step tests of
  // gptq_step rely on these bounds.
  bool yok = true;
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const int c = QL * m + q;
    const float ud = c < L ? su[c * USTR + lane_off(q) + m] : 1.0f;
    R.ys[m] = R.stc[m] == 0.0f ? 0.0f : 1.0f / R.stc[m];  // 0: a zero step (code 0)
    R.yu[m] = 1.0f / ud;
    const float ay = __builtin_fabsf(R.yu[m]);
    yok = yok && ay >= 0x1p-50f && ay <= 0x1p50f && __builtin_fabsf(R.ys[m]) <= 0x1p40f &&
          __builtin_fabsf(R.loc[m]) <= 0x1p40f && __builtin_fabsf(R.stc[m]) <= 0x1p32f;
  }
  R.inexact = __builtin_amdgcn_ballot_w64(!yok);
}
template <bool COMP>
__device__ __forceinline__ void load_row(RowRegs<COMP>& R, const float* __restrict__ wc,
                                         int64_t K, int64_t i1, int L, int64_t rbase,
                                         int nrows, int lr, const int32_t* __restrict__ blk,
                                         int gspan, int gsel, const float* __restrict__ lo,
                                         const float* __restrict__ st, int64_t ldp,
                                         const float* su, int q) {
  int bix[CPL];
  load_row_a<COMP>(R, bix, wc, K, i1, L, rbase, nrows, lr, blk, gspan, gsel, q);
  load_row_b<COMP>(R, bix, rbase, nrows, lr, lo, st, ldp);
  load_row_c<COMP>(R, L, su, q);
}

template <bool COMP>
__device__ __forceinline__ void store_row(const RowRegs<COMP>& R, int64_t K, int64_t i1, int L,
                                          int64_t r, int q, float* __restrict__ err1,
                                          int64_t lde, uint8_t* __restrict__ codes,
                                          float* __restrict__ comp) {
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const int c = QL * m + q;
    if (c < L) {
      err1[r * lde + c] = R.er[m];
      codes[r * K + i1 + c] = (uint8_t)R.qc[m];
      if constexpr (COMP) comp[r * K + i1 + c] = R.cm[m];
    }
  }
}

// Column group M (columns i = 16M + s, s = 0..15) of the block with IEEE division: the
// 16 steps as a rolled loop whose register index M is a compile-time constant, so the
// row state stays in registers (no dynamically indexed array, no scratch memory).  The
// same operations in the same order as gptq_step; w[M] is also updated at s = 15, where
// every lane's column of group M is already rounded (a dead value, as in gptq_step).
template <int M, bool COMP>
__device__ __forceinline__ void exact_group(RowRegs<COMP>& R, int L, int q, float nm,
                                            const float* __restrict__ suq, int lane) {
#pragma unroll 1
  for (int s = 0; s < QL; ++s) {
    const int i = QL * M + s;
    if (i >= L) break;  // L is uniform: the whole wave leaves together
    const float col = R.w[M];
    const float lo_j = R.loc[M], st_j = R.stc[M];
    const float safe = (st_j == 0.0f) ? 1.0f : st_j;
    float qv = clamp_code(__builtin_rintf((col - lo_j) / safe), nm);
    if (st_j == 0.0f) qv = 0.0f;
    const float wq = f16_round(lo_j + qv * st_j);
    const float* ui = suq + i * USTR;
    const float e = (col - wq) / ui[M];  // U[i][i] in the owner lane
    const float eb = __shfl(e, (lane & ~(QL - 1)) + s, 64);
    const bool own = q == s;
    R.er[M] = own ? e : R.er[M];
    R.qc[M] = own ? qv : R.qc[M];
    if constexpr (COMP) R.cm[M] = own ? col : R.cm[M];
#pragma unroll
    for (int mm = M; mm < CPL; ++mm) R.w[mm] = R.w[mm] - eb * ui[mm];
  }
}
template <bool COMP, int... Ms>
__device__ __forceinline__ void exact_groups(std::integer_sequence<int, Ms...>,
                                             RowRegs<COMP>& R, int L, int q, float nm,
                                             const float* __restrict__ suq, int lane) {
  (exact_group<Ms, COMP>(R, L, q, nm, suq, lane), ...);
}

// The block for this lane's row again, from the working copy, with IEEE division, then
// the row's outputs.  Runs only for a wave whose fast pass met an error quotient outside
// the reciprocal iteration's exact range; it reloads the fast pass's register state R
// (dead once the wave has decided to run again) instead of holding a second copy.
template <bool COMP>
__device__ void gptq_rows_exact(RowRegs<COMP>& R, const float* __restrict__ wc, int64_t K,
                                int64_t i1, int L, int64_t rbase, int nrows, int lr,
                                int64_t r, const int32_t* __restrict__ blk, int gspan, int gsel,
                                const float* __restrict__ lo, const float* __restrict__ st,
                                int64_t ldp, const float* su, int q, float nm,
                                float* __restrict__ err1, int64_t lde,
                                uint8_t* __restrict__ codes, float* __restrict__ comp) {
  load_row<COMP>(R, wc, K, i1, L, rbase, nrows, lr, blk, gspan, gsel, lo, st, ldp, su, q);
  exact_groups<COMP>(std::make_integer_sequence<int, CPL>{}, R, L, q, nm, su + lane_off(q),
                     (int)(threadIdx.x & 63));
  store_row<COMP>(R, K, i1, L, r, q, err1, lde, codes, comp);
}

// Last group of the run that starts at group g (groups up to g1): the following groups
// whose factor is the same matrix (equal u_ptrs; the row classes of one input), at most
// as many as keep (ge - g) * K + 128 < 2^29 for the block-map offsets of load_row_a.
// Rows of one run share one pass of the column loop and one tile pass of the cross-block
// update, so a batch needs no padding between them.
__device__ __forceinline__ int factor_run_end(const int64_t* __restrict__ u_ptrs, int g, int g1,
                                              int64_t K) {
  const int64_t ug = u_ptrs[g];
  int ge = g;
  while (ge < g1 && u_ptrs[ge + 1] == ug && (int64_t)(ge + 1 - g) * K + LMAX < (1 << 29)) ++ge;
  return ge;
}

// The column loop of block [i1, i1 + L) for this workgroup's rows, one run of groups
// (factor_run_end) after the other, each row with its own group's block map and highest
// code (su: the workgroup's LDS block of U).  Reads wc, writes err1, codes, comp.  Two
// workgroups per CU: without the bound the per-row highest code took the full blocks'
// variants to 256 VGPRs + AGPRs, one wave per SIMD, and the big batches' column loops
// (gate/up, MoE experts) ran at half rate; with it they fit in 256 VGPRs, no scratch.
template <bool FULL, bool COMP>
__global__ __launch_bounds__(RPG * QL, 2) void gptq_block_kernel(
    const float* __restrict__ wc, int64_t N, int64_t K, int64_t i1, int L,
    float* __restrict__ err1, int64_t lde, uint8_t* __restrict__ codes,
    const float* __restrict__ lo, const float* __restrict__ st, int64_t ldp,
    const int32_t* __restrict__ row_grp, const int64_t* __restrict__ u_ptrs,
    const int32_t* __restrict__ blk, const float* __restrict__ nmax,
    float* __restrict__ comp) {
  __shared__ float su[LMAX * USTR];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int q = lane & (QL - 1);
  const int64_t rbase = (int64_t)blockIdx.x * RPG;
  const int lr = wave * RPW + lane / QL;  // row within the workgroup
  const int64_t r = rbase + lr;
  const bool live = r < N;
  const int64_t rend = ((rbase + RPG < N) ? rbase + RPG : N) - 1;
  const int nrows = (int)(rend - rbase + 1);
  const int g0 = row_grp[rbase];
  const int g1 = row_grp[rend];
  const int gr = live ? row_grp[r] : -1;

  // Global reads go through buffer resources that end at the last valid element, so
  // they need no branches (a branch around a load makes the compiler wait for each load
  // in turn): all loads of a phase are issued before the first is used.
  for (int g = g0, ge = g0; g <= g1; g = ge + 1) {
    ge = factor_run_end(u_ptrs, g, g1, K);
    const bool mine = gr >= g && gr <= ge;  // uniform over the row's 16 lanes
    const int gsel = mine ? gr - g : 0;
    // the row's working copy and ladder indices first, so that the dependent load of its
    // ladders runs while the U block is in flight
    RowRegs<COMP> R;
    int bix[CPL];
    load_row_a<COMP>(R, bix, wc, K, i1, L, rbase, nrows, lr, blk + (int64_t)g * K, ge - g, gsel,
                     q);
    __syncthreads();  // LDS of the previous group is no longer read
    {
      // U[i1:i1+L, i1:i1+L]: rows >= L read zero, columns >= L are zeroed here
      const float* U = reinterpret_cast<const float*>(u_ptrs[g]);
      const __amdgpu_buffer_rsrc_t ur = mg_rsrc(U + i1 * K + i1, (int64_t)(L - 1) * K + L);
      constexpr int NV = LMAX * LMAX / 4 / (RPG * QL);  // 16-byte vectors per thread
      f32x4 uv[NV];
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        const int idx = tid + RPG * QL * t, i = idx / (LMAX / 4), c = 4 * (idx % (LMAX / 4));
        const uint32_t off = i < L ? (uint32_t)(((int64_t)i * K + c) * 4) : MG_OOB;
        uv[t] = mg_load4(ur, off);
      }
      load_row_b<COMP>(R, bix, rbase, nrows, lr, lo, st, ldp);
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        const int idx = tid + RPG * QL * t, i = idx / (LMAX / 4), c = 4 * (idx % (LMAX / 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int cc = c + e;
          const float v = uv[t][e];
          su[i * USTR + lane_off(cc % QL) + cc / QL] = (cc < L) ? v : 0.0f;
        }
      }
    }
    __syncthreads();
    if (!mine) continue;

    const float nm = nmax[gr];
    load_row_c<COMP>(R, L, su, q);
    const float* suq = su + lane_off(q);
    float ub[2][CPL];
    load_urow<0>(ub[0], suq);
    gptq_steps<FULL, COMP, false>(std::make_integer_sequence<int, LMAX>{}, R, L, q, nm, suq, ub);
    if (R.inexact != 0) {
      // some row of this wave met an error quotient outside the iteration's exact range
      // (subnormal or negative-zero numerators, extreme magnitudes): the wave runs the
      // block again from the working copy with IEEE division
      gptq_rows_exact<COMP>(R, wc, K, i1, L, rbase, nrows, lr, r, blk + (int64_t)g * K, ge - g,
                            gsel, lo, st, ldp, su, q, nm, err1, lde, codes, comp);
      continue;
    }
    store_row<COMP>(R, K, i1, L, r, q, err1, lde, codes, comp);
  }
}

// ---------------------------------------------------------------------------------
// Cross-block update on fp32 MFMA.
//
//   wc[r, c] -= sum_k err1[r, t*128 + k] * U_g[i1 + 128t + k, c]     (t = 0..nblk-1, in order)
//
// Each product is accumulated from zero with v_mfma_f32_32x32x2_f32, which evaluates
// fma(a1, b1, fma(a0, b0, acc)) in k order: the same sequential fp32 FMA chain as the
// reference's CPU GEMM, then one subtraction per block.  One launch applies the nblk
// blocks of a super-block to the far columns (lazy batching) and every block's product
// is subtracted separately, in block order, so the result equals the per-block schedule
// bit for bit.
// Workgroup tile 128 x 128 (4 waves as 2 x 2 of 64 x 64), rank streamed in chunks of
// 32 through LDS.  When the whole tile belongs to one factor, the wc tile is read once,
// held in registers while the blocks stream through as one pipelined rank (the next
// chunk in flight across block boundaries), and written once.  A tile shared by two
// factors runs one pass per factor: rows of another group are masked in A and left
// untouched in that pass's epilogue.
// ---------------------------------------------------------------------------------
struct GroupMask {  // A rows of the current group pass (this thread's staged row)
  static constexpr bool kElem = false;
  bool mine;
  __device__ __forceinline__ bool row(int64_t) const { return mine; }
  __device__ __forceinline__ bool elem(int64_t, int64_t) const { return true; }
};

// T: workgroup tile edge, 128 (2 x 2 accumulators per wave, two workgroups per CU) or 64
// (one accumulator per wave, for launches with too few 128-tiles to fill the chip).
template <int T>
__global__ __launch_bounds__(256, T == MG_T ? 2 : 4) void gptq_trailing_kernel(
    float* __restrict__ wc, int64_t N, int64_t K, int64_t i1, int nblk,
    const float* __restrict__ err1, int64_t lde, int64_t c0, int64_t c1,
    const int32_t* __restrict__ row_grp, const int64_t* __restrict__ u_ptrs, int64_t tn,
    int64_t ntiles, const unsigned long long* __restrict__ skip) {
  constexpr int NA = T / 64;
  __shared__ MgSmemT<T> sm;
  const int64_t tile = xcd_tile(blockIdx.x, ntiles);
  if (tile < 0) return;
  if (skip != nullptr && *skip == 0ull) return;  // a caller's device-side "nothing to do"
  const int64_t r0 = (tile / tn) * T;
  const int64_t cc0 = c0 + (tile % tn) * T;
  const int64_t rlast = ((r0 + T < N) ? r0 + T : N) - 1;
  const int g0 = row_grp[r0], g1 = row_grp[rlast];
  const int tid = threadIdx.x;
  const int64_t my_row = r0 + tid / (256 / T);  // row this thread stages for the A operand
  const int my_grp = my_row < N ? row_grp[my_row] : -1;
  const CTile<T> ct(wc, K, N, c1, r0, cc0);
  bool one = true;  // every group of the tile has the same factor (the row classes of one input)
  for (int g = g0 + 1; g <= g1; ++g) one = one && u_ptrs[g] == u_ptrs[g0];

  if (one) {  // one factor for the whole tile: the blocks as one pipelined rank stream
    const float* U = reinterpret_cast<const float*>(u_ptrs[g0]);
    const int64_t R = (K - i1 < (int64_t)nblk * LMAX) ? K - i1 : (int64_t)nblk * LMAX;
    RowsLoader<GroupMask, T> al{err1, lde, N, R, GroupMask{my_grp >= 0}};
    ColsLoader<NoMask, T> bl{U + i1 * K, K, c1, R, NoMask{}};
    f32x16 acc[NA][NA], cv[NA][NA];
    mg_zero(acc);
    // the wc tile stays in registers across the blocks; it is loaded during the first
    // chunk's MFMAs (first needed at the end of the first block)
    mg_mainloop_seg<NA, T, LMAX>(
        acc, sm, al, bl, r0, cc0, 0, R, []() {},
        [&](f32x16(&a)[NA][NA]) {
#pragma unroll
          for (int x = 0; x < NA; ++x)
#pragma unroll
            for (int y = 0; y < NA; ++y)
#pragma unroll
              for (int j = 0; j < 16; ++j) {
                cv[x][y][j] = cv[x][y][j] - a[x][y][j];
                a[x][y][j] = 0.0f;
              }
        },
        [&]() { ct.load(cv); });
    ct.store(cv, [](int, int, int) { return true; });
    return;
  }
  // a tile shared by several factors: one masked pass per run of groups with one factor
  for (int g = g0, ge = g0; g <= g1; g = ge + 1) {
    for (ge = g; ge < g1 && u_ptrs[ge + 1] == u_ptrs[g];) ++ge;
    const float* U = reinterpret_cast<const float*>(u_ptrs[g]);
    for (int t = 0; t < nblk; ++t) {
      const int64_t ib = i1 + (int64_t)t * LMAX;
      const int64_t L = (K - ib < LMAX) ? K - ib : LMAX;
      f32x16 acc[NA][NA];
      mg_zero(acc);
      RowsLoader<GroupMask, T> al{err1 + t * LMAX, lde, N, L,
                                  GroupMask{my_grp >= g && my_grp <= ge}};
      ColsLoader<NoMask, T> bl{U + ib * K, K, c1, L, NoMask{}};
      mg_mainloop(acc, sm, al, bl, r0, cc0, 0, L);
      // wc tile -= this block's product (read-modify-write: the tile is not held in
      // registers across the rank loop, which keeps two workgroups per CU resident)
      f32x16 cv[NA][NA];
      ct.load(cv);
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NA; ++b)
#pragma unroll
          for (int j = 0; j < 16; ++j) cv[a][b][j] = cv[a][b][j] - acc[a][b][j];
      // bit a*16+j: row (a, j) is in the run [g, ge]
      uint32_t in_g = 0;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int64_t rr = r0 + mg_row<T>(a, j);
          const int gg = rr < N ? row_grp[rr] : -1;
          in_g |= (uint32_t)(gg >= g && gg <= ge) << (a * 16 + j);
        }
      ct.store(cv, [&](int a, int j, int) { return (in_g >> (a * 16 + j)) & 1u; });
    }
  }
}

int launch_block(const float* wc, int64_t n, int64_t k, int64_t i1, int64_t len, float* err1,
                 int64_t lde, uint8_t* codes, const float* lo, const float* st, int64_t ldp,
                 const int32_t* row_grp, const int64_t* u_ptrs, const int32_t* blk,
                 const float* nmax, float* comp, hipStream_t s) {
  const dim3 grid((unsigned)((n + RPG - 1) / RPG));
  LaunchTimer timer(HI2X_TIME_GPTQ_BLOCK, (double)n * len * (len - 1), s);
#define HI2X_BLOCK_LAUNCH(F, C)                                                            \
  hipLaunchKernelGGL((gptq_block_kernel<F, C>), grid, dim3(RPG * QL), 0, s, wc, n, k, i1,   \
                     (int)len, err1, lde, codes, lo, st, ldp, row_grp, u_ptrs, blk, nmax, comp)
  const bool full = len == LMAX;
  if (comp) {
    if (full) HI2X_BLOCK_LAUNCH(true, true);
    else HI2X_BLOCK_LAUNCH(false, true);
  } else {
    if (full) HI2X_BLOCK_LAUNCH(true, false);
    else HI2X_BLOCK_LAUNCH(false, false);
  }
#undef HI2X_BLOCK_LAUNCH
  return launch_status("gptq_block_kernel");
}

int launch_trailing(float* wc, int64_t n, int64_t k, int64_t i1, int nblk, const float* err1,
                    int64_t lde, int64_t c0, int64_t c1, const int32_t* row_grp,
                    const int64_t* u_ptrs, hipStream_t s,
                    const unsigned long long* skip = nullptr,
                    int timing_kind = HI2X_TIME_GPTQ_TRAILING) {
  if (c1 <= c0 || n == 0) return HI2X_OK;
  double rank = 0.0;
  for (int t = 0; t < nblk; ++t) rank += (double)std::min<int64_t>(LMAX, k - (i1 + (int64_t)t * LMAX));
  LaunchTimer timer(timing_kind, 2.0 * n * rank * (c1 - c0), s);
  // 128-tiles fill the chip from two rounds of its 512 workgroup slots on; smaller grids
  // (the near updates of a super-block) run on 64-tiles, four times as many workgroups
  // on a background stream the workgroups hold unused LDS on top of their own (72 + 28 KB
  // for 128-tiles: one per CU instead of two; 36 + 24 KB for 64-tiles: two instead of
  // four), which leaves each CU room for another stream's small products or leaves
  const bool bg = stream_background(s);
  const int64_t tn128 = (c1 - c0 + MG_T - 1) / MG_T, tm128 = (n + MG_T - 1) / MG_T;
  if (tn128 * tm128 >= 512) {
    const int64_t ntiles = tn128 * tm128;
    hipLaunchKernelGGL(gptq_trailing_kernel<MG_T>, dim3((unsigned)((ntiles + 7) / 8 * 8)),
                       dim3(256), bg ? 28 * 1024 : 0, s, wc, n, k, i1, nblk, err1, lde, c0, c1,
                       row_grp, u_ptrs, tn128, ntiles, skip);
  } else {
    const int64_t tn = (c1 - c0 + 63) / 64, tm = (n + 63) / 64, ntiles = tn * tm;
    hipLaunchKernelGGL(gptq_trailing_kernel<64>, dim3((unsigned)((ntiles + 7) / 8 * 8)),
                       dim3(256), bg ? 24 * 1024 : 0, s, wc, n, k, i1, nblk, err1, lde, c0, c1,
                       row_grp, u_ptrs, tn, ntiles, skip);
  }
  return launch_status("gptq_trailing_kernel");
}

}  // namespace

int trailing_update(float* wc, int64_t n, int64_t k, int64_t i1, int nblk, const float* err1,
                    int64_t lde, int64_t c0, int64_t c1, const int32_t* row_grp,
                    const int64_t* u_ptrs, hipStream_t s, const unsigned long long* skip,
                    int timing_kind) {
  return launch_trailing(wc, n, k, i1, nblk, err1, lde, c0, c1, row_grp, u_ptrs, s, skip,
                         timing_kind);
}

}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_gptq_block(const float* wc, int64_t n, int64_t k, int64_t i1, int64_t len,
                               float* err1, uint8_t* codes, const float* lo, const float* st,
                               int64_t ldp, const int32_t* row_grp, const int64_t* u_ptrs,
                               const int32_t* blk, const float* nmax, float* comp,
                               void* stream) {
  clear_error();
  HI2X_REQUIRE(n >= 0 && k > 0, "gptq_block: bad shape n=%lld k=%lld", (long long)n,
               (long long)k);
  HI2X_REQUIRE(len > 0 && len <= LMAX, "gptq_block: block length %lld not in (0, 128]",
               (long long)len);
  HI2X_REQUIRE(i1 >= 0 && i1 + len <= k, "gptq_block: block [%lld, %lld) outside K=%lld",
               (long long)i1, (long long)(i1 + len), (long long)k);
  if (n == 0) return HI2X_OK;
  HI2X_REQUIRE(wc && err1 && codes && lo && st && row_grp && u_ptrs && blk && nmax,
               "gptq_block: null buffer");
  return launch_block(wc, n, k, i1, len, err1, len, codes, lo, st, ldp, row_grp, u_ptrs, blk,
                      nmax, comp, as_stream(stream));
}

extern "C" int hi2x_gptq_trailing(float* wc, int64_t n, int64_t k, int64_t i1, int64_t len,
                                  const float* err1, int64_t lde, int64_t c0, int64_t c1,
                                  const int32_t* row_grp, const int64_t* u_ptrs,
                                  void* stream) {
  clear_error();
  HI2X_REQUIRE(len > 0 && len <= LMAX && i1 >= 0 && i1 + len <= k,
               "gptq_trailing: bad block [%lld, +%lld) for K=%lld", (long long)i1,
               (long long)len, (long long)k);
  HI2X_REQUIRE(c0 >= i1 + len && c1 <= k, "gptq_trailing: columns [%lld, %lld) invalid",
               (long long)c0, (long long)c1);
  HI2X_REQUIRE(lde >= len, "gptq_trailing: lde < len");
  if (n == 0 || c1 <= c0) return HI2X_OK;
  return launch_trailing(wc, n, k, i1, 1, err1, lde, c0, c1, row_grp, u_ptrs,
                         as_stream(stream));
}

extern "C" int hi2x_gptq_run(float* wc, int64_t n, int64_t k, uint8_t* codes, const float* lo,
                             const float* st, int64_t ldp, const int32_t* row_grp,
                             const int64_t* u_ptrs, const int32_t* blk, const float* nmax,
                             float* comp, float* err_ws, int64_t super_blocks, void* stream) {
  clear_error();
  HI2X_REQUIRE(n >= 0 && k > 0 && k % 16 == 0, "gptq_run: bad shape n=%lld k=%lld",
               (long long)n, (long long)k);
  HI2X_REQUIRE(super_blocks >= 1 && super_blocks <= 64, "gptq_run: super_blocks=%lld",
               (long long)super_blocks);
  if (n == 0) return HI2X_OK;
  HI2X_REQUIRE(wc && codes && lo && st && row_grp && u_ptrs && blk && nmax && err_ws,
               "gptq_run: null buffer");
  hipStream_t s = as_stream(stream);
  const int64_t nblocks = (k + LMAX - 1) / LMAX;
  const int64_t lde = super_blocks * LMAX;
  for (int64_t sb = 0; sb < nblocks; sb += super_blocks) {
    const int64_t sb_end = (sb + super_blocks < nblocks) ? sb + super_blocks : nblocks;
    const int64_t cs_end = (sb_end * LMAX < k) ? sb_end * LMAX : k;
    for (int64_t b = sb; b < sb_end; ++b) {
      const int64_t i1 = b * LMAX;
      const int64_t len = (k - i1 < LMAX) ? k - i1 : LMAX;
      float* eb = err_ws + (b - sb) * LMAX;
      int rc = launch_block(wc, n, k, i1, len, eb, lde, codes, lo, st, ldp, row_grp, u_ptrs,
                            blk, nmax, comp, s);
      if (rc) return rc;
      rc = launch_trailing(wc, n, k, i1, 1, eb, lde, i1 + len, cs_end, row_grp, u_ptrs, s);
      if (rc) return rc;
    }
    int rc = launch_trailing(wc, n, k, sb * LMAX, (int)(sb_end - sb), err_ws, lde, cs_end, k,
                             row_grp, u_ptrs, s);
    if (rc) return rc;
  }
  return HI2X_OK;
}

// ---- the column loop without allocation -------------------------------------------------
// hi2x_gptq_run's error workspace taken from a file-scope device array instead of the
// caller's buffer: for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).  Each GPU the library
// runs on holds its own copy of the array until the process ends; its address on a device
// is looked up once (hipGetSymbolAddress with that device current) and kept.
namespace {
constexpr int64_t kScratchBytes = int64_t(64) << 20;  // 64 MiB per device
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The array's device address on the current device (host code never uses the symbol
// itself: on the host it names a stand-in, not device memory).
int scratch_on_current_device(float** out) {
  int dev = -1;
  HI2X_HIP(hipGetDevice(&dev));
  HI2X_REQUIRE(dev >= 0 && dev < kMaxDevices, "gptq_run_noalloc: device %d", dev);
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !addr) {
        set_error("gptq_run_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                  hipGetErrorString(e));
        return HI2X_ELAUNCH;
      }
      p = static_cast<float*>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return HI2X_OK;
}
}  // namespace

extern "C" int hi2x_gptq_run_noalloc(float* wc, int64_t n, int64_t k, uint8_t* codes,
                                     const float* lo, const float* st, int64_t ldp,
                                     const int32_t* row_grp, const int64_t* u_ptrs,
                                     const int32_t* blk, const float* nmax, float* comp,
                                     int64_t super_blocks, void* stream) {
  clear_error();
  HI2X_REQUIRE(n >= 0 && n <= (int64_t(1) << 40) && super_blocks >= 1 && super_blocks <= 64,
               "gptq_run_noalloc: n=%lld super_blocks=%lld", (long long)n,
               (long long)super_blocks);
  const int64_t need = n * LMAX * super_blocks * (int64_t)sizeof(float);
  HI2X_REQUIRE(need <= kScratchBytes,
               "gptq_run_noalloc: %lld rows x %lld super-blocks need %lld bytes of error "
               "scratch, more than its %lld (64 MiB); use hi2x_gptq_run with a workspace",
               (long long)n, (long long)super_blocks, (long long)need,
               (long long)kScratchBytes);
  if (n == 0) return HI2X_OK;
  float* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  return hi2x_gptq_run(wc, n, k, codes, lo, st, ldp, row_grp, u_ptrs, blk, nmax, comp, ws,
                       super_blocks, stream);
}
