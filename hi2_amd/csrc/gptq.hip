// GPTQ column loop on gfx950: the intra-block rounding kernel, the cross-block
// (trailing) update on fp32 MFMA, and the block schedule that drives them.
//
// Reference: hi2/hessian.py:235-315 (_round_reference / _round_kernel) and the op-by-op
// rounding spec of hi2/gptq_kernel.py:82-100.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace hi2x {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------------
// Intra-block kernel.
//
// One row is owned by a quad of lanes (16 rows per wave, 64 per workgroup).  Lane q of
// the quad holds the row's columns c = 4m + q (m = 0..31) of the 128-column block in
// registers, together with the decoded (lo, step) of each column's ladder block.  The
// factor block U[i1:i1+128, i1:i1+128] of the row's group sits in LDS, laid out so that
// lane q reads its 32 columns of a U row contiguously: su[i][q][m] = U[i1+i][i1+4m+q].
//
// Step i (fully unrolled): every lane runs the rounding chain on its own column m=i/4;
// only lane q = i%4 owns column i, so its error e is broadcast to the quad with a DPP
// quad_perm, recorded by the owner, and the quad applies w[c] -= e * U[i][c] to the
// columns it holds.  Columns <= i of the other lanes are dead (already rounded), so
// updating them is harmless.  Every product and difference is rounded separately
// (-ffp-contract=off), division is IEEE, rounding to an integer is half-to-even: the
// codes, errors and compensated values are bit-identical to the reference loop.
// ---------------------------------------------------------------------------------
constexpr int LMAX = 128;
constexpr int QL = 4;                 // lanes per row
constexpr int CPL = LMAX / QL;        // columns per lane
constexpr int RPW = 64 / QL;          // rows per wave
constexpr int WPG = 4;                // waves per workgroup
constexpr int RPG = RPW * WPG;        // rows per workgroup
constexpr int QSTR = CPL + 4;         // per-lane stride in an LDS U row (bank spread)
constexpr int USTR = QL * QSTR;       // LDS U row stride (floats)

template <int S>
__device__ __forceinline__ float quad_bcast_t(float v) {
  constexpr int ctrl = S * 0x55;  // quad_perm(S, S, S, S)
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl,
                                                            0xf, 0xf, false));
}

__device__ __forceinline__ float quad_bcast(float v, int s) {
  switch (s) {
    case 0: return quad_bcast_t<0>(v);
    case 1: return quad_bcast_t<1>(v);
    case 2: return quad_bcast_t<2>(v);
    default: return quad_bcast_t<3>(v);
  }
}

__global__ __launch_bounds__(RPG * QL) void gptq_block_kernel(
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
  const int q = lane & 3;
  const int64_t rbase = (int64_t)blockIdx.x * RPG;
  const int64_t r = rbase + wave * RPW + (lane >> 2);
  const bool live = r < N;
  const int64_t rend = ((rbase + RPG < N) ? rbase + RPG : N) - 1;
  const int g0 = row_grp[rbase];
  const int g1 = row_grp[rend];
  const int gr = live ? row_grp[r] : -1;

  for (int g = g0; g <= g1; ++g) {
    __syncthreads();  // LDS of the previous group is no longer read
    {
      const float* U = reinterpret_cast<const float*>(u_ptrs[g]);
      for (int idx = tid; idx < LMAX * LMAX; idx += RPG * QL) {
        const int i = idx / LMAX, c = idx % LMAX;
        const float v = (i < L && c < L) ? U[(i1 + i) * K + i1 + c] : 0.0f;
        su[i * USTR + (c & 3) * QSTR + (c >> 2)] = v;
      }
    }
    __syncthreads();
    if (gr != g) continue;  // uniform over the quad (one row)

    const int32_t* bl = blk + (int64_t)g * K;
    const float nm = nmax[g];
    float w[CPL], loc[CPL], stc[CPL], er[CPL];
    uint32_t cq[CPL / 4];
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int c = QL * m + q;
      float wv = 0.0f, lv = 0.0f, sv = 0.0f;
      if (c < L) {
        wv = wc[r * K + i1 + c];
        const int b = bl[i1 + c];
        lv = lo[r * ldp + b];
        sv = st[r * ldp + b];
      }
      w[m] = wv;
      loc[m] = lv;
      stc[m] = sv;
      er[m] = 0.0f;
    }
#pragma unroll
    for (int m = 0; m < CPL / 4; ++m) cq[m] = 0u;

    const float* qrow = su + q * QSTR;
#pragma unroll
    for (int i = 0; i < LMAX; ++i) {
      if (i >= L) break;
      const int m = i / QL, s = i % QL;
      const float col = w[m];
      const float lo_j = loc[m], st_j = stc[m];
      const float safe = (st_j == 0.0f) ? 1.0f : st_j;
      float qv = clamp_code(__builtin_rintf((col - lo_j) / safe), nm);
      if (st_j == 0.0f) qv = 0.0f;
      const float wq = f16_round(lo_j + qv * st_j);
      const float ujj = su[i * USTR + s * QSTR + m];
      const float e = (col - wq) / ujj;
      const float eb = quad_bcast(e, s);
      if (q == s) {
        er[m] = e;
        cq[m >> 2] |= ((uint32_t)qv & 0xffu) << (8 * (m & 3));
        if (comp) comp[r * K + i1 + i] = col;
      }
      const float* urow = qrow + i * USTR;
#pragma unroll
      for (int mm = (i + 1) / QL; mm < CPL; ++mm) w[mm] = w[mm] - eb * urow[mm];
    }

#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int c = QL * m + q;
      if (c < L) {
        err1[r * lde + c] = er[m];
        codes[r * K + i1 + c] = (uint8_t)((cq[m >> 2] >> (8 * (m & 3))) & 0xffu);
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Cross-block update on fp32 MFMA.
//
//   wc[r, c] -= sum_k err1[r, t*128 + k] * U_g[i1 + 128t + k, c]     (t = 0..nblk-1, in order)
//
// Each product is accumulated from zero with v_mfma_f32_32x32x2_f32, which evaluates
// fma(a1, b1, fma(a0, b0, acc)) in k order: the same sequential fp32 FMA chain as the
// reference's CPU GEMM, then one subtraction per block.  The wc tile stays in registers
// across the nblk blocks (lazy batching of the far columns) and every block's product
// is subtracted separately, so the result equals the per-block schedule bit for bit.
// Workgroup tile 128 x 128 (4 waves as 2 x 2 of 64 x 64), rank streamed in chunks of
// 16 through LDS.  Rows of another group than the pass's are masked in A and left
// untouched in the epilogue.
// ---------------------------------------------------------------------------------
constexpr int TM = 128, TN = 128, KC = 16;

__global__ __launch_bounds__(256) void gptq_trailing_kernel(
    float* __restrict__ wc, int64_t N, int64_t K, int64_t i1, int nblk,
    const float* __restrict__ err1, int64_t lde, int64_t c0, int64_t c1,
    const int32_t* __restrict__ row_grp, const int64_t* __restrict__ u_ptrs) {
  __shared__ float As[KC][TM];
  __shared__ float Bs[KC][TN];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  const int64_t r0 = (int64_t)blockIdx.y * TM;
  const int64_t cc0 = c0 + (int64_t)blockIdx.x * TN;
  const int64_t rlast = ((r0 + TM < N) ? r0 + TM : N) - 1;
  const int g0 = row_grp[r0], g1 = row_grp[rlast];

  // C tile in the MFMA accumulator layout: tile (a, b), register j, lane l ->
  // row 8*(j/4) + 4*(l/32) + j%4 (+32a, +64wr), col l%32 (+32b, +64wcn).
  f32x16 cv[2][2];
  const int64_t row_base = r0 + wr * 64 + 4 * (lane >> 5);
  const int64_t col_base = cc0 + wcn * 64 + (lane & 31);
#define TROW(a, j) (row_base + (a) * 32 + 8 * ((j) >> 2) + ((j) & 3))
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t cc = col_base + b * 32;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t rr = TROW(a, j);
        cv[a][b][j] = (rr < N && cc < c1) ? wc[rr * K + cc] : 0.0f;
      }
    }

  for (int g = g0; g <= g1; ++g) {
    const float* U = reinterpret_cast<const float*>(u_ptrs[g]);
    for (int t = 0; t < nblk; ++t) {
      const int64_t ib = i1 + (int64_t)t * LMAX;
      const int L = (int)((K - ib < LMAX) ? K - ib : LMAX);
      f32x16 acc[2][2];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;

      for (int kk = 0; kk < L; kk += KC) {
        __syncthreads();
        {  // A chunk: As[k][m] = err1[r0+m, t*128 + kk + k] (rows of group g only)
          const int m = tid >> 1, h = tid & 1;
          const int64_t rr = r0 + m;
          const bool ok = rr < N && row_grp[rr] == g;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int k = h * 8 + j;
            As[k][m] = (ok && kk + k < L) ? err1[rr * lde + t * LMAX + kk + k] : 0.0f;
          }
        }
        {  // B chunk: Bs[k][n] = U[ib + kk + k, cc0 + n]
          const int k = tid >> 4, nb = (tid & 15) * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int64_t cc = cc0 + nb + j;
            Bs[k][nb + j] = (kk + k < L && cc < c1) ? U[(ib + kk + k) * K + cc] : 0.0f;
          }
        }
        __syncthreads();
#pragma unroll
        for (int k2 = 0; k2 < KC; k2 += 2) {
          const int kr = k2 + (lane >> 5);
          float av[2], bv[2];
#pragma unroll
          for (int a = 0; a < 2; ++a) av[a] = As[kr][wr * 64 + a * 32 + (lane & 31)];
#pragma unroll
          for (int b = 0; b < 2; ++b) bv[b] = Bs[kr][wcn * 64 + b * 32 + (lane & 31)];
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
              acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
      }
      if (g0 == g1) {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int j = 0; j < 16; ++j) cv[a][b][j] = cv[a][b][j] - acc[a][b][j];
      } else {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int64_t rr = TROW(a, j);
            const bool mine = rr < N && row_grp[rr] == g;
#pragma unroll
            for (int b = 0; b < 2; ++b)
              cv[a][b][j] = mine ? cv[a][b][j] - acc[a][b][j] : cv[a][b][j];
          }
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t cc = col_base + b * 32;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t rr = TROW(a, j);
        if (rr < N && cc < c1) wc[rr * K + cc] = cv[a][b][j];
      }
    }
#undef TROW
}

int launch_block(const float* wc, int64_t n, int64_t k, int64_t i1, int64_t len, float* err1,
                 int64_t lde, uint8_t* codes, const float* lo, const float* st, int64_t ldp,
                 const int32_t* row_grp, const int64_t* u_ptrs, const int32_t* blk,
                 const float* nmax, float* comp, hipStream_t s) {
  const dim3 grid((unsigned)((n + RPG - 1) / RPG));
  hipLaunchKernelGGL(gptq_block_kernel, grid, dim3(RPG * QL), 0, s, wc, n, k, i1, (int)len,
                     err1, lde, codes, lo, st, ldp, row_grp, u_ptrs, blk, nmax, comp);
  return launch_status("gptq_block_kernel");
}

int launch_trailing(float* wc, int64_t n, int64_t k, int64_t i1, int nblk, const float* err1,
                    int64_t lde, int64_t c0, int64_t c1, const int32_t* row_grp,
                    const int64_t* u_ptrs, hipStream_t s) {
  if (c1 <= c0 || n == 0) return HI2X_OK;
  const dim3 grid((unsigned)((c1 - c0 + TN - 1) / TN), (unsigned)((n + TM - 1) / TM));
  hipLaunchKernelGGL(gptq_trailing_kernel, grid, dim3(256), 0, s, wc, n, k, i1, nblk, err1,
                     lde, c0, c1, row_grp, u_ptrs);
  return launch_status("gptq_trailing_kernel");
}

}  // namespace
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
