// Damped Cholesky chain of inverse_factor (hi2/hessian.py:71-86) on gfx950.
//
// The reference evaluates U = chol_upper(sym(cholesky_inverse(chol(H)))) with
// H = Hs + lam I: three O(K^3) passes (4K^3/3 flops).  The same matrix is
//   U = (J L J)^-1 = J L^-1 J,   L = chol(J H J),   J = the reversal permutation,
// because J L J is upper triangular with H = (J L J)(J L J)^T, so (J L J)^-1 is the
// upper triangular factor of H^-1 with positive diagonal, which is unique.  Only L^-1
// is needed, never L: 2K^3/3 flops.
//
// L^-1 is built recursively on P = J H J, in place in its lower triangle:
//   leaf (n <= 128): one workgroup runs the same recursion on the block in LDS down to
//     16 x 16 bases, each one wave's fused factor-and-invert sweep in registers; a node
//     of up to 256 columns (two leaves and its four products) is one workgroup too;
//   node [A11 0; A21 A22], n1 + n2 = n, after inv_chol(A11) left A11 = L11^-1:
//     T1  = A21 A11^T               (= L21)
//     A22 = A22 - T1 T1^T           (lower triangle)
//     inv_chol(A22)                 (A22 = L22^-1)
//     T2  = T1 A11                  (= L21 L11^-1)
//     A21 = -A22 T2                 (= -L22^-1 L21 L11^-1, the lower-left block of L^-1)
//   every product on the fp32 MFMA GEMM of mfma_gemm.h with triangular operands masked.
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>
#include <vector>

#include "mfma_gemm.h"

namespace hi2x {
namespace {

constexpr int NB = 128;  // leaf size

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_u16(const uint16_t* base, int64_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, (int)(n * 2),
                                           0x00020000);
}

// ---- triangular GEMM ----------------------------------------------------------------
// C[M, N] = alpha * A[M, Kd] * op(B) + beta * C (beta 0 or 1).
// AMODE 1: A lower triangular.  BMODE 1 / 2: op(B) lower / upper triangular.
// TB: B is given as [N, Kd] (op(B) = B^T).  CLOW: only the lower triangle of C.
struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, Kd, lda, ldb, ldc;
  float alpha, beta;
  int64_t sA = 0, sB = 0, sC = 0;  // batch strides (elements): operand z at + z * s
};

struct MaskLower {  // keep (r, k) with k <= r
  static constexpr bool kElem = true;
  __device__ __forceinline__ bool row(int64_t) const { return true; }
  __device__ __forceinline__ bool elem(int64_t r, int64_t k) const { return k <= r; }
};
struct MaskUpper {  // keep (r, k) with k >= r
  static constexpr bool kElem = true;
  __device__ __forceinline__ bool row(int64_t) const { return true; }
  __device__ __forceinline__ bool elem(int64_t r, int64_t k) const { return k >= r; }
};

// where the heavy tiles of each product are (its rank grows along rows or columns)
template <int AMODE, int BMODE>
constexpr int tri_order() {
  return AMODE == 1 ? 1 : (BMODE == 2 ? 2 : (BMODE == 1 ? 3 : 0));
}

// rank range [kbeg, kend) of output tile (r0, c0): the triangular operand's nonzeros
template <int AMODE, int BMODE>
__host__ __device__ inline void tri_krange(int64_t r0, int64_t c0, int64_t T, int64_t Kd,
                                           int64_t& kbeg, int64_t& kend) {
  kbeg = 0;
  kend = Kd;
  if (AMODE == 1) kend = (r0 + T < kend) ? r0 + T : kend;
  if (BMODE == 1) kbeg = c0;
  if (BMODE == 2) kend = (c0 + T < kend) ? c0 + T : kend;
}

// One output tile of the product (workgroup bid of the launch's tile mapping).
template <int AMODE, int BMODE, bool TB, bool CLOW, int T>
__device__ __forceinline__ void tri_gemm_tile(const GemmArgs& g0, MgSmemT<T>& sm, int64_t tm,
                                              int64_t tn, int super, const MgSched& sched,
                                              int64_t bid) {
  constexpr int NA = T / 64;
  GemmArgs g = g0;
  g.A += (int64_t)blockIdx.z * g.sA;
  g.B += (int64_t)blockIdx.z * g.sB;
  g.C += (int64_t)blockIdx.z * g.sC;
  int64_t tr, tc;
  if (sched.per_xcd > 0) {
    if (!mg_sched_tile<CLOW>(bid, sched, tm, tn, tr, tc)) return;
  } else if (super) {
    if (!mg_super_tile<tri_order<AMODE, BMODE>(), CLOW>(bid, tm, tn, tr, tc)) return;
  } else {
    const int64_t t = xcd_tile(bid, tm * tn);
    if (t < 0) return;
    tr = t / tn;
    tc = t % tn;
  }
  const int64_t r0 = tr * T, c0 = tc * T;
  if (CLOW && c0 > r0 + T - 1) return;
  int64_t kbeg, kend;
  tri_krange<AMODE, BMODE>(r0, c0, T, g.Kd, kbeg, kend);
  f32x16 acc[NA][NA];
  mg_zero<NA>(acc);
  using AMask = typename std::conditional<AMODE == 1, MaskLower, NoMask>::type;
  RowsLoader<AMask, T> al{g.A, g.lda, g.M, kend, AMask{}};
  if (TB) {
    // op(B)[k][j] = B[j][k]: lower op(B) keeps k >= j, upper keeps k <= j
    using BMask = typename std::conditional<
        BMODE == 1, MaskUpper, typename std::conditional<BMODE == 2, MaskLower, NoMask>::type>::type;
    RowsLoader<BMask, T> bl{g.B, g.ldb, g.N, kend, BMask{}};
    mg_mainloop<NA, T>(acc, sm, al, bl, r0, c0, kbeg, kend);
  } else {
    // op(B)[k][c] = B[k][c]: lower keeps c <= k (mask(k, c)), upper keeps c >= k
    using BMask = typename std::conditional<
        BMODE == 1, MaskLower, typename std::conditional<BMODE == 2, MaskUpper, NoMask>::type>::type;
    ColsLoader<BMask, T> bl{g.B, g.ldb, g.N, kend, BMask{}};
    mg_mainloop<NA, T>(acc, sm, al, bl, r0, c0, kbeg, kend);
  }
  const CTile<T> ct(g.C, g.ldc, g.M, g.N, r0, c0);
  f32x16 cv[NA][NA];
  if (g.beta != 0.0f) {
    ct.load(cv);
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < NA; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) cv[a][b][j] = cv[a][b][j] + g.alpha * acc[a][b][j];
  } else {
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < NA; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) cv[a][b][j] = g.alpha * acc[a][b][j];
  }
  ct.store(cv, [&](int a, int j, int b) {
    return !CLOW || c0 + mg_col<T>(b) <= r0 + mg_row<T>(a, j);
  });
}

template <int AMODE, int BMODE, bool TB, bool CLOW, int T>
__global__ __launch_bounds__(256) void tri_gemm_kernel(GemmArgs g0, int64_t tm, int64_t tn,
                                                       int super, MgSched sched) {
  __shared__ MgSmemT<T> sm;
  tri_gemm_tile<AMODE, BMODE, TB, CLOW, T>(g0, sm, tm, tn, super, sched, blockIdx.x);
}

// Two independent small products in one launch (64-tiles, xcd-spread tiles): workgroups
// [0, grid1) run the first, the rest the second.  The recursion pairs A22 -= T1 T1^T with
// T2 = T1 A11, which needs the same inputs and none of the other's output.
template <int A1, int B1, bool TB1, bool C1, int A2, int B2, bool TB2, bool C2>
__global__ __launch_bounds__(256) void tri_gemm_pair_kernel(GemmArgs g1, int64_t tm1,
                                                            int64_t tn1, int64_t grid1,
                                                            GemmArgs g2, int64_t tm2,
                                                            int64_t tn2) {
  __shared__ MgSmemT<64> sm;
  const int64_t bid = blockIdx.x;
  if (bid < grid1)
    tri_gemm_tile<A1, B1, TB1, C1, 64>(g1, sm, tm1, tn1, 0, MgSched{}, bid);
  else
    tri_gemm_tile<A2, B2, TB2, C2, 64>(g2, sm, tm2, tn2, 0, MgSched{}, bid - grid1);
}

// ---- products of the big levels on fp16 MFMA through a scaled two-way split ----------
// Every fp32 operand row is scaled by a power of two, s_r = 2^(14 - e_r) with
// e_r = floor(log2 max_k |x[r][k]|), which puts the row's largest element in [2^14, 2^15)
// (inside fp16's range), and written once, before the product, as two fp16 planes
// x1 = fp16(s_r x), x2 = fp16(s_r x - x1) (the difference is exact in fp32): s_r x =
// x1 + x2 to within 2^-22 of the row's largest element.  The planes are laid out
// [row][k] with k contiguous (a transposed copy where the product needs one; stored in
// chunks of 16 k), the operand's structural zeros written as zeros.  The product keeps
// the three terms x1 y1 + x1 y2 + x2 y1 (the dropped x2 y2 is below 2^-22 of the largest
// |x_k y_k|); fp16 products are exact and v_mfma_f32_32x32x16_f16 accumulates in fp32,
// and the epilogue multiplies by 1 / (s_r s_c) (exact: powers of two).  Three MFMAs of 32
// cycles cover 16 k where the fp32 MFMA needs eight of 64, with the rounding of an fp32
// GEMM (not bit-identical to one).

// Operand row maxima: G2_NS slices of the rank, one partial per (slice, row).
constexpr int G2_NS = 16;
constexpr int G3_NP = 2;  // planes per operand

__device__ __forceinline__ int split_load_block(float (&t)[64][65], const float* X, int64_t ldx,
                                                int64_t R, int64_t Kk, int trans, int64_t r0,
                                                int64_t k0) {
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  // input block: rows of X are contiguous along k (!trans) or along r (trans)
  const int64_t xr0 = trans ? k0 : r0, xc0 = trans ? r0 : k0;
  const int64_t xrows = trans ? Kk : R, xcols = trans ? R : Kk;
  const int rows = (int)((xrows - xr0 < 64) ? (xrows - xr0 > 0 ? xrows - xr0 : 0) : 64);
  const int cols = (int)((xcols - xc0 < 64) ? (xcols - xc0 > 0 ? xcols - xc0 : 0) : 64);
  const __amdgpu_buffer_rsrc_t rs =
      mg_rsrc(X + xr0 * ldx + xc0, rows > 0 && cols > 0 ? (int64_t)(rows - 1) * ldx + cols : 0);
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int y = ty + 4 * q;
    const uint32_t off = (y < rows && tx < cols) ? (uint32_t)(((int64_t)y * ldx + tx) * 4) : MG_OOB;
    t[y][tx] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0));
  }
  return 0;
}

__device__ __forceinline__ bool split_keep(int mask, int64_t r, int64_t k) {
  return mask == 1 ? k <= r : (mask == 2 ? k >= r : true);
}

// Grid (G2_NS, row groups): slice s covers k in [s L, (s + 1) L), L = ceil(Kk / G2_NS)
// rounded up to a multiple of 256.  !trans (operand rows contiguous): one wave per row,
// each lane 16-byte pieces along k; trans (operand rows are columns of X): 256 rows per
// workgroup, each lane a 16-byte piece of 4 rows, the four waves taking every fourth k,
// combined through LDS.  Loads go through buffer resources that end at the last valid
// element (past it they read zero).  VEC: X and ldx allow 16-byte pieces (else 4-byte
// loads).  mask as in split2_kernel.
// One operand of a split: rows R of X (layouts as in split2_kernel) into the planes at out.
struct SplitOp {
  const float* X;
  int64_t ldx, R, Kk, Kp, sx, sout;  // batch strides sx (floats) and sout (16-bit values)
  int trans, mask;
  uint16_t* out;
};

// The operand of this workgroup: grid rows below y0 belong to o0, the rest to o1 (two
// operands of a product split by one launch); by is the row group within the operand.
__device__ __forceinline__ SplitOp split_operand(const SplitOp& o0, const SplitOp& o1, int y0,
                                                 int64_t& by) {
  const bool second = (int)blockIdx.y >= y0;
  by = second ? (int64_t)blockIdx.y - y0 : (int64_t)blockIdx.y;
  return second ? o1 : o0;
}

template <bool VEC>
__global__ __launch_bounds__(256) void rowmax_kernel(SplitOp o0, SplitOp o1, int y0) {
  int64_t by;
  const SplitOp o = split_operand(o0, o1, y0, by);
  const float* __restrict__ X = o.X + (int64_t)blockIdx.z * o.sx;
  const int64_t ldx = o.ldx, R = o.R, Kk = o.Kk;
  const int trans = o.trans, mask = o.mask;
  float* __restrict__ pm =
      reinterpret_cast<float*>(o.out + (int64_t)blockIdx.z * o.sout + G3_NP * R * o.Kp) + R;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t L = ((Kk + G2_NS - 1) / G2_NS + 255) / 256 * 256;
  const int64_t ks = (int64_t)blockIdx.x * L;
  const int64_t ke = (ks + L < Kk) ? ks + L : Kk;
  float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // fmaxf skips NaN elements
  auto take = [&](int i, float x, int64_t r, int64_t k) {
    m[i] = (k < ke && split_keep(mask, r, k)) ? fmaxf(m[i], fabsf(x)) : m[i];
  };
  if (!trans) {
    const int64_t r = by * 4 + wave;
    if (r >= R) return;
    if (ks < ke) {
      const __amdgpu_buffer_rsrc_t rs = mg_rsrc(X + r * ldx + ks, ke - ks);
      for (int64_t k0 = 0; k0 < ke - ks; k0 += 256) {
        const int64_t k = k0 + 4 * lane;
        if (VEC) {
          const f32x4 v = mg_load4(rs, (uint32_t)(k * 4));
#pragma unroll
          for (int i = 0; i < 4; ++i) take(i, v[i], r, ks + k + i);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            take(i, __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)((k + i) * 4), 0, 0)), r, ks + k + i);
        }
      }
    }
    float mm = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) mm = fmaxf(mm, __shfl_xor(mm, sh));
    if (lane == 0) pm[blockIdx.x * R + r] = mm;
    return;
  }
  __shared__ float part[4][256];
  const int64_t rb = by * 256, r = rb + 4 * lane;
  const int nr = (int)((R - rb < 256) ? R - rb : 256);
  if (ks < ke) {
    const __amdgpu_buffer_rsrc_t rs = mg_rsrc(X + ks * ldx + rb, (ke - ks - 1) * ldx + nr);
#pragma unroll 8
    for (int64_t k = wave; k < ke - ks; k += 4) {
      const uint32_t o = 4 * lane < nr ? (uint32_t)((k * ldx + 4 * lane) * 4) : MG_OOB;
      if (VEC) {
        const f32x4 v = mg_load4(rs, o);
#pragma unroll
        for (int i = 0; i < 4; ++i) take(i, v[i], r + i, ks + k);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          take(i, __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, o == MG_OOB ? (int)MG_OOB : (int)(o + 4 * i), 0, 0)), r + i, ks + k);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave][4 * lane + i] = m[i];
  __syncthreads();
  const int c = threadIdx.x;
  if (c < nr)
    pm[blockIdx.x * R + rb + c] = fmaxf(fmaxf(part[0][c], part[1][c]), fmaxf(part[2][c], part[3][c]));
}

// Planes of R x Kp fp16 from X, each stored in chunks of 16 k: element (r, k) of plane p
// at out[p][k / 16][r][k % 16] (a chunk of a tile's rows is contiguous, so the product
// reads whole cache lines), followed by the R inverse row scales 1 / s_r (fp32) and the
// row maxima partials of rowmax_kernel ([slice][R]).  !trans: x = X[r][k] (X is R x Kk,
// ld ldx), trans: x = X[k][r] (X is Kk x R).  mask 1 keeps k <= r, 2 keeps k >= r; k >= Kk
// and masked elements are zero.  A workgroup converts a 64 x 64 block through LDS: 4
// threads per output row, 16 consecutive k (one chunk row) each.
__global__ __launch_bounds__(256) void split2_kernel(SplitOp o0, SplitOp o1, int y0) {
  __shared__ float t[64][65];
  int64_t by;
  const SplitOp o = split_operand(o0, o1, y0, by);
  const float* __restrict__ X = o.X + (int64_t)blockIdx.z * o.sx;
  uint16_t* __restrict__ out = o.out + (int64_t)blockIdx.z * o.sout;
  const int64_t ldx = o.ldx, R = o.R, Kk = o.Kk, Kp = o.Kp;
  const int trans = o.trans, mask = o.mask;
  const int64_t r0 = by * 64, k0 = (int64_t)blockIdx.x * 64;
  if (k0 >= Kp) return;  // the other operand of the launch has more rank
  split_load_block(t, X, ldx, R, Kk, trans, r0, k0);
  __syncthreads();
  const int orow = threadIdx.x >> 2, kq = threadIdx.x & 3;  // output row, 16-k quarter
  const int64_t r = r0 + orow;
  if (r >= R) return;
  float* inv = reinterpret_cast<float*>(out + G3_NP * R * Kp);
  const float* pm = inv + R;
  float m = 0.0f;  // the row's maximum: four partials per thread, then over the row's lanes
#pragma unroll
  for (int i = 0; i < G2_NS / 4; ++i) m = fmaxf(m, pm[(G2_NS / 4 * kq + i) * R + r]);
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  int ex = 0;
  (void)frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1): floor(log2 m) = ex - 1
  // e in [-100, 127]: the scale 2^(14 - e) and its inverse stay normal for every finite m
  const int e = m > 0.0f ? (ex - 1 < -100 ? -100 : (ex - 1 > 127 ? 127 : ex - 1)) : 0;
  const float sc = ldexpf(1.0f, 14 - e);
  if (blockIdx.x == 0 && kq == 0) inv[r] = ldexpf(1.0f, e - 14);
  mg_u16x8 p1[2], p2[2];
#pragma unroll
  for (int e2 = 0; e2 < 16; ++e2) {
    const int kk = 16 * kq + e2;
    float x = trans ? t[kk][orow] : t[orow][kk];
    x = split_keep(mask, r, k0 + kk) ? x * sc : 0.0f;
    const _Float16 h1 = (_Float16)x;
    const _Float16 h2 = (_Float16)(x - (float)h1);
    p1[e2 >> 3][e2 & 7] = __builtin_bit_cast(unsigned short, h1);
    p2[e2 >> 3][e2 & 7] = __builtin_bit_cast(unsigned short, h2);
  }
  const int64_t kb = k0 + 16 * kq;
  if (kb >= Kp) return;
  const int64_t plane = R * Kp;
  uint16_t* dst = out + ((kb >> 4) * R + r) * 16;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    *reinterpret_cast<mg_u16x8*>(dst + 8 * g) = p1[g];
    *reinterpret_cast<mg_u16x8*>(dst + plane + 8 * g) = p2[g];
  }
}

// The planes and inverse row scales of split2_kernel, for a row-major operand (!trans),
// in one pass over it (rowmax_kernel and split2_kernel read the operand twice): one wave
// per row, the row in registers (lane l holds k = 4 (l + 64 q) .. + 3 for q < NV, so each
// load instruction reads 1 KB of the row), its maximum by a wave reduction, then both
// planes.  The same elements, maxima and conversions as the pair, so the same bits.  No
// LDS, so the workgroups share CUs with whatever else runs.  Grid (1, groups of 4 rows of
// o0 then of o1, batch); X and ldx allow 16-byte loads (the host checks).
constexpr int SR_NV_MAX = 28;  // rank up to 7168 (28 x 256)

template <int NV>
__global__ __launch_bounds__(256) void split_rows_kernel(SplitOp o0, SplitOp o1, int y0) {
  int64_t by;
  const SplitOp o = split_operand(o0, o1, y0, by);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t R = o.R, r = by * 4 + wave;
  if (r >= R) return;
  const float* __restrict__ X = o.X + (int64_t)blockIdx.z * o.sx;
  uint16_t* __restrict__ out = o.out + (int64_t)blockIdx.z * o.sout;
  const int64_t Kp = o.Kp;
  const int mask = o.mask;
  const __amdgpu_buffer_rsrc_t rs = mg_rsrc(X + r * o.ldx, o.Kk);  // k >= Kk reads zero
  f32x4 v[NV];
#pragma unroll
  for (int q = 0; q < NV; ++q) v[q] = mg_load4(rs, (uint32_t)(16 * (lane + 64 * q)));
  float m = 0.0f;  // fmaxf skips NaN elements
  const int r32 = (int)r;  // rows and ranks stay below 2^31
#pragma unroll
  for (int q = 0; q < NV; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = 4 * lane + 256 * q + e;
      const bool keep = mask == 1 ? k <= r32 : (mask == 2 ? k >= r32 : true);
      v[q][e] = keep ? v[q][e] : 0.0f;
      m = fmaxf(m, fabsf(v[q][e]));
    }
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) m = fmaxf(m, __shfl_xor(m, sh));
  int ex = 0;  // the row scale as split2_kernel forms it
  (void)frexpf(m, &ex);
  const int e = m > 0.0f ? (ex - 1 < -100 ? -100 : (ex - 1 > 127 ? 127 : ex - 1)) : 0;
  const float sc = ldexpf(1.0f, 14 - e);
  if (lane == 0) reinterpret_cast<float*>(out + G3_NP * R * Kp)[r] = ldexpf(1.0f, e - 14);
  const int64_t plane = R * Kp;
#pragma unroll
  for (int q = 0; q < NV; ++q) {
    const int k0 = 4 * lane + 256 * q;
    if (k0 >= Kp) continue;
    uint32_t p1[2], p2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t w1 = 0, w2 = 0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float x = v[q][2 * h + t] * sc;
        const _Float16 a = (_Float16)x;
        const _Float16 b = (_Float16)(x - (float)a);
        w1 |= (uint32_t)__builtin_bit_cast(unsigned short, a) << (16 * t);
        w2 |= (uint32_t)__builtin_bit_cast(unsigned short, b) << (16 * t);
      }
      p1[h] = w1;
      p2[h] = w2;
    }
    uint16_t* dst = out + ((int64_t)(k0 >> 4) * R + r) * 16 + (k0 & 15);
    *reinterpret_cast<uint2*>(dst) = make_uint2(p1[0], p1[1]);
    *reinterpret_cast<uint2*>(dst + plane) = make_uint2(p2[0], p2[1]);
  }
}

// C[M, N] = alpha * A B^T + beta * C over k in [kbeg, kend) of each 128 x 128 output tile
// (tri_krange), A and B given as split planes (16-k chunks).  Workgroup: 4 waves of
// 64 x 64 (2 x 2 accumulators), two workgroups per CU (48 KB of LDS each), so each SIMD
// has a second wave to issue MFMAs while one waits at a stage barrier.  Stages of 16 k
// go from L2 straight into LDS through a ring of three (prefetch distance two): each load
// instruction of a wave writes 1 KB = 32 rows x 2 16-byte slots of one plane, slot q of
// row r holding piece q ^ ((r / 8) % 2) so that the MFMA operand reads are free of bank
// conflicts.
struct G3Args {
  const uint16_t* A;
  const uint16_t* B;
  float* C;
  int64_t M, N, Kd, Kp, ldc;
  float alpha, beta;
  int64_t sA = 0, sB = 0, sC = 0;  // batch strides (elements): operand z at + z * s
};
constexpr int G3_KC = 16;                 // k per stage (one MFMA k-step)
constexpr int G3_KA = 32;                 // k alignment of the planes (Kp)
constexpr int G3_NB = 3;                  // stages in the ring
constexpr int G3_PL = MG_T * G3_KC;       // fp16 per plane per stage
constexpr int G3_PER_STAGE = 2 * G3_NP;   // load instructions per wave and stage (2 x 2 x 4 / 4)

typedef _Float16 mg_f16x8 __attribute__((ext_vector_type(8)));

// The inverse row scales of an operand's planes (rows x Kp per plane, then the scales)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_scales(const uint16_t* planes,
                                                               int64_t rows, int64_t Kp) {
  return mg_rsrc(reinterpret_cast<const float*>(planes + G3_NP * rows * Kp), rows);
}
__device__ __forceinline__ float scale_at(__amdgpu_buffer_rsrc_t rs, int64_t i, bool ok) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                       rs, ok ? (int)(i * 4) : (int)MG_OOB, 0, 0));
}

__device__ __forceinline__ void g3_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, void* lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(
      (uint32_t)(size_t)(__attribute__((address_space(3))) void*)lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  // as inline assembly: the compiler would otherwise take the asynchronous LDS write for
  // an alias of every later LDS read and wait for all loads in flight before each one
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(la), "v"(voff), "s"(rs)
               : "m0");
#pragma clang diagnostic pop
}

constexpr int g3_waitcnt(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

typedef uint16_t G3Stage[G3_NB][G3_NP][G3_PL];

// Output tile (tr, tc) of the product (SA, SB: the workgroup's LDS rings).
template <int AMODE, int BMODE, bool CLOW>
__device__ __forceinline__ void gemm3_tile(const G3Args& g0, G3Stage& SA, G3Stage& SB,
                                           int64_t tr, int64_t tc) {
  G3Args g = g0;
  g.A += (int64_t)blockIdx.z * g.sA;
  g.B += (int64_t)blockIdx.z * g.sB;
  g.C += (int64_t)blockIdx.z * g.sC;
  const int64_t r0 = tr * MG_T, c0 = tc * MG_T;
  if (CLOW && c0 > r0 + MG_T - 1) return;
  int64_t kbeg, kend;
  tri_krange<AMODE, BMODE>(r0, c0, MG_T, g.Kd, kbeg, kend);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  f32x16 acc[2][2];
  mg_zero<2>(acc);
  // plane p of the operand tile rows: a buffer per plane that ends at the last valid row
  const int rowsA = (int)((g.M - r0 < MG_T) ? g.M - r0 : MG_T);
  const int rowsB = (int)((g.N - c0 < MG_T) ? g.N - c0 : MG_T);
  const int64_t plA = g.M * g.Kp, plB = g.N * g.Kp;
  // load j (0..3) of a stage: operand j / 2, plane j % 2, rows 32 wv .. 32 wv + 31
  const int prow = lane >> 1, piece = (lane & 1) ^ ((lane >> 4) & 1);
  auto dma_one = [&](int j, int64_t k0, int buf, bool live) {
    const int opd = j / G3_NP, pl = j % G3_NP;
    const int row = 32 * wv + prow;
    // chunk k0 / 16 of the tile's rows: rows x 16 contiguous fp16
    const uint16_t* base = opd == 0 ? g.A + pl * plA + ((k0 >> 4) * g.M + r0) * G3_KC
                                    : g.B + pl * plB + ((k0 >> 4) * g.N + c0) * G3_KC;
    const int rows = opd == 0 ? rowsA : rowsB;
    const __amdgpu_buffer_rsrc_t rs = rsrc_u16(base, (int64_t)rows * G3_KC);
    const uint32_t o = (uint32_t)(row * G3_KC * 2 + 16 * piece);
    uint16_t* dst = opd == 0 ? &SA[buf][pl][wv * 32 * G3_KC] : &SB[buf][pl][wv * 32 * G3_KC];
    g3_dma16(rs, (live && row < rows) ? o : MG_OOB, dst);
  };
  auto dma = [&](int64_t k0, int buf, bool live) {
#pragma unroll
    for (int j = 0; j < G3_PER_STAGE; ++j) dma_one(j, k0, buf, live);
  };
  // operand reads: rows wr * 64 + 32 t + lane % 32 (A) / wcn * 64 + ... (B), piece
  // lane / 32 (k 8 h .. 8 h + 7 of the stage) in slot h ^ ((row / 8) % 2)
  const int rA = wr * 64 + (lane & 31), rB = wcn * 64 + (lane & 31);
  const int so = 8 * ((lane >> 5) ^ ((lane >> 3) & 1));
  typedef mg_f16x8 V;
  V a0[G3_NP][2], b0[G3_NP][2], a1[G3_NP][2], b1[G3_NP][2];  // [plane][tile], stage sets
  auto read = [&](V (&av)[G3_NP][2], V (&bv)[G3_NP][2], int buf) {
#pragma unroll
    for (int pl = 0; pl < G3_NP; ++pl)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        av[pl][t] = __builtin_bit_cast(V, *reinterpret_cast<const mg_u16x8*>(&SA[buf][pl][(rA + 32 * t) * G3_KC + so]));
        bv[pl][t] = __builtin_bit_cast(V, *reinterpret_cast<const mg_u16x8*>(&SB[buf][pl][(rB + 32 * t) * G3_KC + so]));
      }
  };
  // the three products of a k-step, small terms first (planes (1,0) (0,1) (0,0)), each
  // over the four tiles in turn so that consecutive MFMAs use different accumulators
  constexpr int PA[3] = {1, 0, 0}, PB[3] = {0, 1, 0};
#define G3_ONE(AV, BV, n)                                                                    \
  acc[((n) & 3) >> 1][(n) & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(                      \
      AV[PA[(n) >> 2]][((n) & 3) >> 1], BV[PB[(n) >> 2]][(n) & 1], acc[((n) & 3) >> 1][(n) & 1], \
      0, 0, 0);
  auto sync = [&]() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  // nst stages carry data; the loop runs an even count (a last stage of zeros, loaded
  // from past the end, when nst is odd) so that its body has no branch around the MFMAs
  const int nst = kend > kbeg ? (int)((kend - kbeg + G3_KC - 1) / G3_KC) : 0;
  const int nst2 = (nst + 1) & ~1;
  if (nst > 0) {
#pragma unroll
    for (int p = 0; p < G3_NB; ++p) dma(kbeg + (int64_t)p * G3_KC, p, p < nst);
    __builtin_amdgcn_s_waitcnt(g3_waitcnt(2 * G3_PER_STAGE, 15));  // stage 0 landed
    sync();
    read(a0, b0, 0);
  }
  // Stage st: wait until stage st + 1 has landed (every stage issues G3_PER_STAGE loads,
  // so that is "at most stage st + 2's loads outstanding") and this wave's reads of stage
  // st are done; after the barrier no wave reads buffer st % 3 any more.  Then the reads
  // of stage st + 1 are issued, and stage st's MFMAs run with the loads of stage st + 3
  // into buffer st % 3 in between (one after every third MFMA).
#define G3_STAGE(XA, XB, YA, YB, ST)                                                       \
  {                                                                                        \
    const int st_ = (ST);                                                                  \
    const int cb = st_ % G3_NB, nb = (st_ + 1) % G3_NB;                                    \
    __builtin_amdgcn_s_waitcnt(g3_waitcnt(G3_PER_STAGE, 0));                               \
    sync();                                                                                \
    read(YA, YB, nb);                                                                      \
    __builtin_amdgcn_sched_barrier(0);                                                     \
    const int64_t kn = kbeg + (int64_t)(st_ + G3_NB) * G3_KC;                              \
    const bool live = st_ + G3_NB < nst;                                                   \
    _Pragma("unroll") for (int n = 0; n < 12; ++n) {                                       \
      G3_ONE(XA, XB, n)                                                                    \
      if (n % 3 == 2) {                                                                    \
        dma_one(n / 3, kn, cb, live);                                                      \
        __builtin_amdgcn_sched_barrier(0);                                                 \
      }                                                                                    \
    }                                                                                      \
  }
  for (int st = 0; st < nst2; st += 2) {
    G3_STAGE(a0, b0, a1, b1, st)
    G3_STAGE(a1, b1, a0, b0, st + 1)
  }
#undef G3_STAGE
#undef G3_ONE
  // undo the row scales: acc (1 / s_r) (1 / s_c), exact (powers of two)
  {
    const __amdgpu_buffer_rsrc_t sa = plane_scales(g.A, g.M, g.Kp);
    const __amdgpu_buffer_rsrc_t sb = plane_scales(g.B, g.N, g.Kp);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t cc = c0 + mg_col<MG_T>(b);
      const float vc = scale_at(sb, cc, cc < g.N);
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int64_t rr = r0 + mg_row<MG_T>(a, j);
          acc[a][b][j] = (acc[a][b][j] * scale_at(sa, rr, rr < g.M)) * vc;
        }
    }
  }
  const CTile<MG_T> ct(g.C, g.ldc, g.M, g.N, r0, c0);
  f32x16 cv[2][2];
  if (g.beta != 0.0f) {
    ct.load(cv);
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) cv[a][b][j] = cv[a][b][j] + g.alpha * acc[a][b][j];
  } else {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j) cv[a][b][j] = g.alpha * acc[a][b][j];
  }
  ct.store(cv, [&](int a, int j, int b) {
    return !CLOW || c0 + mg_col<MG_T>(b) <= r0 + mg_row<MG_T>(a, j);
  });
  __syncthreads();  // no wave leaves while loads it issued may still write LDS
}

template <int AMODE, int BMODE, bool CLOW>
__global__ __launch_bounds__(256, 2) void gemm3_kernel(G3Args g0, int64_t tm, int64_t tn,
                                                       MgSched sched) {
  __shared__ __attribute__((aligned(1024))) G3Stage SA;
  __shared__ __attribute__((aligned(1024))) G3Stage SB;
  int64_t tr, tc;
  if (sched.per_xcd > 0) {
    if (!mg_sched_tile<CLOW>(blockIdx.x, sched, tm, tn, tr, tc)) return;
  } else {
    const int64_t t = xcd_tile(blockIdx.x, tm * tn);
    if (t < 0) return;
    tr = t / tn;
    tc = t % tn;
  }
  gemm3_tile<AMODE, BMODE, CLOW>(g0, SA, SB, tr, tc);
}

// Two products in one launch on 128-tiles: the table as gemm3x_pair_kernel's (GxPair),
// over super-tiles of MG_SUP x MG_SUP tiles.
struct GxPair {
  int32_t per_xcd = 0;
  int32_t nsc[2] = {0, 0};
  uint16_t st[MG_SCHED_MAX] = {};
};

template <int A1, int B1, bool C1, int A2, int B2, bool C2>
__global__ __launch_bounds__(256, 2) void gemm3_pair_kernel(G3Args g1, int64_t tm1, int64_t tn1,
                                                            G3Args g2, int64_t tm2, int64_t tn2,
                                                            GxPair sched) {
  __shared__ __attribute__((aligned(1024))) G3Stage SA;
  __shared__ __attribute__((aligned(1024))) G3Stage SB;
  const int x = (int)(blockIdx.x & 7);
  const int64_t slot = blockIdx.x >> 3;
  const int j = (int)(slot / (MG_SUP * MG_SUP)), w = (int)(slot % (MG_SUP * MG_SUP));
  if (j >= sched.per_xcd) return;
  const int u = sched.st[x * sched.per_xcd + j];
  if (u == 0xffff) return;
  const int p = u >> 15, id = u & 0x7fff, nsc = sched.nsc[p];
  const int64_t tr = (int64_t)(id / nsc) * MG_SUP + w / MG_SUP;
  const int64_t tc = (int64_t)(id % nsc) * MG_SUP + w % MG_SUP;
  if (p == 0) {
    if (tr >= tm1 || tc >= tn1 || (C1 && tc > tr)) return;
    gemm3_tile<A1, B1, C1>(g1, SA, SB, tr, tc);
  } else {
    if (tr >= tm2 || tc >= tn2 || (C2 && tc > tr)) return;
    gemm3_tile<A2, B2, C2>(g2, SA, SB, tr, tc);
  }
}

// The same product on 256 x 256 tiles for the largest grids: one workgroup of 8 waves per
// CU, each wave 128 x 64 (4 x 2 accumulators), on the planes' three-stage ring of 32 KB
// stages.  Per 16 k a wave reads 12 fragment planes for 24 MFMAs (gemm3_kernel: 8 for 12)
// and the CU brings 32 KB into LDS per 16 k of a 256 x 256 tile (gemm3_kernel: 2 x 16 KB
// per 16 k of two 128 x 128 tiles), half the LDS and L2 traffic per MFMA.  Each output
// element accumulates the same terms in the same order as in gemm3_kernel (a 256-tile may
// run some stages more than a 128-tile of it, whose masked planes add exact zeros) and
// is scaled the same way.
constexpr int GX_T = 256;                // tile edge
constexpr int GX_SUP = 4;                // super-tile edge of the balanced schedule (tiles)
constexpr int GX_PL = GX_T * G3_KC;      // fp16 per plane per stage

typedef uint16_t GxStage[G3_NB][G3_NP][GX_PL];

// Output tile (tr, tc) of the product (SA, SB: the workgroup's LDS rings).
template <int AMODE, int BMODE, bool CLOW>
__device__ __forceinline__ void gemm3x_tile(const G3Args& g0, GxStage& SA, GxStage& SB,
                                            int64_t tr, int64_t tc) {
  G3Args g = g0;
  g.A += (int64_t)blockIdx.z * g.sA;
  g.B += (int64_t)blockIdx.z * g.sB;
  g.C += (int64_t)blockIdx.z * g.sC;
  const int64_t r0 = tr * GX_T, c0 = tc * GX_T;
  if (CLOW && c0 > r0 + GX_T - 1) return;
  int64_t kbeg, kend;
  tri_krange<AMODE, BMODE>(r0, c0, GX_T, g.Kd, kbeg, kend);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 2, wc = wave & 3;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;
  const int rowsA = (int)((g.M - r0 < GX_T) ? g.M - r0 : GX_T);
  const int rowsB = (int)((g.N - c0 < GX_T) ? g.N - c0 : GX_T);
  const int64_t plA = g.M * g.Kp, plB = g.N * g.Kp;
  // load j (0..3) of a stage: operand j / 2, plane j % 2, rows 32 wv .. 32 wv + 31 (the
  // slot swizzle of gemm3_kernel)
  const int prow = lane >> 1, piece = (lane & 1) ^ ((lane >> 4) & 1);
  auto dma_one = [&](int j, int64_t k0, int buf, bool live) {
    const int opd = j / G3_NP, pl = j % G3_NP;
    const int row = 32 * wv + prow;
    const uint16_t* base = opd == 0 ? g.A + pl * plA + ((k0 >> 4) * g.M + r0) * G3_KC
                                    : g.B + pl * plB + ((k0 >> 4) * g.N + c0) * G3_KC;
    const int rows = opd == 0 ? rowsA : rowsB;
    const __amdgpu_buffer_rsrc_t rs = rsrc_u16(base, (int64_t)rows * G3_KC);
    const uint32_t o = (uint32_t)(row * G3_KC * 2 + 16 * piece);
    uint16_t* dst = opd == 0 ? &SA[buf][pl][wv * 32 * G3_KC] : &SB[buf][pl][wv * 32 * G3_KC];
    g3_dma16(rs, (live && row < rows) ? o : MG_OOB, dst);
  };
  // fragment reads: A rows wr * 128 + 32 ta + lane % 32, B rows (output columns) wc * 64 +
  // 32 tb + lane % 32, piece lane / 32 in slot h ^ ((row / 8) % 2)
  const int so = 8 * ((lane >> 5) ^ ((lane >> 3) & 1));
  const int rA = wr * 128 + (lane & 31), rB = wc * 64 + (lane & 31);
  typedef mg_f16x8 V;
  auto rdA = [&](V (&av)[G3_NP][4], int pl, int buf) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      av[pl][t] = __builtin_bit_cast(V, *reinterpret_cast<const mg_u16x8*>(&SA[buf][pl][(rA + 32 * t) * G3_KC + so]));
  };
  auto rdB = [&](V (&bv)[G3_NP][2], int pl, int buf) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
      bv[pl][t] = __builtin_bit_cast(V, *reinterpret_cast<const mg_u16x8*>(&SB[buf][pl][(rB + 32 * t) * G3_KC + so]));
  };
  constexpr int PA[3] = {1, 0, 0}, PB[3] = {0, 1, 0};
  auto term = [&](auto P, const V (&av)[G3_NP][4], const V (&bv)[G3_NP][2]) {
    constexpr int pr = decltype(P)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[i >> 1][i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          av[PA[pr]][i >> 1], bv[PB[pr]][i & 1], acc[i >> 1][i & 1], 0, 0, 0);
  };
  auto sync = [&]() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  const int nst = kend > kbeg ? (int)((kend - kbeg + G3_KC - 1) / G3_KC) : 0;
  const int nst2 = (nst + 1) & ~1;
  V a0[G3_NP][4], b0[G3_NP][2], a1[G3_NP][4], b1[G3_NP][2];  // [plane][tile], stage sets
  if (nst > 0) {
#pragma unroll
    for (int p = 0; p < G3_NB; ++p) {
#pragma unroll
      for (int j = 0; j < G3_PER_STAGE; ++j) dma_one(j, kbeg + (int64_t)p * G3_KC, p, p < nst);
    }
    __builtin_amdgcn_s_waitcnt(g3_waitcnt(2 * G3_PER_STAGE, 15));  // stage 0 landed
    sync();
#pragma unroll
    for (int pl = 0; pl < G3_NP; ++pl) {
      rdA(a0, pl, 0);
      rdB(b0, pl, 0);
    }
  }
  // Stage st (planes x): wait until stage st + 1 has landed and every wave's reads of
  // stage st (made during stage st - 1) are done, then the reads of the next stage and
  // the three terms, with the four DMAs of stage st + 3 into buffer st % 3 between them.
  auto stage = [&](const V (&xa)[G3_NP][4], const V (&xb)[G3_NP][2], V (&ya)[G3_NP][4],
                   V (&yb)[G3_NP][2], int st) {
    const int cb = st % G3_NB, nb = (st + 1) % G3_NB;
    __builtin_amdgcn_s_waitcnt(g3_waitcnt(G3_PER_STAGE, 0));
    sync();
#pragma unroll
    for (int pl = 0; pl < G3_NP; ++pl) {
      rdB(yb, pl, nb);
      rdA(ya, pl, nb);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int64_t kn = kbeg + (int64_t)(st + G3_NB) * G3_KC;
    const bool live = st + G3_NB < nst;
    term(std::integral_constant<int, 0>{}, xa, xb);
    dma_one(0, kn, cb, live);
    __builtin_amdgcn_sched_barrier(0);
    term(std::integral_constant<int, 1>{}, xa, xb);
    dma_one(1, kn, cb, live);
    dma_one(2, kn, cb, live);
    __builtin_amdgcn_sched_barrier(0);
    term(std::integral_constant<int, 2>{}, xa, xb);
    dma_one(3, kn, cb, live);
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int st = 0; st < nst2; st += 2) {
    stage(a0, b0, a1, b1, st);
    stage(a1, b1, a0, b0, st + 1);
  }
  // C = alpha acc (+ C): register j of tile (ta, tb) at row wr * 128 + 32 ta + 8 (j / 4) +
  // 4 (lane / 32) + j % 4, column wc * 64 + 32 tb + lane % 32; rows and columns outside
  // C, and with CLOW the elements above the diagonal, are left alone
  const __amdgpu_buffer_rsrc_t rc = mg_rsrc(g.C + r0 * g.ldc + c0, (int64_t)(rowsA - 1) * g.ldc + rowsB);
  const __amdgpu_buffer_rsrc_t sa = plane_scales(g.A, g.M, g.Kp);
  const __amdgpu_buffer_rsrc_t sb = plane_scales(g.B, g.N, g.Kp);
  const int lr0 = wr * 128 + 4 * (lane >> 5), lc0 = wc * 64 + (lane & 31);
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const int cc = lc0 + 32 * tb;
    const float vc = scale_at(sb, c0 + cc, cc < rowsB);
#pragma unroll
    for (int ta = 0; ta < 4; ++ta)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int rr = lr0 + 32 * ta + 8 * (j >> 2) + (j & 3);
        const bool ok = rr < rowsA && cc < rowsB && (!CLOW || c0 + cc <= r0 + rr);
        const uint32_t o = ok ? (uint32_t)(((int64_t)rr * g.ldc + cc) * 4) : MG_OOB;
        // undo the row scales: acc (1 / s_r) (1 / s_c), exact (powers of two)
        const float x = (acc[ta][tb][j] * scale_at(sa, r0 + rr, rr < rowsA)) * vc;
        float v = g.alpha * x;
        if (g.beta != 0.0f)
          v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc, (int)o, 0, 0)) + v;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rc, (int)o, 0, 0);
      }
  }
  __syncthreads();  // no wave leaves while loads it issued may still write LDS
}

template <int AMODE, int BMODE, bool CLOW>
__global__ __launch_bounds__(512, 1) void gemm3x_kernel(G3Args g0, int64_t tm, int64_t tn,
                                                        MgSched sched) {
  __shared__ __attribute__((aligned(1024))) GxStage SA;
  __shared__ __attribute__((aligned(1024))) GxStage SB;
  int64_t tr, tc;
  if (sched.per_xcd > 0) {
    if (!mg_sched_tile<CLOW, GX_SUP>(blockIdx.x, sched, tm, tn, tr, tc)) return;
  } else {
    const int64_t t = xcd_tile(blockIdx.x, tm * tn);
    if (t < 0) return;
    tr = t / tn;
    tc = t % tn;
  }
  gemm3x_tile<AMODE, BMODE, CLOW>(g0, SA, SB, tr, tc);
}

// Two products in one launch: the node's A22 -= T1 T1^T (lower) and T2 = T1 A11 share T1's
// planes and each fills the other's last round of tiles.  The table (GxPair) deals both
// products' super-tiles to the XCDs by summed rank, longest first; an entry is
// (product << 15) | super-tile index (row-major over that product's super-tile grid of
// nsc[product] columns), 0xffff none.

template <int A1, int B1, bool C1, int A2, int B2, bool C2>
__global__ __launch_bounds__(512, 1) void gemm3x_pair_kernel(G3Args g1, int64_t tm1,
                                                             int64_t tn1, G3Args g2,
                                                             int64_t tm2, int64_t tn2,
                                                             GxPair sched) {
  __shared__ __attribute__((aligned(1024))) GxStage SA;
  __shared__ __attribute__((aligned(1024))) GxStage SB;
  const int x = (int)(blockIdx.x & 7);
  const int64_t slot = blockIdx.x >> 3;
  const int j = (int)(slot / (GX_SUP * GX_SUP)), w = (int)(slot % (GX_SUP * GX_SUP));
  if (j >= sched.per_xcd) return;
  const int u = sched.st[x * sched.per_xcd + j];
  if (u == 0xffff) return;
  const int p = u >> 15, id = u & 0x7fff, nsc = sched.nsc[p];
  const int64_t tr = (int64_t)(id / nsc) * GX_SUP + w / GX_SUP;
  const int64_t tc = (int64_t)(id % nsc) * GX_SUP + w % GX_SUP;
  if (p == 0) {
    if (tr >= tm1 || tc >= tn1 || (C1 && tc > tr)) return;
    gemm3x_tile<A1, B1, C1>(g1, SA, SB, tr, tc);
  } else {
    if (tr >= tm2 || tc >= tn2 || (C2 && tc > tr)) return;
    gemm3x_tile<A2, B2, C2>(g2, SA, SB, tr, tc);
  }
}

// The planes of one or two operands of a product (split2_kernel's layout at out, batch
// stride sout): the row maxima first, then the scaled split, each one launch for both
// operands.  out holds 2 R Kp fp16 then (1 + G2_NS) R floats, within the 3 R Kp fp16 a
// plane buffer holds (Kp >= 34).
// One-pass splits of row-major operands (split_rows_kernel); HI2X_CHOL_SPLIT_ROWS=0 keeps
// the rowmax_kernel + split2_kernel pair for every operand (read once per process; the
// two give the same planes, which the tests compare).
static bool chol_split_rows() {
  static const bool on = [] {
    const char* e = getenv("HI2X_CHOL_SPLIT_ROWS");
    return !(e && *e && strcmp(e, "0") == 0);
  }();
  return on;
}

int split2(const SplitOp& a, const SplitOp* b, hipStream_t s, int batch = 1) {
  const SplitOp none{a.X, a.ldx, 0, a.Kk, a.Kp, a.sx, a.sout, a.trans, a.mask, a.out};
  const SplitOp& o1 = b ? *b : none;
  for (const SplitOp* o : {&a, &o1})
    if (o->R > 0 && o->Kp < 2 * (1 + G2_NS)) {  // split products have ranks in the hundreds
      set_error("split2: rank %lld too small for the scale partials", (long long)o->Kp);
      return HI2X_EINVAL;
    }
  auto groups = [](const SplitOp& o) {  // rowmax_kernel row groups of an operand
    return (unsigned)(o.trans ? (o.R + 255) / 256 : (o.R + 3) / 4);
  };
  auto vec = [](const SplitOp& o) {
    return o.R <= 0 || ((reinterpret_cast<uintptr_t>(o.X) & 15) == 0 && o.ldx % 4 == 0 &&
                        o.sx % 4 == 0);
  };
  // a row-major operand of rank up to SR_NV_MAX x 256 in one pass
  auto one_pass = [&](const SplitOp& o) {
    return chol_split_rows() && o.R > 0 && !o.trans && vec(o) && o.Kp <= 256 * SR_NV_MAX;
  };
  if (one_pass(a)) {
    const bool both = o1.R > 0 && one_pass(o1);  // then one launch (they share Kp)
    const unsigned ya = (unsigned)((a.R + 3) / 4), yb = both ? (unsigned)((o1.R + 3) / 4) : 0;
    const dim3 grid(1, ya + yb, (unsigned)batch);
    const SplitOp& ob = both ? o1 : none;
    const int nv = (int)((a.Kp + 255) / 256);
    if (nv <= 4)
      hipLaunchKernelGGL(split_rows_kernel<4>, grid, dim3(256), 0, s, a, ob, (int)ya);
    else if (nv <= 8)
      hipLaunchKernelGGL(split_rows_kernel<8>, grid, dim3(256), 0, s, a, ob, (int)ya);
    else if (nv <= 12)
      hipLaunchKernelGGL(split_rows_kernel<12>, grid, dim3(256), 0, s, a, ob, (int)ya);
    else if (nv <= 16)
      hipLaunchKernelGGL(split_rows_kernel<16>, grid, dim3(256), 0, s, a, ob, (int)ya);
    else if (nv <= 20)
      hipLaunchKernelGGL(split_rows_kernel<20>, grid, dim3(256), 0, s, a, ob, (int)ya);
    else if (nv <= 24)
      hipLaunchKernelGGL(split_rows_kernel<24>, grid, dim3(256), 0, s, a, ob, (int)ya);
    else
      hipLaunchKernelGGL(split_rows_kernel<SR_NV_MAX>, grid, dim3(256), 0, s, a, ob, (int)ya);
    const int rc = launch_status("split_rows_kernel");
    if (rc || both || o1.R <= 0) return rc;
    return split2(o1, nullptr, s, batch);  // the transposed operand: the pair
  }
  const unsigned ga = groups(a), gb = o1.R > 0 ? groups(o1) : 0;
  if (ga + gb == 0) return HI2X_OK;
  {
    const dim3 gm((unsigned)G2_NS, ga + gb, (unsigned)batch);
    if (vec(a) && vec(o1))
      hipLaunchKernelGGL(rowmax_kernel<true>, gm, dim3(256), 0, s, a, o1, (int)ga);
    else
      hipLaunchKernelGGL(rowmax_kernel<false>, gm, dim3(256), 0, s, a, o1, (int)ga);
    const int rc = launch_status("rowmax_kernel");
    if (rc) return rc;
  }
  const unsigned ya = (unsigned)((a.R + 63) / 64), yb = (unsigned)((o1.R + 63) / 64);
  const int64_t kp = std::max(a.Kp, o1.R > 0 ? o1.Kp : 0);
  const dim3 grid((unsigned)((kp + 63) / 64), ya + yb, (unsigned)batch);
  hipLaunchKernelGGL(split2_kernel, grid, dim3(256), 0, s, a, o1, (int)ya);
  return launch_status("split2_kernel");
}

template <int AMODE, int BMODE, bool CLOW>
int gemm3x(const G3Args& a, hipStream_t s, int batch);
static bool chol_tile256();

template <int AMODE, int BMODE, bool CLOW>
int gemm3(const G3Args& a, hipStream_t s, int batch = 1) {
  if (a.M <= 0 || a.N <= 0) return HI2X_OK;
  {
    const int64_t tm2 = (a.M + GX_T - 1) / GX_T, tn2 = (a.N + GX_T - 1) / GX_T;
    const int64_t live2 = CLOW ? tm2 * (tm2 + 1) / 2 : tm2 * tn2;
    if (live2 >= 256 && chol_tile256()) return gemm3x<AMODE, BMODE, CLOW>(a, s, batch);
  }
  const int64_t tm = (a.M + MG_T - 1) / MG_T, tn = (a.N + MG_T - 1) / MG_T;
  LaunchTimer timer(HI2X_TIME_CHOL_SPLIT, 3.0 * a.M * a.N * a.Kd * batch, s);
  MgSched sched = mg_balance(tm, tn, [&](int64_t sr, int64_t sc) {
    double w = 0.0;
    for (int64_t i = 0; i < MG_SUP; ++i)
      for (int64_t j = 0; j < MG_SUP; ++j) {
        const int64_t tr = sr * MG_SUP + i, tc = sc * MG_SUP + j;
        if (tr >= tm || tc >= tn || (CLOW && tc > tr)) continue;
        int64_t kb, ke;
        tri_krange<AMODE, BMODE>(tr * MG_T, tc * MG_T, MG_T, a.Kd, kb, ke);
        w += (double)std::max<int64_t>(0, ke - kb) + 2.0 * G3_KC;
      }
    return w;
  });
  const int64_t grid = sched.per_xcd > 0 ? mg_sched_grid(sched) : (tm * tn + 7) / 8 * 8;
  hipLaunchKernelGGL((gemm3_kernel<AMODE, BMODE, CLOW>), dim3((unsigned)grid, 1, (unsigned)batch),
                     dim3(256), 0, s, a, tm, tn, sched);
  return launch_status("gemm3_kernel");
}

// 256-tiles where they fill the chip (at least one 256-CU round of live tiles);
// HI2X_CHOL_TILE256=0 keeps the 128-tiles (read at every product, for comparisons)
static bool chol_tile256() {
  const char* e = getenv("HI2X_CHOL_TILE256");
  return !(e && *e && strcmp(e, "0") == 0);
}

template <int AMODE, int BMODE, bool CLOW>
int gemm3x(const G3Args& a, hipStream_t s, int batch) {
  const int64_t tm = (a.M + GX_T - 1) / GX_T, tn = (a.N + GX_T - 1) / GX_T;
  LaunchTimer timer(HI2X_TIME_CHOL_SPLIT, 3.0 * a.M * a.N * a.Kd * batch, s);
  MgSched sched = mg_balance(tm, tn, [&](int64_t sr, int64_t sc) {
    double w = 0.0;
    for (int64_t i = 0; i < GX_SUP; ++i)
      for (int64_t j = 0; j < GX_SUP; ++j) {
        const int64_t tr = sr * GX_SUP + i, tc = sc * GX_SUP + j;
        if (tr >= tm || tc >= tn || (CLOW && tc > tr)) continue;
        int64_t kb, ke;
        tri_krange<AMODE, BMODE>(tr * GX_T, tc * GX_T, GX_T, a.Kd, kb, ke);
        w += (double)std::max<int64_t>(0, ke - kb) + 2.0 * G3_KC;
      }
    return w;
  }, GX_SUP);
  const int64_t grid = sched.per_xcd > 0 ? mg_sched_grid(sched) : (tm * tn + 7) / 8 * 8;
  hipLaunchKernelGGL((gemm3x_kernel<AMODE, BMODE, CLOW>), dim3((unsigned)grid, 1, (unsigned)batch),
                     dim3(512), 0, s, a, tm, tn, sched);
  return launch_status("gemm3x_kernel");
}

// A22 -= T1 T1^T (lower) and T2 = T1 A11 in one launch, on 64-tiles (pair_small).
int tri_gemm_pair(GemmArgs a1, GemmArgs a2, hipStream_t s, int batch) {
  const int64_t tm1 = (a1.M + 63) / 64, tn1 = (a1.N + 63) / 64;
  const int64_t tm2 = (a2.M + 63) / 64, tn2 = (a2.N + 63) / 64;
  const int64_t grid1 = (tm1 * tn1 + 7) / 8 * 8, grid2 = (tm2 * tn2 + 7) / 8 * 8;
  LaunchTimer timer(HI2X_TIME_CHOL_GEMM,
                    ((double)a1.M * a1.N * a1.Kd + (double)a2.M * a2.N * a2.Kd) * batch, s);
  hipLaunchKernelGGL((tri_gemm_pair_kernel<0, 0, true, true, 0, 1, false, false>),
                     dim3((unsigned)(grid1 + grid2), 1, (unsigned)batch), dim3(256), 0, s, a1,
                     tm1, tn1, grid1, a2, tm2, tn2);
  return launch_status("tri_gemm_pair_kernel");
}

// weight of super-tile (sr, sc) (SUP x SUP tiles of T) of a product (0: no live tile)
template <int AMODE, int BMODE, bool CLOW, int T, int SUP>
static double pair_weight(const G3Args& a, int64_t tm, int64_t tn, int64_t sr, int64_t sc) {
  double w = 0.0;
  for (int64_t i = 0; i < SUP; ++i)
    for (int64_t j = 0; j < SUP; ++j) {
      const int64_t tr = sr * SUP + i, tc = sc * SUP + j;
      if (tr >= tm || tc >= tn || (CLOW && tc > tr)) continue;
      int64_t kb, ke;
      tri_krange<AMODE, BMODE>(tr * T, tc * T, T, a.Kd, kb, ke);
      w += (double)std::max<int64_t>(0, ke - kb) + 2.0 * G3_KC;
    }
  return w;
}

// Both products in one launch on T-tiles (T = GX_T: gemm3x_pair_kernel, MG_T:
// gemm3_pair_kernel); 1 when the table would not hold their super-tiles (nothing
// launched: the caller runs them apart).
template <int T, int A1, int B1, bool C1, int A2, int B2, bool C2>
int g3_pair(const G3Args& a1, const G3Args& a2, hipStream_t s, int batch) {
  constexpr int SUP = T == GX_T ? GX_SUP : MG_SUP;
  const int64_t tm1 = (a1.M + T - 1) / T, tn1 = (a1.N + T - 1) / T;
  const int64_t tm2 = (a2.M + T - 1) / T, tn2 = (a2.N + T - 1) / T;
  GxPair sched;
  sched.nsc[0] = (int32_t)((tn1 + SUP - 1) / SUP);
  sched.nsc[1] = (int32_t)((tn2 + SUP - 1) / SUP);
  std::vector<std::pair<double, int>> items;
  for (int p = 0; p < 2; ++p) {
    const int64_t tm = p ? tm2 : tm1, tn = p ? tn2 : tn1, nsc = sched.nsc[p];
    const int64_t nsr = (tm + SUP - 1) / SUP;
    if (nsr * nsc >= 0x7fff) return 1;
    for (int64_t sr = 0; sr < nsr; ++sr)
      for (int64_t sc = 0; sc < nsc; ++sc) {
        const double w = p ? pair_weight<A2, B2, C2, T, SUP>(a2, tm, tn, sr, sc)
                           : pair_weight<A1, B1, C1, T, SUP>(a1, tm, tn, sr, sc);
        if (w > 0.0) items.push_back({w, (p << 15) | (int)(sr * nsc + sc)});
      }
  }
  if (items.empty() || (int64_t)items.size() > MG_SCHED_MAX) return 1;
  std::stable_sort(items.begin(), items.end(),
                   [](const std::pair<double, int>& x, const std::pair<double, int>& y) {
                     return x.first > y.first;
                   });
  double load[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  std::vector<int> lists[8];
  for (const auto& it : items) {
    int best = 0;
    for (int x = 1; x < 8; ++x)
      if (load[x] < load[best]) best = x;
    load[best] += it.first;
    lists[best].push_back(it.second);
  }
  int per = 0;
  for (int x = 0; x < 8; ++x) per = std::max(per, (int)lists[x].size());
  if ((int64_t)per * 8 > MG_SCHED_MAX) return 1;
  sched.per_xcd = per;
  for (int x = 0; x < 8; ++x)
    for (int j = 0; j < per; ++j)
      sched.st[x * per + j] = j < (int)lists[x].size() ? (uint16_t)lists[x][j] : (uint16_t)0xffff;
  LaunchTimer timer(HI2X_TIME_CHOL_SPLIT,
                    3.0 * ((double)a1.M * a1.N * a1.Kd + (double)a2.M * a2.N * a2.Kd) * batch, s);
  const int64_t grid = (int64_t)8 * per * SUP * SUP;
  if constexpr (T == GX_T) {
    hipLaunchKernelGGL((gemm3x_pair_kernel<A1, B1, C1, A2, B2, C2>),
                       dim3((unsigned)grid, 1, (unsigned)batch), dim3(512), 0, s, a1, tm1, tn1,
                       a2, tm2, tn2, sched);
    return launch_status("gemm3x_pair_kernel");
  } else {
    hipLaunchKernelGGL((gemm3_pair_kernel<A1, B1, C1, A2, B2, C2>),
                       dim3((unsigned)grid, 1, (unsigned)batch), dim3(256), 0, s, a1, tm1, tn1,
                       a2, tm2, tn2, sched);
    return launch_status("gemm3_pair_kernel");
  }
}

// Products of the big grids: fp16 MFMA on the two scaled split planes (default), or the
// fp32 MFMA GEMM when HI2X_CHOL_FP32 is set to a nonzero value (read once per process).
static bool chol_split() {
  static const bool split = [] {
    const char* e = getenv("HI2X_CHOL_FP32");
    return !(e && *e && strcmp(e, "0") != 0);
  }();
  return split;
}

template <int AMODE, int BMODE, bool TB, bool CLOW>
int tri_gemm(const GemmArgs& a, hipStream_t s, int batch = 1) {
  if (a.M <= 0 || a.N <= 0) return HI2X_OK;
  const int64_t tm = (a.M + MG_T - 1) / MG_T, tn = (a.N + MG_T - 1) / MG_T;
  const int64_t ntiles = tm * tn;
  // every product here has one triangular operand or output: M*N*rank useful flops
  LaunchTimer timer(HI2X_TIME_CHOL_GEMM, (double)a.M * a.N * a.Kd * batch, s);
  if ((CLOW ? ntiles / 2 : ntiles) < 128) {
    // a small grid: 64-tiles, four times the workgroups for a quarter of the work each
    const int64_t tm6 = (a.M + 63) / 64, tn6 = (a.N + 63) / 64;
    const int64_t grid = (tm6 * tn6 + 7) / 8 * 8;
    hipLaunchKernelGGL((tri_gemm_kernel<AMODE, BMODE, TB, CLOW, 64>),
                       dim3((unsigned)grid, 1, (unsigned)batch), dim3(256), 0, s, a, tm6, tn6, 0,
                       MgSched{});
    return launch_status("tri_gemm_kernel");
  }
  // big grids (several rounds of the 512 workgroup slots): super-tiles balanced over the
  // XCDs by their rank (plus two chunks' worth of per-tile overhead)
  const int super = (CLOW ? ntiles / 2 : ntiles) >= 256 ? 1 : 0;
  MgSched sched;
  if (super) {
    sched = mg_balance(tm, tn, [&](int64_t sr, int64_t sc) {
      double w = 0.0;
      for (int64_t i = 0; i < MG_SUP; ++i)
        for (int64_t j = 0; j < MG_SUP; ++j) {
          const int64_t tr = sr * MG_SUP + i, tc = sc * MG_SUP + j;
          if (tr >= tm || tc >= tn || (CLOW && tc > tr)) continue;
          int64_t kb, ke;
          tri_krange<AMODE, BMODE>(tr * MG_T, tc * MG_T, MG_T, a.Kd, kb, ke);
          w += (double)std::max<int64_t>(0, ke - kb) + 2.0 * MG_KC;
        }
      return w;
    });
  }
  const int64_t grid = sched.per_xcd > 0 ? mg_sched_grid(sched)
                       : super            ? mg_super_grid(tm, tn, CLOW)
                                          : (ntiles + 7) / 8 * 8;
  hipLaunchKernelGGL((tri_gemm_kernel<AMODE, BMODE, TB, CLOW, MG_T>),
                     dim3((unsigned)grid, 1, (unsigned)batch), dim3(256), 0, s, a, tm, tn, super,
                     sched);
  return launch_status("tri_gemm_kernel");
}

// ---- lam = damp * max(mean(diag hs), 1e-12) * 10^attempt ---------------------------------
// mean(diag) as the reference's torch CPU reduction of the strided diagonal: 4 scalar
// accumulators over rows of 4 elements, the 4-level cascade (base 2^max(4,
// ceil_log2(rows)/4)), the tail into accumulator 0, the accumulators folded, / K.
// Thread q < 4 runs accumulator q; the diagonal is staged through LDS in chunks.
__global__ __launch_bounds__(256) void diag_mean_kernel(const float* __restrict__ hs, int64_t K,
                                                        float damp, float p10,
                                                        float* __restrict__ lam_out,
                                                        int64_t shs, int64_t slam) {
  hs += (int64_t)blockIdx.z * shs;
  lam_out += (int64_t)blockIdx.z * slam;
  // Accumulator q adds element q of every row of 4 in row order; within a step of
  // `step` rows it starts from zero (the cascade moved it up at the previous step end),
  // so the step sums are independent: all threads form them in parallel (each one the
  // same sequential chain as the reference), then thread q runs the cascade over them.
  constexpr int SC = 1024;  // steps per round
  __shared__ float ssum[SC][4];
  __shared__ float part[4];
  const int tid = threadIdx.x;
  const int64_t size_ilp = K / 4;
  int64_t lp = 1;
  if (size_ilp > 2) lp = 64 - __builtin_clzll((unsigned long long)(size_ilp - 1));
  lp /= 4;
  if (lp < 4) lp = 4;
  const int64_t step = (int64_t)1 << lp, lmask = step - 1;
  const int64_t nsteps = size_ilp / step;  // full steps; rows past them are the remainder
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int64_t i = 0;  // rows of 4 consumed by full steps
  for (int64_t s0 = 0; s0 < nsteps; s0 += SC) {
    const int64_t ns = (nsteps - s0 < SC) ? nsteps - s0 : SC;
    __syncthreads();
    for (int64_t task = tid; task < ns * 4; task += 256) {
      const int64_t sidx = task >> 2, q = task & 3;
      const int64_t row0 = (s0 + sidx) * step;
      float a = 0.0f;
      if (step == 16) {  // every K below 2^22: the 16 loads issued before the first add
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t e = 4 * (row0 + r) + q;
          v[r] = hs[e * K + e];
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) a += v[r];
      } else {
        for (int64_t r = 0; r < step; ++r) {
          const int64_t e = 4 * (row0 + r) + q;
          a += hs[e * K + e];
        }
      }
      ssum[sidx][q] = a;
    }
    __syncthreads();
    if (tid < 4) {
      for (int64_t sidx = 0; sidx < ns; ++sidx) {
        acc[0] = ssum[sidx][tid];  // acc[0] is zero at a step start
        i += step;
        for (int lev = 1; lev < 4; ++lev) {
          acc[lev] += acc[lev - 1];
          acc[lev - 1] = 0.0f;
          if (i & (lmask << (lev * lp))) break;
        }
      }
    }
  }
  if (tid < 4) {  // the remaining rows after the last full step, in order
    for (int64_t row = nsteps * step; row < size_ilp; ++row) {
      const int64_t e = 4 * row + tid;
      acc[0] += hs[e * K + e];
    }
    part[tid] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  }
  __syncthreads();
  if (tid == 0) {
    float p0 = part[0];
    for (int64_t e = size_ilp * 4; e < K; ++e) p0 += hs[e * K + e];  // tail, in order
    const float sum = ((p0 + part[1]) + part[2]) + part[3];
    float mean = sum / (float)K;
    mean = mean < 1e-12f ? 1e-12f : mean;
    *lam_out = (damp * mean) * p10;
  }
}

// P[i][j] = hs[K-1-i][K-1-j] (+ lam on the diagonal), lower triangle only.
__global__ __launch_bounds__(256) void reverse_damp_kernel(const float* __restrict__ hs,
                                                           int64_t K,
                                                           const float* __restrict__ lam,
                                                           float* __restrict__ P, int64_t shs,
                                                           int64_t slam, int64_t sP) {
  hs += (int64_t)blockIdx.z * shs;
  lam += (int64_t)blockIdx.z * slam;
  P += (int64_t)blockIdx.z * sP;
  const int64_t i = (int64_t)blockIdx.y;
  const float l = *lam;
  for (int64_t j = threadIdx.x + (int64_t)blockIdx.x * blockDim.x; j <= i;
       j += (int64_t)gridDim.x * blockDim.x) {
    const float v = hs[(K - 1 - i) * K + (K - 1 - j)];
    P[i * K + j] = (i == j) ? v + l : v;
  }
}

// The same with 16-byte vectors (K a multiple of 4, 16-byte aligned matrices): vector v of
// row i (columns 4v .. 4v + 3, 4v <= i) is row K-1-i's vector at K-4-4v reversed.  In the
// vector that holds the diagonal, the columns past i get the reversed values too: that
// part of P is above the diagonal, which nothing reads before reverse_out4_kernel writes
// it.
__global__ __launch_bounds__(256) void reverse_damp4_kernel(const float* __restrict__ hs,
                                                            int64_t K,
                                                            const float* __restrict__ lam,
                                                            float* __restrict__ P, int64_t shs,
                                                            int64_t slam, int64_t sP) {
  hs += (int64_t)blockIdx.z * shs;
  lam += (int64_t)blockIdx.z * slam;
  P += (int64_t)blockIdx.z * sP;
  const int64_t i = (int64_t)blockIdx.y;
  const float l = *lam;
  const float* src = hs + (K - 1 - i) * K + (K - 4);
  float* dst = P + i * K;
  for (int64_t v = threadIdx.x + (int64_t)blockIdx.x * blockDim.x; 4 * v <= i;
       v += (int64_t)gridDim.x * blockDim.x) {
    const float4 x = *reinterpret_cast<const float4*>(src - 4 * v);
    float4 y = make_float4(x.w, x.z, x.y, x.x);
    const int64_t e = i - 4 * v;  // the diagonal's place in the vector (if < 4)
    y.x = e == 0 ? y.x + l : y.x;
    y.y = e == 1 ? y.y + l : y.y;
    y.z = e == 2 ? y.z + l : y.z;
    y.w = e == 3 ? y.w + l : y.w;
    *reinterpret_cast<float4*>(dst + 4 * v) = y;
  }
}

// ---- leaf: L^-1 of chol(P[r0:r0+n, r0:r0+n]) in place (lower triangle) ---------------------
// One workgroup of 4 waves holds the 128 x 128 block in LDS (identity beyond n, zeros
// above the diagonal) and runs the same recursion as the host on it, down to 16 x 16:
//   node [A11 0; A21 A22]: leaf(A11); T1 = A21 A11^T; A22 -= T1 T1^T (lower);
//                          leaf(A22); T2 = T1 A11; A21 = -A22 T2
// with the products on v_mfma_f32_16x16x4f32 (each product is read into registers,
// then written back in place after a barrier).
//
// The 16 x 16 base is one wave's fused factor-and-invert sweep, lane i (< 16) holding row
// i of the symmetric block in 16 registers (the upper triangle mirrored from the lower one
// on load).  For c = 0..15, with d = M[c][c], r = 1/sqrt(d) and g_i = -M[i][c] r^2 on
// the rows i > c (0 on the others):
//   every j != c:  M[i][j] += g_i M[c][j]
//     (j > c: the Schur update T[i][j] -= l_i l_j, l_k = T[k][c] r, with T[j][c] = T[c][j]
//      by symmetry; j < c: the forward substitution B[i][j] -= l_i X[c][j], where row c of
//      L^-1 is X[c][j] = B[c][j] r)
//   rows i > c:    M[i][c] = g_i   (= -l_i r, column c of L^-1 before row i's scaling).
// Row c is then final up to its scale, which is applied once after the sweep:
// X[c][j] = M[c][j] r_c (j < c), X[c][c] = r_c.  Every multiplier is one of lane c's own
// registers, broadcast to each row of 16 lanes by DPP (row_newbcast) inside
// v_fmac_f32_dpp: one instruction per register and column, no barrier and no LDS traffic
// in the sweep.  The reciprocal and square root are the hardware approximations (the
// factor is compared to a tolerance, not bit for bit).
constexpr int LP = NB + 4;  // LDS pitch of the leaf block (floats)
#ifndef HI2X_LEAF_SPLIT
#define HI2X_LEAF_SPLIT 1
#endif
constexpr bool LEAF_SPLIT = HI2X_LEAF_SPLIT;

typedef float f32x4v __attribute__((ext_vector_type(4)));

// v[j] += bcast_C(v[j]) * g for the 15 registers j != C, bcast_C = lane C of each row of 16
// lanes.  The compiler does not fold a DPP move into an FMA (v_fma_f32 has no DPP form on
// this target), so the fused instructions are written out.  The leading s_nop 4 gives the
// five wait states a DPP instruction needs after a VALU write of its source VGPR (two) or
// of EXEC (five); inside the block no instruction reads a register another one writes.
#define HI2X_FMAC_DPP(k, C) \
  "v_fmac_f32_dpp %" #k ", %" #k ", %15 row_newbcast:" #C " row_mask:0xf bank_mask:0xf\n\t"
#define HI2X_FMAC15(C)                                                                     \
  "s_nop 4\n\t" HI2X_FMAC_DPP(0, C) HI2X_FMAC_DPP(1, C) HI2X_FMAC_DPP(2, C)              \
      HI2X_FMAC_DPP(3, C) HI2X_FMAC_DPP(4, C) HI2X_FMAC_DPP(5, C) HI2X_FMAC_DPP(6, C)     \
          HI2X_FMAC_DPP(7, C) HI2X_FMAC_DPP(8, C) HI2X_FMAC_DPP(9, C) HI2X_FMAC_DPP(10, C) \
              HI2X_FMAC_DPP(11, C) HI2X_FMAC_DPP(12, C) HI2X_FMAC_DPP(13, C)               \
                  HI2X_FMAC_DPP(14, C)
#define HI2X_J(k) ((k) < C ? (k) : (k) + 1)
#define HI2X_ROW_OPS                                                                   \
  "+v"(v[HI2X_J(0)]), "+v"(v[HI2X_J(1)]), "+v"(v[HI2X_J(2)]), "+v"(v[HI2X_J(3)]),     \
      "+v"(v[HI2X_J(4)]), "+v"(v[HI2X_J(5)]), "+v"(v[HI2X_J(6)]), "+v"(v[HI2X_J(7)]), \
      "+v"(v[HI2X_J(8)]), "+v"(v[HI2X_J(9)]), "+v"(v[HI2X_J(10)]),                    \
      "+v"(v[HI2X_J(11)]), "+v"(v[HI2X_J(12)]), "+v"(v[HI2X_J(13)]),                  \
      "+v"(v[HI2X_J(14)])
template <int C>
__device__ __forceinline__ void fmac_row(float (&v)[16], float g) {
  static_assert(C >= 0 && C < 16, "column of the 16 x 16 base");
  if constexpr (C == 0) asm(HI2X_FMAC15(0) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 1) asm(HI2X_FMAC15(1) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 2) asm(HI2X_FMAC15(2) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 3) asm(HI2X_FMAC15(3) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 4) asm(HI2X_FMAC15(4) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 5) asm(HI2X_FMAC15(5) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 6) asm(HI2X_FMAC15(6) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 7) asm(HI2X_FMAC15(7) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 8) asm(HI2X_FMAC15(8) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 9) asm(HI2X_FMAC15(9) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 10) asm(HI2X_FMAC15(10) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 11) asm(HI2X_FMAC15(11) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 12) asm(HI2X_FMAC15(12) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 13) asm(HI2X_FMAC15(13) : HI2X_ROW_OPS : "v"(g));
  else if constexpr (C == 14) asm(HI2X_FMAC15(14) : HI2X_ROW_OPS : "v"(g));
  else asm(HI2X_FMAC15(15) : HI2X_ROW_OPS : "v"(g));
}
#undef HI2X_ROW_OPS
#undef HI2X_J
#undef HI2X_FMAC15
#undef HI2X_FMAC_DPP

// Column C of the sweep.  Lane i keeps its own pivot in pv (rows below C take theirs at
// their own column, so i >= C is the previous column's i > C).  M[i][C] becomes g on every
// row: the rows below need it, and lane C's and the finished rows' registers C are not
// read again before the final scaling overwrites them.
template <int C>
__device__ __forceinline__ void base_step(float (&v)[16], int i, float& pv) {
  const float d = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[C]), C));  // pivot M[c][c]
  const float rp = __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(d));
  const float gv = v[C] * -(rp * rp);
  fmac_row<C>(v, i > C ? gv : 0.0f);
  v[C] = gv;
  pv = i >= C ? d : pv;
}

template <int... Cs>
__device__ __forceinline__ void base_steps(float (&v)[16], int i, float& pv,
                                           std::integer_sequence<int, Cs...>) {
  (base_step<Cs>(v, i, pv), ...);
}

// 16 x 16 block at (o, o): one wave (the caller's wave 0), lane i holds row i % 16 (lanes
// 16..63 repeat rows 0..15 and do not write back).  Only the block's lower triangle is
// read: row i below the diagonal, column i (M[j][i] for j > i) as the upper half.
__device__ __forceinline__ void leaf_base16(float* S, int o, bool& bad) {
  const int l = threadIdx.x & 63, i = l & 15;
  float* row = &S[(o + i) * LP + o];
  float v[16], t[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 x = *reinterpret_cast<const float4*>(row + 4 * q);
    v[4 * q] = x.x;
    v[4 * q + 1] = x.y;
    v[4 * q + 2] = x.z;
    v[4 * q + 3] = x.w;
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) t[j] = S[(o + j) * LP + o + i];
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = j > i ? t[j] : v[j];
  float pv = 0.0f;
  base_steps(v, i, pv, std::make_integer_sequence<int, 16>{});
  // a pivot not positive (or NaN) anywhere in the block; the same r_i as in the sweep
  bad = bad || __builtin_amdgcn_ballot_w64(!(pv > 0.0f)) != 0;
  const float r = __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(pv));
  // row i of L^-1: X[i][j] = M[i][j] r_i (j < i), X[i][i] = r_i; the block stays lower
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = j < i ? v[j] * r : (j == i ? r : 0.0f);
  if (l < 16) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(row + 4 * q) =
          make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  }
}

// C[H x H] at (cr, cc) = alpha * A (at (ar, ac)) * op(B) (at (br, bc)), op(B) = B^T when
// TB; with LOWER, C += alpha * A op(B) on the lower triangle of C only.  Every block is in
// the leaf's LDS; the result is written after all inputs have been read (C may alias).
// For each 16 k: lane group g = l/16 supplies k = 16 kb + 4 g + s at MFMA step s, so a
// lane reads its 4 k of A (and of B^T) as one 16-byte vector.
template <int H>
struct ProdAcc {  // this wave's tiles of an H x H product (tile t = wave + 4p, p < PER)
  static constexpr int NT = H / 16, TILES = NT * NT, PER = (TILES + 3) / 4;
  f32x4v acc[PER];
};

// Three bf16 planes of 8 consecutive k of one lane's fragment: x1 = bf16(x),
// x2 = bf16(x - x1), x3 = bf16(x - x1 - x2) (the differences are exact in fp32; bf16 has
// fp32's exponent range, so no row scale is needed).  Pairs go through
// v_cvt_pk_bf16_f32; a bf16 back to fp32 is its bits in the upper half of the word.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split8(const float4 x0, const float4 x1, bf16x8 (&o)[3]) {
  const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  uint32_t w[3][4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float lo = x[2 * e], hi = x[2 * e + 1];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
      const uint32_t u =
          __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, bf16x2));
      w[pl][e] = u;
      if (pl < 2) {
        lo = lo - __builtin_bit_cast(float, u << 16);
        hi = hi - __builtin_bit_cast(float, u & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int pl = 0; pl < 3; ++pl)
    o[pl] = __builtin_bit_cast(bf16x8, (uint4){w[pl][0], w[pl][1], w[pl][2], w[pl][3]});
}

// acc = A op(B) for the node's 128 x 128 blocks on bf16 MFMA through the three-way split
// (the six terms x_i y_j with i + j <= 2, small terms first; the big products' scaled
// two-plane fp16 split measured slower here, its row maxima and conversions back to
// fp32 costing the VALU time its halved MFMAs save):
// v_mfma_f32_16x16x32_bf16 (lane l: row or column l % 16, k 8 (l / 16) .. + 7; the
// accumulator layout of the fp32 16x16x4 MFMA), six 16-cycle MFMAs per 32 k where the
// fp32 MFMA takes eight of 32 cycles.  The wave's tiles t = wave + 4p are tile row p / 2,
// column wave + 4 (p % 2): per 32 k its two column fragments are split first, then the
// eight row fragments two at a time, each pair's 24 MFMAs (four accumulators in turn)
// covering the split of the next pair.  fp32-level rounding, not bit-identical to the
// fp32 MFMA.  (Blocks of 64 and below stay on fp32 MFMA: with a row fragment used by
// one tile, the split costs more VALU time than the MFMA time it saves.)
template <bool TB>
__device__ __forceinline__ void node_mma3(const float* S, int ar, int ac, int br, int bc,
                                          ProdAcc<128>& P) {
  constexpr int PER = ProdAcc<128>::PER;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lr = l & 15, lg = l >> 4;
#pragma unroll
  for (int p = 0; p < PER; ++p) P.acc[p] = (f32x4v){0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int PA[6] = {2, 1, 0, 1, 0, 0}, PB[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll 1
  for (int kb = 0; kb < 128; kb += 32) {
    const int k = kb + 8 * lg;
    bf16x8 b[2][3];
#pragma unroll
    for (int ci = 0; ci < 2; ++ci) {
      const int tc = wave + 4 * ci;
      float4 x0, x1;
      if (TB) {
        const float* bp = &S[(br + tc * 16 + lr) * LP + bc + k];
        x0 = *reinterpret_cast<const float4*>(bp);
        x1 = *reinterpret_cast<const float4*>(bp + 4);
      } else {
        const float* bp = &S[(br + k) * LP + bc + tc * 16 + lr];
        x0 = make_float4(bp[0], bp[LP], bp[2 * LP], bp[3 * LP]);
        x1 = make_float4(bp[4 * LP], bp[5 * LP], bp[6 * LP], bp[7 * LP]);
      }
      split8(x0, x1, b[ci]);
    }
#pragma unroll
    for (int rp = 0; rp < 4; ++rp) {
      bf16x8 a[2][3];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float* ap = &S[(ar + (2 * rp + q) * 16 + lr) * LP + ac + k];
        split8(*reinterpret_cast<const float4*>(ap), *reinterpret_cast<const float4*>(ap + 4),
               a[q]);
      }
#pragma unroll
      for (int pr = 0; pr < 6; ++pr)
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int ci = 0; ci < 2; ++ci) {
            const int p = 2 * (2 * rp + q) + ci;
            P.acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[q][PA[pr]], b[ci][PB[pr]],
                                                                P.acc[p], 0, 0, 0);
          }
    }
  }
}

// acc = A (at (ar, ac)) * op(B) (at (br, bc)), H x H blocks of the leaf's LDS, op(B) = B^T
// when TB (the 128 blocks take the split product above).  For each 16 k: lane group g = l/16 supplies k = 16 kb + 4 g + s at MFMA step
// s, so a lane reads its 4 k of A (and of B^T) as one 16-byte vector.
template <int H, bool TB>
__device__ __forceinline__ void leaf_mma(const float* S, int ar, int ac, int br, int bc,
                                         ProdAcc<H>& P) {
  if constexpr (H == 128 && LEAF_SPLIT) {
    node_mma3<TB>(S, ar, ac, br, bc, P);
    return;
  }
  constexpr int NT = ProdAcc<H>::NT, TILES = ProdAcc<H>::TILES, PER = ProdAcc<H>::PER;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lr = l & 15, lg = l >> 4;
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int t = wave + 4 * p;
    P.acc[p] = (f32x4v){0.0f, 0.0f, 0.0f, 0.0f};
    if (t < TILES) {
      const int tr = t / NT, tc = t % NT;
#pragma unroll
      for (int kb = 0; kb < H; kb += 16) {
        const int k = kb + 4 * lg;
        const float4 a = *reinterpret_cast<const float4*>(&S[(ar + tr * 16 + lr) * LP + ac + k]);
        float4 b;
        if (TB) {
          b = *reinterpret_cast<const float4*>(&S[(br + tc * 16 + lr) * LP + bc + k]);
        } else {
          const float* bp = &S[(br + k) * LP + bc + tc * 16 + lr];
          b = make_float4(bp[0], bp[LP], bp[2 * LP], bp[3 * LP]);
        }
        P.acc[p] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, P.acc[p], 0, 0, 0);
        P.acc[p] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, P.acc[p], 0, 0, 0);
        P.acc[p] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, P.acc[p], 0, 0, 0);
        P.acc[p] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, P.acc[p], 0, 0, 0);
      }
    }
  }
}

// (row, col) within the H x H product of register j of tile p of this lane
template <int H>
__device__ __forceinline__ int prod_row(int p, int j) {
  const int t = (threadIdx.x >> 6) + 4 * p;
  return (t / ProdAcc<H>::NT) * 16 + 4 * ((threadIdx.x & 63) >> 4) + j;
}
template <int H>
__device__ __forceinline__ int prod_col(int p) {
  const int t = (threadIdx.x >> 6) + 4 * p;
  return (t % ProdAcc<H>::NT) * 16 + (threadIdx.x & 15);
}
template <int H>
__device__ __forceinline__ bool prod_live(int p) {
  return (threadIdx.x >> 6) + 4 * p < ProdAcc<H>::TILES;
}

// C[H x H] at (cr, cc) = alpha * A op(B); with LOWER, C += alpha * A op(B) on the lower
// triangle of C only.  The result is written after all inputs have been read (C may
// alias an input).
template <int H, bool TB, bool LOWER>
__device__ __forceinline__ void leaf_prod(float* S, int ar, int ac, int br, int bc, int cr,
                                          int cc, float alpha) {
  ProdAcc<H> P;
  leaf_mma<H, TB>(S, ar, ac, br, bc, P);
  __syncthreads();
#pragma unroll
  for (int p = 0; p < ProdAcc<H>::PER; ++p) {
    if (!prod_live<H>(p)) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = prod_row<H>(p, j), c = prod_col<H>(p);
      const float x = P.acc[p][j];
      float* d = &S[(cr + r) * LP + cc + c];
      if (LOWER) {
        if (c <= r) *d = *d + alpha * x;
      } else {
        *d = alpha * x;
      }
    }
  }
  __syncthreads();
}

// returns true when a pivot of this block was not positive (wave 0's view)
template <int N>
__device__ __forceinline__ bool leaf_rec(float* S, int o) {
  if constexpr (N == 16) {
    bool bad = false;
    if ((threadIdx.x >> 6) == 0) leaf_base16(S, o, bad);
    __syncthreads();
    return bad;
  } else {
    constexpr int H = N / 2;
    bool bad = leaf_rec<H>(S, o);
    leaf_prod<H, true, false>(S, o + H, o, o, o, o + H, o, 1.0f);             // T1
    leaf_prod<H, true, true>(S, o + H, o, o + H, o, o + H, o + H, -1.0f);      // A22 -= T1 T1^T
    bad = leaf_rec<H>(S, o + H) || bad;
    leaf_prod<H, false, false>(S, o + H, o, o, o, o + H, o, 1.0f);            // T2 = T1 A11
    leaf_prod<H, false, false>(S, o + H, o + H, o + H, o, o + H, o, -1.0f);   // -A22 T2
    return bad;
  }
}

// Rows [0, n) x columns [0, n) of the n x n diagonal block at P (row stride K) into the
// LDS block at row offset so of S: lower triangle, zeros above, identity beyond n.  The
// buffer ends at the block's last element: rows past n read zero; n and K are multiples
// of 4 (the entry points require it of K), so every 16-byte vector is all in or all out.
__device__ __forceinline__ void leaf_load(float* S, int so, const float* P, int64_t K, int n) {
  const __amdgpu_buffer_rsrc_t rs = mg_rsrc(P, (int64_t)(n - 1) * K + n);
  constexpr int V = NB / 4;  // float4 per row
  const int tid = threadIdx.x;
  float4 x[NB * V / 256];
#pragma unroll
  for (int q = 0; q < NB * V / 256; ++q) {
    const int idx = tid + 256 * q, i = idx / V, j = 4 * (idx % V);
    const uint32_t off = (i < n && j < n) ? (uint32_t)(((int64_t)i * K + j) * 4) : MG_OOB;
    x[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0));
  }
#pragma unroll
  for (int q = 0; q < NB * V / 256; ++q) {
    const int idx = tid + 256 * q, i = idx / V, j = 4 * (idx % V);
    float e[4] = {x[q].x, x[q].y, x[q].z, x[q].w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int jj = j + t;
      e[t] = (i < n && jj < n) ? (jj <= i ? e[t] : 0.0f) : (i == jj ? 1.0f : 0.0f);
    }
    *reinterpret_cast<float4*>(&S[(so + i) * LP + j]) = make_float4(e[0], e[1], e[2], e[3]);
  }
}

// The LDS block at row offset so back to rows [0, n) x columns [0, n) at P in full
// vectors: the zeros above the diagonal land in P's upper triangle, which nothing reads
// before the final reflection overwrites it.
__device__ __forceinline__ void leaf_store(const float* S, int so, float* P, int64_t K, int n) {
  const __amdgpu_buffer_rsrc_t rs = mg_rsrc(P, (int64_t)(n - 1) * K + n);
  constexpr int V = NB / 4;
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < NB * V / 256; ++q) {
    const int idx = tid + 256 * q, i = idx / V, j = 4 * (idx % V);
    const uint32_t off = (i < n && j < n) ? (uint32_t)(((int64_t)i * K + j) * 4) : MG_OOB;
    const float4 v = *reinterpret_cast<const float4*>(&S[(so + i) * LP + j]);
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), rs, (int)off, 0, 0);
  }
}

__global__ __launch_bounds__(256) void leaf_kernel(float* __restrict__ P, int64_t K, int64_t r0,
                                                   int n, int* __restrict__ status, int64_t sP) {
  __shared__ float S[NB * LP];
  P += (int64_t)blockIdx.z * sP;
  status += blockIdx.z;
  float* blk = P + r0 * K + r0;
  leaf_load(S, 0, blk, K, n);
  __syncthreads();
  const bool bad = leaf_rec<NB>(S, 0);
  if (threadIdx.x == 0 && bad) atomicMin(status, (int)(r0 + 1));
  leaf_store(S, 0, blk, K, n);
}

// A whole recursion node of m = 128 + m2 columns (0 < m2 <= 128) in one workgroup: both
// diagonal blocks live in LDS (rows 0..127 and 128..255 of S), so the node's two leaves
// and four 128 x 128 products run without a launch in between:
//   S_A = leaf(A11) -> A11;  S_B = A21;  T1 = S_B S_A^T -> S_B;  T2 = T1 S_A -> S_A;
//   S_B = A22 - T1 T1^T (lower);  S_B = leaf(S_B) -> A22;  A21 = -S_B T2.
__global__ __launch_bounds__(256) void node_kernel(float* __restrict__ P, int64_t K, int64_t r0,
                                                   int m2, int* __restrict__ status, int64_t sP) {
  __shared__ float S[2 * NB * LP];
  P += (int64_t)blockIdx.z * sP;
  status += blockIdx.z;
  float* a11 = P + r0 * K + r0;
  float* a21 = P + (r0 + NB) * K + r0;
  float* a22 = P + (r0 + NB) * K + (r0 + NB);
  leaf_load(S, 0, a11, K, NB);
  {  // A21 [m2 x 128] into S_B (rows past m2 zero)
    const __amdgpu_buffer_rsrc_t rs = mg_rsrc(a21, (int64_t)(m2 - 1) * K + NB);
    constexpr int V = NB / 4;
    const int tid = threadIdx.x;
    float4 x[NB * V / 256];
#pragma unroll
    for (int q = 0; q < NB * V / 256; ++q) {
      const int idx = tid + 256 * q, i = idx / V, j = 4 * (idx % V);
      const uint32_t off = i < m2 ? (uint32_t)(((int64_t)i * K + j) * 4) : MG_OOB;
      x[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0));
    }
#pragma unroll
    for (int q = 0; q < NB * V / 256; ++q) {
      const int idx = tid + 256 * q, i = idx / V, j = 4 * (idx % V);
      *reinterpret_cast<float4*>(&S[(NB + i) * LP + j]) = x[q];
    }
  }
  __syncthreads();
  bool bad1 = leaf_rec<NB>(S, 0);
  leaf_store(S, 0, a11, K, NB);
  leaf_prod<NB, true, false>(S, NB, 0, 0, 0, NB, 0, 1.0f);   // T1 = A21 A11^T
  leaf_prod<NB, false, false>(S, NB, 0, 0, 0, 0, 0, 1.0f);   // T2 = T1 A11 (over S_A)
  {  // S_B = A22 - T1 T1^T: lower triangle, zeros above, identity beyond m2
    // (A22 is requested from memory first, so that its loads are in flight during the
    // product)
    const __amdgpu_buffer_rsrc_t rs = mg_rsrc(a22, (int64_t)(m2 - 1) * K + m2);
    float g[ProdAcc<NB>::PER][4];
#pragma unroll
    for (int p = 0; p < ProdAcc<NB>::PER; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = prod_row<NB>(p, j), c = prod_col<NB>(p);
        const uint32_t off = (r < m2 && c <= r) ? (uint32_t)(((int64_t)r * K + c) * 4) : MG_OOB;
        g[p][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0));
      }
    ProdAcc<NB> Q;
    leaf_mma<NB, true>(S, NB, 0, NB, 0, Q);
    __syncthreads();  // T1 has been read
#pragma unroll
    for (int p = 0; p < ProdAcc<NB>::PER; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = prod_row<NB>(p, j), c = prod_col<NB>(p);
        const float x = Q.acc[p][j];
        const float v = (r < m2 && c < m2) ? (c <= r ? g[p][j] - x : 0.0f) : (r == c ? 1.0f : 0.0f);
        S[(NB + r) * LP + c] = v;
      }
    __syncthreads();
  }
  bool bad2 = leaf_rec<NB>(S + NB * LP, 0);
  if (threadIdx.x == 0 && (bad1 || bad2)) atomicMin(status, (int)(r0 + (bad1 ? 1 : NB + 1)));
  leaf_store(S, NB, a22, K, m2);
  {  // A21 = -S_B T2 (rows < m2)
    ProdAcc<NB> Q;
    leaf_mma<NB, false>(S, NB, 0, 0, 0, Q);
    const __amdgpu_buffer_rsrc_t rs = mg_rsrc(a21, (int64_t)(m2 - 1) * K + NB);
#pragma unroll
    for (int p = 0; p < ProdAcc<NB>::PER; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = prod_row<NB>(p, j), c = prod_col<NB>(p);
        const uint32_t off = r < m2 ? (uint32_t)(((int64_t)r * K + c) * 4) : MG_OOB;
        const float x = Q.acc[p][j];
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(-x), rs, (int)off, 0, 0);
      }
  }
}

// U[i][j] = Linv[K-1-i][K-1-j] for j >= i, 0 below: in place over pairs
// {(i, j), (K-1-i, K-1-j)}, one thread per element of the upper triangle.
__global__ __launch_bounds__(256) void reverse_out_kernel(float* __restrict__ P, int64_t K,
                                                          int64_t sP) {
  P += (int64_t)blockIdx.z * sP;
  const int64_t i = (int64_t)blockIdx.y;
  for (int64_t j = i + threadIdx.x + (int64_t)blockIdx.x * blockDim.x; j < K;
       j += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ri = K - 1 - i, rj = K - 1 - j;  // (ri, rj) is in the lower triangle
    if (j == i) {
      if (i < ri) {
        const float a = P[i * K + i], b = P[ri * K + ri];
        P[i * K + i] = b;
        P[ri * K + ri] = a;
      }
    } else {
      P[i * K + j] = P[ri * K + rj];
      P[ri * K + rj] = 0.0f;
    }
  }
}

// The same with 16-byte vectors (K a multiple of 4, 16-byte aligned P): vector v of row i
// (columns 4v .. 4v + 3, 4v + 3 > i) receives row K-1-i's vector at K-4-4v reversed, which
// is then zeroed; in the vector that holds the diagonal only the columns past i move (one
// element at a time: the others are row i's lower part, the source of row K-1-i's), and
// the diagonal is swapped.  Every element moves or is zeroed by exactly one thread.
__global__ __launch_bounds__(256) void reverse_out4_kernel(float* __restrict__ P, int64_t K,
                                                           int64_t sP) {
  P += (int64_t)blockIdx.z * sP;
  const int64_t i = (int64_t)blockIdx.y, ri = K - 1 - i;
  float* row = P + i * K;
  float* mir = P + ri * K + (K - 4);
  for (int64_t v = i / 4 + threadIdx.x + (int64_t)blockIdx.x * blockDim.x; 4 * v < K;
       v += (int64_t)gridDim.x * blockDim.x) {
    if (4 * v > i) {  // every column of the vector is past the diagonal
      const float4 x = *reinterpret_cast<const float4*>(mir - 4 * v);
      *reinterpret_cast<float4*>(row + 4 * v) = make_float4(x.w, x.z, x.y, x.x);
      *reinterpret_cast<float4*>(mir - 4 * v) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t j = 4 * v + e, rj = K - 1 - j;
        if (j > i) {
          row[j] = P[ri * K + rj];
          P[ri * K + rj] = 0.0f;
        } else if (j == i && i < ri) {
          const float a = row[i], b = P[ri * K + ri];
          row[i] = b;
          P[ri * K + ri] = a;
        }
      }
    }
  }
}

__global__ void status_init_kernel(int* __restrict__ status, int v, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) status[i] = v;
}

// ---- host recursion -------------------------------------------------------------------
struct Plan {
  std::vector<int64_t> t1_off;  // per depth offsets into the workspace: T1
  std::vector<int64_t> t2_off;  // and T2 (made before the A22 recursion, used after it)
  int64_t total = 0;
  int64_t pa_off = 0, pb_off = 0;  // the two split-plane buffers (offsets in floats)
};

// Whether a node's A22 update and its T2 = T1 A11 both take the small-grid path (64-tiles,
// fewer than 128 live tiles of 128): they then run as one launch, before the A22
// recursion, with T2 in a buffer of the node's depth.
static bool pair_small(int64_t m1, int64_t m2) {
  const int64_t a = (m2 + MG_T - 1) / MG_T, b = (m1 + MG_T - 1) / MG_T;
  return (a * a) / 2 < 128 && a * b < 128;
}

void plan_sizes(int64_t m, int depth, std::vector<int64_t>& t12) {
  if (m <= 2 * NB) return;  // nodes and leaves work in LDS
  const int64_t nbk = (m + NB - 1) / NB;
  const int64_t m1 = ((nbk + 1) / 2) * NB, m2 = m - m1;
  if ((int)t12.size() <= depth) t12.resize(depth + 1, 0);
  t12[depth] = std::max(t12[depth], m1 * m2);
  plan_sizes(m1, depth + 1, t12);
  plan_sizes(m2, depth + 1, t12);
}

struct Ctx {
  float* P;
  int64_t K;
  float* ws;
  const Plan* plan;
  int* status;
  hipStream_t s;
  int batch = 1;     // factors of one launch sequence (grid z)
  int64_t sP = 0;    // floats between consecutive factors' matrices
  int64_t sW = 0;    // floats between consecutive factors' workspaces
  // batch stride of an operand: the workspace's for pointers into it, else the matrix's
  int64_t stride(const void* p) const {
    const float* f = static_cast<const float*>(p);
    return (f >= ws && f < ws + plan->total + 64) ? sW : sP;
  }
};

// op(B) mask of a TB / !TB product in split coordinates (row = output column j, k)
constexpr int split_mask_b(int bmode) { return bmode == 1 ? 2 : (bmode == 2 ? 1 : 0); }

// Whether a product runs through the split planes: grids of at least 128 tiles of 128,
// a lower-triangular output from 96 (14 x 14 tiles: the fp16 split's three MFMAs per 16 k
// on 105 tiles beat the fp32 MFMA's 406 tiles of 64).
static bool split_worth(int64_t tm, int64_t tn, bool clow) {
  return clow ? tm * (tm + 1) / 2 >= 96 : tm * tn >= 128;
}

// One product of the recursion: the big grids through the split planes, the small ones
// on the fp32 MFMA GEMM.
template <int AMODE, int BMODE, bool TB, bool CLOW>
int product(const Ctx& c, GemmArgs a) {
  const int64_t tm = (a.M + MG_T - 1) / MG_T, tn = (a.N + MG_T - 1) / MG_T;
  a.sA = c.stride(a.A);
  a.sB = c.stride(a.B);
  a.sC = c.stride(a.C);
  if (!chol_split() || !split_worth(tm, tn, CLOW))
    return tri_gemm<AMODE, BMODE, TB, CLOW>(a, c.s, c.batch);
  const int64_t Kp = (a.Kd + G3_KA - 1) / G3_KA * G3_KA;
  uint16_t* pa = reinterpret_cast<uint16_t*>(c.ws + c.plan->pa_off);
  uint16_t* pb = reinterpret_cast<uint16_t*>(c.ws + c.plan->pb_off);
  const int64_t sPl = 2 * c.sW;  // planes live in the workspace (16-bit elements)
  const SplitOp oa{a.A, a.lda, a.M, a.Kd, Kp, a.sA, sPl, 0, AMODE == 1 ? 1 : 0, pa};
  const SplitOp ob{a.B, a.ldb, a.N, a.Kd, Kp, a.sB, sPl, TB ? 0 : 1, split_mask_b(BMODE), pb};
  // B is A itself in the symmetric update: one operand's planes serve both
  const bool same = TB && a.B == a.A && a.ldb == a.lda && a.N == a.M && AMODE == 0 && BMODE == 0;
  const int rc = split2(oa, same ? nullptr : &ob, c.s, c.batch);
  if (rc) return rc;
  const uint16_t* bp = same ? pa : pb;
  G3Args g{pa, bp, a.C, a.M, a.N, a.Kd, Kp, a.ldc, a.alpha, a.beta};
  g.sA = sPl;
  g.sB = sPl;
  g.sC = a.sC;
  return gemm3<AMODE, BMODE, CLOW>(g, c.s, c.batch);
}

// The split-plane tile edge a product runs on (as product() and gemm3() decide): 256,
// 128, or 0 when it takes the fp32 path.
static int split_tile(const GemmArgs& a, bool clow) {
  const int64_t tm = (a.M + MG_T - 1) / MG_T, tn = (a.N + MG_T - 1) / MG_T;
  if (!chol_split() || !split_worth(tm, tn, clow)) return 0;
  const int64_t tm2 = (a.M + GX_T - 1) / GX_T, tn2 = (a.N + GX_T - 1) / GX_T;
  return ((clow ? tm2 * (tm2 + 1) / 2 : tm2 * tn2) >= 256 && chol_tile256()) ? GX_T : MG_T;
}

// A22 -= T1 T1^T (lower) and T2 = T1 A11: where both run on split planes with the same
// tile edge, T1 is split once for both and they share one launch; otherwise one product
// after the other.
int product_pair(const Ctx& c, GemmArgs upd, GemmArgs t2) {
  const int tile = split_tile(upd, true);
  if (tile != 0 && tile == split_tile(t2, false)) {
    upd.sA = c.stride(upd.A);
    upd.sC = c.stride(upd.C);
    t2.sB = c.stride(t2.B);
    t2.sC = c.stride(t2.C);
    const int64_t Kp = (upd.Kd + G3_KA - 1) / G3_KA * G3_KA;
    uint16_t* pa = reinterpret_cast<uint16_t*>(c.ws + c.plan->pa_off);
    uint16_t* pb = reinterpret_cast<uint16_t*>(c.ws + c.plan->pb_off);
    const int64_t sPl = 2 * c.sW;
    const SplitOp oa{upd.A, upd.lda, upd.M, upd.Kd, Kp, upd.sA, sPl, 0, 0, pa};
    const SplitOp ob{t2.B, t2.ldb, t2.N, t2.Kd, Kp, t2.sB, sPl, 1, split_mask_b(1), pb};
    int rc = split2(oa, &ob, c.s, c.batch);
    if (rc) return rc;
    G3Args g1{pa, pa, upd.C, upd.M, upd.N, upd.Kd, Kp, upd.ldc, upd.alpha, upd.beta};
    G3Args g2{pa, pb, t2.C, t2.M, t2.N, t2.Kd, Kp, t2.ldc, t2.alpha, t2.beta};
    g1.sA = g1.sB = g2.sA = g2.sB = sPl;
    g1.sC = upd.sC;
    g2.sC = t2.sC;
    rc = tile == GX_T ? g3_pair<GX_T, 0, 0, true, 0, 1, false>(g1, g2, c.s, c.batch)
                      : g3_pair<MG_T, 0, 0, true, 0, 1, false>(g1, g2, c.s, c.batch);
    if (rc != 1) return rc;
    rc = gemm3<0, 0, true>(g1, c.s, c.batch);  // the table was too small: apart
    if (rc) return rc;
    return gemm3<0, 1, false>(g2, c.s, c.batch);
  }
  int rc = product<0, 0, true, true>(c, upd);
  if (rc) return rc;
  return product<0, 1, false, false>(c, t2);
}

int inv_chol(const Ctx& c, int64_t r0, int64_t m, int depth) {
  const int64_t K = c.K;
  if (m <= NB) {
    LaunchTimer timer(HI2X_TIME_CHOL_LEAF, 2.0 * m * m * m / 3.0 * c.batch, c.s);
    hipLaunchKernelGGL(leaf_kernel, dim3(1, 1, (unsigned)c.batch), dim3(256), 0, c.s, c.P, K, r0,
                       (int)m, c.status, c.sP);
    return launch_status("leaf_kernel");
  }
  if (m <= 2 * NB) {  // the node's split is 128 + (m - 128): one fused kernel
    LaunchTimer timer(HI2X_TIME_CHOL_LEAF, 2.0 * m * m * m / 3.0 * c.batch, c.s);
    hipLaunchKernelGGL(node_kernel, dim3(1, 1, (unsigned)c.batch), dim3(256), 0, c.s, c.P, K, r0,
                       (int)(m - NB), c.status, c.sP);
    return launch_status("node_kernel");
  }
  const int64_t nbk = (m + NB - 1) / NB;
  const int64_t m1 = ((nbk + 1) / 2) * NB, m2 = m - m1;
  float* A11 = c.P + r0 * K + r0;
  float* A21 = c.P + (r0 + m1) * K + r0;
  float* A22 = c.P + (r0 + m1) * K + (r0 + m1);
  float* T1 = c.ws + c.plan->t1_off[depth];
  int rc = inv_chol(c, r0, m1, depth + 1);
  if (rc) return rc;
  // T1 = A21 A11^T  (op(B) = A11^T upper)
  rc = product<0, 2, true, false>(c, GemmArgs{A21, A11, T1, m2, m1, m1, K, K, m1, 1.0f, 0.0f});
  if (rc) return rc;
  // A22 -= T1 T1^T (lower) and T2 = T1 A11 (op(B) = A11 lower), both from T1 and A11 alone:
  // at once, before the A22 recursion (T2 in this depth's buffer, the recursion uses the
  // deeper ones)
  float* T2 = c.ws + c.plan->t2_off[depth];
  GemmArgs upd{T1, T1, A22, m2, m2, m1, m1, m1, K, -1.0f, 1.0f};
  GemmArgs t2{T1, A11, T2, m2, m1, m1, m1, K, m1, 1.0f, 0.0f};
  if (pair_small(m1, m2)) {
    upd.sA = c.stride(upd.A);
    upd.sB = c.stride(upd.B);
    upd.sC = c.stride(upd.C);
    t2.sA = c.stride(t2.A);
    t2.sB = c.stride(t2.B);
    t2.sC = c.stride(t2.C);
    rc = tri_gemm_pair(upd, t2, c.s, c.batch);
  } else {
    rc = product_pair(c, upd, t2);
  }
  if (rc) return rc;
  rc = inv_chol(c, r0 + m1, m2, depth + 1);
  if (rc) return rc;
  // A21 = -A22 T2  (A = A22 lower)
  return product<1, 0, false, false>(c, GemmArgs{A22, T2, A21, m2, m1, m2, K, m1, K, -1.0f, 0.0f});
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

// Workspace layout (floats): the recursion's T1 (one per depth) and T2, then lam and the
// status word of the synchronous entry.
static Plan make_plan(int64_t k) {
  Plan plan;
  std::vector<int64_t> t12;
  plan_sizes(k, 0, t12);
  int64_t off = 0;
  for (int64_t sz : t12) {
    plan.t1_off.push_back(off);
    off += (sz + 63) / 64 * 64;
    plan.t2_off.push_back(off);
    off += (sz + 63) / 64 * 64;
  }
  // split planes: 3 x rows x Kp 16-bit values for the largest operand of the top-level
  // products (split2_kernel's layout: two fp16 planes, then the inverse row scales and
  // the row-maximum partials in fp32)
  int64_t m1 = 0;
  if (k > NB) {
    const int64_t nbk = (k + NB - 1) / NB;
    m1 = ((nbk + 1) / 2) * NB;
  }
  const int64_t kp = (m1 + G3_KA - 1) / G3_KA * G3_KA;
  const int64_t plane_floats = (3 * m1 * kp * 2 + 255) / 256 * 64;  // bytes / 4, 256-aligned
  plan.pa_off = off;
  off += plane_floats;
  plan.pb_off = off;
  off += plane_floats;
  plan.total = off;
  return plan;
}
static int64_t ws_floats(const Plan& p) { return p.total + 64; }

// The whole chain for `batch` matrices of one size: matrix z at hs + z shs, its factor at
// u + z su, its workspace at ws + z sw (floats), its status word at status_out + z.
static int chol_launch(const float* hs, int64_t k, float damp, int attempt, float* u,
                       int* status_out, float* ws, const Plan& plan, hipStream_t s,
                       int batch = 1, int64_t shs = 0, int64_t su = 0, int64_t sw = 0) {
  float* lam = ws + plan.total;
  const int big = 0x7fffffff;
  int rc = HI2X_OK;
  hipLaunchKernelGGL(status_init_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s,
                     status_out, big, batch);
  rc = launch_status("status_init_kernel");
  float p10 = 1.0f;
  for (int a = 0; a < attempt; ++a) p10 *= 10.0f;
  if (!rc) {
    hipLaunchKernelGGL(diag_mean_kernel, dim3(1, 1, (unsigned)batch), dim3(256), 0, s, hs, k, damp,
                       p10, lam, shs, sw);
    rc = launch_status("diag_mean_kernel");
  }
  // 16-byte vectors where every row and matrix start is 16-byte aligned
  const bool vec4 = k % 4 == 0 && shs % 4 == 0 && su % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(hs) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(u) & 15) == 0;
  if (!rc && vec4) {
    const dim3 g((unsigned)((k + 1023) / 1024 < 16 ? (k + 1023) / 1024 : 16), (unsigned)k,
                 (unsigned)batch);
    hipLaunchKernelGGL(reverse_damp4_kernel, g, dim3(256), 0, s, hs, k, lam, u, shs, sw, su);
    rc = launch_status("reverse_damp4_kernel");
  } else if (!rc) {
    const dim3 g((unsigned)((k + 255) / 256 < 16 ? (k + 255) / 256 : 16), (unsigned)k,
                 (unsigned)batch);
    hipLaunchKernelGGL(reverse_damp_kernel, g, dim3(256), 0, s, hs, k, lam, u, shs, sw, su);
    rc = launch_status("reverse_damp_kernel");
  }
  Ctx c{u, k, ws, &plan, status_out, s, batch, su, sw};
  if (!rc) rc = inv_chol(c, 0, k, 0);
  if (!rc && vec4) {  // U = J L^-1 J (garbage if the factorisation failed; the status says so)
    const dim3 g((unsigned)((k + 1023) / 1024 < 16 ? (k + 1023) / 1024 : 16), (unsigned)k,
                 (unsigned)batch);
    hipLaunchKernelGGL(reverse_out4_kernel, g, dim3(256), 0, s, u, k, su);
    rc = launch_status("reverse_out4_kernel");
  } else if (!rc) {
    const dim3 g((unsigned)((k + 255) / 256 < 16 ? (k + 255) / 256 : 16), (unsigned)k,
                 (unsigned)batch);
    hipLaunchKernelGGL(reverse_out_kernel, g, dim3(256), 0, s, u, k, su);
    rc = launch_status("reverse_out_kernel");
  }
  return rc;
}

extern "C" int hi2x_chol_lambda(const float* hs, int64_t k, float damp, int attempt,
                                float* lam, void* stream) {
  clear_error();
  HI2X_REQUIRE(hs && lam && k > 0, "chol_lambda: bad arguments");
  HI2X_REQUIRE(attempt >= 0 && attempt <= 30, "chol_lambda: attempt %d", attempt);
  float p10 = 1.0f;
  for (int a = 0; a < attempt; ++a) p10 *= 10.0f;
  hipLaunchKernelGGL(diag_mean_kernel, dim3(1), dim3(256), 0, as_stream(stream), hs, k, damp,
                     p10, lam, (int64_t)0, (int64_t)0);
  return launch_status("diag_mean_kernel");
}

extern "C" int64_t hi2x_chol_workspace_bytes(int64_t k) {
  if (k <= 0) return -1;
  return ws_floats(make_plan(k)) * (int64_t)sizeof(float);
}

extern "C" int hi2x_chol_inv_upper_async(const float* hs, int64_t k, float damp, int attempt,
                                         float* u, int32_t* status, void* ws, int64_t ws_bytes,
                                         void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && hs && u && hs != u && status, "chol_inv_upper_async: bad arguments");
  HI2X_REQUIRE(k % 4 == 0, "chol_inv_upper_async: k=%lld is not a multiple of 4", (long long)k);
  HI2X_REQUIRE(attempt >= 0 && attempt < 10, "chol_inv_upper_async: attempt %d", attempt);
  hipStream_t s = as_stream(stream);
  const Plan plan = make_plan(k);
  Workspace w;
  const int rc = take_workspace(w, ws, ws_bytes, (size_t)ws_floats(plan) * sizeof(float), s,
                                "chol_inv_upper_async");
  if (rc) return rc;
  return chol_launch(hs, k, damp, attempt, u, status, reinterpret_cast<float*>(w.p), plan, s);
}

extern "C" int hi2x_chol_inv_upper(const float* hs, int64_t k, float damp, int attempt,
                                   float* u, void* ws, int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && hs && u && hs != u, "chol_inv_upper: bad arguments");
  HI2X_REQUIRE(k % 4 == 0, "chol_inv_upper: k=%lld is not a multiple of 4", (long long)k);
  HI2X_REQUIRE(attempt >= 0 && attempt < 10, "chol_inv_upper: attempt %d", attempt);
  hipStream_t s = as_stream(stream);
  const Plan plan = make_plan(k);
  Workspace w;
  int rc = take_workspace(w, ws, ws_bytes, (size_t)ws_floats(plan) * sizeof(float), s,
                          "chol_inv_upper");
  if (rc) return rc;
  float* wsf = reinterpret_cast<float*>(w.p);
  int* status = reinterpret_cast<int*>(wsf + plan.total + 1);
  rc = chol_launch(hs, k, damp, attempt, u, status, wsf, plan, s);
  int st = 0x7fffffff;
  if (!rc) {
    hipError_t e = hipMemcpyAsync(&st, status, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      set_error("chol_inv_upper: status read: %s", hipGetErrorString(e));
      rc = HI2X_ELAUNCH;
    }
  }
  if (!rc && st != 0x7fffffff) {
    set_error("chol_inv_upper: not positive definite in the block at %d (attempt %d)", st - 1,
              attempt);
    rc = HI2X_ENOTPD;
  }
  return rc;
}

// Workspace of one factor of a batch, rounded to 256 bytes.
static int64_t batch_ws_floats(const Plan& p) { return (ws_floats(p) + 63) / 64 * 64; }

extern "C" int64_t hi2x_chol_batched_workspace_bytes(int64_t k, int64_t batch) {
  if (k <= 0 || batch <= 0 || batch > 65535) return -1;
  return batch_ws_floats(make_plan(k)) * batch * (int64_t)sizeof(float);
}

extern "C" int hi2x_chol_inv_upper_batched_async(const float* hs, int64_t hs_stride, int64_t k,
                                                 int64_t batch, float damp, int attempt,
                                                 float* u, int64_t u_stride, int32_t* status,
                                                 void* ws, int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && hs && u && status && batch > 0 && batch <= 65535,
               "chol_inv_upper_batched_async: bad arguments");
  HI2X_REQUIRE(k % 4 == 0, "chol_inv_upper_batched: k=%lld is not a multiple of 4",
               (long long)k);
  HI2X_REQUIRE(hs_stride >= k * k && u_stride >= k * k,
               "chol_inv_upper_batched_async: strides %lld / %lld below k * k",
               (long long)hs_stride, (long long)u_stride);
  HI2X_REQUIRE(!(u < hs + hs_stride * batch && hs < u + u_stride * batch),
               "chol_inv_upper_batched_async: hs and u overlap");
  HI2X_REQUIRE(attempt >= 0 && attempt < 10, "chol_inv_upper_batched_async: attempt %d",
               attempt);
  hipStream_t s = as_stream(stream);
  const Plan plan = make_plan(k);
  const int64_t sw = batch_ws_floats(plan);
  Workspace w;
  const int rc = take_workspace(w, ws, ws_bytes, (size_t)(sw * batch) * sizeof(float), s,
                                "chol_inv_upper_batched_async");
  if (rc) return rc;
  return chol_launch(hs, k, damp, attempt, u, status, reinterpret_cast<float*>(w.p), plan, s,
                     (int)batch, hs_stride, u_stride, sw);
}
