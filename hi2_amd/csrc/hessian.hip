// Calibration Hessian S += X^T X on MFMA, and its transform to the stored basis.
//
// Reference: hi2/hessian.py:26-47 (HessianStats.update/merge/mean),
// hi2/hessian.py:50-68 (transform_sigma), hi2/moe.py:83-100 (routed token subsets).
#include "common.h"

namespace hi2x {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int HT = 128;  // output tile (features x features)
constexpr int TCB = 32;  // tokens per LDS stage (bf16): two 32x32x16 steps
constexpr int TCF = 8;   // tokens per LDS stage (f32): four 32x32x2 steps
constexpr int XSB = TCB + 8;  // LDS row stride in bf16 elements (bank spread)

__device__ __forceinline__ void upper_tile(int nT, int idx, int& ta, int& tb) {
  int a = 0;
  while (idx >= nT - a) {
    idx -= nT - a;
    ++a;
  }
  ta = a;
  tb = a + idx;
}

// Adds the accumulator tiles of one 128 x 128 output tile (rows a0.., cols b0..) into S,
// mirrored so that S stays exactly symmetric: a diagonal tile writes (i, j) and (j, i)
// from the i <= j element; an off-diagonal tile writes both (i, j) and (j, i).
__device__ __forceinline__ void store_sym(float* __restrict__ s, int64_t K, int64_t a0,
                                          int64_t b0, bool diag, int wr, int wcn, int lane,
                                          const f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t row = a0 + wr * 64 + a * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        const int64_t col = b0 + wcn * 64 + b * 32 + (lane & 31);
        if (row >= K || col >= K) continue;
        if (diag && row > col) continue;
        const float v = s[row * K + col] + acc[a][b][j];
        s[row * K + col] = v;
        if (row != col) s[col * K + row] = v;
      }
}

// bf16 X [T, K]: one workgroup per upper 128 x 128 tile; the two feature slabs of a
// 32-token stage are staged feature-major in LDS so every lane reads its 8 tokens as
// one 16-byte vector; v_mfma_f32_32x32x16_bf16 accumulates in f32 (products exact).
__global__ __launch_bounds__(256) void syrk_bf16_kernel(const uint16_t* __restrict__ x,
                                                        int64_t T, int64_t K, int nT,
                                                        float* __restrict__ s) {
  __shared__ __attribute__((aligned(16))) uint16_t Xa[HT * XSB];
  __shared__ __attribute__((aligned(16))) uint16_t Xb[HT * XSB];
  int ta, tb;
  upper_tile(nT, blockIdx.x, ta, tb);
  const bool diag = ta == tb;
  const int64_t a0 = (int64_t)ta * HT, b0 = (int64_t)tb * HT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;

  const int f = tid & (HT - 1), tg = tid >> 7;  // feature, 16-token half
  for (int64_t t0 = 0; t0 < T; t0 += TCB) {
    __syncthreads();
    {
      u16x8 va0, va1, vb0, vb1;
      const int64_t fa = a0 + f, fb = b0 + f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t t1 = t0 + tg * 16 + e, t2 = t1 + 8;
        va0[e] = (t1 < T && fa < K) ? x[t1 * K + fa] : (uint16_t)0;
        va1[e] = (t2 < T && fa < K) ? x[t2 * K + fa] : (uint16_t)0;
        if (!diag) {
          vb0[e] = (t1 < T && fb < K) ? x[t1 * K + fb] : (uint16_t)0;
          vb1[e] = (t2 < T && fb < K) ? x[t2 * K + fb] : (uint16_t)0;
        }
      }
      *reinterpret_cast<u16x8*>(&Xa[f * XSB + tg * 16]) = va0;
      *reinterpret_cast<u16x8*>(&Xa[f * XSB + tg * 16 + 8]) = va1;
      if (!diag) {
        *reinterpret_cast<u16x8*>(&Xb[f * XSB + tg * 16]) = vb0;
        *reinterpret_cast<u16x8*>(&Xb[f * XSB + tg * 16 + 8]) = vb1;
      }
    }
    __syncthreads();
    const uint16_t* XB = diag ? Xa : Xb;
#pragma unroll
    for (int ks = 0; ks < TCB; ks += 16) {
      const int ko = ks + 8 * (lane >> 5);
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int a = 0; a < 2; ++a)
        av[a] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u16x8*>(&Xa[(wr * 64 + a * 32 + (lane & 31)) * XSB + ko]));
#pragma unroll
      for (int b = 0; b < 2; ++b)
        bv[b] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u16x8*>(&XB[(wcn * 64 + b * 32 + (lane & 31)) * XSB + ko]));
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[a], bv[b], acc[a][b], 0, 0, 0);
    }
  }
  store_sym(s, K, a0, b0, diag, wr, wcn, lane, acc);
}

// f32 X [T, K]: same tiling on v_mfma_f32_32x32x2_f32.
__global__ __launch_bounds__(256) void syrk_f32_kernel(const float* __restrict__ x, int64_t T,
                                                       int64_t K, int nT,
                                                       float* __restrict__ s) {
  __shared__ float Xa[TCF][HT];
  __shared__ float Xb[TCF][HT];
  int ta, tb;
  upper_tile(nT, blockIdx.x, ta, tb);
  const bool diag = ta == tb;
  const int64_t a0 = (int64_t)ta * HT, b0 = (int64_t)tb * HT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;
  const int f = tid & (HT - 1), tg = tid >> 7;
  for (int64_t t0 = 0; t0 < T; t0 += TCF) {
    __syncthreads();
#pragma unroll
    for (int e = 0; e < TCF / 2; ++e) {
      const int tt = tg * (TCF / 2) + e;
      const int64_t t1 = t0 + tt;
      Xa[tt][f] = (t1 < T && a0 + f < K) ? x[t1 * K + a0 + f] : 0.0f;
      if (!diag) Xb[tt][f] = (t1 < T && b0 + f < K) ? x[t1 * K + b0 + f] : 0.0f;
    }
    __syncthreads();
    const float(*XB)[HT] = diag ? Xa : Xb;
#pragma unroll
    for (int ks = 0; ks < TCF; ks += 2) {
      const int kr = ks + (lane >> 5);
      float av[2], bv[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) av[a] = Xa[kr][wr * 64 + a * 32 + (lane & 31)];
#pragma unroll
      for (int b = 0; b < 2; ++b) bv[b] = XB[kr][wcn * 64 + b * 32 + (lane & 31)];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
    }
  }
  store_sym(s, K, a0, b0, diag, wr, wcn, lane, acc);
}

// transform_sigma, one workgroup (16 x 16 threads) per upper pair of 16 x 16 blocks
// (gi <= gh).  Evaluates, as the reference's fp32 einsums do:
//   s = (sigma * inv_i) * inv_j                       (smoothing, when col_scale given)
//   t1[i][k] = sum_j m_gi[i][j] s[j][k]                (sequential FMA chain from 0)
//   t2[i][l] = sum_k t1[i][k] m_gh[l][k]               (sequential FMA chain from 0)
//   out = 0.5 * (t2 + t2^T)
// with m = H16/4 on flagged groups and I elsewhere; an identity product reduces to
// x + 0 (the chain maps -0 to +0), so both orders give the reference's bits.
__device__ __forceinline__ float hsgn(int i, int j) {
  return (__builtin_popcount(i & j) & 1) ? -0.25f : 0.25f;
}

__global__ __launch_bounds__(256) void sigma_transform_kernel(
    const float* __restrict__ sigma, const uint16_t* __restrict__ col_scale,
    const uint8_t* __restrict__ had, int64_t K, int G, float* __restrict__ hs) {
  __shared__ float S1[16][17], S2[16][17], T1[16][17], T2[16][17];
  int gi, gh;
  upper_tile(G, blockIdx.x, gi, gh);
  const int i = threadIdx.x >> 4, l = threadIdx.x & 15;
  const bool same = gi == gh;
  const int64_t ri = (int64_t)gi * 16, rh = (int64_t)gh * 16;
  {
    float a = sigma[(ri + i) * K + rh + l];
    float b = sigma[(rh + i) * K + ri + l];
    if (col_scale) {
      const float ii = 1.0f / f16_from_bits(col_scale[ri + i]);
      const float il = 1.0f / f16_from_bits(col_scale[rh + l]);
      const float hi = 1.0f / f16_from_bits(col_scale[rh + i]);
      const float hl = 1.0f / f16_from_bits(col_scale[ri + l]);
      a = (a * ii) * il;
      b = (b * hi) * hl;
    }
    S1[i][l] = a;  // block (gi, gh)
    S2[i][l] = b;  // block (gh, gi)
  }
  __syncthreads();
  const bool fi = had[gi] != 0, fh = had[gh] != 0;
  // left products: rows of block (gi, gh) by m_gi, rows of block (gh, gi) by m_gh
  {
    float a = 0.0f, b = 0.0f;
    if (fi) {
#pragma unroll
      for (int j = 0; j < 16; ++j) a = __builtin_fmaf(hsgn(i, j), S1[j][l], a);
    } else {
      a = S1[i][l] + 0.0f;
    }
    if (fh) {
#pragma unroll
      for (int j = 0; j < 16; ++j) b = __builtin_fmaf(hsgn(i, j), S2[j][l], b);
    } else {
      b = S2[i][l] + 0.0f;
    }
    T1[i][l] = a;
    T2[i][l] = b;
  }
  __syncthreads();
  // right products: block (gi, gh) by m_gh^T, block (gh, gi) by m_gi^T
  float u1 = 0.0f, u2 = 0.0f;
  if (fh) {
#pragma unroll
    for (int k = 0; k < 16; ++k) u1 = __builtin_fmaf(T1[i][k], hsgn(l, k), u1);
  } else {
    u1 = T1[i][l] + 0.0f;
  }
  if (fi) {
#pragma unroll
    for (int k = 0; k < 16; ++k) u2 = __builtin_fmaf(T2[i][k], hsgn(l, k), u2);
  } else {
    u2 = T2[i][l] + 0.0f;
  }
  __syncthreads();
  S1[i][l] = u1;  // t2 of block (gi, gh)
  S2[i][l] = u2;  // t2 of block (gh, gi)
  __syncthreads();
  // out(gi, gh)[i][l] = 0.5 * (t2(gi,gh)[i][l] + t2(gh,gi)[l][i]); out(gh, gi) is its transpose
  const float o = 0.5f * (S1[i][l] + (same ? S1[l][i] : S2[l][i]));
  hs[(ri + i) * K + rh + l] = o;
  if (!same) hs[(rh + l) * K + ri + i] = o;
}

int launch_syrk(const void* x, int dtype, int64_t t, int64_t k, float* s, hipStream_t st) {
  const int nT = (int)((k + HT - 1) / HT);
  const int64_t tiles = (int64_t)nT * (nT + 1) / 2;
  if (dtype == 2)
    hipLaunchKernelGGL(syrk_bf16_kernel, dim3((unsigned)tiles), dim3(256), 0, st,
                       (const uint16_t*)x, t, k, nT, s);
  else
    hipLaunchKernelGGL(syrk_f32_kernel, dim3((unsigned)tiles), dim3(256), 0, st,
                       (const float*)x, t, k, nT, s);
  return launch_status("syrk_kernel");
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_hessian_syrk(const void* x, int dtype, int64_t t, int64_t k, float* s,
                                 void* stream) {
  clear_error();
  HI2X_REQUIRE(dtype == 0 || dtype == 2, "hessian_syrk: dtype %d (0 = f32, 2 = bf16)", dtype);
  HI2X_REQUIRE(k > 0 && t >= 0, "hessian_syrk: bad shape");
  if (t == 0) return HI2X_OK;
  return launch_syrk(x, dtype, t, k, s, as_stream(stream));
}

extern "C" int hi2x_hessian_syrk_varlen(const void* x, int dtype, const int64_t* offs,
                                        int64_t n_groups, int64_t k, float* const* s_ptrs,
                                        void* stream) {
  clear_error();
  HI2X_REQUIRE(dtype == 0 || dtype == 2, "hessian_syrk_varlen: dtype %d", dtype);
  const size_t esz = dtype == 2 ? 2 : 4;
  for (int64_t e = 0; e < n_groups; ++e) {
    const int64_t t = offs[e + 1] - offs[e];
    HI2X_REQUIRE(t >= 0, "hessian_syrk_varlen: offsets not ascending");
    if (t == 0) continue;
    const char* xe = static_cast<const char*>(x) + (size_t)offs[e] * (size_t)k * esz;
    const int rc = launch_syrk(xe, dtype, t, k, s_ptrs[e], as_stream(stream));
    if (rc) return rc;
  }
  return HI2X_OK;
}

extern "C" int hi2x_sigma_transform(const float* sigma, const uint16_t* col_scale,
                                    const uint8_t* had, int64_t k, float* hs, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0, "sigma_transform: K=%lld not a multiple of 16",
               (long long)k);
  HI2X_REQUIRE(sigma != hs, "sigma_transform: in-place not supported");
  const int G = (int)(k / 16);
  const int64_t pairs = (int64_t)G * (G + 1) / 2;
  hipLaunchKernelGGL(sigma_transform_kernel, dim3((unsigned)pairs), dim3(256), 0,
                     as_stream(stream), sigma, col_scale, had, k, G, hs);
  return launch_status("sigma_transform_kernel");
}
