// Ladder fit, 8-bit block parameters, decode, and the GPTQ finish (un-permute + SSE).
//
// Reference: hi2/encode.py:18-119 (EFFORT, _recon, _lsq, fit_ladder, quantize_params),
// hi2/ladder_kernel.py:44-86 (the grid search), hi2/format.py:45-69 (decode_params,
// ladder_dequantize), hi2/hessian.py:318-345 (_finish).
#include "common.h"

namespace hi2x {
namespace {

struct Grid {
  float v[8];
};

// One thread per (row, block).  Grid search then `ls` weighted least-squares refits,
// every elementwise op rounded as the reference's torch ops and every block sum in
// torch's CPU order (torch_sum_small), so lo/step are bit-identical to fit_ladder.
template <int B>
__global__ __launch_bounds__(256) void ladder_fit_kernel(
    const float* __restrict__ w, const float* __restrict__ d, int64_t rows, int64_t k,
    int nlev, Grid grid, int G, int ls, float* __restrict__ out_lo,
    float* __restrict__ out_st, float* __restrict__ out_err,
    const int32_t* __restrict__ d_row) {
  const int64_t nb = k / B;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nb) return;
  const int64_t r = i / nb, b = i % nb;
  const float* wp = w + r * k + b * B;
  const float* dp = d + (d_row ? (int64_t)d_row[r] * k : 0) + b * B;
  float x[B], dd[B];
#pragma unroll
  for (int t = 0; t < B; t += 4) {
    const float4 v = *reinterpret_cast<const float4*>(wp + t);
    x[t] = v.x;
    x[t + 1] = v.y;
    x[t + 2] = v.z;
    x[t + 3] = v.w;
    const float4 e = *reinterpret_cast<const float4*>(dp + t);
    dd[t] = e.x;
    dd[t + 1] = e.y;
    dd[t + 2] = e.z;
    dd[t + 3] = e.w;
  }
  const float nm = (float)(nlev - 1);
  float mn = x[0], mx = x[0];
#pragma unroll
  for (int t = 1; t < B; ++t) {
    mn = (x[t] < mn) ? x[t] : mn;
    mx = (x[t] > mx) ? x[t] : mx;
  }
  const float span = mx - mn;

  // (x - lo) / safe through the correctly rounded reciprocal of safe (div_rcp_code):
  // the same codes as the IEEE division.  A subnormal candidate step (spans below about
  // 2^-120) takes the IEEE division instead, in a branch the wave takes only when one of
  // its lanes has such a step.
  auto err_with = [&](float lo, float step, float safe, float ys, auto div) {
    return torch_sum_small<B>([&](int t) {
      const float c = clamp_code(__builtin_rintf(div(x[t] - lo, safe, ys)), nm);
      const float rec = lo + c * step;
      const float df = rec - x[t];
      return dd[t] * (df * df);
    });
  };
  auto err_of = [&](float lo, float step) {
    const float safe = (step == 0.0f) ? 1.0f : step;
    const float ys = 1.0f / safe;
    if (__builtin_amdgcn_ballot_w64(!div_code_ok(safe)) == 0)
      return err_with(lo, step, safe, ys,
                      [](float a, float b, float y) { return div_rcp_code(a, b, y); });
    return err_with(lo, step, safe, ys,
                    [](float a, float b, float y) { return div_code(a, b, y); });
  };

  float best_lo = 0.0f, best_st = 0.0f, best_err = 0.0f;
  bool first = true;
  for (int a = 0; a < G; ++a) {
    const float lo = mn + grid.v[a] * span;
    for (int bb = 0; bb < G; ++bb) {
      const float step = ((mx - grid.v[bb] * span) - lo) / nm;
      const float err = err_of(lo, step);
      if (first || err < best_err) {
        best_lo = lo;
        best_st = step;
        best_err = err;
        first = false;
      }
    }
  }
  for (int it = 0; it < ls; ++it) {
    const float safe = (best_st == 0.0f) ? 1.0f : best_st;
    const float ys = 1.0f / safe;
    float c[B];
    if (__builtin_amdgcn_ballot_w64(!div_code_ok(safe)) == 0) {
#pragma unroll
      for (int t = 0; t < B; ++t)
        c[t] = clamp_code(__builtin_rintf(div_rcp_code(x[t] - best_lo, safe, ys)), nm);
    } else {
#pragma unroll
      for (int t = 0; t < B; ++t)
        c[t] = clamp_code(__builtin_rintf(div_code(x[t] - best_lo, safe, ys)), nm);
    }
    const float sd = torch_sum_small<B>([&](int t) { return dd[t]; });
    const float sc = torch_sum_small<B>([&](int t) { return dd[t] * c[t]; });
    const float scc = torch_sum_small<B>([&](int t) { return (dd[t] * c[t]) * c[t]; });
    const float sw = torch_sum_small<B>([&](int t) { return dd[t] * x[t]; });
    const float scw = torch_sum_small<B>([&](int t) { return (dd[t] * c[t]) * x[t]; });
    const float det = sd * scc - sc * sc;
    const bool ok = __builtin_fabsf(det) > 1e-20f;
    const float step = ok ? (sd * scw - sc * sw) / det : 0.0f;
    const float sdc = (sd < 1e-20f) ? 1e-20f : sd;
    const float lo =
        ok ? (sw - step * sc) / sdc : torch_sum_small<B>([&](int t) { return x[t]; }) / (float)B;
    const float err = err_of(lo, step);
    if (err < best_err && step > 0.0f) {
      best_lo = lo;
      best_st = step;
      best_err = err;
    }
  }
  out_lo[i] = best_lo;
  out_st[i] = best_st;
  if (out_err) out_err[i] = best_err;
}

// The same fit with NL lanes (2 or 4) per (row, block), for B = 32 and 64: the one-lane
// kernel holds 2B values per lane (x and d) and runs one wave per SIMD at B = 64, too
// few to hide its dependent chains.  Torch's CPU sum of a block runs over 8-wide vectors
// (position e % 8); lane h of a group owns the positions [h P, h P + P), P = 8 / NL,
// B / NL elements, as local slot j = P (e / 8) + e % 8 - h P.  Every sum is torch's order
// split at the vector position: each lane forms the per-position partials of its
// positions in that order, lane 0 starts the sum over positions from zero and each lane
// in turn continues it with its own (one lane-to-lane move per lane), and the last
// lane's total goes to the whole group, so every decision below is taken identically by
// all NL lanes and equals the one-lane kernel's.
template <int NL>
struct LaneGroup {  // DPP moves within aligned groups of NL lanes (quad_perm patterns)
  static_assert(NL == 2 || NL == 4, "lanes per group");
  // from the previous lane of the group (lane 0 reads itself)
  static constexpr int PREV = NL == 2 ? 0xA0 : 0x90;  // [0,0,2,2] / [0,0,1,2]
  static constexpr int LAST = NL == 2 ? 0xF5 : 0xFF;  // [1,1,3,3] / [3,3,3,3]
  static constexpr int X1 = 0xB1, X2 = 0x4E;           // lane ^ 1: [1,0,3,2]; ^ 2: [2,3,0,1]
  static constexpr int FIRST = NL == 2 ? 0xA0 : 0x00;  // lane 0 of the group
  template <int CTRL>
  static __device__ __forceinline__ float mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
  }
  template <int CTRL>
  static __device__ __forceinline__ int movi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
  }
};

// torch_sum_small<B> of fn over the group's elements; fn(j) yields the element in local
// slot j.  B / 32 rows of 4 vectors, no tail vectors for B = 32 and 64.
template <int B, int NL, class F>
__device__ __forceinline__ float group_sum(F fn) {
  static_assert(B % 32 == 0 && B <= 64, "block size");
  constexpr int SI = B / 32, P = 8 / NL;
  using LG = LaneGroup<NL>;
  float Q[P];
#pragma unroll
  for (int vv = 0; vv < P; ++vv) {
    float p[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) p[kk] = 0.0f;
#pragma unroll
    for (int i = 0; i < SI; ++i)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) p[kk] += fn((i * 4 + kk) * P + vv);
    Q[vv] = ((p[0] + p[1]) + p[2]) + p[3];
  }
  float acc = 0.0f;
#pragma unroll
  for (int vv = 0; vv < P; ++vv) acc += Q[vv];
  // after move m, lane m holds the sum over positions [0, (m + 1) P)
#pragma unroll
  for (int m = 1; m < NL; ++m) {
    float t = LG::template mov<LG::PREV>(acc);
#pragma unroll
    for (int vv = 0; vv < P; ++vv) t += Q[vv];
    acc = t;
  }
  return LG::template mov<LG::LAST>(acc);
}

template <int B, int NL>
__global__ __launch_bounds__(256) void ladder_fit_group_kernel(
    const float* __restrict__ w, const float* __restrict__ d, int64_t rows, int64_t k,
    int nlev, Grid grid, int G, int ls, float* __restrict__ out_lo,
    float* __restrict__ out_st, float* __restrict__ out_err,
    const int32_t* __restrict__ d_row) {
  constexpr int NE = B / NL, P = 8 / NL;  // elements and positions per lane
  using LG = LaneGroup<NL>;
  const int64_t nb = k / B;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = gid / NL;
  const int h = (int)(gid % NL);
  if (i >= rows * nb) return;  // the lanes of a group leave together
  const int64_t r = i / nb, b = i % nb;
  const float* wp = w + r * k + b * B + P * h;
  const float* dp = d + (d_row ? (int64_t)d_row[r] * k : 0) + b * B + P * h;
  float x[NE], dd[NE];
#pragma unroll
  for (int q = 0; q < B / 8; ++q) {  // vector q: elements 8q + P h .. 8q + P h + P - 1
    if constexpr (P == 4) {
      const float4 v = *reinterpret_cast<const float4*>(wp + 8 * q);
      const float4 e = *reinterpret_cast<const float4*>(dp + 8 * q);
      x[4 * q] = v.x;
      x[4 * q + 1] = v.y;
      x[4 * q + 2] = v.z;
      x[4 * q + 3] = v.w;
      dd[4 * q] = e.x;
      dd[4 * q + 1] = e.y;
      dd[4 * q + 2] = e.z;
      dd[4 * q + 3] = e.w;
    } else {
      const float2 v = *reinterpret_cast<const float2*>(wp + 8 * q);
      const float2 e = *reinterpret_cast<const float2*>(dp + 8 * q);
      x[2 * q] = v.x;
      x[2 * q + 1] = v.y;
      dd[2 * q] = e.x;
      dd[2 * q + 1] = e.y;
    }
  }
  const float nm = (float)(nlev - 1);
  // min / max as the sequential scan from x[0] with strict comparisons: the first
  // element (in index order) equal to the extreme.  Each lane scans its elements from
  // x[0]; the group then keeps the smaller (larger) value, on a tie the earlier element.
  const float x0 = LG::template mov<LG::FIRST>(x[0]);
  float mn = x0, mx = x0;
  int imn = 0, imx = 0;
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const int e = 8 * (j / P) + P * h + (j % P);
    if (x[j] < mn) {
      mn = x[j];
      imn = e;
    }
    if (x[j] > mx) {
      mx = x[j];
      imx = e;
    }
  }
  auto merge = [&](float omn, int oin, float omx, int oix) {
    const bool tmn = omn < mn || (omn == mn && oin < imn);
    const bool tmx = omx > mx || (omx == mx && oix < imx);
    mn = tmn ? omn : mn;
    imn = tmn ? oin : imn;
    mx = tmx ? omx : mx;
    imx = tmx ? oix : imx;
  };
  merge(LG::template mov<LG::X1>(mn), LG::template movi<LG::X1>(imn),
        LG::template mov<LG::X1>(mx), LG::template movi<LG::X1>(imx));
  if constexpr (NL == 4)
    merge(LG::template mov<LG::X2>(mn), LG::template movi<LG::X2>(imn),
          LG::template mov<LG::X2>(mx), LG::template movi<LG::X2>(imx));
  const float span = mx - mn;

  // The code of an element is clamp(rint((x - lo) / safe)).  q0 = (x - lo) * (1 / safe)
  // is within 2 ulp of the quotient, so rint(q0) is the quotient's rint unless q0 lies
  // within 2 ulp of a half-integer: |q0 - rint(q0)| >= 0.5 - tol, tol = (nm + 1) 2^-22
  // covering 2 ulp everywhere below nm + 1 (farther out both clamp to the same end).
  // The error of a candidate is summed from those cheap codes, and the wave sums it
  // again with the exact quotients (div_code) when any of its lanes met a near-tie or
  // has a subnormal candidate step (spans below about 2^-120, where the reciprocal
  // overflows and the IEEE division gives the codes).  A zero code may come out as -0
  // here and +0 there: it only ever multiplies into a term that is squared or added to +0
  // first, so the sums are the same.
  const float tol = (nm + 1.0f) * 0x1p-22f;
  auto err_exact = [&](float lo, float step, float safe, float ys) {
    return group_sum<B, NL>([&](int j) {
      const float c = clamp_code(__builtin_rintf(div_code(x[j] - lo, safe, ys)), nm);
      const float rec = lo + c * step;
      const float df = rec - x[j];
      return dd[j] * (df * df);
    });
  };
  auto err_of = [&](float lo, float step) {
    const float safe = (step == 0.0f) ? 1.0f : step;
    const float ys = 1.0f / safe;
    bool near = !div_code_ok(safe);
    const float e = group_sum<B, NL>([&](int j) {
      const float q0 = (x[j] - lo) * ys;
      const float r0 = __builtin_rintf(q0);
      near = near || __builtin_fabsf(q0 - r0) >= 0.5f - tol;
      const float c = __builtin_amdgcn_fmed3f(r0, 0.0f, nm);
      const float rec = lo + c * step;
      const float df = rec - x[j];
      return dd[j] * (df * df);
    });
    if (__builtin_amdgcn_ballot_w64(near) == 0) return e;
    return err_exact(lo, step, safe, ys);
  };

  float best_lo = 0.0f, best_st = 0.0f, best_err = 0.0f;
  bool first = true;
  for (int a = 0; a < G; ++a) {
    const float lo = mn + grid.v[a] * span;
    for (int bb = 0; bb < G; ++bb) {
      const float step = ((mx - grid.v[bb] * span) - lo) / nm;
      const float err = err_of(lo, step);
      if (first || err < best_err) {
        best_lo = lo;
        best_st = step;
        best_err = err;
        first = false;
      }
    }
  }
  for (int it = 0; it < ls; ++it) {
    const float safe = (best_st == 0.0f) ? 1.0f : best_st;
    const float ys = 1.0f / safe;
    float c[NE];
    if (__builtin_amdgcn_ballot_w64(!div_code_ok(safe)) == 0) {
#pragma unroll
      for (int j = 0; j < NE; ++j)
        c[j] = clamp_code(__builtin_rintf(div_rcp_code(x[j] - best_lo, safe, ys)), nm);
    } else {
#pragma unroll
      for (int j = 0; j < NE; ++j)
        c[j] = clamp_code(__builtin_rintf(div_code(x[j] - best_lo, safe, ys)), nm);
    }
    const float sd = group_sum<B, NL>([&](int j) { return dd[j]; });
    const float sc = group_sum<B, NL>([&](int j) { return dd[j] * c[j]; });
    const float scc = group_sum<B, NL>([&](int j) { return (dd[j] * c[j]) * c[j]; });
    const float sw = group_sum<B, NL>([&](int j) { return dd[j] * x[j]; });
    const float scw = group_sum<B, NL>([&](int j) { return (dd[j] * c[j]) * x[j]; });
    const float det = sd * scc - sc * sc;
    const bool ok = __builtin_fabsf(det) > 1e-20f;
    const float step = ok ? (sd * scw - sc * sw) / det : 0.0f;
    const float sdc = (sd < 1e-20f) ? 1e-20f : sd;
    const float lo =
        ok ? (sw - step * sc) / sdc : group_sum<B, NL>([&](int j) { return x[j]; }) / (float)B;
    const float err = err_of(lo, step);
    if (err < best_err && step > 0.0f) {
      best_lo = lo;
      best_st = step;
      best_err = err;
    }
  }
  if (h == 0) {
    out_lo[i] = best_lo;
    out_st[i] = best_st;
    if (out_err) out_err[i] = best_err;
  }
}

// quantize_params + decode_params, one wave per row (max/min reductions are exact).
__global__ __launch_bounds__(256) void params_kernel(
    const float* __restrict__ lo, const float* __restrict__ step, int64_t rows, int64_t nb,
    uint8_t* __restrict__ lo_u8, uint8_t* __restrict__ st_u8, uint16_t* __restrict__ consts,
    float* __restrict__ lo_d, float* __restrict__ st_d, int64_t ldd) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* l = lo + r * nb;
  const float* s = step + r * nb;
  float smax = 0.0f, lmin = __builtin_inff(), lmax = -__builtin_inff();
  bool any = false;
  for (int64_t b = lane; b < nb; b += 64) {
    const float sv = s[b] < 0.0f ? 0.0f : s[b];
    smax = (!any || sv > smax) ? sv : smax;
    lmin = (l[b] < lmin) ? l[b] : lmin;
    lmax = (l[b] > lmax) ? l[b] : lmax;
    any = true;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float so = __shfl_xor(smax, off);
    const float no = __shfl_xor(lmin, off);
    const float xo = __shfl_xor(lmax, off);
    const int ao = __shfl_xor((int)any, off);
    smax = (ao && (!any || so > smax)) ? so : smax;
    lmin = (no < lmin) ? no : lmin;
    lmax = (xo > lmax) ? xo : lmax;
    any = any || ao;
  }
  const uint16_t ss_h = f16_bits(smax / 255.0f);
  const float ss = f16_from_bits(ss_h);
  const uint16_t lm_h = f16_bits(lmin);
  const float lmf = f16_from_bits(lm_h);
  float span = lmax - lmf;
  span = span < 0.0f ? 0.0f : span;
  const uint16_t ls_h = f16_bits(span / 255.0f);
  const float lsf = f16_from_bits(ls_h);
  if (lane == 0) {
    consts[r * 3 + 0] = lm_h;
    consts[r * 3 + 1] = ls_h;
    consts[r * 3 + 2] = ss_h;
  }
  for (int64_t b = lane; b < nb; b += 64) {
    const float sv = s[b] < 0.0f ? 0.0f : s[b];
    float su = 0.0f;
    if (ss > 0.0f) su = __builtin_rintf(sv / (ss < 1e-30f ? 1e-30f : ss));
    su = su < 0.0f ? 0.0f : (su > 255.0f ? 255.0f : su);
    float lu = 0.0f;
    if (lsf > 0.0f) lu = __builtin_rintf((l[b] - lmf) / (lsf < 1e-30f ? 1e-30f : lsf));
    lu = lu < 0.0f ? 0.0f : (lu > 255.0f ? 255.0f : lu);
    const uint8_t lub = (uint8_t)lu, sub = (uint8_t)su;
    lo_u8[r * nb + b] = lub;
    st_u8[r * nb + b] = sub;
    if (lo_d) {
      const double v = (double)lub * (double)lsf + (double)lmf;
      lo_d[r * ldd + b] = f16_round((float)v);
      st_d[r * ldd + b] = f16_round((float)sub * ss);
    }
  }
}

__global__ void decode_kernel(const uint8_t* __restrict__ lo_u8, const uint8_t* __restrict__ st_u8,
                              const uint16_t* __restrict__ consts, int64_t rows, int64_t nb,
                              uint16_t* __restrict__ lo_h, uint16_t* __restrict__ st_h) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nb) return;
  const int64_t r = i / nb;
  const float lm = f16_from_bits(consts[r * 3 + 0]);
  const float ls = f16_from_bits(consts[r * 3 + 1]);
  const float ss = f16_from_bits(consts[r * 3 + 2]);
  const double v = (double)lo_u8[i] * (double)ls + (double)lm;
  lo_h[i] = f16_bits((float)v);
  st_h[i] = f16_bits((float)st_u8[i] * ss);
}

__global__ void dequant_kernel(const uint8_t* __restrict__ codes, const float* __restrict__ lo,
                               const float* __restrict__ st, int64_t rows, int64_t nb, int64_t B,
                               int exact, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nb * B) return;
  const int64_t rb = i / B;
  const float c = (float)codes[i];
  if (exact) {
    const double v = (double)lo[rb] + (double)c * (double)st[rb];
    out[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
  } else {
    out[i] = f16_bits(lo[rb] + c * st[rb]);
  }
}

// Un-permute codes / comp: out[r, perm[j]] = in[r, j].
__global__ void unpermute_kernel(const uint8_t* __restrict__ codes_ro, const float* __restrict__ comp_ro,
                                 const int64_t* __restrict__ perm, int64_t n, int64_t k,
                                 uint8_t* __restrict__ codes, float* __restrict__ comp) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * k) return;
  const int64_t r = i / k, j = i % k;
  const int64_t c = perm ? perm[j] : j;
  codes[r * k + c] = codes_ro[i];
  if (comp && comp_ro) comp[r * k + c] = comp_ro[i];
}

// sse[r] = sum_c d_c (fp16(lo + code*step) - w)^2 in torch's CPU sum order for a
// contiguous row of k floats: 8 vector lanes x 4 vector accumulators, the 4-level
// cascade over rows of 32 floats (base 2^max(4, ceil_log2(rows)/4)), the extra vectors
// into accumulator 0, the accumulators folded, then the 8 lanes in order.  Two rows per
// wave; lane (kq, v) = (l/8 % 4, l%8) of a 32-lane half holds p[kq][v].
__device__ __forceinline__ int64_t ceil_log2_dev(int64_t x) {
  if (x <= 2) return 1;
  return 64 - __builtin_clzll((unsigned long long)(x - 1));
}

// The torch CPU order above for one row, term(c) giving element c's term: returns the
// row's sum on lane hl == 0 of the half-wave (every lane of the wave takes part in the
// shuffles).
template <class F>
__device__ __forceinline__ float sse_row_sum(int64_t k, int kq, int v, int base, F term) {
  const int64_t vec_size = k / 8;
  const int64_t size_ilp = vec_size / 4;
  float p = 0.0f;
  if (size_ilp > 0) {
    int64_t lp = ceil_log2_dev(size_ilp) / 4;
    if (lp < 4) lp = 4;
    const int64_t step = (int64_t)1 << lp, lmask = step - 1;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t i = 0;
    while (i + step <= size_ilp) {
      // step is a power of two >= 16: the terms of 16 consecutive vectors are loaded
      // together, then added in order (the loads of a group are all in flight at once)
      for (int64_t j = 0; j < step; j += 16) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = term(((i + j + u) * 4 + kq) * 8 + v);
#pragma unroll
        for (int u = 0; u < 16; ++u) acc[0] += t[u];
      }
      i += step;
      for (int lev = 1; lev < 4; ++lev) {
        acc[lev] += acc[lev - 1];
        acc[lev - 1] = 0.0f;
        if (i & (lmask << (lev * lp))) break;
      }
    }
    for (; i < size_ilp; ++i) acc[0] += term((i * 4 + kq) * 8 + v);
    p = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  }
  if (kq == 0)
    for (int64_t i = size_ilp * 4; i < vec_size; ++i) p += term(i * 8 + v);
  // fold the 4 accumulators of lane v: ((p0 + p1) + p2) + p3
  const float p1 = __shfl(p, base + 8 + v);
  const float p2 = __shfl(p, base + 16 + v);
  const float p3 = __shfl(p, base + 24 + v);
  const float p0 = ((p + p1) + p2) + p3;  // valid on kq == 0
  float out = 0.0f;
  for (int64_t i = vec_size * 8; i < k; ++i) out += term(i);
#pragma unroll
  for (int vv = 0; vv < 8; ++vv) out += __shfl(p0, base + vv);
  return out;
}

// With groups (not null), row r of the batch belongs to group row_grp[r]: its
// uncompensated row is row r - row0 of the group's w, its weights the group's d and its
// ladder block the group's; rows past the group's own (padding) are skipped.
__global__ __launch_bounds__(256) void sse_kernel(const uint8_t* __restrict__ codes,
                                                  int64_t n, int64_t k, int64_t B,
                                                  const float* __restrict__ lo_d,
                                                  const float* __restrict__ st_d, int64_t ldd,
                                                  const float* __restrict__ w,
                                                  const float* __restrict__ d,
                                                  float* __restrict__ sse,
                                                  const int32_t* __restrict__ row_grp,
                                                  const hi2x_rows_group* __restrict__ groups) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5, hl = lane & 31;
  const int kq = hl >> 3, v = hl & 7;
  const int64_t r = ((int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)) * 2 + half;
  bool live = r < n;
  const int64_t rr = live ? r : 0;
  const float* wr = w + rr * k;
  if (groups) {
    const hi2x_rows_group& gp = groups[row_grp[rr]];
    const int64_t lr = rr - gp.row0;
    live = live && lr < gp.rows;
    wr = gp.w + (live ? lr : 0) * k;
    d = gp.d;
    B = gp.block;
  }
  auto row_sum = [&](auto blk) {
    return sse_row_sum(k, kq, v, half * 32, [&](int64_t c) -> float {
      const int64_t b = blk(c);
      const float rec =
          f16_round(lo_d[rr * ldd + b] + (float)codes[rr * k + c] * st_d[rr * ldd + b]);
      const float df = rec - wr[c];
      return d[c] * (df * df);
    });
  };
  // the element's ladder block c / B (c < k): for k B < 2^32, floor(c M / 2^32) with
  // M = ceil(2^32 / B) is floor(c / B) exactly (c M / 2^32 exceeds c / B by
  // c (M B - 2^32) / (B 2^32) < c / 2^32 < 1 / B), one multiply-high; the 64-bit division
  // otherwise (the wave decides together, so its loop has one form)
  const uint32_t Bu = (uint32_t)B;
  const bool by_mul = B >= 2 && B < (1ll << 32) && (uint64_t)k * Bu < (1ull << 32);
  const uint32_t M = by_mul ? (uint32_t)(((1ull << 32) + Bu - 1) / Bu) : 0u;
  const float out = __builtin_amdgcn_ballot_w64(!by_mul) == 0
                        ? row_sum([&](int64_t c) { return (int64_t)__umulhi((uint32_t)c, M); })
                        : row_sum([&](int64_t c) { return c / B; });
  if (live && hl == 0) sse[r] = out;
}

// encode_rows' codes (hi2/encode.py:151-155): q = clamp(st == 0 ? 0 : rint((w - lo) /
// st), 0, nm) with the row's decoded ladder of the element's block, the quotient by IEEE
// division.  Four consecutive elements per thread (one 16-byte read of w).
__global__ __launch_bounds__(256) void nearest_codes_kernel(
    const float* __restrict__ w, int64_t rows, int64_t k, int64_t block,
    const float* __restrict__ lo_d, const float* __restrict__ st_d, int64_t ldd, float nm,
    uint8_t* __restrict__ codes) {
  const int64_t q4 = k / 4;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * q4) return;
  const int64_t r = i / q4, c0 = (i % q4) * 4;
  const float4 v = *reinterpret_cast<const float4*>(w + r * k + c0);
  const float* lr = lo_d + r * ldd;
  const float* sr = st_d + r * ldd;
  const float x[4] = {v.x, v.y, v.z, v.w};
  uint32_t packed = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t b = (c0 + t) / block;
    const float lo = lr[b], st = sr[b];
    const float safe = st == 0.0f ? 1.0f : st;
    float q = __builtin_rintf((x[t] - lo) / safe);
    q = st == 0.0f ? 0.0f : q;
    q = clamp_code(q, nm);
    packed |= (uint32_t)(uint8_t)q << (8 * t);
  }
  *reinterpret_cast<uint32_t*>(codes + r * k + c0) = packed;
}

#ifndef LADDER_LANES
#define LADDER_LANES 2  // measured: 4 lanes (twice the occupancy) lose more to the moves
#endif

template <int B>
int launch_fit(const float* w, const float* d, int64_t rows, int64_t k, int nlev,
               const Grid& grid, int g, int ls, float* lo, float* step, float* err,
               hipStream_t s, const int32_t* d_row = nullptr) {
  const int64_t total = rows * (k / B);
  LaunchTimer timer(HI2X_TIME_LADDER_FIT, 4.0 * rows * k, s);
  if constexpr (B == 32 || B == 64) {  // a group of lanes per (row, block)
    constexpr int NL = LADDER_LANES;
    const dim3 blocks((unsigned)((NL * total + 255) / 256));
    hipLaunchKernelGGL((ladder_fit_group_kernel<B, NL>), blocks, dim3(256), 0, s, w, d, rows, k,
                       nlev, grid, g, ls, lo, step, err, d_row);
  } else {
    const dim3 blocks((unsigned)((total + 255) / 256));
    hipLaunchKernelGGL(ladder_fit_kernel<B>, blocks, dim3(256), 0, s, w, d, rows, k, nlev,
                       grid, g, ls, lo, step, err, d_row);
  }
  return launch_status("ladder_fit_kernel");
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_ladder_fit(const float* w, const float* d, int64_t rows, int64_t k,
                               int64_t block, int nlev, const float* grid, int g, int ls,
                               float* lo, float* step, float* err, void* stream) {
  clear_error();
  HI2X_REQUIRE(block == 16 || block == 32 || block == 64, "ladder_fit: block %lld",
               (long long)block);
  HI2X_REQUIRE(k > 0 && k % block == 0, "ladder_fit: K=%lld not a multiple of %lld",
               (long long)k, (long long)block);
  HI2X_REQUIRE(g >= 1 && g <= 8 && grid, "ladder_fit: grid of %d points", g);
  HI2X_REQUIRE(nlev >= 2 && nlev <= 256 && ls >= 0, "ladder_fit: nlev=%d ls=%d", nlev, ls);
  if (rows == 0) return HI2X_OK;
  Grid gr{};
  for (int i = 0; i < g; ++i) gr.v[i] = grid[i];
  hipStream_t s = as_stream(stream);
  switch (block) {
    case 16: return launch_fit<16>(w, d, rows, k, nlev, gr, g, ls, lo, step, err, s);
    case 32: return launch_fit<32>(w, d, rows, k, nlev, gr, g, ls, lo, step, err, s);
    default: return launch_fit<64>(w, d, rows, k, nlev, gr, g, ls, lo, step, err, s);
  }
}

extern "C" int hi2x_ladder_fit_rows(const float* w, const float* d, const int32_t* d_row,
                                    int64_t rows, int64_t k, int64_t block, int nlev,
                                    const float* grid, int g, int ls, float* lo, float* step,
                                    float* err, void* stream) {
  clear_error();
  HI2X_REQUIRE(block == 16 || block == 32 || block == 64, "ladder_fit_rows: block %lld",
               (long long)block);
  HI2X_REQUIRE(k > 0 && k % block == 0, "ladder_fit_rows: K=%lld not a multiple of %lld",
               (long long)k, (long long)block);
  HI2X_REQUIRE(g >= 1 && g <= 8 && grid, "ladder_fit_rows: grid of %d points", g);
  HI2X_REQUIRE(nlev >= 2 && nlev <= 256 && ls >= 0, "ladder_fit_rows: nlev=%d ls=%d", nlev, ls);
  if (rows == 0) return HI2X_OK;
  HI2X_REQUIRE(w && d && d_row && lo && step, "ladder_fit_rows: null buffer");
  Grid gr{};
  for (int i = 0; i < g; ++i) gr.v[i] = grid[i];
  hipStream_t s = as_stream(stream);
  switch (block) {
    case 16: return launch_fit<16>(w, d, rows, k, nlev, gr, g, ls, lo, step, err, s, d_row);
    case 32: return launch_fit<32>(w, d, rows, k, nlev, gr, g, ls, lo, step, err, s, d_row);
    default: return launch_fit<64>(w, d, rows, k, nlev, gr, g, ls, lo, step, err, s, d_row);
  }
}

extern "C" int hi2x_params(const float* lo, const float* step, int64_t rows, int64_t nb,
                           uint8_t* lo_u8, uint8_t* step_u8, uint16_t* consts, float* lo_d,
                           float* step_d, int64_t ldd, void* stream) {
  clear_error();
  HI2X_REQUIRE(nb > 0 && rows >= 0, "params: bad shape");
  HI2X_REQUIRE(!lo_d || ldd >= nb, "params: ldd < nb");
  HI2X_REQUIRE((lo_d == nullptr) == (step_d == nullptr), "params: lo_d/step_d pairing");
  if (rows == 0) return HI2X_OK;
  const dim3 blocks((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL(params_kernel, blocks, dim3(256), 0, as_stream(stream), lo, step, rows, nb,
                     lo_u8, step_u8, consts, lo_d, step_d, ldd);
  return launch_status("params_kernel");
}

extern "C" int hi2x_decode_params(const uint8_t* lo_u8, const uint8_t* step_u8,
                                  const uint16_t* consts, int64_t rows, int64_t nb,
                                  uint16_t* lo_h, uint16_t* step_h, void* stream) {
  clear_error();
  HI2X_REQUIRE(rows >= 0 && nb > 0, "decode_params: bad shape");
  if (rows == 0) return HI2X_OK;
  const int64_t total = rows * nb;
  hipLaunchKernelGGL(decode_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), lo_u8, step_u8, consts, rows, nb, lo_h, step_h);
  return launch_status("decode_kernel");
}

extern "C" int hi2x_ladder_dequantize(const uint8_t* codes, const float* lo, const float* step,
                                      int64_t rows, int64_t nb, int64_t block, int exact,
                                      uint16_t* out_h, void* stream) {
  clear_error();
  HI2X_REQUIRE(rows >= 0 && nb > 0 && block > 0, "ladder_dequantize: bad shape");
  if (rows == 0) return HI2X_OK;
  const int64_t total = rows * nb * block;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), codes, lo, step, rows, nb, block, exact, out_h);
  return launch_status("dequant_kernel");
}

extern "C" int hi2x_nearest_codes(const float* w, int64_t rows, int64_t k, int64_t block,
                                  const float* lo_d, const float* st_d, int64_t ldd, int nbits,
                                  uint8_t* codes, void* stream) {
  clear_error();
  HI2X_REQUIRE(rows >= 0 && k > 0 && k % 4 == 0 && block > 0 && k % block == 0,
               "nearest_codes: bad shape");
  HI2X_REQUIRE(ldd >= k / block, "nearest_codes: ldd < nb");
  HI2X_REQUIRE(nbits >= 1 && nbits <= 8, "nearest_codes: nbits=%d", nbits);
  HI2X_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)codes & 3) == 0,
               "nearest_codes: w must be 16-byte and codes 4-byte aligned");
  if (rows == 0) return HI2X_OK;
  const int64_t total = rows * (k / 4);
  hipLaunchKernelGGL(nearest_codes_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), w, rows, k, block, lo_d, st_d, ldd,
                     (float)((1 << nbits) - 1), codes);
  return launch_status("nearest_codes_kernel");
}

extern "C" int hi2x_finish(const uint8_t* codes_ro, const float* comp_ro, const int64_t* perm,
                           int64_t n, int64_t k, int64_t block, const float* lo_d,
                           const float* step_d, int64_t ldd, const float* w, const float* d,
                           uint8_t* codes, float* comp, float* sse, void* stream) {
  clear_error();
  HI2X_REQUIRE(n >= 0 && k > 0 && block > 0 && k % block == 0, "finish: bad shape");
  HI2X_REQUIRE(ldd >= k / block, "finish: ldd < nb");
  if (n == 0) return HI2X_OK;
  hipStream_t s = as_stream(stream);
  const int64_t total = n * k;
  const bool moves = !(perm == nullptr && codes == codes_ro && comp == comp_ro);
  LaunchTimer timer(HI2X_TIME_FINISH,
                    (double)n * k * (5 + (moves ? 2 + (comp ? 8 : 0) : 0)), s);
  // without a permutation the outputs may alias the inputs: nothing to move then
  if (!(perm == nullptr && codes == codes_ro && comp == comp_ro)) {
    hipLaunchKernelGGL(unpermute_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       codes_ro, comp_ro, perm, n, k, codes, comp);
    const int rc = launch_status("unpermute_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(sse_kernel, dim3((unsigned)((n + 7) / 8)), dim3(256), 0, s, codes, n, k,
                     block, lo_d, step_d, ldd, w, d, sse, (const int32_t*)nullptr,
                     (const hi2x_rows_group*)nullptr);
  return launch_status("sse_kernel");
}

extern "C" int hi2x_finish_rows(const uint8_t* codes, int64_t n, int64_t k, const float* lo_d,
                                const float* step_d, int64_t ldd, const int32_t* row_grp,
                                const hi2x_rows_group* groups, float* sse, void* stream) {
  clear_error();
  HI2X_REQUIRE(n >= 0 && k > 0 && k % 16 == 0 && ldd >= k / 16, "finish_rows: bad shape");
  if (n == 0) return HI2X_OK;
  HI2X_REQUIRE(codes && lo_d && step_d && row_grp && groups && sse, "finish_rows: null buffer");
  hipStream_t s = as_stream(stream);
  LaunchTimer timer(HI2X_TIME_FINISH, (double)n * k * 5, s);
  hipLaunchKernelGGL(sse_kernel, dim3((unsigned)((n + 7) / 8)), dim3(256), 0, s, codes, n, k,
                     (int64_t)64, lo_d, step_d, ldd, (const float*)nullptr, (const float*)nullptr,
                     sse, row_grp, groups);
  return launch_status("sse_kernel");
}
