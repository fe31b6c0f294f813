// QAD decode of the fake-quantised weights, forward and backward, and the fused
// Hadamard-and-scale transform (HBM-bound elementwise kernels).
//
// Reference: hi2/qad_kernel.py:57-176 (the decode_fwd / decode_bwd / wht_scale contract:
// per-element arithmetic, the per-block gradient sums as a pairwise tree over the block,
// the butterfly of the normalised order-16 Walsh-Hadamard transform) and hi2/qad.py:366-400
// (FakeQuantLinear._group, the torch graph whose values and gradients they are).
//
// Layout: every thread owns 4 consecutive columns of one row (16-byte loads and stores),
// threads are numbered row-major over (row, column quad), so a ladder block of B columns
// is B/4 consecutive lanes of one wave (B in {16, 32, 64}: 4, 8 or 16 lanes) and a
// 16-column rotation group is 4 lanes.  Per-block sums and the butterfly's cross-column
// steps are lane shuffles; no LDS.
#include "common.h"

namespace hi2x {
namespace {

constexpr int QT = 256;

struct Ladder {
  float lo, st;
};

// The two continuous bytes of a block -> fp16 lo and step (as float):
// byte = clamp(rint(u), 0, 255); lo = fp16(f32(f64(byte) * f64(lo_scale) + f64(lo_min)))
// (exact in f64), step = fp16(f32(byte) * step_scale).
__device__ __forceinline__ Ladder block_ladder(float lo_u, float st_u,
                                               const uint16_t* __restrict__ c) {
  const float lb = fminf(fmaxf(rintf(lo_u), 0.0f), 255.0f);
  const float sb = fminf(fmaxf(rintf(st_u), 0.0f), 255.0f);
  const double lo = (double)lb * (double)f16_from_bits(c[1]) + (double)f16_from_bits(c[0]);
  Ladder l;
  l.lo = f16_round((float)lo);
  l.st = f16_round(sb * f16_from_bits(c[2]));
  return l;
}

// code = clamp(rint(z), 0, nmax) with NaN propagated (torch.clamp), 0 for a zero step.
__device__ __forceinline__ float code_of(float z, float nmax, bool zero) {
  float q = rintf(z);
  q = q < 0.0f ? 0.0f : q;
  q = q > nmax ? nmax : q;
  return zero ? 0.0f : q;
}

__device__ __forceinline__ float4 ld4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ float& at(float4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ float at(const float4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// out[rows[r], :] = fp16(lo + q * step) (the sum in f64), for the group's
// rows r; v = latent (times unit when given).
// The block's divisions by safe (the fp32 divisions of the torch graph) as div_rcp
// through one reciprocal per thread: bit-identical to IEEE division for every numerator.
template <int SHIFT>
__global__ __launch_bounds__(QT) void qad_decode_fwd_kernel(
    const float* __restrict__ latent, const float* __restrict__ unit,
    const float* __restrict__ lo_u, const float* __restrict__ st_u,
    const uint16_t* __restrict__ consts, const int64_t* __restrict__ rows, int64_t n_rows,
    int64_t r_total, int64_t k, float nmax, float* __restrict__ out) {
  constexpr int shift = SHIFT;
  // thread (row, column quad); the host keeps n_rows * k / 4 below 2^31, so the index
  // arithmetic is 32-bit (a 64-bit division is a long emulated sequence on the SIMD)
  const uint32_t k4 = (uint32_t)(k >> 2);
  const uint32_t i = blockIdx.x * QT + threadIdx.x;
  if (i >= (uint32_t)n_rows * k4) return;
  const uint32_t r32 = i / k4;
  const int64_t r = r32, c0 = (int64_t)(i - r32 * k4) << 2;
  const int64_t row = rows[r];
  if (row < 0 || row >= r_total) return;  // a row outside the latent is skipped
  const int64_t nblk = k >> shift, b = c0 >> shift;
  const Ladder l = block_ladder(lo_u[r * nblk + b], st_u[r * nblk + b], consts + r * 3);
  const bool zero = l.st == 0.0f;
  const float safe = zero ? 1.0f : l.st;
  const float ys = 1.0f / safe;
  const int64_t off = row * k + c0;
  float4 v = ld4(latent + off);
  if (unit) {
    const float4 u = ld4(unit + off);
    v.x *= u.x; v.y *= u.y; v.z *= u.z; v.w *= u.w;
  }
  float4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float z = div_rcp(at(v, e) - l.lo, safe, ys);
    const float q = code_of(z, nmax, zero);
    // lo + q * step in f64 (exact), then torch's f64 -> fp16 conversion (through f32)
    const double val = (double)l.lo + (double)q * (double)l.st;
    at(o, e) = f16_round((float)val);
  }
  st4(out + off, o);
}

// Gradients of the STE graph: with G the gradient of the decoded value,
//   gz = G * step inside the clamp range [0, nmax] of z, else 0;  d latent = gz / safe
//   (times unit);  d lo_byte = lo_scale * sum_block(G - gz / safe);
//   d step_byte = step_scale * sum_block(G * q - [step != 0] gz * (z / safe)).
// The block sums are the pairwise tree s[i] += s[i + h] for h = B/2 .. 1: the levels
// h >= 4 are shuffles between the block's lanes, h = 2 and 1 inside the lane.
// Lane j + D of this lane's row of 16 (DPP row_shl; past the row's end 0: such lanes'
// sums are never read).  Written as update_dpp so that the add folds it in.
template <int D>
__device__ __forceinline__ float from_lane_plus(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + D, 0xf, 0xf, true));
}

// The tree levels h = H .. 4 of the block sums across the block's lanes (lane j += lane
// j + h/4, within the block's aligned run of B/4 <= 16 lanes, one DPP row).
template <int H>
__device__ __forceinline__ void block_tree(float4& a_lo, float4& a_st) {
  if constexpr (H >= 4) {
    constexpr int D = H >> 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      at(a_lo, e) = at(a_lo, e) + from_lane_plus<D>(at(a_lo, e));
      at(a_st, e) = at(a_st, e) + from_lane_plus<D>(at(a_st, e));
    }
    block_tree<H / 2>(a_lo, a_st);
  }
}

template <int SHIFT>
__global__ __launch_bounds__(QT) void qad_decode_bwd_kernel(
    const float* __restrict__ grad, const float* __restrict__ latent,
    const float* __restrict__ unit, const float* __restrict__ lo_u,
    const float* __restrict__ st_u, const uint16_t* __restrict__ consts,
    const int64_t* __restrict__ rows, int64_t n_rows, int64_t r_total, int64_t k,
    float nmax, float* __restrict__ g_latent, float* __restrict__ g_lo,
    float* __restrict__ g_st) {
  constexpr int shift = SHIFT;
  const uint32_t k4 = (uint32_t)(k >> 2);
  const uint32_t i = blockIdx.x * QT + threadIdx.x;
  const bool valid = i < (uint32_t)n_rows * k4;
  float4 a_lo = make_float4(0.f, 0.f, 0.f, 0.f), a_st = a_lo;
  int64_t r = 0, c0 = 0, b = 0;
  const int64_t nblk = k >> shift;
  if (valid) {
    const uint32_t r32 = i / k4;
    r = r32;
    c0 = (int64_t)(i - r32 * k4) << 2;
    b = c0 >> shift;
  }
  // a row outside the latent is skipped: no access, its block gradients read 0
  const int64_t row = valid ? rows[r] : -1;
  if (row >= 0 && row < r_total) {
    const Ladder l = block_ladder(lo_u[r * nblk + b], st_u[r * nblk + b], consts + r * 3);
    const bool zero = l.st == 0.0f;
    const float safe = zero ? 1.0f : l.st;
    const float ys = 1.0f / safe;
    const int64_t off = row * k + c0;
    float4 v = ld4(latent + off);
    float4 u = make_float4(1.f, 1.f, 1.f, 1.f);
    if (unit) {
      u = ld4(unit + off);
      v.x *= u.x; v.y *= u.y; v.z *= u.z; v.w *= u.w;
    }
    const float4 g = ld4(grad + off);
    float4 gl;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float z = div_rcp(at(v, e) - l.lo, safe, ys);
      const float q = code_of(z, nmax, zero);
      const float G = at(g, e);
      const bool inside = z >= 0.0f && z <= nmax;
      const float gz = inside ? G * l.st : 0.0f;
      const float gv = div_rcp(gz, safe, ys);
      at(gl, e) = unit ? gv * at(u, e) : gv;
      at(a_lo, e) = G - gv;
      float s = G * q;
      if (!zero) s = s + (-gz) * div_rcp(z, safe, ys);
      at(a_st, e) = s;
    }
    st4(g_latent + off, gl);
  }
  // tree levels h = B/2 .. 4 across the block's lanes (lane j += lane j + h/4); the
  // lanes that are not read again compute values nobody uses
  constexpr int block = 1 << shift;
  block_tree<block / 2>(a_lo, a_st);
  if (valid && (c0 & (block - 1)) == 0) {
    const float slo = (a_lo.x + a_lo.z) + (a_lo.y + a_lo.w);
    const float sst = (a_st.x + a_st.z) + (a_st.y + a_st.w);
    const uint16_t* c = consts + r * 3;
    g_lo[r * nblk + b] = slo * f16_from_bits(c[1]);
    g_st[r * nblk + b] = sst * f16_from_bits(c[2]);
  }
}

// out = H16(x) / scale over the flagged 16-column groups (x / scale elsewhere), or with
// pre_div the division first: H16(x / scale).  H16 is the butterfly
// y[t] = (t & h) ? y[t ^ h] - y[t] : y[t] + y[t ^ h] for h = 1, 2, 4, 8, then * 0.25.
// h = 1, 2 act inside a lane's 4 columns, h = 4, 8 between the group's 4 lanes.
// One cross-lane level of the butterfly: partner lane ^ M of the 4-lane group (CTRL its
// DPP quad_perm), the upper lane keeping the difference.
template <int M, int CTRL>
__device__ __forceinline__ void butterfly_step(float4& v, int lane) {
  const bool upper = (lane & M) != 0;
  float4 p;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    at(p, e) = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, at(v, e)), CTRL, 0xf, 0xf,
                                           true));
#pragma unroll
  for (int e = 0; e < 4; ++e) at(v, e) = upper ? at(p, e) - at(v, e) : at(v, e) + at(p, e);
}

__global__ __launch_bounds__(QT) void qad_wht_scale_kernel(
    const float* __restrict__ x, int64_t n_rows, int64_t k, const uint8_t* __restrict__ flags,
    const uint16_t* __restrict__ scale, int pre_div, float* __restrict__ out) {
  const uint32_t k4 = (uint32_t)(k >> 2);
  const uint32_t i = blockIdx.x * QT + threadIdx.x;
  const bool valid = i < (uint32_t)n_rows * k4;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f), s = make_float4(1.f, 1.f, 1.f, 1.f);
  int64_t c0 = 0, r = 0;
  if (valid) {
    const uint32_t r32 = i / k4;
    r = r32;
    c0 = (int64_t)(i - r32 * k4) << 2;
    v = ld4(x + r * k + c0);
    if (scale) {
#pragma unroll
      for (int e = 0; e < 4; ++e) at(s, e) = f16_from_bits(scale[c0 + e]);
      if (pre_div) {
        v.x = v.x / s.x; v.y = v.y / s.y; v.z = v.z / s.z; v.w = v.w / s.w;
      }
    }
  }
  const float4 orig = v;
  // h = 1
  float4 y;
  y.x = v.x + v.y; y.y = v.x - v.y; y.z = v.z + v.w; y.w = v.z - v.w;
  // h = 2
  v.x = y.x + y.z; v.z = y.x - y.z; v.y = y.y + y.w; v.w = y.y - y.w;
  // h = 4, 8: partner lane j ^ 1, j ^ 2 of the group (lanes 4-aligned in the wave)
  const int lane = threadIdx.x & 63;
  butterfly_step<1, 0xB1>(v, lane);  // DPP quad_perm [1,0,3,2]: lane ^ 1
  butterfly_step<2, 0x4E>(v, lane);  // [2,3,0,1]: lane ^ 2
  if (!valid) return;
  const bool flagged = flags[c0 >> 4] != 0;
  float4 o = flagged ? make_float4(v.x * 0.25f, v.y * 0.25f, v.z * 0.25f, v.w * 0.25f) : orig;
  if (scale && !pre_div) {
    o.x = o.x / s.x; o.y = o.y / s.y; o.z = o.z / s.z; o.w = o.w / s.w;
  }
  st4(out + r * k + c0, o);
}

int block_shift(int block) { return block == 16 ? 4 : (block == 32 ? 5 : (block == 64 ? 6 : -1)); }

bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_qad_decode_fwd(const float* latent, const float* unit, const float* lo_u,
                                   const float* st_u, const uint16_t* consts,
                                   const int64_t* rows, int64_t n_rows, int64_t r_total,
                                   int64_t k, int block, float nmax, float* out, void* stream) {
  clear_error();
  const int shift = block_shift(block);
  HI2X_REQUIRE(shift > 0, "qad_decode_fwd: block %d must be 16, 32 or 64", block);
  HI2X_REQUIRE(n_rows >= 0 && r_total >= 0 && k > 0 && k % block == 0,
               "qad_decode_fwd: K=%lld must be a positive multiple of the block", (long long)k);
  HI2X_REQUIRE(aligned16(latent) && aligned16(unit) && aligned16(out),
               "qad_decode_fwd: latent, unit and out must be 16-byte aligned");
  if (n_rows == 0) return HI2X_OK;
  const int64_t total = n_rows * (k / 4);
  HI2X_REQUIRE(total < (int64_t(1) << 31), "qad_decode_fwd: %lld rows x K too large", (long long)n_rows);
  const dim3 grid((unsigned)((total + QT - 1) / QT));
#define HI2X_QAD_FWD(S)                                                                     \
  hipLaunchKernelGGL(qad_decode_fwd_kernel<S>, grid, dim3(QT), 0, as_stream(stream), latent, \
                     unit, lo_u, st_u, consts, rows, n_rows, r_total, k, nmax, out)
  if (shift == 4) HI2X_QAD_FWD(4);
  else if (shift == 5) HI2X_QAD_FWD(5);
  else HI2X_QAD_FWD(6);
#undef HI2X_QAD_FWD
  return launch_status("qad_decode_fwd_kernel");
}

extern "C" int hi2x_qad_decode_bwd(const float* grad, const float* latent, const float* unit,
                                   const float* lo_u, const float* st_u, const uint16_t* consts,
                                   const int64_t* rows, int64_t n_rows, int64_t r_total,
                                   int64_t k, int block, float nmax, float* g_latent, float* g_lo,
                                   float* g_st, void* stream) {
  clear_error();
  const int shift = block_shift(block);
  HI2X_REQUIRE(shift > 0, "qad_decode_bwd: block %d must be 16, 32 or 64", block);
  HI2X_REQUIRE(n_rows >= 0 && r_total >= 0 && k > 0 && k % block == 0,
               "qad_decode_bwd: K=%lld must be a positive multiple of the block", (long long)k);
  HI2X_REQUIRE(aligned16(grad) && aligned16(latent) && aligned16(unit) && aligned16(g_latent),
               "qad_decode_bwd: grad, latent, unit and g_latent must be 16-byte aligned");
  if (n_rows == 0) return HI2X_OK;
  const int64_t total = n_rows * (k / 4);
  HI2X_REQUIRE(total < (int64_t(1) << 31), "qad_decode_bwd: %lld rows x K too large", (long long)n_rows);
  const dim3 grid((unsigned)((total + QT - 1) / QT));
#define HI2X_QAD_BWD(S)                                                                    \
  hipLaunchKernelGGL(qad_decode_bwd_kernel<S>, grid, dim3(QT), 0, as_stream(stream), grad, \
                     latent, unit, lo_u, st_u, consts, rows, n_rows, r_total, k, nmax,     \
                     g_latent, g_lo, g_st)
  if (shift == 4) HI2X_QAD_BWD(4);
  else if (shift == 5) HI2X_QAD_BWD(5);
  else HI2X_QAD_BWD(6);
#undef HI2X_QAD_BWD
  return launch_status("qad_decode_bwd_kernel");
}

extern "C" int hi2x_qad_wht_scale(const float* x, int64_t n_rows, int64_t k,
                                  const uint8_t* flags, const uint16_t* scale, int pre_div,
                                  float* out, void* stream) {
  clear_error();
  HI2X_REQUIRE(n_rows >= 0 && k > 0 && k % 16 == 0,
               "qad_wht_scale: K=%lld must be a positive multiple of 16", (long long)k);
  HI2X_REQUIRE(aligned16(x) && aligned16(out), "qad_wht_scale: x and out must be 16-byte aligned");
  if (n_rows == 0) return HI2X_OK;
  const int64_t total = n_rows * (k / 4);
  HI2X_REQUIRE(total < (int64_t(1) << 31), "qad_wht_scale: %lld rows x K too large", (long long)n_rows);
  hipLaunchKernelGGL(qad_wht_scale_kernel, dim3((unsigned)((total + QT - 1) / QT)), dim3(QT), 0,
                     as_stream(stream), x, n_rows, k, flags, scale, pre_div, out);
  return launch_status("qad_wht_scale_kernel");
}
