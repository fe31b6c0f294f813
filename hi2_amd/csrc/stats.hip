// Calibration-side statistics on gfx950: ColumnStats (the 16 x 16 second moments of every
// column group, hi2/stats.py:26-55) and the cached-Sigma payload (the upper triangle of an
// exactly symmetric Sigma, hi2/cache.py:266-277).
#include <stdio.h>

#include "common.h"
#include "mfma_gemm.h"

namespace hi2x {
namespace {

constexpr int CS_CHUNK = 4096;  // tokens per fp32 chunk (hi2/stats.py:13)
constexpr int CS_SUB = 256;     // tokens per sub-chunk (one workgroup)
constexpr int CS_FB = 256;      // features per workgroup (16 groups)
constexpr int CS_ST = 32;       // tokens per LDS stage

// Moments of one sub-chunk of 256 tokens for 16 column groups: thread (group gl, quad q)
// holds the 4 x 4 block (rows 4 (q / 4).., columns 4 (q % 4)..) of group gl's 16 x 16
// moment, a sequential fp32 FMA chain over the sub-chunk's tokens in order from zero.
// Tokens are staged in LDS as f32, 32 at a time; tokens past the end and features past K
// read zero (a zero product leaves a chain unchanged).  partials [nsub, K/16, 16, 16].
template <bool BF16>
__global__ __launch_bounds__(256) void colstats_partial_kernel(const void* __restrict__ x,
                                                               int64_t T, int64_t K,
                                                               float* __restrict__ partials) {
  __shared__ __attribute__((aligned(16))) float sx[CS_ST][CS_FB];
  const int tid = threadIdx.x;
  const int64_t f0 = (int64_t)blockIdx.x * CS_FB;
  const int64_t t0 = (int64_t)blockIdx.y * CS_SUB;
  const int64_t t1 = (t0 + CS_SUB < T) ? t0 + CS_SUB : T;
  const int gl = tid >> 4, ia = (tid >> 2) & 3, jb = tid & 3;
  float acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;
  // staging: 8 consecutive features per thread, 32 threads per token row, 8 rows per pass
  const int srow = tid >> 5, scol = 8 * (tid & 31);
  const int64_t nf = (K - f0 < CS_FB) ? K - f0 : CS_FB;
  for (int64_t s0 = t0; s0 < t1; s0 += CS_ST) {
    __syncthreads();  // the previous stage has been read
#pragma unroll
    for (int p = 0; p < CS_ST / 8; ++p) {
      const int r = srow + 8 * p;
      const int64_t tok = s0 + r;
      float v[8];
      if (tok < t1 && scol < nf) {  // nf is a multiple of 16, so 8 features are all in
        if (BF16) {
          const uint4 raw = *reinterpret_cast<const uint4*>(
              reinterpret_cast<const uint16_t*>(x) + tok * K + f0 + scol);
          const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(w[e] << 16);
            v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
          }
        } else {
          const float* p8 = reinterpret_cast<const float*>(x) + tok * K + f0 + scol;
          const float4 a = *reinterpret_cast<const float4*>(p8);
          const float4 b = *reinterpret_cast<const float4*>(p8 + 4);
          v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
          v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
      }
      *reinterpret_cast<float4*>(&sx[r][scol]) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(&sx[r][scol + 4]) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
#pragma unroll 4
    for (int r = 0; r < CS_ST; ++r) {
      const float4 xi = *reinterpret_cast<const float4*>(&sx[r][16 * gl + 4 * ia]);
      const float4 xj = *reinterpret_cast<const float4*>(&sx[r][16 * gl + 4 * jb]);
      const float ai[4] = {xi.x, xi.y, xi.z, xi.w}, bj[4] = {xj.x, xj.y, xj.z, xj.w};
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = __builtin_fmaf(ai[a], bj[b], acc[a][b]);
    }
  }
  const int64_t g = f0 / 16 + gl;
  if (16 * gl < nf) {
    float* out = partials + (((int64_t)blockIdx.y * (K / 16) + g) * 16) * 16;
#pragma unroll
    for (int a = 0; a < 4; ++a)
      *reinterpret_cast<float4*>(&out[(4 * ia + a) * 16 + 4 * jb]) =
          make_float4(acc[a][0], acc[a][1], acc[a][2], acc[a][3]);
  }
}

// s[e] (f64) += each chunk's fp32 moment, the chunks in order; a chunk's moment is the
// fp32 sum of its sub-chunks' partials in order (hi2/stats.py:30-32: one fp32 einsum per
// chunk, added to the f64 state).
__global__ __launch_bounds__(256) void colstats_reduce_kernel(const float* __restrict__ partials,
                                                              int64_t nsub, int64_t ne,
                                                              double* __restrict__ s) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= ne) return;
  double acc = s[e];
  constexpr int per = CS_CHUNK / CS_SUB;
  for (int64_t c = 0; c < nsub; c += per) {
    const int64_t cend = (c + per < nsub) ? c + per : nsub;
    float sum = 0.0f;
    for (int64_t q = c; q < cend; ++q) sum = sum + partials[q * ne + e];
    acc = acc + (double)sum;
  }
  s[e] = acc;
}

// diag (hi2/stats.py:39-55), thread (group g, i): s = S / max(n, 1), times inv_j inv_k
// with smoothing; plain s_ii, or on a flagged group sum_j h_ij (sum_k s_jk h_ik) with
// h = H16 / 4, each sum sequential in f64 without fused products.
__global__ __launch_bounds__(256) void colstats_diag_kernel(const double* __restrict__ S,
                                                            int64_t K, int64_t n,
                                                            const uint8_t* __restrict__ flags,
                                                            const float* __restrict__ inv_scale,
                                                            float* __restrict__ out) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= K) return;
  const int64_t g = id / 16;
  const int i = (int)(id % 16);
  const double nn = (double)(n > 1 ? n : 1);
  const double* sg = S + g * 256;
  auto sv = [&](int j, int q) {
    double v = sg[j * 16 + q] / nn;
    if (inv_scale) {
      const double vj = (double)inv_scale[g * 16 + j], vq = (double)inv_scale[g * 16 + q];
      v = v * vj;
      v = v * vq;
    }
    return v;
  };
  double v = sv(i, i);
  if (flags && flags[g]) {
    double rot = 0.0;
    for (int j = 0; j < 16; ++j) {
      double tj = 0.0;
      for (int q = 0; q < 16; ++q) {
        const double hq = (__builtin_popcount(i & q) & 1) ? -0.25 : 0.25;
        const double prod = sv(j, q) * hq;
        tj = tj + prod;
      }
      const double hj = (__builtin_popcount(i & j) & 1) ? -0.25 : 0.25;
      const double prod = hj * tj;
      rot = rot + prod;
    }
    v = rot;
  }
  out[id] = (float)v;
}

// The upper triangle of sigma [K, K] row-major (row i: columns i..K-1) as f32 or fp16
// bits, and the number of pairs with sigma[i][j] != sigma[j][i] (torch.equal(s, s.T) is
// "none"; NaN counts as unequal).  Grid: (column blocks, row i).
__global__ __launch_bounds__(256) void sigma_pack_kernel(const float* __restrict__ sigma,
                                                         int64_t K, int fp16,
                                                         void* __restrict__ tri,
                                                         int32_t* __restrict__ asym) {
  const int64_t i = blockIdx.y;
  const int64_t j = i + (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool live = j < K;
  bool bad = false;
  if (live) {
    const float a = sigma[i * K + j];
    bad = !(a == sigma[j * K + i]);
    const int64_t o = i * K - i * (i - 1) / 2 + (j - i);
    if (fp16) {
      reinterpret_cast<uint16_t*>(tri)[o] = f16_bits(a);
    } else {
      reinterpret_cast<float*>(tri)[o] = a;
    }
  }
  const uint64_t m = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && m != 0) atomicAdd(asym, (int32_t)__builtin_popcountll(m));
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int64_t hi2x_colstats_workspace_bytes(int64_t t, int64_t k) {
  if (t < 0 || k <= 0 || k % 16) return -1;
  const int64_t nsub = (t + CS_SUB - 1) / CS_SUB;
  return nsub * k * 16 * (int64_t)sizeof(float);
}

extern "C" int hi2x_colstats_update(const void* x, int dtype, int64_t t, int64_t k, double* s,
                                    void* ws, int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0 && t >= 0, "colstats_update: bad shape t=%lld k=%lld",
               (long long)t, (long long)k);
  HI2X_REQUIRE(dtype == 0 || dtype == 2, "colstats_update: dtype %d (0 f32, 2 bf16)", dtype);
  if (t == 0) return HI2X_OK;
  HI2X_REQUIRE(x && s, "colstats_update: null buffer");
  hipStream_t st = as_stream(stream);
  const int64_t nsub = (t + CS_SUB - 1) / CS_SUB;
  Workspace w;
  int rc = take_workspace(w, ws, ws_bytes, (size_t)(nsub * k * 16) * sizeof(float), st,
                          "colstats_update");
  if (rc) return rc;
  float* parts = reinterpret_cast<float*>(w.p);
  const dim3 grid((unsigned)((k + CS_FB - 1) / CS_FB), (unsigned)nsub);
  if (dtype == 2)
    hipLaunchKernelGGL(colstats_partial_kernel<true>, grid, dim3(256), 0, st, x, t, k, parts);
  else
    hipLaunchKernelGGL(colstats_partial_kernel<false>, grid, dim3(256), 0, st, x, t, k, parts);
  if ((rc = launch_status("colstats_partial_kernel"))) return rc;
  const int64_t ne = k * 16;
  hipLaunchKernelGGL(colstats_reduce_kernel, dim3((unsigned)((ne + 255) / 256)), dim3(256), 0, st,
                     parts, nsub, ne, s);
  return launch_status("colstats_reduce_kernel");
}

extern "C" int hi2x_colstats_diag(const double* s, int64_t k, int64_t n, const uint8_t* flags,
                                  const float* inv_scale, float* out, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0 && n >= 0, "colstats_diag: bad arguments k=%lld n=%lld",
               (long long)k, (long long)n);
  HI2X_REQUIRE(s && out, "colstats_diag: null buffer");
  hipLaunchKernelGGL(colstats_diag_kernel, dim3((unsigned)((k + 255) / 256)), dim3(256), 0,
                     as_stream(stream), s, k, n, flags, inv_scale, out);
  return launch_status("colstats_diag_kernel");
}

extern "C" int hi2x_sigma_pack_upper(const float* sigma, int64_t k, int fp16, void* tri,
                                     int32_t* asym, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k <= 65535, "sigma_pack_upper: k=%lld", (long long)k);
  HI2X_REQUIRE(sigma && tri && asym, "sigma_pack_upper: null buffer");
  const dim3 grid((unsigned)((k + 255) / 256), (unsigned)k);
  hipLaunchKernelGGL(sigma_pack_kernel, grid, dim3(256), 0, as_stream(stream), sigma, k, fp16,
                     tri, asym);
  return launch_status("sigma_pack_kernel");
}
