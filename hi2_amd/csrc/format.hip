// Order-16 Hadamard rotation and rdna_hint_flex packing (HBM-bound kernels).
//
// Reference: hi2/format.py:22-41 (hadamard16, fwht_groups), hi2/format.py:73-85
// (pack_codes) and hi2/format.py:155-171 (the scatters of assemble).
#include "common.h"

namespace hi2x {
namespace {

// Sylvester sign of H16[i][j]: (-1)^popcount(i & j); the entries are +-1/4.
__device__ __forceinline__ bool hneg(int i, int j) { return __builtin_popcount(i & j) & 1; }

// One thread per 16-column group of a row.  y_j = sum_i x_i * H[i][j] as the
// reference's matmul evaluates it: a sequential FMA chain over i from zero (the
// products by +-1/4 are exact).  Unflagged groups are copied.
template <typename T>
__global__ __launch_bounds__(256) void fwht16_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                     int64_t rows, int64_t k,
                                                     const uint8_t* __restrict__ flags) {
  const int64_t ng = k / 16;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * ng) return;
  const int64_t g = i % ng;
  const T* xi = x + i * 16;
  T* yo = y + i * 16;
  T v[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) v[t] = xi[t];
  if (!flags[g]) {
#pragma unroll
    for (int t = 0; t < 16; ++t) yo[t] = v[t];
    return;
  }
  const T q = (T)0.25;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    T acc = (T)0;
#pragma unroll
    for (int t = 0; t < 16; ++t) acc = __builtin_fma(v[t], hneg(t, j) ? -q : q, acc);
    yo[j] = acc;
  }
}

// The weight preparation of a GPTQ unit in one pass: out[i] = fwht16 of row rows[i] of
// (float(w) * col_scale) (rows null: row i; col_scale null: no product).  float(bf16)
// is exact and the product is one rounding, as the reference's elementwise ops; the
// transform is fwht16_kernel's.  A workgroup takes 256 consecutive 16-column groups
// (in row-major order over the selected rows), one per thread for the arithmetic; the
// groups' inputs come in and their outputs go out through LDS in 16-byte pieces with
// consecutive lanes on consecutive pieces, so every global access is coalesced.  The
// LDS slots are 3 (bf16 inputs) or 5 (f32 inputs, outputs) pieces apart: the 16 lanes
// of a 16-byte LDS access fall on distinct banks.
template <typename T>
__global__ __launch_bounds__(256) void rotate_rows_kernel(
    const T* __restrict__ w, int64_t ldw, int64_t nw, const int64_t* __restrict__ rows,
    int64_t n, int64_t k, const float* __restrict__ col_scale,
    const uint8_t* __restrict__ flags, float* __restrict__ out, int64_t ldo) {
  constexpr int CH = 16 * (int)sizeof(T) / 16;  // input pieces per group (2 or 4)
  constexpr int IS = CH + 1;                    // input slot (pieces)
  constexpr int OS = 5;                         // output slot: 4 pieces + 1
  __shared__ uint4 pin[256 * IS];
  __shared__ uint4 pout[256 * OS];
  // group indices fit 32 bits (the host checks n * k / 16 < 2^31): cheap divisions
  const uint32_t ng = (uint32_t)(k / 16), total = (uint32_t)(n * (k / 16));
  const uint32_t base = blockIdx.x * 256u;
  const int tid = threadIdx.x;
  // the inputs: piece c = group c / CH, part c % CH
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = tid + 256 * j, gl = c / CH, part = c % CH;
    const uint32_t t = base + gl;
    if (t < total) {
      const uint32_t i = t / ng, g = t % ng;
      const int64_t src = rows ? rows[i] : (int64_t)i;
      if (src >= 0 && src < nw)
        pin[gl * IS + part] =
            *reinterpret_cast<const uint4*>(w + src * ldw + 16 * g + part * (16 / (int)sizeof(T)));
    }
  }
  __syncthreads();
  {
    const uint32_t t = base + tid;
    if (t < total) {
      const uint32_t i = t / ng, g = t % ng;
      const int64_t src = rows ? rows[i] : (int64_t)i;
      float y[16];
      if (src < 0 || src >= nw) {  // an index out of range: the row reads NaN
#pragma unroll
        for (int j = 0; j < 16; ++j) y[j] = __builtin_nanf("");
      } else {
        float v[16];
        if constexpr (sizeof(T) == 2) {
          const uint4 a = pin[tid * IS], b = pin[tid * IS + 1];
          const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            v[2 * e] = __uint_as_float(u[e] << 16);
            v[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4 a = pin[tid * IS + q];
            v[4 * q] = __uint_as_float(a.x);
            v[4 * q + 1] = __uint_as_float(a.y);
            v[4 * q + 2] = __uint_as_float(a.z);
            v[4 * q + 3] = __uint_as_float(a.w);
          }
        }
        if (col_scale) {
#pragma unroll
          for (int q = 0; q < 16; ++q) v[q] = v[q] * col_scale[16 * g + q];
        }
        if (flags && flags[g]) {
          const float qv = 0.25f;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc = __builtin_fmaf(v[e], hneg(e, j) ? -qv : qv, acc);
            y[j] = acc;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j) y[j] = v[j];
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        pout[tid * OS + q] = make_uint4(__float_as_uint(y[4 * q]), __float_as_uint(y[4 * q + 1]),
                                        __float_as_uint(y[4 * q + 2]),
                                        __float_as_uint(y[4 * q + 3]));
    }
  }
  __syncthreads();
  // the outputs: piece c = group c / 4, part c % 4
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = tid + 256 * j, gl = c / 4, part = c % 4;
    const uint32_t t = base + gl;
    if (t < total) {
      const uint32_t i = t / ng, g = t % ng;
      *reinterpret_cast<uint4*>(out + (int64_t)i * ldo + 16 * g + 4 * part) = pout[gl * OS + part];
    }
  }
}

__device__ __forceinline__ void note_bad(int32_t* bad, int n) {
  if (n && bad) atomicAdd(bad, n);
}

// One thread per output word: 32/nbits codes, LSB first.
__global__ __launch_bounds__(256) void pack_kernel(const uint8_t* __restrict__ codes,
                                                   int64_t rows, int64_t k, int nbits,
                                                   int32_t* __restrict__ words,
                                                   int32_t* __restrict__ bad) {
  const int per = 32 / nbits;
  const int64_t nw = k / per;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nw) return;
  const uint8_t* c = codes + i * per;
  const uint32_t lim = 1u << nbits;
  uint32_t v = 0;
  int nbad = 0;
  for (int t = 0; t < per; ++t) {
    const uint32_t cv = c[t];
    nbad += cv >= lim;
    v |= (cv & (lim - 1u)) << (nbits * t);
  }
  words[i] = (int32_t)v;
  note_bad(bad, nbad);
}

// assemble, one piece: thread (i, wi) packs word wi of piece row i into the flat
// buffer at code_off[rows[i]] + wi; threads (i, b) with b < nblk copy the two bytes
// of block b to param_off[rows[i]] + b; thread (i, 0) copies the row constants.
__global__ __launch_bounds__(256) void assemble_kernel(
    const int64_t* __restrict__ rows, int64_t r, const uint8_t* __restrict__ codes,
    const uint8_t* __restrict__ params, const uint16_t* __restrict__ consts, int64_t k,
    int nbits, int64_t nblk, const int64_t* __restrict__ code_off,
    const int64_t* __restrict__ param_off, int32_t* __restrict__ out_codes,
    uint8_t* __restrict__ out_params, uint16_t* __restrict__ out_consts,
    int32_t* __restrict__ bad) {
  const int per = 32 / nbits;
  const int64_t nw = k / per;
  const int64_t span = nw > nblk ? nw : nblk;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= r * span) return;
  const int64_t i = t / span, j = t % span;
  const int64_t row = rows[i];
  if (j < nw) {
    const uint8_t* c = codes + i * k + j * per;
    const uint32_t lim = 1u << nbits;
    uint32_t v = 0;
    int nbad = 0;
    for (int q = 0; q < per; ++q) {
      const uint32_t cv = c[q];
      nbad += cv >= lim;
      v |= (cv & (lim - 1u)) << (nbits * q);
    }
    out_codes[code_off[row] + j] = (int32_t)v;
    note_bad(bad, nbad);
  }
  if (j < nblk) {
    const int64_t dst = (param_off[row] + j) * 2;
    out_params[dst] = params[(i * nblk + j) * 2];
    out_params[dst + 1] = params[(i * nblk + j) * 2 + 1];
  }
  if (j == 0) {
    out_consts[row * 3 + 0] = consts[i * 3 + 0];
    out_consts[row * 3 + 1] = consts[i * 3 + 1];
    out_consts[row * 3 + 2] = consts[i * 3 + 2];
  }
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_rotate_rows(const void* w, int dtype, int64_t ldw, int64_t nw,
                                const int64_t* rows, int64_t n, int64_t k,
                                const float* col_scale, const uint8_t* flags, float* out,
                                int64_t ldo, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0, "rotate_rows: K=%lld must be a multiple of 16",
               (long long)k);
  HI2X_REQUIRE(dtype == 0 || dtype == 2, "rotate_rows: dtype %d (0 = f32, 2 = bf16)", dtype);
  HI2X_REQUIRE(n >= 0 && nw >= 0 && ldw >= k && ldo >= k, "rotate_rows: bad shape or strides");
  HI2X_REQUIRE(rows || n <= nw, "rotate_rows: %lld rows of a %lld-row matrix", (long long)n,
               (long long)nw);
  if (n == 0) return HI2X_OK;
  HI2X_REQUIRE(w && out, "rotate_rows: null buffer");
  HI2X_REQUIRE(((uintptr_t)w % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                   (ldw * (dtype == 0 ? 4 : 2)) % 16 == 0 && (ldo * 4) % 16 == 0,
               "rotate_rows: rows must start on 16-byte boundaries");
  HI2X_REQUIRE(n * (k / 16) < (int64_t)1 << 31, "rotate_rows: %lld groups (at most 2^31 - 1)",
               (long long)(n * (k / 16)));
  const int64_t total = n * (k / 16);
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t s = as_stream(stream);
  LaunchTimer timer(HI2X_TIME_FWHT, (double)n * k * ((dtype == 0 ? 4 : 2) + 4), s);
  if (dtype == 0)
    hipLaunchKernelGGL(rotate_rows_kernel<float>, grid, dim3(256), 0, s, (const float*)w, ldw,
                       nw, rows, n, k, col_scale, flags, out, ldo);
  else
    hipLaunchKernelGGL(rotate_rows_kernel<uint16_t>, grid, dim3(256), 0, s, (const uint16_t*)w,
                       ldw, nw, rows, n, k, col_scale, flags, out, ldo);
  return launch_status("rotate_rows_kernel");
}

extern "C" int hi2x_fwht16(const void* x, void* y, int dtype, int64_t rows, int64_t k,
                           const uint8_t* flags, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0, "fwht16: K=%lld must be a multiple of 16", (long long)k);
  HI2X_REQUIRE(dtype == 0 || dtype == 1, "fwht16: dtype %d (0 = f32, 1 = f64)", dtype);
  if (rows == 0) return HI2X_OK;
  const int64_t total = rows * (k / 16);
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t s = as_stream(stream);
  LaunchTimer timer(HI2X_TIME_FWHT, 2.0 * rows * k * (dtype == 0 ? 4 : 8), s);
  if (dtype == 0)
    hipLaunchKernelGGL(fwht16_kernel<float>, grid, dim3(256), 0, s, (const float*)x, (float*)y,
                       rows, k, flags);
  else
    hipLaunchKernelGGL(fwht16_kernel<double>, grid, dim3(256), 0, s, (const double*)x,
                       (double*)y, rows, k, flags);
  return launch_status("fwht16_kernel");
}

extern "C" int hi2x_pack_codes(const uint8_t* codes, int64_t rows, int64_t k, int nbits,
                               int32_t* words, int32_t* bad, void* stream) {
  clear_error();
  HI2X_REQUIRE(nbits == 2 || nbits == 4 || nbits == 8, "pack_codes: nbits=%d", nbits);
  HI2X_REQUIRE(k > 0 && k % (32 / nbits) == 0, "pack_codes: %lld codes is not a multiple of %d",
               (long long)k, 32 / nbits);
  if (rows == 0) return HI2X_OK;
  const int64_t total = rows * (k / (32 / nbits));
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), codes, rows, k, nbits, words, bad);
  return launch_status("pack_kernel");
}

extern "C" int hi2x_assemble_batch(const hi2x_piece* pieces, int64_t n_pieces, int32_t* bad,
                                   void* stream) {
  clear_error();
  HI2X_REQUIRE(n_pieces >= 0 && (n_pieces == 0 || pieces), "assemble_batch: bad arguments");
  hipStream_t s = as_stream(stream);
  double bytes = 0.0;
  for (int64_t i = 0; i < n_pieces; ++i) {
    const hi2x_piece& p = pieces[i];
    HI2X_REQUIRE(p.nbits == 2 || p.nbits == 4 || p.nbits == 8, "assemble_batch: piece %lld "
                 "nbits=%d", (long long)i, p.nbits);
    HI2X_REQUIRE(p.block > 0 && p.k % p.block == 0 && p.k % (32 / p.nbits) == 0 && p.r >= 0,
                 "assemble_batch: piece %lld K/block", (long long)i);
    bytes += (double)p.r * (p.k + p.k * p.nbits / 8 + 4 * (p.k / p.block) + 12);
  }
  LaunchTimer timer(HI2X_TIME_PACK, bytes, s);
  for (int64_t i = 0; i < n_pieces; ++i) {
    const hi2x_piece& p = pieces[i];
    if (p.r == 0) continue;
    const int64_t nw = p.k / (32 / p.nbits), nblk = p.k / p.block;
    const int64_t span = nw > nblk ? nw : nblk;
    const int64_t total = p.r * span;
    hipLaunchKernelGGL(assemble_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       p.rows, p.r, p.codes, p.params, p.consts, p.k, p.nbits, nblk, p.code_off,
                       p.param_off, p.out_codes, p.out_params, p.out_consts, bad);
    const int rc = launch_status("assemble_kernel");
    if (rc) return rc;
  }
  return HI2X_OK;
}

extern "C" int hi2x_assemble_piece(const int64_t* rows, int64_t r, const uint8_t* codes,
                                   const uint8_t* params, const uint16_t* consts, int64_t k,
                                   int nbits, int64_t block, const int64_t* code_off,
                                   const int64_t* param_off, int32_t* out_codes,
                                   uint8_t* out_params, uint16_t* out_consts, int32_t* bad,
                                   void* stream) {
  clear_error();
  HI2X_REQUIRE(nbits == 2 || nbits == 4 || nbits == 8, "assemble: nbits=%d", nbits);
  HI2X_REQUIRE(block > 0 && k % block == 0 && k % (32 / nbits) == 0, "assemble: K/block");
  if (r == 0) return HI2X_OK;
  const int64_t nw = k / (32 / nbits), nblk = k / block;
  const int64_t span = nw > nblk ? nw : nblk;
  const int64_t total = r * span;
  LaunchTimer timer(HI2X_TIME_PACK, (double)r * (k + k * nbits / 8 + 4 * nblk + 12),
                    as_stream(stream));
  hipLaunchKernelGGL(assemble_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), rows, r, codes, params, consts, k, nbits, nblk, code_off,
                     param_off, out_codes, out_params, out_consts, bad);
  return launch_status("assemble_kernel");
}
