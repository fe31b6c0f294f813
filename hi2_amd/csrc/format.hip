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

// assemble (hi2/format.py:155-171): the pieces of one or more tensors in one launch.
// Each piece is a group of rows sharing (nbits, B); its descriptor travels in the kernel
// arguments (up to kPackPieces per launch) with the first workgroup of every piece.  A
// wave packs one row: lane l takes words l, l + 64, ... of the row (32/nbits codes, LSB
// first, each from one 4-, 8- or 16-byte load, four loads in flight per round) into the
// flat buffer at code_off[rows[i]] + j, moves the ladder bytes of blocks l, l + 64, ...
// (16-bit pairs) to param_off[rows[i]] + b, and lanes 0..2 move the row's three
// constants.  Codes at or above 2^nbits are counted in bad (packed masked).
constexpr int kPackPieces = 24;
constexpr int kPackRows = 4;  // rows (waves) per workgroup
struct PackPiece {
  const int64_t* rows;
  const uint8_t* codes;
  const uint8_t* params;
  const uint16_t* consts;
  const int64_t* code_off;
  const int64_t* param_off;
  int32_t* out_codes;
  uint8_t* out_params;
  uint16_t* out_consts;
  int32_t k, nbits, nblk, nw, r;
  int32_t vec;  // bit 0: 16-byte code rows, bit 1: 2-byte params
};
struct PackBatch {
  PackPiece p[kPackPieces];
  int32_t wg_start[kPackPieces + 1];
  int32_t n;
};

template <int PER>
__device__ __forceinline__ uint32_t pack_word(const uint32_t (&x)[PER / 4], int& nbad) {
  constexpr int NB = 32 / PER;
  constexpr uint32_t LIM = 1u << NB;
  uint32_t v = 0;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const uint32_t cv = (x[q / 4] >> (8 * (q % 4))) & 0xffu;
    nbad += cv >= LIM;
    v |= (cv & (LIM - 1u)) << (NB * q);
  }
  return v;
}

// Word j of a code row c (PER codes), as PER / 4 dwords.
template <int PER>
__device__ __forceinline__ void load_word(uint32_t (&x)[PER / 4], const uint8_t* c, int j,
                                          bool vec) {
  if (vec) {
    if constexpr (PER == 16) {
      const uint4 y = reinterpret_cast<const uint4*>(c)[j];
      x[0] = y.x, x[1] = y.y, x[2] = y.z, x[3] = y.w;
    } else if constexpr (PER == 8) {
      const uint2 y = reinterpret_cast<const uint2*>(c)[j];
      x[0] = y.x, x[1] = y.y;
    } else {
      x[0] = reinterpret_cast<const uint32_t*>(c)[j];
    }
  } else {
#pragma unroll
    for (int q = 0; q < PER / 4; ++q) {
      const uint8_t* b = c + PER * j + 4 * q;
      x[q] = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
    }
  }
}

template <int PER>
__device__ __forceinline__ int pack_row(const uint8_t* __restrict__ c, int nw, bool vec,
                                        int32_t* __restrict__ out, int lane) {
  constexpr int U = 4;  // loads in flight per lane
  int nbad = 0;
  for (int j0 = lane; j0 < nw; j0 += 64 * U) {
    uint32_t x[U][PER / 4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + 64 * u;
      if (j < nw) load_word<PER>(x[u], c, j, vec);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + 64 * u;
      if (j < nw) out[j] = (int32_t)pack_word<PER>(x[u], nbad);
    }
  }
  return nbad;
}

__global__ __launch_bounds__(64 * kPackRows) void assemble_batch_kernel(
    const PackBatch b, int32_t* __restrict__ bad) {
  const int wg = blockIdx.x;
  int pi = 0;
  while (pi + 1 < b.n && wg >= b.wg_start[pi + 1]) ++pi;  // uniform: scalar registers
  const PackPiece& p = b.p[pi];
  const int lane = threadIdx.x & 63;
  const int i = (wg - b.wg_start[pi]) * kPackRows + (int)(threadIdx.x >> 6);
  if (i >= p.r) return;
  const int64_t row = p.rows[i];
  const uint8_t* c = p.codes + (int64_t)i * p.k;
  int32_t* out = p.out_codes + p.code_off[row];
  const bool vec = (p.vec & 1) != 0;
  int nbad;
  if (p.nbits == 2)
    nbad = pack_row<16>(c, p.nw, vec, out, lane);
  else if (p.nbits == 4)
    nbad = pack_row<8>(c, p.nw, vec, out, lane);
  else
    nbad = pack_row<4>(c, p.nw, vec, out, lane);
  const int64_t src = (int64_t)i * p.nblk, dst = p.param_off[row];
  if (p.vec & 2) {
    const uint16_t* ps = reinterpret_cast<const uint16_t*>(p.params) + src;
    uint16_t* pd = reinterpret_cast<uint16_t*>(p.out_params) + dst;
    for (int j = lane; j < p.nblk; j += 64) pd[j] = ps[j];
  } else {
    for (int j = lane; j < p.nblk; j += 64) {
      p.out_params[2 * (dst + j)] = p.params[2 * (src + j)];
      p.out_params[2 * (dst + j) + 1] = p.params[2 * (src + j) + 1];
    }
  }
  if (lane < 3) p.out_consts[row * 3 + lane] = p.consts[(int64_t)i * 3 + lane];
  note_bad(bad, nbad);
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

// One launch per kPackPieces pieces (the pieces' checks come first, before anything is
// launched).
static int assemble_launch(const hi2x_piece* pieces, int64_t n_pieces, int32_t* bad,
                           hipStream_t s) {
  double bytes = 0.0;
  for (int64_t i = 0; i < n_pieces; ++i) {
    const hi2x_piece& p = pieces[i];
    HI2X_REQUIRE(p.nbits == 2 || p.nbits == 4 || p.nbits == 8, "assemble: piece %lld "
                 "nbits=%d", (long long)i, p.nbits);
    HI2X_REQUIRE(p.block > 0 && p.k > 0 && p.k % p.block == 0 && p.k % (32 / p.nbits) == 0 &&
                     p.r >= 0 && p.k < (int64_t(1) << 30),
                 "assemble: piece %lld K/block", (long long)i);
    HI2X_REQUIRE(p.r == 0 || (p.rows && p.codes && p.params && p.consts && p.code_off &&
                              p.param_off && p.out_codes && p.out_params && p.out_consts),
                 "assemble: piece %lld has a null buffer", (long long)i);
    bytes += (double)p.r * (p.k + p.k * p.nbits / 8 + 4 * (p.k / p.block) + 12);
  }
  LaunchTimer timer(HI2X_TIME_PACK, bytes, s);
  PackBatch b;
  int64_t i = 0;
  while (i < n_pieces) {
    b.n = 0;
    int64_t wgs = 0;
    for (; i < n_pieces && b.n < kPackPieces; ++i) {
      const hi2x_piece& q = pieces[i];
      if (q.r == 0) continue;
      const int64_t nw = q.k / (32 / q.nbits), nblk = q.k / q.block;
      const int64_t nwg = (q.r + kPackRows - 1) / kPackRows;
      HI2X_REQUIRE(q.r < (int64_t(1) << 31) && wgs + nwg < (int64_t(1) << 31),
                   "assemble: too many rows");
      PackPiece& p = b.p[b.n];
      p.rows = q.rows;
      p.codes = q.codes;
      p.params = q.params;
      p.consts = q.consts;
      p.code_off = q.code_off;
      p.param_off = q.param_off;
      p.out_codes = q.out_codes;
      p.out_params = q.out_params;
      p.out_consts = q.out_consts;
      p.k = (int32_t)q.k;
      p.nbits = q.nbits;
      p.nblk = (int32_t)nblk;
      p.nw = (int32_t)nw;
      p.r = (int32_t)q.r;
      p.vec = ((reinterpret_cast<uintptr_t>(q.codes) % 16 == 0 && q.k % 16 == 0) ? 1 : 0) |
              ((reinterpret_cast<uintptr_t>(q.params) % 2 == 0 &&
                reinterpret_cast<uintptr_t>(q.out_params) % 2 == 0) ? 2 : 0);
      b.wg_start[b.n] = (int32_t)wgs;
      wgs += nwg;
      ++b.n;
    }
    if (b.n == 0) break;
    b.wg_start[b.n] = (int32_t)wgs;
    hipLaunchKernelGGL(assemble_batch_kernel, dim3((unsigned)wgs), dim3(64 * kPackRows), 0, s,
                       b, bad);
    const int rc = launch_status("assemble_batch_kernel");
    if (rc) return rc;
  }
  return HI2X_OK;
}

extern "C" int hi2x_assemble_batch(const hi2x_piece* pieces, int64_t n_pieces, int32_t* bad,
                                   void* stream) {
  clear_error();
  HI2X_REQUIRE(n_pieces >= 0 && (n_pieces == 0 || pieces), "assemble_batch: bad arguments");
  return assemble_launch(pieces, n_pieces, bad, as_stream(stream));
}

extern "C" int hi2x_assemble_piece(const int64_t* rows, int64_t r, const uint8_t* codes,
                                   const uint8_t* params, const uint16_t* consts, int64_t k,
                                   int nbits, int64_t block, const int64_t* code_off,
                                   const int64_t* param_off, int32_t* out_codes,
                                   uint8_t* out_params, uint16_t* out_consts, int32_t* bad,
                                   void* stream) {
  clear_error();
  const hi2x_piece p{rows, r, codes, params, consts, k, nbits, 0, block, code_off, param_off,
                     out_codes, out_params, out_consts};
  return assemble_launch(&p, 1, bad, as_stream(stream));
}
