// fp32 MFMA GEMM building block shared by the Cholesky chain and the GPTQ cross-block
// update (gfx950, wave64).
//
// A workgroup of 256 threads computes a 128 x 128 tile of A * op(B) as 2 x 2 waves of
// 64 x 64, each wave holding 2 x 2 accumulators of v_mfma_f32_32x32x2_f32 (16 VGPRs
// each).  The rank is streamed in chunks of 32 through double-buffered LDS: while the
// MFMAs consume one chunk, the next is already in flight from global memory into
// registers.  Accumulation runs from zero in k order, and each MFMA step evaluates
// fma(a1, b1, fma(a0, b0, acc)), so every element of the product is the sequential
// fp32 FMA chain over k.
//
// Operand access is through small loader structs so that triangular operands can mask
// their structural zeros (never reading the unused triangle) and edges can be guarded.
#pragma once
#include "common.h"

namespace hi2x {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int MG_T = 128;          // tile edge
constexpr int MG_KC = 32;          // rank chunk
constexpr int MG_KP = MG_KC / 2;   // k-pairs per chunk
constexpr int MG_RP = MG_KC + 4;   // LDS pitch of one tile row (floats)

// A chunk in LDS: row m of the tile holds [k parity][k pair] = 2 x 16 floats, so the
// lane that feeds MFMA row m with parity h reads all 16 of its k-pairs as 4 x b128.
struct MgSmem {
  float A[2][MG_T][MG_RP];
  float B[2][MG_T][MG_RP];
};

// Row-major operand X[r][k] (k contiguous), read as "rows" of the tile: the A operand,
// or the B operand of a transposed product (op(B) = X^T).  mask(r, k) -> keep.
// Thread t stages row t/2, 16 consecutive k starting at 16*(t%2).
template <class Mask>
struct RowsLoader {
  const float* p;
  int64_t ld, nrows, kend;
  Mask mask;
  __device__ __forceinline__ void load(int64_t r0, int64_t k0, int tid, float (&st)[16]) const {
    const int64_t r = r0 + (tid >> 1);
    const int64_t kb = k0 + 16 * (tid & 1);
    const bool rok = r < nrows;
    const float* src = p + r * ld + kb;
    const bool vec = rok && kb + 16 <= kend && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
    if (vec) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float4 x = *reinterpret_cast<const float4*>(src + 4 * v);
        st[4 * v] = x.x;
        st[4 * v + 1] = x.y;
        st[4 * v + 2] = x.z;
        st[4 * v + 3] = x.w;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) st[e] = mask(r, kb + e) ? st[e] : 0.0f;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st[e] = (rok && kb + e < kend && mask(r, kb + e)) ? src[e] : 0.0f;
    }
  }
  // k = 16h + e -> parity e & 1, pair 8h + e / 2
  __device__ __forceinline__ static void store(float (*S)[MG_RP], int tid, const float (&st)[16]) {
    const int m = tid >> 1, h = tid & 1;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      float* d = &S[m][par * MG_KP + 8 * h];
      *reinterpret_cast<float4*>(d) = make_float4(st[par], st[par + 2], st[par + 4], st[par + 6]);
      *reinterpret_cast<float4*>(d + 4) =
          make_float4(st[par + 8], st[par + 10], st[par + 12], st[par + 14]);
    }
  }
};

// Row-major operand X[k][c] (c contiguous) read as the B operand of a plain product.
// Thread t stages k = t%32 and 16 consecutive columns starting at 16*(t/32).
template <class Mask>
struct ColsLoader {
  const float* p;
  int64_t ld, ncols, kend;
  Mask mask;
  __device__ __forceinline__ void load(int64_t c0, int64_t k0, int tid, float (&st)[16]) const {
    const int64_t k = k0 + (tid & 31);
    const int64_t cb = c0 + 16 * (tid >> 5);
    const bool kok = k < kend;
    const float* src = p + k * ld + cb;
    const bool vec = kok && cb + 16 <= ncols && ((reinterpret_cast<uintptr_t>(src) & 15) == 0);
    if (vec) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float4 x = *reinterpret_cast<const float4*>(src + 4 * v);
        st[4 * v] = x.x;
        st[4 * v + 1] = x.y;
        st[4 * v + 2] = x.z;
        st[4 * v + 3] = x.w;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) st[e] = mask(k, cb + e) ? st[e] : 0.0f;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st[e] = (kok && cb + e < ncols && mask(k, cb + e)) ? src[e] : 0.0f;
    }
  }
  __device__ __forceinline__ static void store(float (*S)[MG_RP], int tid, const float (&st)[16]) {
    const int kk = tid & 31, cb = 16 * (tid >> 5);
    const int off = (kk & 1) * MG_KP + (kk >> 1);
#pragma unroll
    for (int e = 0; e < 16; ++e) S[cb + e][off] = st[e];
  }
};

struct NoMask {
  __device__ __forceinline__ bool operator()(int64_t, int64_t) const { return true; }
};

__device__ __forceinline__ void mg_zero(f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;
}

// acc += A[r0:r0+128, kbeg:kend] * op(B)[kbeg:kend, c0:c0+128], rank chunks in order.
// kbeg must be a multiple of 2 (MFMA k-pairs); loaders mask everything beyond kend.
template <class AL, class BL>
__device__ __forceinline__ void mg_mainloop(f32x16 (&acc)[2][2], MgSmem& sm, const AL& al,
                                            const BL& bl, int64_t r0, int64_t c0,
                                            int64_t kbeg, int64_t kend) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  if (kend <= kbeg) return;
  const int nch = (int)((kend - kbeg + MG_KC - 1) / MG_KC);
  float sa[16], sb[16];
  al.load(r0, kbeg, tid, sa);
  bl.load(c0, kbeg, tid, sb);
  __syncthreads();  // the previous use of the LDS buffers is over
  AL::store(sm.A[0], tid, sa);
  BL::store(sm.B[0], tid, sb);
  __syncthreads();
  const int par = lane >> 5, lr = lane & 31;
  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    if (ch + 1 < nch) {
      al.load(r0, kbeg + (int64_t)(ch + 1) * MG_KC, tid, sa);
      bl.load(c0, kbeg + (int64_t)(ch + 1) * MG_KC, tid, sb);
    }
    // this lane's operands for all 16 k-pairs of the chunk
    float av[2][MG_KP], bv[2][MG_KP];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const float* src = &sm.A[buf][wr * 64 + a * 32 + lr][par * MG_KP];
#pragma unroll
      for (int q = 0; q < MG_KP / 4; ++q) {
        const float4 x = *reinterpret_cast<const float4*>(src + 4 * q);
        av[a][4 * q] = x.x;
        av[a][4 * q + 1] = x.y;
        av[a][4 * q + 2] = x.z;
        av[a][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const float* src = &sm.B[buf][wcn * 64 + b * 32 + lr][par * MG_KP];
#pragma unroll
      for (int q = 0; q < MG_KP / 4; ++q) {
        const float4 x = *reinterpret_cast<const float4*>(src + 4 * q);
        bv[b][4 * q] = x.x;
        bv[b][4 * q + 1] = x.y;
        bv[b][4 * q + 2] = x.z;
        bv[b][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int kp = 0; kp < MG_KP; ++kp)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a][kp], bv[b][kp], acc[a][b], 0, 0, 0);
    if (ch + 1 < nch) {  // buffer buf ^ 1 was last read before the previous barrier
      AL::store(sm.A[buf ^ 1], tid, sa);
      BL::store(sm.B[buf ^ 1], tid, sb);
    }
    __syncthreads();
  }
}

// Row / column of accumulator register j of tile (a, b) for this lane, relative to the
// workgroup tile origin.
__device__ __forceinline__ int mg_row(int a, int j) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave >> 1) * 64 + a * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
}
__device__ __forceinline__ int mg_col(int b) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave & 1) * 64 + b * 32 + (lane & 31);
}

// Workgroup -> tile mapping that keeps neighbouring tiles on one XCD: workgroups are
// dispatched round-robin over the 8 XCDs, so linear id i runs on XCD i % 8; give XCD x
// the contiguous tile range [x * per, (x + 1) * per).
__device__ __forceinline__ int64_t xcd_tile(int64_t id, int64_t ntiles) {
  const int64_t per = (ntiles + 7) / 8;
  const int64_t t = (id % 8) * per + id / 8;
  return t < ntiles ? t : -1;
}

}  // namespace hi2x
