// Calibration Hessian S += X^T X on MFMA, and its transform to the stored basis.
//
// Reference: hi2/hessian.py:26-47 (HessianStats.update/merge/mean),
// hi2/hessian.py:50-68 (transform_sigma), hi2/moe.py:83-100 (routed token subsets).
#include <algorithm>
#include <vector>

#include "common.h"
#include "mfma_gemm.h"

namespace hi2x {
namespace {

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

// ---- bf16 SYRK on the feature-major copy Xt [K, T] -----------------------------------
// X [T, K] is first transposed once (one HBM pass) so that every MFMA operand (8
// consecutive tokens of one feature) is a 16-byte vector in memory and in LDS.  A
// workgroup (4 waves) computes a 256 x 256 upper tile of S; each wave owns 128 x 128 as
// 4 x 4 accumulators of v_mfma_f32_32x32x16_bf16 (f32 accumulation, products of bf16
// exact).  Tokens stream in stages of 64 through double-buffered LDS, loaded with
// branch-free buffer loads (features past K read zero) one stage ahead.  Big grids run
// the super-tile schedule: 4 x 8 tiles of the upper triangle per XCD round, so the 32
// workgroups of an XCD read 12 feature panels instead of up to 33.  Workgroups may split
// the token range (partials combined in a fixed order afterwards) so that small K still
// fills the chip.
constexpr int S2T = 256;          // workgroup tile edge
constexpr int S2C = 32;           // tokens per stage (64 bytes of a feature row)
constexpr int S2NB = 4;           // LDS stage buffers (prefetch distance S2NB - 1)
constexpr int S2Q = S2C / 8;      // 16-byte slots per feature row and stage
constexpr int S2R = 4, S2S = 8;   // super-tile: tile rows x tile columns per XCD round

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_bytes(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Upper-triangular grid of nT x nT tiles (tb >= ta) cut into super-tiles of S2R x S2S
// tiles; super-tile (sr, sc) holds upper tiles when sc >= floor(sr * S2R / S2S).  The
// host deals the super-tiles to the 8 XCDs longest first (by their upper tiles), each
// XCD's in row order; the main launch runs the first `main` tiles of every XCD's list (a
// whole number of rounds of its 32 CUs), and the tiles past them go, token-split, to a
// tail launch (see SyrkSched).
__host__ __device__ inline int syrk_first_sc(int sr) { return (sr * S2R) / S2S; }

// Upper tiles in super-tile (sr, sc): per tile row ta, the columns in [sc S2S, +S2S) at or
// right of ta and below nT.
__host__ __device__ inline int syrk_super_size(int sr, int sc, int nT) {
  int n = 0;
  for (int i = 0; i < S2R; ++i) {
    const int ta = sr * S2R + i;
    if (ta >= nT) break;
    int lo = sc * S2S, hi = sc * S2S + S2S;
    if (hi > nT) hi = nT;
    if (lo < ta) lo = ta;
    if (hi > lo) n += hi - lo;
  }
  return n;
}

constexpr int SYRK_MAX_SUPER = 512;  // super-tiles in a schedule (nT <= 128)
constexpr int SYRK_MAX_TAIL = 256;   // tail tiles (at most one round's worth)
struct SyrkSched {
  uint16_t st[SYRK_MAX_SUPER];     // super-tile ids (sr * nsc + sc), XCD by XCD
  uint16_t xoff[9];                // XCD x's super-tiles: st[xoff[x] .. xoff[x + 1])
  int32_t main;                    // tiles per XCD in the main launch
  uint16_t tail[SYRK_MAX_TAIL];    // tail tiles, ta << 8 | tb
  int32_t ntail;
};

// Tile j (in list order) of XCD x; false when the XCD has fewer tiles.
__device__ __forceinline__ bool syrk_sched_tile(const SyrkSched& sc, int nT, int x, int j,
                                                int& ta, int& tb) {
  const int nsc = (nT + S2S - 1) / S2S;
  for (int i = sc.xoff[x]; i < sc.xoff[x + 1]; ++i) {
    const int sr = sc.st[i] / nsc, c = sc.st[i] % nsc;
    const int n = syrk_super_size(sr, c, nT);
    if (j >= n) {
      j -= n;
      continue;
    }
    for (int w = 0; w < S2R * S2S; ++w) {
      const int a = sr * S2R + w / S2S, b = c * S2S + w % S2S;
      if (a < nT && b < nT && b >= a && j-- == 0) {
        ta = a;
        tb = b;
        return true;
      }
    }
    return false;
  }
  return false;
}

// xt [K, Tp] = x^T with the token range padded with zeros to Tp (a multiple of 64).
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ x,
                                                             int64_t T, int64_t K, int64_t Tp,
                                                             uint16_t* __restrict__ xt) {
  __shared__ uint16_t tile[64][66];
  const int64_t t0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int y = ty; y < 64; y += 4) {
    const int64_t t = t0 + y, k = k0 + tx;
    tile[y][tx] = (t < T && k < K) ? x[t * K + k] : (uint16_t)0;
  }
  __syncthreads();
  for (int y = ty; y < 64; y += 4) {
    const int64_t k = k0 + y, t = t0 + tx;
    if (k < K && t < Tp) xt[k * Tp + t] = tile[tx][y];
  }
}

// The same with 16-byte accesses (K a multiple of 8, x 16-byte aligned): a 64 x 64 tile
// read as 8-element row vectors and written as 8-token column vectors gathered from LDS
// (row pitch 66: the 8 rows a gather step reads from lie on distinct banks).
__global__ __launch_bounds__(256) void transpose8_bf16_kernel(const uint16_t* __restrict__ x,
                                                              int64_t T, int64_t K, int64_t Tp,
                                                              uint16_t* __restrict__ xt) {
  __shared__ uint32_t tile[64][33];  // 64 tokens x 66 features (bf16 pairs)
  const int64_t t0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  const int tid = threadIdx.x, c = tid & 7;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int r = (tid >> 3) + 32 * p;
    const int64_t t = t0 + r, k = k0 + 8 * c;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (t < T && k < K) v = *reinterpret_cast<const uint4*>(x + t * K + k);
    tile[r][4 * c] = v.x;
    tile[r][4 * c + 1] = v.y;
    tile[r][4 * c + 2] = v.z;
    tile[r][4 * c + 3] = v.w;
  }
  __syncthreads();
  const uint16_t* t16 = reinterpret_cast<const uint16_t*>(&tile[0][0]);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int kk = (tid >> 3) + 32 * p;
    const int64_t k = k0 + kk;
    if (k >= K) continue;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (uint32_t)t16[(8 * c + 2 * e) * 66 + kk] |
             ((uint32_t)t16[(8 * c + 2 * e + 1) * 66 + kk] << 16);
    *reinterpret_cast<uint4*>(xt + k * Tp + t0 + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---- routed (grouped) accumulation: one launch for every group of a token batch --------
// Group e is the tokens j in [offs[e], offs[e+1]) of a routed batch (the rows an MoE
// router sent to expert e, hi2/moe.py:83-100); token j is row rows[j] of x (rows NULL:
// row j).  The plan (on the device, so the caller never waits for the counts) gives every
// group a 64-aligned token window of the shared transposed copy and orders the groups by
// descending token count (largest first: the longest tiles start first).
struct SyrkGroups {
  const int32_t* order;  // [G] groups by descending token count (ties by index)
  const int64_t* toff;   // [G] first column of the group's window in xt
  const int64_t* tp;     // [G] window width: the token count rounded up to 64
  int64_t sstride;       // floats between consecutive groups' S
  int64_t ntiles;        // upper 256-tiles per group
};

__global__ __launch_bounds__(256) void grouped_plan_kernel(const int64_t* __restrict__ offs,
                                                           int G, int64_t t_total, int64_t cap,
                                                           int32_t* __restrict__ order,
                                                           int64_t* __restrict__ toff,
                                                           int64_t* __restrict__ tp) {
  // counts (a group outside [0, t_total] or descending offsets counts as empty)
  for (int e = threadIdx.x; e < G; e += blockDim.x) {
    const int64_t a = offs[e], b = offs[e + 1];
    const bool ok = a >= 0 && b >= a && b <= t_total;
    tp[e] = ok ? (b - a + 63) / 64 * 64 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // windows in group order, never past the capacity
    int64_t o = 0;
    for (int e = 0; e < G; ++e) {
      if (o + tp[e] > cap) tp[e] = 0;
      toff[e] = o;
      o += tp[e];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G; e += blockDim.x) {
    const int64_t te = tp[e] ? offs[e + 1] - offs[e] : 0;
    int rank = 0;
    for (int f = 0; f < G; ++f) {
      const int64_t tf = tp[f] ? offs[f + 1] - offs[f] : 0;
      rank += (tf > te || (tf == te && f < e)) ? 1 : 0;
    }
    order[rank] = e;
  }
}

// xt [K, cap]: column toff[e] + i of group e = token offs[e] + i (zeros past the group's
// count); the row of token j is rows[j] (rows NULL: j), rows outside [0, x_rows) read zero.
__global__ __launch_bounds__(256) void grouped_transpose_kernel(
    const uint16_t* __restrict__ x, int64_t x_rows, const int64_t* __restrict__ rows,
    const int64_t* __restrict__ offs, int G, const int64_t* __restrict__ toff,
    const int64_t* __restrict__ tp, int64_t K, int64_t cap, uint16_t* __restrict__ xt) {
  __shared__ uint16_t tile[64][66];
  __shared__ int64_t grp[2];  // group of this 64-column block, its first token
  const int64_t c0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  if (threadIdx.x == 0) {
    int lo = 0, hi = G - 1, e = -1;  // last group whose window starts at or before c0
    while (lo <= hi) {
      const int mid = (lo + hi) / 2;
      if (toff[mid] <= c0) {
        e = mid;
        lo = mid + 1;
      } else {
        hi = mid - 1;
      }
    }
    // empty windows share their start with the next group: step to the one holding c0
    while (e >= 0 && e < G && c0 >= toff[e] + tp[e]) e = (e + 1 < G && toff[e + 1] <= c0) ? e + 1 : -1;
    grp[0] = e;
  }
  __syncthreads();
  const int e = (int)grp[0];
  if (e < 0) return;
  const int64_t first = offs[e] + (c0 - toff[e]), end = offs[e + 1];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int y = ty; y < 64; y += 4) {
    const int64_t j = first + y, k = k0 + tx;
    int64_t r = -1;
    if (j < end) r = rows ? rows[j] : j;
    tile[y][tx] = (r >= 0 && r < x_rows && k < K) ? x[r * K + k] : (uint16_t)0;
  }
  __syncthreads();
  for (int y = ty; y < 64; y += 4) {
    const int64_t k = k0 + y, c = c0 + tx;
    if (k < K && c < cap) xt[k * cap + c] = tile[tx][y];
  }
}

// Operands of one k-step (16 tokens) of the current stage: XA / XB point at this lane's
// operand row (tile t adds 32 rows), so its 16-byte slot.
__device__ __forceinline__ void syrk_read(bf16x8 (&av)[4], bf16x8 (&bv)[4], const uint16_t* XA,
                                          const uint16_t* XB, int so) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    av[t] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(&XA[32 * t * S2C + so]));
    bv[t] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(&XB[32 * t * S2C + so]));
  }
}
__device__ __forceinline__ void syrk_mma(f32x16 (&acc)[4][4], const bf16x8 (&av)[4],
                                         const bf16x8 (&bv)[4]) {
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[a], bv[b], acc[a][b], 0, 0, 0);
}

// 16 bytes per lane from a buffer straight into LDS: lane L writes lds + 16 L (lds is
// wave-uniform).  Issued as inline assembly so that the compiler does not treat the
// asynchronous LDS write as aliasing every later LDS read (it would wait for all loads
// in flight before the first one); the kernel orders the writes itself with vmcnt waits
// and barriers.  m0 holds the LDS address only for this instruction.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, void* lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(
      (uint32_t)(size_t)(__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(la), "v"(voff), "s"(rs)
               : "m0");
}
#pragma clang diagnostic pop

// s_waitcnt immediate: wait until at most vm vector memory and lgkm LDS operations of this
// wave are outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left at
// its maximum, lgkmcnt 11:8)
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

// T is xt's row stride (its padded token count); with grouped (gr.order not null) item
// blockIdx.x is tile (id % ntiles) of the group of rank id / ntiles, over its window.
//
// mode 0: every upper tile (row-major id = blockIdx / splits, dealt to the XCDs in
// contiguous ranges), each split over the token range into a [K, K] slice of out per
// split (or S itself with one split); mode 1 (super): XCD blockIdx % 8 runs tile
// blockIdx / 8 of its list in sched, into S; mode 2 (tail): tail tile blockIdx / splits
// of sched, split over the tokens, each (tile, split) partial a 256 x 256 block of out.
__global__ __launch_bounds__(256) void syrk2_bf16_kernel(const uint16_t* __restrict__ xt,
                                                         int64_t T, int64_t K, int nT,
                                                         int64_t ntiles, int splits,
                                                         int64_t tchunk, float* __restrict__ out,
                                                         int64_t out_stride, int mode,
                                                         SyrkGroups gr, const SyrkSched sched) {
  __shared__ __attribute__((aligned(1024))) uint16_t Xa[S2NB][S2T * S2C];
  __shared__ __attribute__((aligned(1024))) uint16_t Xb[S2NB][S2T * S2C];
  const int64_t id = (int64_t)blockIdx.x;
  int ta, tb, sp = 0;
  int64_t tbeg, tend;
  float* so;    // the tile's output origin
  int64_t ldo;  // and its row stride
  if (gr.order) {
    const int e = gr.order[id / gr.ntiles];
    const int64_t w = gr.tp[e];
    if (w == 0) return;
    upper_tile(nT, (int)(id % gr.ntiles), ta, tb);
    tbeg = gr.toff[e];
    tend = tbeg + w;
    so = out + (int64_t)e * gr.sstride + (int64_t)ta * S2T * K + (int64_t)tb * S2T;
    ldo = K;
  } else {
    int64_t tile = 0;
    if (mode == 1) {
      const int j = (int)(id >> 3);
      if (j >= sched.main || !syrk_sched_tile(sched, nT, (int)(id & 7), j, ta, tb)) return;
    } else if (mode == 2) {
      sp = (int)(id % splits);
      tile = id / splits;
      if (tile >= sched.ntail) return;
      ta = sched.tail[tile] >> 8;
      tb = sched.tail[tile] & 0xff;
    } else {
      sp = (int)(id % splits);
      tile = xcd_tile(id / splits, ntiles);
      if (tile < 0) return;
      upper_tile(nT, (int)tile, ta, tb);
    }
    tbeg = (int64_t)sp * tchunk;
    tend = (tbeg + tchunk < T) ? tbeg + tchunk : T;
    if (mode == 2) {
      so = out + (tile * splits + sp) * (int64_t)S2T * S2T;
      ldo = S2T;
    } else {
      so = out + (int64_t)sp * out_stride + (int64_t)ta * S2T * K + (int64_t)tb * S2T;
      ldo = K;
    }
  }
  const bool diag = ta == tb;
  const int64_t a0 = (int64_t)ta * S2T, b0 = (int64_t)tb * S2T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  f32x16 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;

  // feature panels [a0, a0 + 256) and [b0, b0 + 256) of xt: features past K read zero
  // (T is the padded token count: every stage is whole, pad tokens are zero)
  const int rowsA = (int)((K - a0 < S2T) ? K - a0 : S2T);
  const int rowsB = (int)((K - b0 < S2T) ? K - b0 : S2T);
  const __amdgpu_buffer_rsrc_t rsa = rsrc_bytes(xt + a0 * T, (int64_t)rowsA * T * 2);
  const __amdgpu_buffer_rsrc_t rsb = rsrc_bytes(xt + b0 * T, (int64_t)rowsB * T * 2);
  // A stage of a panel (256 feature rows x 32 tokens = 64 bytes per row) goes from L2
  // straight into LDS (no registers, no LDS store instructions): each load instruction
  // of a wave writes 1 KB, 16 rows of 4 16-byte slots, lane L into slot L % 4 of row
  // L / 4.  Rows carry no padding; slot q of row r holds the row's piece q ^ ((r / 4) % 4),
  // so that the 16 consecutive rows an MFMA operand read touches (same piece) fall on 16
  // different 16-byte bank groups.  S2NB stages are in flight: the stage S2NB - 1 ahead
  // is requested while the current one is multiplied.
  constexpr int NC = S2T * S2C * 2 / 1024 / 4;  // 1 KB chunks per wave and panel
  const int prow = lane >> 2, piece = (lane & 3) ^ ((lane >> 4) & 3);
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // uniform: LDS addresses in SGPRs
  // load instruction j of a stage (chunk j / 2 of panel A or B, j % 2); b is this lane's
  // byte offset of the stage in its first row
  // (live = false: a load that reads nothing and writes zeros, for stages past the end,
  // so that every stage issues the same number of loads)
  auto dma_one = [&](int j, uint32_t b, int buf, bool live) {
    const int i = j >> 1, c = NC * wv + i, row = 16 * c + prow;
    const uint32_t o = b + (uint32_t)((int64_t)16 * i * T * 2);
    if ((j & 1) == 0) {
      lds_dma16(rsa, (live && row < rowsA) ? o : MG_OOB, &Xa[buf][c * 512]);
    } else {  // diagonal tiles load the A panel twice (uniform count of loads per stage)
      lds_dma16(diag ? rsa : rsb, (live && row < (diag ? rowsA : rowsB)) ? o : MG_OOB,
                &Xb[buf][c * 512]);
    }
  };
  auto stage_off = [&](int64_t t0) {
    uint32_t b = (uint32_t)(((int64_t)(16 * NC * wv + prow)) * T * 2 + t0 * 2 + 16 * piece);
    asm volatile("" : "+v"(b));
    return b;
  };
  auto dma = [&](int64_t t0, int buf, bool live) {
    const uint32_t b = stage_off(t0);
#pragma unroll
    for (int j = 0; j < 2 * NC; ++j) dma_one(j, b, buf, live);
  };
  constexpr int PER_STAGE = 2 * NC;  // load instructions per wave and stage
  static_assert(S2C == 32 && S2NB == 4, "the loop below reads two k-steps per stage");
  // operand rows of this lane (+ 32 t for tile t) and its slots of pieces h and 2 + h:
  // rows within a 32-row tile start at a multiple of 16, so (row / 4) % 4 = (lane / 4) % 4
  const int rowA = wr * 128 + (lane & 31), rowB = wcn * 128 + (lane & 31);
  const int so0 = 8 * ((lane >> 5) ^ ((lane >> 2) & 3));
  const int so1 = 8 * ((2 + (lane >> 5)) ^ ((lane >> 2) & 3));
  const int nst = (int)((tend - tbeg + S2C - 1) / S2C);
  // Pipeline: stage st + 1's k-step 0 operands are read, and stage st + 4 requested,
  // between the two k-steps of stage st, so that no LDS latency is exposed at the stage
  // boundary.  The ring holds stages st .. st + 3; every stage issues PER_STAGE loads
  // (stages past the end load nothing), so "stage j has landed" is always "at most the
  // two later stages' loads outstanding".  The loop body has no branch: MFMA chains on
  // one path only keep the accumulators in place.
  auto sync = [&]() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no LDS access moves across the barrier
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  bf16x8 oa0[4], ob0[4], oa1[4], ob1[4];
  if (nst > 0) {
#pragma unroll
    for (int p = 0; p < S2NB; ++p) dma(tbeg + (int64_t)p * S2C, p, p < nst);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(3 * PER_STAGE, 15));  // stage 0 landed
    sync();
    syrk_read(oa0, ob0, &Xa[0][rowA * S2C], &Xb[0][rowB * S2C], so0);
  }
  for (int st = 0; st < nst; ++st) {
    const int cb = st % S2NB, nb = (st + 1) % S2NB;
    syrk_read(oa1, ob1, &Xa[cb][rowA * S2C], &Xb[cb][rowB * S2C], so1);
    __builtin_amdgcn_sched_barrier(0);
    syrk_mma(acc, oa0, ob0);
    __builtin_amdgcn_sched_barrier(0);
    // this wave's reads of stage st are done and stage st + 1 has landed; after the
    // barrier no wave reads buffer cb any more (past the end: reads of unused zeros)
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * PER_STAGE, 0));
    sync();
    syrk_read(oa0, ob0, &Xa[nb][rowA * S2C], &Xb[nb][rowB * S2C], so0);
    __builtin_amdgcn_sched_barrier(0);
    // stage st + 4 into buffer cb, one load after every second MFMA (a single wave per
    // SIMD issues in order: a block of loads would leave the MFMA pipe idle)
    const uint32_t b = stage_off(tbeg + (int64_t)(st + S2NB) * S2C);
    const bool live = st + S2NB < nst;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[a][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa1[a], ob1[q], acc[a][q], 0, 0, 0);
        if (q & 1) {
          dma_one(2 * a + (q >> 1), b, cb, live);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();
  // upper part of the tile (i <= j on the diagonal tile); the lower triangle is mirrored
  // from it afterwards.  Branch-free: one buffer over the tile, rejected elements get an
  // offset past it.
  const __amdgpu_buffer_rsrc_t rss = mg_rsrc(so, (int64_t)(rowsA - 1) * ldo + rowsB);
  uint32_t base = (uint32_t)((((int64_t)wr * 128 + 4 * (lane >> 5)) * ldo + wcn * 128 + (lane & 31)) * 4);
  asm volatile("" : "+v"(base));
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      uint32_t offs[16];
      float cur[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = wr * 128 + a * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        const int c = wcn * 128 + b * 32 + (lane & 31);
        const bool ok = r < rowsA && c < rowsB && !(diag && r > c);
        offs[j] = ok ? base + (uint32_t)((((int64_t)(a * 32 + 8 * (j >> 2) + (j & 3))) * ldo + b * 32) * 4)
                     : MG_OOB;
        cur[j] = 0.0f;
      }
      if (splits == 1) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
          cur[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rss, (int)offs[j], 0, 0));
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float v = cur[j] + acc[a][b][j];
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rss, (int)offs[j], 0, 0);
      }
    }
}

// S (upper triangle) += partial_0 + partial_1 + ... in split order.  Grid (row i, pieces of
// the row): VEC (K a multiple of 4, 16-byte aligned buffers) gives each thread 4
// consecutive columns, the elements below the diagonal written back as read; a piece
// wholly below the diagonal returns at once.
template <bool VEC>
__global__ __launch_bounds__(256) void split_sum_kernel(float* __restrict__ s,
                                                        const float* __restrict__ parts,
                                                        int splits, int64_t K) {
  const int64_t i = blockIdx.x;
  constexpr int W = VEC ? 4 : 1;
  const int64_t j = ((int64_t)blockIdx.y * 256 + threadIdx.x) * W;
  if (j >= K || j + W - 1 < i) return;
  const int64_t idx = i * K + j;
  if constexpr (VEC) {
    f32x4 v = *reinterpret_cast<const f32x4*>(s + idx);
    const f32x4 v0 = v;
    for (int p = 0; p < splits; ++p) {
      const f32x4 q = *reinterpret_cast<const f32x4*>(parts + (int64_t)p * K * K + idx);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = v[e] + q[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = j + e < i ? v0[e] : v[e];
    *reinterpret_cast<f32x4*>(s + idx) = v;
  } else {
    float v = s[idx];
    for (int p = 0; p < splits; ++p) v = v + parts[(int64_t)p * K * K + idx];
    s[idx] = v;
  }
}

// The tail tiles' partials (compact blocks, split s of tail tile t at parts + (t * splits
// + s) * 256 * 256) into S: S[i][j] += p_0 + p_1 + ... in split order, the upper part of
// each tile.  Four workgroups per tile, 64 rows each; thread c walks column c of its rows.
__global__ __launch_bounds__(256) void syrk_tail_sum_kernel(float* __restrict__ s, int64_t K,
                                                            const SyrkSched sched, int splits,
                                                            const float* __restrict__ parts) {
  const int64_t t = blockIdx.x / 4;
  const int r0 = (int)(blockIdx.x % 4) * 64, c = threadIdx.x;
  const int ta = sched.tail[t] >> 8, tb = sched.tail[t] & 0xff;
  const int64_t a0 = (int64_t)ta * S2T, b0 = (int64_t)tb * S2T;
  if (b0 + c >= K) return;
  const float* pt = parts + t * splits * (int64_t)S2T * S2T;
  for (int r = r0; r < r0 + 64; ++r) {
    if (a0 + r >= K || (ta == tb && r > c)) break;  // rows only grow: the rest is out too
    float v = s[(a0 + r) * K + b0 + c];
    for (int p = 0; p < splits; ++p) v = v + pt[((int64_t)p * S2T + r) * S2T + c];
    s[(a0 + r) * K + b0 + c] = v;
  }
}

// Element access to the 64 x 64 tile at (r0, c0) of a row-major [K, K] matrix through a
// buffer resource that ends at the tile's last valid element: loads and stores need no
// branch (a branch around a load makes the compiler wait for it on the spot); elements
// outside the matrix read zero and are not written.
struct TileIO {
  __amdgpu_buffer_rsrc_t rs;
  int64_t ld;
  int rows, cols;
  __device__ __forceinline__ TileIO(const float* p, int64_t K, int64_t r0, int64_t c0) : ld(K) {
    rows = (int)((K - r0 < 64) ? K - r0 : 64);
    cols = (int)((K - c0 < 64) ? K - c0 : 64);
    rs = mg_rsrc(p + r0 * K + c0, (int64_t)(rows - 1) * K + cols);
  }
  __device__ __forceinline__ uint32_t off(int y, int x, bool keep) const {
    return (keep && y < rows && x < cols) ? (uint32_t)(((int64_t)y * ld + x) * 4) : MG_OOB;
  }
  __device__ __forceinline__ float load(int y, int x) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off(y, x, true), 0, 0));
  }
  __device__ __forceinline__ void store(int y, int x, float v, bool keep = true) const {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rs, (int)off(y, x, keep), 0, 0);
  }
};

// S[j][i] = S[i][j] for i < j: 64 x 64 tile pairs (ti <= tj) through LDS, rows of 256
// bytes on both sides; grid (tj, ti), the workgroups below the diagonal exit at once.
constexpr int MT = 64, MTP = MT + 1;
__global__ __launch_bounds__(256) void mirror_kernel(float* __restrict__ s, int64_t K,
                                                     int64_t sstride) {
  __shared__ float A[MT][MTP];
  s += (int64_t)blockIdx.z * sstride;
  const int ti = blockIdx.y, tj = blockIdx.x;
  if (ti > tj) return;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t i0 = (int64_t)ti * MT, j0 = (int64_t)tj * MT;
  const TileIO up(s, K, i0, j0), lo(s, K, j0, i0);
#pragma unroll
  for (int q = 0; q < MT / 4; ++q) A[ty + 4 * q][tx] = up.load(ty + 4 * q, tx);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < MT / 4; ++q) {
    const int y = ty + 4 * q;  // lower element (j0 + y, i0 + tx) = upper (i0 + tx, j0 + y)
    lo.store(y, tx, A[tx][y], j0 + y > i0 + tx);
  }
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

// transform_sigma in three coalesced passes over HBM, evaluating what the reference's
// fp32 ops evaluate (hi2/hessian.py:57-68):
//   (a) t1[16g+i][c] = sum_j m_g[i][j] s[16g+j][c], s = (sigma * inv_r) * inv_c
//   (b) t2[r][16h+l] = sum_k t1[r][16h+k] m_h[l][k]          (in place)
//   (c) out = 0.5 * (t2 + t2^T)                              (in place, tile pairs)
// with m = H16/4 on flagged groups (sequential FMA chains from zero, the products by
// +-1/4 exact) and I elsewhere; an identity product reduces to x + 0 (the chain maps
// -0 to +0), so the bits are the reference einsums'.
__device__ __forceinline__ float hsgn(int i, int j) {
  return (__builtin_popcount(i & j) & 1) ? -0.25f : 0.25f;
}

__global__ __launch_bounds__(256) void st_left_kernel(const float* __restrict__ sigma,
                                                      const uint16_t* __restrict__ col_scale,
                                                      const uint8_t* __restrict__ had, int64_t K,
                                                      float* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t g = blockIdx.y;
  if (c >= K) return;
  float x[16];
  const float ic = col_scale ? 1.0f / f16_from_bits(col_scale[c]) : 1.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t r = g * 16 + j;
    float v = sigma[r * K + c];
    if (col_scale) v = (v * (1.0f / f16_from_bits(col_scale[r]))) * ic;
    x[j] = v;
  }
  if (had[g]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) a = __builtin_fmaf(hsgn(i, j), x[j], a);
      out[(g * 16 + i) * K + c] = a;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[(g * 16 + i) * K + c] = x[i] + 0.0f;
  }
}

__global__ __launch_bounds__(256) void st_right_kernel(const uint8_t* __restrict__ had, int64_t K,
                                                       float* __restrict__ t) {
  const int64_t G = K / 16;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= K * G) return;
  const int64_t r = idx / G, h = idx % G;
  float* p = t + r * K + h * 16;
  float x[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 v = *reinterpret_cast<const float4*>(p + 4 * q);
    x[4 * q] = v.x;
    x[4 * q + 1] = v.y;
    x[4 * q + 2] = v.z;
    x[4 * q + 3] = v.w;
  }
  float y[16];
  if (had[h]) {
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) a = __builtin_fmaf(x[k], hsgn(l, k), a);
      y[l] = a;
    }
  } else {
#pragma unroll
    for (int l = 0; l < 16; ++l) y[l] = x[l] + 0.0f;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<float4*>(p + 4 * q) =
        make_float4(y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]);
}

// 32 x 32 tile pairs (I <= J): out[i][j] = out[j][i] = 0.5 * (t[i][j] + t[j][i]).
__global__ __launch_bounds__(256) void st_sym_kernel(int64_t K, int nT, float* __restrict__ t) {
  __shared__ float A[32][33], B[32][33];
  int ti, tj;
  upper_tile(nT, blockIdx.x, ti, tj);
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const int64_t i0 = (int64_t)ti * 32, j0 = (int64_t)tj * 32;
  for (int y = ty; y < 32; y += 8) {
    const int64_t r1 = i0 + y, c1 = j0 + tx, r2 = j0 + y, c2 = i0 + tx;
    A[y][tx] = (r1 < K && c1 < K) ? t[r1 * K + c1] : 0.0f;
    B[y][tx] = (r2 < K && c2 < K) ? t[r2 * K + c2] : 0.0f;
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int64_t r1 = i0 + y, c1 = j0 + tx, r2 = j0 + y, c2 = i0 + tx;
    const float o1 = 0.5f * (A[y][tx] + B[tx][y]);
    const float o2 = 0.5f * (B[y][tx] + A[tx][y]);
    if (r1 < K && c1 < K) t[r1 * K + c1] = o1;
    if (ti != tj && r2 < K && c2 < K) t[r2 * K + c2] = o2;
  }
}

// transform_sigma of the mean S / n straight from the upper triangle of the running sum
// S, in one pass: each workgroup takes the 64 x 64 tile pair (I, J), I <= J, reads only
// S's upper tile (I, J) (a diagonal tile's lower half from its upper half), and evaluates
// the same fp32 ops in the same order as the unfused path:
//   x = S / n (IEEE division), then (x * inv_r) * inv_c with the block's own (r, c),
//   the left group products, the right group products (sequential FMA chains from zero;
//   x + 0 on unflagged groups), and out[r][c] = out[c][r] = 0.5 * (t[r][c] + t[c][r]).
// Block (J, I) is built from the transposed values with its own (r, c) order of the
// column scaling, so both blocks are exactly what the full-matrix passes would compute.
constexpr int FT = 64, FTP = FT + 1;

__device__ __forceinline__ void group_left(float (*B)[FTP], int col, int lg, bool flag) {
  float x[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = B[16 * lg + j][col];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float a;
    if (flag) {
      a = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) a = __builtin_fmaf(hsgn(i, j), x[j], a);
    } else {
      a = x[i] + 0.0f;
    }
    B[16 * lg + i][col] = a;
  }
}

__device__ __forceinline__ void group_right(float (*B)[FTP], int row, int h, bool flag) {
  float x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = B[row][16 * h + k];
#pragma unroll
  for (int l = 0; l < 16; ++l) {
    float a;
    if (flag) {
      a = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) a = __builtin_fmaf(x[k], hsgn(l, k), a);
    } else {
      a = x[l] + 0.0f;
    }
    B[row][16 * h + l] = a;
  }
}

// nf: the token count (as the reference's mean divides by it); batched (ns not null):
// matrix z = blockIdx.z at s + z * sstride / out + z * ostride over max(ns[z], 1) tokens.
__global__ __launch_bounds__(256) void st_upper_kernel(const float* __restrict__ s, float nf,
                                                       const uint16_t* __restrict__ col_scale,
                                                       const uint8_t* __restrict__ had,
                                                       int64_t K, float* __restrict__ out,
                                                       const int64_t* __restrict__ ns,
                                                       int64_t sstride, int64_t ostride) {
  __shared__ float X[FT][FTP], Y[FT][FTP];
  if (ns) {
    const int64_t z = blockIdx.z, n = ns[z];
    s += z * sstride;
    out += z * ostride;
    nf = (float)(n > 1 ? n : 1);
  }
  const int ti = blockIdx.y, tj = blockIdx.x;
  if (ti > tj) return;
  const bool diag = ti == tj;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t R0 = (int64_t)ti * FT, C0 = (int64_t)tj * FT;
  const int64_t G = K / 16;
  // raw upper tile
  const TileIO in(s, K, R0, C0);
#pragma unroll
  for (int q = 0; q < FT / 4; ++q) X[ty + 4 * q][tx] = in.load(ty + 4 * q, tx);
  __syncthreads();
  float v[FT / 4];
#pragma unroll
  for (int q = 0; q < FT / 4; ++q) {
    const int y = ty + 4 * q;
    v[q] = (diag && y > tx) ? X[tx][y] : X[y][tx];
  }
  __syncthreads();
  // X block (rows R0.., cols C0..) and the transposed Y block (rows C0.., cols R0..)
  const float ic = (col_scale && C0 + tx < K) ? 1.0f / f16_from_bits(col_scale[C0 + tx]) : 1.0f;
#pragma unroll
  for (int q = 0; q < FT / 4; ++q) {
    const int y = ty + 4 * q;
    const float m = v[q] / nf;
    float xv = m, yv = m;
    if (col_scale) {
      const float ir = R0 + y < K ? 1.0f / f16_from_bits(col_scale[R0 + y]) : 1.0f;
      xv = (m * ir) * ic;
      yv = (m * ic) * ir;
    }
    X[y][tx] = xv;
    Y[tx][y] = yv;
  }
  __syncthreads();
  // left products: X over the row groups of I, Y over those of J
  {
    const int lg = ty;  // 4 groups of 16 rows, column tx
    const int64_t gx = R0 / 16 + lg, gy = C0 / 16 + lg;
    group_left(X, tx, lg, gx < G && had[gx]);
    group_left(Y, tx, lg, gy < G && had[gy]);
  }
  __syncthreads();
  // right products: X over the column groups of J, Y over those of I
  {
    const int h = ty;  // row tx, 4 groups of 16 columns
    const int64_t gx = C0 / 16 + h, gy = R0 / 16 + h;
    group_right(X, tx, h, gx < G && had[gx]);
    group_right(Y, tx, h, gy < G && had[gy]);
  }
  __syncthreads();
  const TileIO o1(out, K, R0, C0), o2(out, K, C0, R0);
#pragma unroll
  for (int q = 0; q < FT / 4; ++q) {
    const int y = ty + 4 * q;
    o1.store(y, tx, 0.5f * (X[y][tx] + Y[tx][y]));
  }
  if (!diag) {
#pragma unroll
    for (int q = 0; q < FT / 4; ++q) {
      const int y = ty + 4 * q;
      o2.store(y, tx, 0.5f * (Y[y][tx] + X[tx][y]));
    }
  }
}

// Work split of the bf16 SYRK and the workspace it needs: the transposed X (tokens
// padded to 64); when the 256-tiles are fewer than the 512 of the super-tile schedule,
// one partial [k, k] per token split; on the super-tile schedule, the compact partials of
// the tail tiles (the last tiles in row-major order past the last whole round of 256,
// each split over the token range so that they fill one round of the CUs).
struct SyrkPlan {
  int64_t tp = 0, tchunk = 0, ntiles = 0;
  int nT = 0, splits = 1;
  int super = 0;
  int64_t main_grid = 0;             // super: workgroups of the main launch
  int tail_splits = 1;
  int64_t tail_tchunk = 0;
  SyrkSched sched{};
  size_t xt_bytes = 0, parts_bytes = 0;
  size_t total() const { return xt_bytes + parts_bytes; }
};

// Token chunk of s splits of tp tokens (a multiple of the stage), and the splits that
// chunk gives.
static void syrk_chunk(int64_t tp, int s, int64_t& tchunk, int& splits) {
  tchunk = (tp + s - 1) / s;
  tchunk = (tchunk + S2C - 1) / S2C * S2C;
  splits = (int)((tp + tchunk - 1) / tchunk);
  if (splits < 1) splits = 1;
}

// The super-tile schedule: super-tiles dealt to the XCDs longest first (to the least
// loaded, lowest index on ties), each XCD's list in row order; every XCD runs its first
// 32 floor(max load / 32) tiles in the main launch and the rest (at most a round) go to
// the tail, split over the tokens.  False when the grid does not fit the tables.
static bool syrk_schedule(SyrkPlan& p) {
  const int nT = p.nT, nsr = (nT + S2R - 1) / S2R, nsc = (nT + S2S - 1) / S2S;
  if (nT > 255) return false;
  std::vector<std::pair<int, int>> items;  // (weight, super id)
  for (int sr = 0; sr < nsr; ++sr)
    for (int sc = syrk_first_sc(sr); sc < nsc; ++sc) {
      const int w = syrk_super_size(sr, sc, nT);
      if (w > 0) items.push_back({w, sr * nsc + sc});
    }
  if ((int)items.size() > SYRK_MAX_SUPER) return false;
  std::stable_sort(items.begin(), items.end(),
                   [](const std::pair<int, int>& a, const std::pair<int, int>& b) {
                     return a.first > b.first;
                   });
  std::vector<int> lists[8];
  int64_t load[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (const auto& it : items) {
    int best = 0;
    for (int x = 1; x < 8; ++x)
      if (load[x] < load[best]) best = x;
    load[best] += it.first;
    lists[best].push_back(it.second);
  }
  int64_t maxl = 0;
  SyrkSched& sc = p.sched;
  int n = 0;
  for (int x = 0; x < 8; ++x) {
    std::sort(lists[x].begin(), lists[x].end());
    sc.xoff[x] = (uint16_t)n;
    for (int id : lists[x]) sc.st[n++] = (uint16_t)id;
    maxl = std::max(maxl, load[x]);
  }
  sc.xoff[8] = (uint16_t)n;
  // the tail: tiles past the last whole round of the most loaded XCD
  const int64_t main = maxl / 32 * 32;
  int64_t tail = 0;
  for (int x = 0; x < 8; ++x) tail += load[x] > main ? load[x] - main : 0;
  int ts = tail > 0 ? (int)(256 / tail) : 1;
  if (ts > 8) ts = 8;
  if (tail == 0 || tail > SYRK_MAX_TAIL || ts < 2 || p.tp < 4 * S2C * ts) {
    sc.main = (int32_t)maxl;  // no tail: every tile in the main launch
    sc.ntail = 0;
    p.main_grid = 8 * maxl;
    return true;
  }
  sc.main = (int32_t)main;
  sc.ntail = 0;
  for (int x = 0; x < 8; ++x) {  // each XCD's tiles from `main` on, in list order
    int64_t j = 0;
    for (int i = sc.xoff[x]; i < sc.xoff[x + 1]; ++i) {
      const int sr = sc.st[i] / nsc, c = sc.st[i] % nsc;
      for (int w = 0; w < S2R * S2S; ++w) {
        const int a = sr * S2R + w / S2S, b = c * S2S + w % S2S;
        if (a < nT && b < nT && b >= a) {
          if (j >= main) sc.tail[sc.ntail++] = (uint16_t)(a << 8 | b);
          ++j;
        }
      }
    }
  }
  p.main_grid = 8 * main;
  syrk_chunk(p.tp, ts, p.tail_tchunk, p.tail_splits);
  p.parts_bytes = (size_t)sc.ntail * p.tail_splits * S2T * S2T * sizeof(float);
  return true;
}

SyrkPlan syrk_plan(int dtype, int64_t t, int64_t k) {
  SyrkPlan p;
  if (dtype != 2 || t == 0) return p;
  p.tp = (t + 63) / 64 * 64;
  p.nT = (int)((k + S2T - 1) / S2T);
  p.ntiles = (int64_t)p.nT * (p.nT + 1) / 2;
  p.xt_bytes = ((size_t)p.tp * (size_t)k * 2 + 255) / 256 * 256;
  if (p.ntiles >= 512) {
    // super-tile schedule, one workgroup per CU (else every tile at once, no tail)
    p.tchunk = p.tp;
    p.super = syrk_schedule(p) ? 1 : 0;
    return p;
  }
  // fewer tiles than the super-tile schedule takes: split the tokens.  From 128 tiles on,
  // s ways (1..8) for the fewest rounds of whole tiles (rounds(s) / s, each split costing a
  // little partial traffic: 136 tiles at K = 4096 take 3 splits, 408 workgroups, where
  // ceil(256 / 136) = 2 gave 272, a second round of 16); below, enough splits for one
  // workgroup per CU
  int best = (int)((256 + p.ntiles - 1) / p.ntiles);
  if (p.ntiles >= 128) {
    double cost = 1e30;
    for (int sp = 1; sp <= 8; ++sp) {
      const double rounds = (double)((p.ntiles * sp + 255) / 256);
      const double c = rounds / sp + 0.05 * (sp - 1);
      if (c < cost - 1e-9) cost = c, best = sp;
    }
  }
  syrk_chunk(p.tp, best, p.tchunk, p.splits);
  p.parts_bytes = p.splits > 1 ? (size_t)p.splits * k * k * sizeof(float) : 0;
  return p;
}

int launch_mirror(float* s, int64_t k, hipStream_t st) {
  const unsigned nM = (unsigned)((k + MT - 1) / MT);
  hipLaunchKernelGGL(mirror_kernel, dim3(nM, nM), dim3(256), 0, st, s, k, (int64_t)0);
  return launch_status("mirror_kernel");
}

// ws: device workspace of at least syrk_plan(...).total() bytes, 256-byte aligned.
// mirror = false leaves the lower triangle of a bf16 accumulation stale (the f32 path
// always writes both triangles).
int launch_syrk(const void* x, int dtype, int64_t t, int64_t k, float* s, char* ws,
                hipStream_t st, bool mirror = true) {
  if (dtype != 2) {
    const int nT = (int)((k + HT - 1) / HT);
    const int64_t tiles = (int64_t)nT * (nT + 1) / 2;
    LaunchTimer timer(HI2X_TIME_HESSIAN_SYRK, (double)t * k * (k + 1), st);  // upper triangle
    hipLaunchKernelGGL(syrk_f32_kernel, dim3((unsigned)tiles), dim3(256), 0, st,
                       (const float*)x, t, k, nT, s);
    return launch_status("syrk_f32_kernel");
  }
  // bf16: transpose, tiles of 256 (token range split when the tiles are few), mirror
  const SyrkPlan p = syrk_plan(dtype, t, k);
  uint16_t* xt = reinterpret_cast<uint16_t*>(ws);
  float* parts = p.parts_bytes > 0 ? reinterpret_cast<float*>(ws + p.xt_bytes) : nullptr;
  const dim3 tg((unsigned)((k + 63) / 64), (unsigned)(p.tp / 64));
  if (k % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0)
    hipLaunchKernelGGL(transpose8_bf16_kernel, tg, dim3(256), 0, st, (const uint16_t*)x, t, k,
                       p.tp, xt);
  else
    hipLaunchKernelGGL(transpose_bf16_kernel, tg, dim3(256), 0, st, (const uint16_t*)x, t, k, p.tp,
                       xt);
  int rc = launch_status("transpose_bf16_kernel");
  if (!rc) {
    // one workgroup per CU: super-tile rounds once the tiles fill several rounds
    LaunchTimer timer(HI2X_TIME_HESSIAN_SYRK, (double)t * k * (k + 1), st);  // upper triangle
    const int64_t grid = p.super ? p.main_grid : (p.ntiles + 7) / 8 * 8 * p.splits;
    hipLaunchKernelGGL(syrk2_bf16_kernel, dim3((unsigned)grid), dim3(256), 0, st, xt, p.tp, k,
                       p.nT, p.ntiles, p.splits, p.tchunk, p.splits > 1 ? parts : s, k * k,
                       p.super, SyrkGroups{}, p.sched);
    rc = launch_status("syrk2_bf16_kernel");
    const int ntail = p.super ? p.sched.ntail : 0;
    if (!rc && ntail > 0) {  // the tail tiles, token-split, then summed in split order
      hipLaunchKernelGGL(syrk2_bf16_kernel, dim3((unsigned)(ntail * p.tail_splits)), dim3(256), 0,
                         st, xt, p.tp, k, p.nT, (int64_t)ntail, p.tail_splits, p.tail_tchunk,
                         parts, (int64_t)0, 2, SyrkGroups{}, p.sched);
      rc = launch_status("syrk2_bf16_kernel");
      if (!rc) {
        hipLaunchKernelGGL(syrk_tail_sum_kernel, dim3((unsigned)(4 * ntail)), dim3(256), 0, st, s,
                           k, p.sched, p.tail_splits, parts);
        rc = launch_status("syrk_tail_sum_kernel");
      }
    }
  }
  if (!rc && parts && !p.super) {
    const bool vec = k % 4 == 0 && (reinterpret_cast<uintptr_t>(s) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(parts) & 15) == 0;
    const int64_t w = vec ? 4 : 1;
    const dim3 grid((unsigned)k, (unsigned)((k + 256 * w - 1) / (256 * w)));
    if (vec)
      hipLaunchKernelGGL(split_sum_kernel<true>, grid, dim3(256), 0, st, s, parts, p.splits, k);
    else
      hipLaunchKernelGGL(split_sum_kernel<false>, grid, dim3(256), 0, st, s, parts, p.splits, k);
    rc = launch_status("split_sum_kernel");
  }
  if (!rc && mirror) rc = launch_mirror(s, k, st);
  return rc;
}

// Workspace of the grouped accumulation: xt [k, cap] bf16 (cap = tokens + 64 per group,
// the windows' worst case) and the plan tables.
struct GroupedPlan {
  int64_t cap = 0;
  size_t xt_bytes = 0, order_off = 0, toff_off = 0, tp_off = 0, total = 0;
};

GroupedPlan grouped_plan(int64_t t_total, int64_t G, int64_t k) {
  GroupedPlan p;
  p.cap = (t_total + 64 * G + 63) / 64 * 64;
  p.xt_bytes = ((size_t)p.cap * (size_t)k * 2 + 255) / 256 * 256;
  p.order_off = p.xt_bytes;
  p.toff_off = p.order_off + ((size_t)G * 4 + 255) / 256 * 256;
  p.tp_off = p.toff_off + ((size_t)G * 8 + 255) / 256 * 256;
  p.total = p.tp_off + ((size_t)G * 8 + 255) / 256 * 256;
  return p;
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int64_t hi2x_hessian_workspace_bytes(int dtype, int64_t t, int64_t k) {
  if ((dtype != 0 && dtype != 2) || k <= 0 || t < 0) return -1;
  return (int64_t)syrk_plan(dtype, t, k).total();
}

extern "C" int hi2x_hessian_syrk(const void* x, int dtype, int64_t t, int64_t k, float* s,
                                 void* ws, int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(dtype == 0 || dtype == 2, "hessian_syrk: dtype %d (0 = f32, 2 = bf16)", dtype);
  HI2X_REQUIRE(k > 0 && t >= 0, "hessian_syrk: bad shape");
  if (t == 0) return HI2X_OK;
  hipStream_t st = as_stream(stream);
  Workspace w;
  const int rc = take_workspace(w, ws, ws_bytes, syrk_plan(dtype, t, k).total(), st,
                                "hessian_syrk");
  if (rc) return rc;
  return launch_syrk(x, dtype, t, k, s, w.p, st);
}

extern "C" int hi2x_hessian_syrk_upper(const void* x, int dtype, int64_t t, int64_t k,
                                       float* s, void* ws, int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(dtype == 0 || dtype == 2, "hessian_syrk_upper: dtype %d (0 = f32, 2 = bf16)",
               dtype);
  HI2X_REQUIRE(k > 0 && t >= 0, "hessian_syrk_upper: bad shape");
  if (t == 0) return HI2X_OK;
  hipStream_t st = as_stream(stream);
  Workspace w;
  const int rc = take_workspace(w, ws, ws_bytes, syrk_plan(dtype, t, k).total(), st,
                                "hessian_syrk_upper");
  if (rc) return rc;
  return launch_syrk(x, dtype, t, k, s, w.p, st, false);
}

extern "C" int hi2x_hessian_mirror(float* s, int64_t k, void* stream) {
  clear_error();
  HI2X_REQUIRE(s && k > 0, "hessian_mirror: bad arguments");
  return launch_mirror(s, k, as_stream(stream));
}

extern "C" int64_t hi2x_hessian_grouped_workspace_bytes(int64_t t_total, int64_t n_groups,
                                                       int64_t k) {
  if (t_total < 0 || n_groups <= 0 || n_groups > 65535 || k <= 0) return -1;
  return (int64_t)grouped_plan(t_total, n_groups, k).total;
}

extern "C" int hi2x_hessian_syrk_grouped(const void* x, int64_t x_rows, int dtype,
                                         const int64_t* rows, const int64_t* offs,
                                         int64_t n_groups, int64_t t_total, int64_t k, float* s,
                                         int64_t s_stride, int upper_only, void* ws,
                                         int64_t ws_bytes, void* stream) {
  clear_error();
  HI2X_REQUIRE(dtype == 2, "hessian_syrk_grouped: dtype %d (bf16 tokens only: 2)", dtype);
  HI2X_REQUIRE(x && offs && s && k > 0 && x_rows >= 0 && t_total >= 0 && n_groups > 0 &&
                   n_groups <= 65535,
               "hessian_syrk_grouped: bad arguments");
  HI2X_REQUIRE(s_stride >= k * k, "hessian_syrk_grouped: s_stride %lld below k * k",
               (long long)s_stride);
  if (t_total == 0) return HI2X_OK;
  hipStream_t st = as_stream(stream);
  const GroupedPlan p = grouped_plan(t_total, n_groups, k);
  HI2X_REQUIRE(p.cap <= (int64_t(1) << 22),
               "hessian_syrk_grouped: %lld tokens (plus 64 per group) exceed 4M per call",
               (long long)t_total);
  Workspace w;
  int rc = take_workspace(w, ws, ws_bytes, p.total, st, "hessian_syrk_grouped");
  if (rc) return rc;
  uint16_t* xt = reinterpret_cast<uint16_t*>(w.p);
  int32_t* order = reinterpret_cast<int32_t*>(w.p + p.order_off);
  int64_t* toff = reinterpret_cast<int64_t*>(w.p + p.toff_off);
  int64_t* tp = reinterpret_cast<int64_t*>(w.p + p.tp_off);
  const int G = (int)n_groups;
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(256), 0, st, offs, G, t_total, p.cap,
                     order, toff, tp);
  rc = launch_status("grouped_plan_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(grouped_transpose_kernel,
                     dim3((unsigned)((k + 63) / 64), (unsigned)(p.cap / 64)), dim3(256), 0, st,
                     (const uint16_t*)x, x_rows, rows, offs, G, toff, tp, k, p.cap, xt);
  rc = launch_status("grouped_transpose_kernel");
  if (rc) return rc;
  const int nT = (int)((k + S2T - 1) / S2T);
  const int64_t ntiles = (int64_t)nT * (nT + 1) / 2;
  {
    LaunchTimer timer(HI2X_TIME_HESSIAN_SYRK, (double)t_total * k * (k + 1), st);
    hipLaunchKernelGGL(syrk2_bf16_kernel, dim3((unsigned)(ntiles * G)), dim3(256), 0, st, xt,
                       p.cap, k, nT, ntiles, 1, (int64_t)0, s, (int64_t)0, 0,
                       SyrkGroups{order, toff, tp, s_stride, ntiles}, SyrkSched{});
    rc = launch_status("syrk2_bf16_kernel");
  }
  if (rc || upper_only) return rc;
  const unsigned nM = (unsigned)((k + MT - 1) / MT);
  hipLaunchKernelGGL(mirror_kernel, dim3(nM, nM, (unsigned)G), dim3(256), 0, st, s, k, s_stride);
  return launch_status("mirror_kernel");
}

extern "C" int hi2x_sigma_transform(const float* sigma, const uint16_t* col_scale,
                                    const uint8_t* had, int64_t k, float* hs, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0, "sigma_transform: K=%lld not a multiple of 16",
               (long long)k);
  HI2X_REQUIRE(sigma != hs, "sigma_transform: in-place not supported");
  hipStream_t s = as_stream(stream);
  const int64_t G = k / 16;
  hipLaunchKernelGGL(st_left_kernel, dim3((unsigned)((k + 255) / 256), (unsigned)G), dim3(256),
                     0, s, sigma, col_scale, had, k, hs);
  int rc = launch_status("st_left_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(st_right_kernel, dim3((unsigned)((k * G + 255) / 256)), dim3(256), 0, s,
                     had, k, hs);
  rc = launch_status("st_right_kernel");
  if (rc) return rc;
  const int nT = (int)((k + 31) / 32);
  hipLaunchKernelGGL(st_sym_kernel, dim3((unsigned)((int64_t)nT * (nT + 1) / 2)), dim3(256), 0,
                     s, k, nT, hs);
  return launch_status("st_sym_kernel");
}

extern "C" int hi2x_sigma_transform_upper(const float* s, int64_t n, const uint16_t* col_scale,
                                          const uint8_t* had, int64_t k, float* hs,
                                          void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0, "sigma_transform_upper: K=%lld not a multiple of 16",
               (long long)k);
  HI2X_REQUIRE(s && had && hs && s != hs, "sigma_transform_upper: bad buffers");
  HI2X_REQUIRE(n >= 0, "sigma_transform_upper: n=%lld", (long long)n);
  const unsigned nT = (unsigned)((k + FT - 1) / FT);
  const float nf = (float)(n > 1 ? n : 1);
  hipLaunchKernelGGL(st_upper_kernel, dim3(nT, nT), dim3(256), 0, as_stream(stream), s, nf,
                     col_scale, had, k, hs, (const int64_t*)nullptr, (int64_t)0, (int64_t)0);
  return launch_status("st_upper_kernel");
}

extern "C" int hi2x_sigma_transform_upper_batched(const float* s, int64_t s_stride,
                                                  const int64_t* n, int64_t batch,
                                                  const uint16_t* col_scale, const uint8_t* had,
                                                  int64_t k, float* hs, int64_t hs_stride,
                                                  void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && k % 16 == 0, "sigma_transform_upper_batched: K=%lld not a multiple "
               "of 16", (long long)k);
  HI2X_REQUIRE(s && n && had && hs && batch > 0 && batch <= 65535,
               "sigma_transform_upper_batched: bad arguments");
  HI2X_REQUIRE(s_stride >= k * k && hs_stride >= k * k,
               "sigma_transform_upper_batched: strides below k * k");
  HI2X_REQUIRE(!(hs < s + s_stride * batch && s < hs + hs_stride * batch),
               "sigma_transform_upper_batched: s and hs overlap");
  const unsigned nT = (unsigned)((k + FT - 1) / FT);
  hipLaunchKernelGGL(st_upper_kernel, dim3(nT, nT, (unsigned)batch), dim3(256), 0,
                     as_stream(stream), s, 1.0f, col_scale, had, k, hs, n, s_stride, hs_stride);
  return launch_status("st_upper_kernel");
}

// ---- MoE token floor (hi2/layerwise.py:245-257 with blend, hi2/moe.py:152-156) ----------
// tot = ((0 + S_0) + S_1) + ... + S_{G-1} elementwise in fp32 (the reference's Python sum
// over the experts' sums, taken before any is changed), then for every expert with
// mask[e]: S_e = S_e + fill[e] * tot (fill the fp32 value of (need - n_e) / n_total).
// Upper triangle only (upper != 0) or every element.
// Grid (row i, pieces of 256 columns): no index division per element, and a piece wholly
// below the diagonal returns at once when only the upper triangle is blended.
__global__ __launch_bounds__(256) void blend_kernel(float* __restrict__ s, int64_t sstride,
                                                    int G, int64_t K,
                                                    const float* __restrict__ fill,
                                                    const uint8_t* __restrict__ mask,
                                                    int upper) {
  const int64_t i = blockIdx.x, j = (int64_t)blockIdx.y * 256 + threadIdx.x;
  if (j >= K || (upper && j < i)) return;
  const int64_t idx = i * K + j;
  float tot = s[idx] + 0.0f;
  for (int e = 1; e < G; ++e) tot = tot + s[(int64_t)e * sstride + idx];
  for (int e = 0; e < G; ++e)
    if (mask[e]) {
      float* p = s + (int64_t)e * sstride + idx;
      *p = *p + fill[e] * tot;
    }
}

extern "C" int hi2x_hessian_blend(float* s, int64_t s_stride, int64_t n_groups, int64_t k,
                                  const float* fill, const uint8_t* mask, int upper_only,
                                  void* stream) {
  clear_error();
  HI2X_REQUIRE(s && fill && mask && k > 0 && n_groups > 0 && s_stride >= k * k,
               "hessian_blend: bad arguments");
  hipLaunchKernelGGL(blend_kernel, dim3((unsigned)k, (unsigned)((k + 255) / 256)), dim3(256), 0,
                     as_stream(stream), s, s_stride, (int)n_groups, k, fill, mask, upper_only);
  return launch_status("blend_kernel");
}
