// fp32 MFMA GEMM building block shared by the Cholesky chain and the GPTQ cross-block
// update (gfx950, wave64).
//
// A workgroup of 256 threads computes a 128 x 128 tile of A * op(B) as 2 x 2 waves of
// 64 x 64, each wave holding 2 x 2 accumulators of v_mfma_f32_32x32x2_f32 (16 VGPRs
// each); a 64 x 64 variant (one accumulator per wave) serves grids too small for the
// chip.  The rank is streamed in chunks of 32 through double-buffered LDS: while the
// MFMAs consume one chunk, the next is already in flight from global memory into
// registers.  Accumulation runs from zero in k order, and each MFMA step evaluates
// fma(a1, b1, fma(a0, b0, acc)), so every element of the product is the sequential
// fp32 FMA chain over k.
//
// Operand access is through small loader structs: edges and masked rows read as zero
// through the buffer-load range check, and triangular operands zero their structural
// zeros when a chunk is staged, so the unused triangle never enters a product.
#pragma once
#include <algorithm>
#include <utility>
#include <vector>

#include "common.h"

namespace hi2x {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int MG_T = 128;          // tile edge
constexpr int MG_KC = 32;          // rank chunk
constexpr int MG_KP = MG_KC / 2;   // k-pairs per chunk
constexpr int MG_RP = MG_KC + 4;   // LDS pitch of one tile row (floats)

// A chunk in LDS: row m of the tile holds [k parity][k pair] = 2 x 16 floats, so the
// lane that feeds MFMA row m with parity h reads all 16 of its k-pairs as 4 x b128.
// T is the workgroup tile edge: 128 (2 x 2 accumulators per wave) or 64 (one per wave,
// for grids too small to fill the chip with 128-tiles).
template <int T = MG_T>
struct MgSmemT {
  float A[2][T][MG_RP];
  float B[2][T][MG_RP];
};
using MgSmem = MgSmemT<MG_T>;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Operand fetches go through buffer loads whose resource covers exactly the valid part
// of the chunk's panel: an access past it returns zero without touching memory, so the
// loads need no branches (a branch around a load makes the compiler wait for it right
// there, before the MFMAs, instead of after them).  Offsets stay far below 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mg_rsrc(const float* base, int64_t nfloats) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0,
                                           (int)(nfloats * 4), 0x00020000);
}
__device__ __forceinline__ f32x4 mg_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}
constexpr uint32_t MG_OOB = 0x80000000u;  // byte offset past every panel: reads as zero

// Masks: row(r) drops a whole staged row (applied through the load offset); elem(r, k)
// drops single elements (applied when the chunk is written to LDS, after the MFMAs).
struct NoMask {
  static constexpr bool kElem = false;
  __device__ __forceinline__ bool row(int64_t) const { return true; }
  __device__ __forceinline__ bool elem(int64_t, int64_t) const { return true; }
};

// Row-major operand X[r][k] (k contiguous), read as "rows" of the tile: the A operand,
// or the B operand of a transposed product (op(B) = X^T).  Rows >= nrows and k >= kend
// read as zero.  TPR threads stage one tile row, KPT consecutive k each.
template <class Mask, int T = MG_T>
struct RowsLoader {
  static constexpr int TPR = 256 / T, KPT = MG_KC / TPR, NV = KPT / 4;
  const float* p;
  int64_t ld, nrows, kend;
  Mask mask;
  __device__ __forceinline__ void load(int64_t r0, int64_t k0, int tid, f32x4 (&st)[NV]) const {
    const int64_t rows = (nrows - r0 < T) ? nrows - r0 : T;
    const int64_t kv = kend - k0;
    // last valid element of the panel: row rows-1, column kend-1
    const __amdgpu_buffer_rsrc_t rs = mg_rsrc(p + r0 * ld + k0, (rows - 1) * ld + kv);
    const int rr = tid / TPR;
    uint32_t off = (uint32_t)((rr * ld + KPT * (tid % TPR)) * 4);
    off = (rr < rows && mask.row(r0 + rr)) ? off : MG_OOB;
#pragma unroll
    for (int v = 0; v < NV; ++v) st[v] = mg_load4(rs, off + 16 * v);
  }
  // k = KPT h + e -> parity e & 1, pair (KPT/2) h + e / 2.  Elements at k >= kend of rows
  // before the last are real memory of the next columns: zeroed here.
  __device__ __forceinline__ void store(float (*S)[MG_RP], int64_t r0, int64_t k0, int tid,
                                        f32x4 (&st)[NV]) const {
    const int m = tid / TPR, h = tid % TPR;
    const int64_t kb = k0 + KPT * h;
    if (Mask::kElem || k0 + MG_KC > kend) {
#pragma unroll
      for (int e = 0; e < KPT; ++e) {
        const bool keep = kb + e < kend && mask.elem(r0 + m, kb + e);
        st[e >> 2][e & 3] = keep ? st[e >> 2][e & 3] : 0.0f;
      }
    }
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      float* d = &S[m][par * MG_KP + (KPT / 2) * h];
#pragma unroll
      for (int g = 0; g < KPT / 8; ++g) {
        // elements e = par + 2 (4g + i), i < 4
        *reinterpret_cast<float4*>(d + 4 * g) =
            make_float4(st[(par + 8 * g) >> 2][(par + 8 * g) & 3],
                        st[(par + 8 * g + 2) >> 2][(par + 8 * g + 2) & 3],
                        st[(par + 8 * g + 4) >> 2][(par + 8 * g + 4) & 3],
                        st[(par + 8 * g + 6) >> 2][(par + 8 * g + 6) & 3]);
      }
    }
  }
};

// Row-major operand X[k][c] (c contiguous) read as the B operand of a plain product.
// k >= kend reads as zero; columns >= ncols feed only output columns that are never
// stored.  Thread t stages k = t%32 and CPT consecutive columns starting at CPT*(t/32).
template <class Mask, int T = MG_T>
struct ColsLoader {
  static constexpr int CPT = T / 8, NV = CPT / 4;
  const float* p;
  int64_t ld, ncols, kend;
  Mask mask;
  __device__ __forceinline__ void load(int64_t c0, int64_t k0, int tid, f32x4 (&st)[NV]) const {
    const int64_t kv = (kend - k0 < MG_KC) ? kend - k0 : MG_KC;
    const __amdgpu_buffer_rsrc_t rs = mg_rsrc(p + k0 * ld + c0, (kv - 1) * ld + (ncols - c0));
    const uint32_t off = (uint32_t)(((tid & 31) * ld + CPT * (tid >> 5)) * 4);
#pragma unroll
    for (int v = 0; v < NV; ++v) st[v] = mg_load4(rs, off + 16 * v);
  }
  __device__ __forceinline__ void store(float (*S)[MG_RP], int64_t c0, int64_t k0, int tid,
                                        f32x4 (&st)[NV]) const {
    const int kk = tid & 31, cb = CPT * (tid >> 5);
    if (Mask::kElem) {
#pragma unroll
      for (int e = 0; e < CPT; ++e)
        st[e >> 2][e & 3] = mask.elem(k0 + kk, c0 + cb + e) ? st[e >> 2][e & 3] : 0.0f;
    }
    const int off = (kk & 1) * MG_KP + (kk >> 1);
#pragma unroll
    for (int e = 0; e < CPT; ++e) S[cb + e][off] = st[e >> 2][e & 3];
  }
};

template <int NA>
__device__ __forceinline__ void mg_zero(f32x16 (&acc)[NA][NA]) {
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < NA; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;
}

// The MFMAs of one LDS chunk (16 k-pairs x NA x NA tiles), in k order.  Operands are
// read in 4 groups of 4 k-pairs (one ds_read_b128 per operand and group) with the next
// group's reads issued before the current group's MFMAs.  The wave owns rows
// wr*(32 NA) + 32a + ... and columns wcn*(32 NA) + 32b + ... of the workgroup tile.
template <int NA>
__device__ __forceinline__ void mg_chunk(f32x16 (&acc)[NA][NA], const float (*A)[MG_RP],
                                         const float (*B)[MG_RP], int wr, int wcn, int par,
                                         int lr) {
  const float* pa[NA];
  const float* pb[NA];
#pragma unroll
  for (int t = 0; t < NA; ++t) {
    pa[t] = &A[wr * 32 * NA + 32 * t + lr][par * MG_KP];
    pb[t] = &B[wcn * 32 * NA + 32 * t + lr][par * MG_KP];
  }
  f32x4 av[2][NA], bv[2][NA];  // [set][tile]
#pragma unroll
  for (int t = 0; t < NA; ++t) {
    av[0][t] = *reinterpret_cast<const f32x4*>(pa[t]);
    bv[0][t] = *reinterpret_cast<const f32x4*>(pb[t]);
  }
#pragma unroll
  for (int g = 0; g < MG_KP / 4; ++g) {
    const int cur = g & 1;
    if (g + 1 < MG_KP / 4) {
#pragma unroll
      for (int t = 0; t < NA; ++t) {
        av[cur ^ 1][t] = *reinterpret_cast<const f32x4*>(pa[t] + 4 * (g + 1));
        bv[cur ^ 1][t] = *reinterpret_cast<const f32x4*>(pb[t] + 4 * (g + 1));
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NA; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[cur][a][q], bv[cur][b][q],
                                                          acc[a][b], 0, 0, 0);
  }
}

// acc += A[r0:r0+T, kbeg:kend] * op(B)[kbeg:kend, c0:c0+T], rank chunks in order.
// kbeg must be a multiple of 2 (MFMA k-pairs); loaders zero everything beyond kend.
// Per chunk: the next chunk's global loads are issued first, the chunk's MFMAs run from
// LDS, and only then are the loaded values masked and written to the other LDS buffer.
template <int NA, int T, class AL, class BL>
__device__ __forceinline__ void mg_mainloop(f32x16 (&acc)[NA][NA], MgSmemT<T>& sm, const AL& al,
                                            const BL& bl, int64_t r0, int64_t c0,
                                            int64_t kbeg, int64_t kend) {
  static_assert(NA * 64 == T, "accumulators must cover the tile");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  if (kend <= kbeg) return;
  const int nch = (int)((kend - kbeg + MG_KC - 1) / MG_KC);
  f32x4 sa[AL::NV], sb[BL::NV];
  al.load(r0, kbeg, tid, sa);
  bl.load(c0, kbeg, tid, sb);
  __syncthreads();  // the previous use of the LDS buffers is over
  al.store(sm.A[0], r0, kbeg, tid, sa);
  bl.store(sm.B[0], c0, kbeg, tid, sb);
  __syncthreads();
  const int par = lane >> 5, lr = lane & 31;
  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    const int64_t kn = kbeg + (int64_t)(ch + 1) * MG_KC;
    const bool more = ch + 1 < nch;
    if (more) {
      al.load(r0, kn, tid, sa);
      bl.load(c0, kn, tid, sb);
    }
    mg_chunk<NA>(acc, sm.A[buf], sm.B[buf], wr, wcn, par, lr);
    __builtin_amdgcn_sched_barrier(0);
    if (more) {  // buffer buf ^ 1 was last read before the previous barrier
      al.store(sm.A[buf ^ 1], r0, kn, tid, sa);
      bl.store(sm.B[buf ^ 1], c0, kn, tid, sb);
    }
    __syncthreads();
  }
}

// The rank [kbeg, kend) as consecutive segments of SEG (a multiple of MG_KC), each
// accumulated from zero: after the MFMAs of a segment's last chunk, end(acc) consumes the
// segment's product and must leave acc zero again; pre() runs at the start of that last
// chunk, before its MFMAs (the place to issue the epilogue's global loads, so that they
// are in flight while the MFMAs run).  The next chunk's loads are issued before every
// chunk's MFMAs, across segment boundaries too, so only the first chunk's load latency
// is exposed.
// first() runs once, in the first chunk, before the second chunk's loads are issued (the
// place for loads the first segment's end needs: they are in flight during the first
// chunk's MFMAs instead of ahead of the first chunk's wait).
template <int NA, int T, int SEG, class AL, class BL, class Pre, class End, class First>
__device__ __forceinline__ void mg_mainloop_seg(f32x16 (&acc)[NA][NA], MgSmemT<T>& sm,
                                                const AL& al, const BL& bl, int64_t r0,
                                                int64_t c0, int64_t kbeg, int64_t kend,
                                                Pre pre, End end, First first) {
  static_assert(NA * 64 == T, "accumulators must cover the tile");
  static_assert(SEG % MG_KC == 0, "segments are whole chunks");
  constexpr int CPS = SEG / MG_KC;  // chunks per segment
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  if (kend <= kbeg) return;
  const int nch = (int)((kend - kbeg + MG_KC - 1) / MG_KC);
  f32x4 sa[AL::NV], sb[BL::NV];
  al.load(r0, kbeg, tid, sa);
  bl.load(c0, kbeg, tid, sb);
  __syncthreads();  // the previous use of the LDS buffers is over
  al.store(sm.A[0], r0, kbeg, tid, sa);
  bl.store(sm.B[0], c0, kbeg, tid, sb);
  __syncthreads();
  const int par = lane >> 5, lr = lane & 31;
  for (int ch = 0; ch < nch; ++ch) {
    const int buf = ch & 1;
    const int64_t kn = kbeg + (int64_t)(ch + 1) * MG_KC;
    const bool more = ch + 1 < nch;
    const bool seg_last = !more || (ch + 1) % CPS == 0;
    if (ch == 0) first();
    if (seg_last) pre();
    if (more) {
      al.load(r0, kn, tid, sa);
      bl.load(c0, kn, tid, sb);
    }
    mg_chunk<NA>(acc, sm.A[buf], sm.B[buf], wr, wcn, par, lr);
    __builtin_amdgcn_sched_barrier(0);
    if (seg_last) end(acc);
    if (more) {  // buffer buf ^ 1 was last read before the previous barrier
      al.store(sm.A[buf ^ 1], r0, kn, tid, sa);
      bl.store(sm.B[buf ^ 1], c0, kn, tid, sb);
    }
    __syncthreads();
  }
}

typedef __bf16 mg_bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short mg_u16x8 __attribute__((ext_vector_type(8)));

// Row / column of accumulator register j of tile (a, b) for this lane, relative to the
// workgroup tile origin.
template <int T = MG_T>
__device__ __forceinline__ int mg_row(int a, int j) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave >> 1) * (T / 2) + a * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
}
template <int T = MG_T>
__device__ __forceinline__ int mg_col(int b) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave & 1) * (T / 2) + b * 32 + (lane & 31);
}

// The T x T tile of a row-major [nrows, ncols] matrix at (r0, c0), accessed in the
// accumulator layout through a buffer resource that ends at the tile's last valid element:
// loads are branch-free (rows past the end read zero, columns past the end of rows before
// the last read real memory that is never stored back), stores drop every element the
// predicate rejects or that lies outside [nrows, ncols).
//
// Offsets are one per-lane base plus a uniform term per register; the base passes
// through an empty asm so the offsets are rebuilt at each access instead of being
// hoisted out of the caller's loops and held in registers across them.
template <int T = MG_T>
struct CTile {
  static constexpr int NA = T / 64;
  __amdgpu_buffer_rsrc_t rs;
  int64_t ld;
  uint32_t vbase;  // byte offset of this lane's (row 0, column 0) element
  int rows, cols;
  __device__ __forceinline__ CTile(float* p, int64_t ld_, int64_t nrows, int64_t ncols,
                                   int64_t r0, int64_t c0)
      : ld(ld_) {
    rows = (int)((nrows - r0 < T) ? nrows - r0 : T);
    cols = (int)((ncols - c0 < T) ? ncols - c0 : T);
    rs = mg_rsrc(p + r0 * ld + c0, (int64_t)(rows - 1) * ld + cols);
    vbase = (uint32_t)(((int64_t)mg_row<T>(0, 0) * ld + mg_col<T>(0)) * 4);
  }
  // byte offset of register j of tile (a, b) relative to vbase (uniform)
  __device__ __forceinline__ uint32_t uoff(int a, int b, int j) const {
    return (uint32_t)(((int64_t)(a * 32 + 8 * (j >> 2) + (j & 3)) * ld + b * 32) * 4);
  }
  __device__ __forceinline__ uint32_t base() const {
    uint32_t v = vbase;
    asm volatile("" : "+v"(v));
    return v;
  }
  __device__ __forceinline__ void load(f32x16 (&v)[NA][NA]) const {
    const uint32_t vb = base();
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < NA; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          v[a][b][j] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(vb + uoff(a, b, j)), 0, 0));
  }
  // keep(a, j, b): predicate for register j of tile (a, b) (rows and columns outside the
  // matrix are dropped regardless)
  template <class Keep>
  __device__ __forceinline__ void store(const f32x16 (&v)[NA][NA], Keep keep) const {
    const uint32_t vb = base();
#pragma unroll
    for (int b = 0; b < NA; ++b) {
      const bool cok = mg_col<T>(b) < cols;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t o = (cok && keep(a, j, b)) ? vb + uoff(a, b, j) : MG_OOB;
          // copy the element to a scalar first: this compiler's __builtin_bit_cast of a
          // vector-element lvalue reads element 0
          const float x = v[a][b][j];
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rs, (int)o, 0, 0);
        }
    }
  }
};

// Workgroup -> tile mapping that keeps neighbouring tiles on one XCD: workgroups are
// dispatched round-robin over the 8 XCDs, so linear id i runs on XCD i % 8; give XCD x
// the contiguous tile range [x * per, (x + 1) * per).
__device__ __forceinline__ int64_t xcd_tile(int64_t id, int64_t ntiles) {
  const int64_t per = (ntiles + 7) / 8;
  const int64_t t = (id % 8) * per + id / 8;
  return t < ntiles ? t : -1;
}

// Super-tile schedule for large grids: groups of 8 x 8 tiles (64 tiles, one per
// workgroup slot of an XCD at two workgroups per CU) go whole to one XCD, so the 8 row
// panels and 8 column panels they read are shared in that XCD's L2; groups are dealt to
// the 8 XCDs in turn, heaviest first.  ORDER says where the heavy tiles are (the rank
// of a triangular product grows along rows or columns):
//   0 uniform, 1 heaviest at the bottom rows, 2 at the right columns, 3 at the left.
// TRI enumerates only the lower triangle of a square grid (uniform work).
constexpr int MG_SUP = 8;  // super-tile edge (tiles)

__host__ __device__ inline int64_t mg_super_count(int64_t tm, int64_t tn, bool tri) {
  const int64_t nsr = (tm + MG_SUP - 1) / MG_SUP, nsc = (tn + MG_SUP - 1) / MG_SUP;
  return tri ? nsr * (nsr + 1) / 2 : nsr * nsc;
}

// workgroups to launch for the super-tile schedule (8 XCDs x 64 slots per group round)
__host__ inline int64_t mg_super_grid(int64_t tm, int64_t tn, bool tri) {
  const int64_t nsup = mg_super_count(tm, tn, tri);
  return (nsup + 7) / 8 * 8 * MG_SUP * MG_SUP;
}

// Balanced schedule: the host weighs every super-tile (the summed rank of its tiles plus
// a per-tile overhead) and deals them to the 8 XCDs longest-processing-time first (each
// to the least loaded XCD so far), so that no XCD ends long after the others.  Workgroup
// slot j * 64 + w of XCD x runs tile w of the XCD's j-th super-tile.
constexpr int MG_SCHED_MAX = 448;  // super-tiles a table holds (else round-robin)
struct MgSched {
  int32_t per_xcd = 0;                 // super-tiles of the busiest XCD (0: no table)
  int32_t nsc = 0;                     // super-tile columns
  int32_t sup = MG_SUP;                // super-tile edge (tiles)
  uint16_t st[MG_SCHED_MAX] = {};      // [x * per_xcd + j]: sr * nsc + sc, 0xffff: none
};

// weight(sr, sc) -> work of super-tile (sr, sc) (0: empty); super-tiles of sup x sup tiles
template <class Weight>
__host__ inline MgSched mg_balance(int64_t tm, int64_t tn, Weight weight, int sup = MG_SUP) {
  MgSched s;
  s.sup = sup;
  const int64_t nsr = (tm + sup - 1) / sup, nsc = (tn + sup - 1) / sup;
  std::vector<std::pair<double, int>> items;
  for (int64_t sr = 0; sr < nsr; ++sr)
    for (int64_t sc = 0; sc < nsc; ++sc) {
      const double w = weight(sr, sc);
      if (w > 0.0) items.push_back({w, (int)(sr * nsc + sc)});
    }
  if (items.empty() || (int64_t)items.size() > MG_SCHED_MAX || nsr * nsc > 0xffff) return s;
  std::stable_sort(items.begin(), items.end(),
                   [](const std::pair<double, int>& a, const std::pair<double, int>& b) {
                     return a.first > b.first;
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
  if ((int64_t)per * 8 > MG_SCHED_MAX) return s;
  s.per_xcd = per;
  s.nsc = (int)nsc;
  for (int x = 0; x < 8; ++x)
    for (int j = 0; j < per; ++j)
      s.st[x * per + j] = j < (int)lists[x].size() ? (uint16_t)lists[x][j] : (uint16_t)0xffff;
  return s;
}

__host__ inline int64_t mg_sched_grid(const MgSched& s) {
  return (int64_t)8 * s.per_xcd * s.sup * s.sup;
}

// SUP: the table's super-tile edge (MgSched::sup)
template <bool TRI, int SUP = MG_SUP>
__device__ __forceinline__ bool mg_sched_tile(int64_t bid, const MgSched& s, int64_t tm,
                                              int64_t tn, int64_t& tr, int64_t& tc) {
  const int x = (int)(bid & 7);
  const int64_t slot = bid >> 3;
  const int j = (int)(slot / (SUP * SUP)), w = (int)(slot % (SUP * SUP));
  if (j >= s.per_xcd) return false;
  const int u = s.st[x * s.per_xcd + j];
  if (u == 0xffff) return false;
  tr = (int64_t)(u / s.nsc) * SUP + w / SUP;
  tc = (int64_t)(u % s.nsc) * SUP + w % SUP;
  if (tr >= tm || tc >= tn) return false;
  if (TRI && tc > tr) return false;
  return true;
}

template <int ORDER, bool TRI>
__device__ __forceinline__ bool mg_super_tile(int64_t bid, int64_t tm, int64_t tn, int64_t& tr,
                                              int64_t& tc) {
  const int64_t x = bid & 7, slot = bid >> 3;
  const int64_t u = (slot / (MG_SUP * MG_SUP)) * 8 + x;  // super-tile, dealt round-robin
  const int w = (int)(slot % (MG_SUP * MG_SUP));
  const int64_t nsr = (tm + MG_SUP - 1) / MG_SUP, nsc = (tn + MG_SUP - 1) / MG_SUP;
  int64_t sr, sc;
  if (TRI) {
    if (u >= nsr * (nsr + 1) / 2) return false;
    sr = (int64_t)((sqrtf(8.0f * (float)u + 1.0f) - 1.0f) * 0.5f);
    while (sr * (sr + 1) / 2 > u) --sr;
    while ((sr + 1) * (sr + 2) / 2 <= u) ++sr;
    sc = u - sr * (sr + 1) / 2;
  } else {
    if (u >= nsr * nsc) return false;
    if (ORDER == 1) {
      sr = nsr - 1 - u / nsc;
      sc = u % nsc;
    } else if (ORDER == 2) {
      sc = nsc - 1 - u / nsr;
      sr = u % nsr;
    } else if (ORDER == 3) {
      sc = u / nsr;
      sr = u % nsr;
    } else {
      sr = u / nsc;
      sc = u % nsc;
    }
  }
  tr = sr * MG_SUP + w / MG_SUP;
  tc = sc * MG_SUP + w % MG_SUP;
  if (tr >= tm || tc >= tn) return false;
  if (TRI && tc > tr) return false;
  return true;
}

}  // namespace hi2x
