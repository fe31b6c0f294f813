// Shared helpers of the hi2x HIP library (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hi2x.h"

namespace hi2x {

// Thread-local last-error text (hi2x_last_error).
void set_error(const char* fmt, ...);
void clear_error();

// Status of the last launch on this thread: HI2X_OK or HI2X_ELAUNCH (message set).
int launch_status(const char* what);

// Whether the caller marked stream s as background (hi2x_stream_background): kernels of
// the many-workgroup GEMMs launched there hold more LDS per workgroup than they use, so
// fewer of them share a CU and latency-bound kernels of other streams find room.
bool stream_background(hipStream_t s);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// The cross-block update of gptq.hip on `s`, for other kernels' schedules:
//   wc[r, c] -= sum_k err1[r, 128 t + k] * U_g[i1 + 128 t + k, c]   (c in [c0, c1), t < nblk)
// each block's product a sequential fp32 FMA chain subtracted in block order.  When skip
// is not null the launch does nothing if *skip reads zero once it runs; its launches are
// timed under timing_kind.
int trailing_update(float* wc, int64_t n, int64_t k, int64_t i1, int nblk, const float* err1,
                    int64_t lde, int64_t c0, int64_t c1, const int32_t* row_grp,
                    const int64_t* u_ptrs, hipStream_t s, const unsigned long long* skip,
                    int timing_kind);

// Launch timing (hi2x_timing_enable): while the kind is enabled, a LaunchTimer brackets
// the launch it scopes with HIP events on the launch's stream and records its algorithmic
// work.  Construct it right before the launch, let it go out of scope right after.
class LaunchTimer {
 public:
  LaunchTimer(int kind, double work, hipStream_t s);
  ~LaunchTimer();
  LaunchTimer(const LaunchTimer&) = delete;
  LaunchTimer& operator=(const LaunchTimer&) = delete;

 private:
  int kind_;
  double work_;
  hipStream_t s_;
  hipEvent_t e0_ = nullptr;
};

}  // namespace hi2x

#define HI2X_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      hi2x::set_error(__VA_ARGS__);      \
      return HI2X_EINVAL;                \
    }                                    \
  } while (0)

#define HI2X_HIP(call)                                                        \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess) {                                                   \
      hi2x::set_error("%s: %s", #call, hipGetErrorString(e_));                \
      return HI2X_ELAUNCH;                                                    \
    }                                                                         \
  } while (0)

namespace hi2x {

// The caller's device workspace (checked for size and 256-byte alignment), or else a
// stream-ordered allocation of the library's own, released in stream order when the
// Workspace goes out of scope.  Callers that run work on several streams at once pass
// their own workspaces: blocks freed on one stream and reused on another make the
// allocator order the two streams.
struct Workspace {
  char* p = nullptr;
  bool owned = false;
  hipStream_t s = nullptr;
  ~Workspace() {
    if (owned && p) (void)hipFreeAsync(p, s);
  }
};

inline int take_workspace(Workspace& w, void* given, int64_t given_bytes, size_t need,
                          hipStream_t s, const char* what) {
  w.s = s;
  if (need == 0) return HI2X_OK;
  if (given) {
    HI2X_REQUIRE(given_bytes >= (int64_t)need, "%s: workspace of %lld bytes, %lld needed", what,
                 (long long)given_bytes, (long long)need);
    HI2X_REQUIRE(((uintptr_t)given & 255) == 0, "%s: workspace not 256-byte aligned", what);
    w.p = static_cast<char*>(given);
    return HI2X_OK;
  }
  HI2X_HIP(hipMallocAsync((void**)&w.p, need, s));
  w.owned = true;
  return HI2X_OK;
}

}  // namespace hi2x

// ---- device helpers ------------------------------------------------------------------

// fp32 -> fp16 -> fp32 with round-to-nearest-even (torch's .to(float16).float()).
__device__ __forceinline__ float f16_round(float x) { return (float)(_Float16)x; }

__device__ __forceinline__ uint16_t f16_bits(float x) {
  _Float16 h = (_Float16)x;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_from_bits(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

#include "divrcp.h"

// torch.clamp(q, 0, n - 1): NaN propagates through both compares.
__device__ __forceinline__ float clamp_code(float q, float nm) {
  q = (q < 0.0f) ? 0.0f : q;
  q = (q > nm) ? nm : q;
  return q;
}

// Sum of x[0..B) in torch's CPU order for a contiguous inner reduction of B <= 64
// floats (8 vector lanes, 4 vector accumulators; the cascade needs >= 16 rows of 4
// vectors, i.e. B >= 512, so it never triggers here).  fn(t) yields x[t].
template <int B, class F>
__device__ __forceinline__ float torch_sum_small(F fn) {
  static_assert(B % 8 == 0 && B <= 64, "block size");
  constexpr int VS = B / 8;   // vectors
  constexpr int SI = VS / 4;  // rows of 4 vectors
  float p[4][8];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int v = 0; v < 8; ++v) p[k][v] = 0.0f;
#pragma unroll
  for (int i = 0; i < SI; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int v = 0; v < 8; ++v) p[k][v] += fn((i * 4 + k) * 8 + v);
#pragma unroll
  for (int i = SI * 4; i < VS; ++i)
#pragma unroll
    for (int v = 0; v < 8; ++v) p[0][v] += fn(i * 8 + v);
#pragma unroll
  for (int k = 1; k < 4; ++k)
#pragma unroll
    for (int v = 0; v < 8; ++v) p[0][v] += p[k][v];
  float out = 0.0f;
#pragma unroll
  for (int v = 0; v < 8; ++v) out += p[0][v];
  return out;
}

