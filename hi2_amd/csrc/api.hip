// Library identity and error reporting of the hi2x C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "common.h"

namespace hi2x {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return HI2X_ELAUNCH;
  }
  return HI2X_OK;
}

// ---- launch timing ----------------------------------------------------------------------
// Process-wide record (measurement only; the encode path never reads it).
namespace {
struct Timed {
  int kind;
  double work;
  hipEvent_t e0, e1;
};
std::atomic<unsigned> g_timing_mask{0};
std::mutex g_timing_mu;
std::vector<Timed> g_timed;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
  {
    std::lock_guard<std::mutex> lk(g_timing_mu);
    if (!g_event_pool.empty()) {
      hipEvent_t e = g_event_pool.back();
      g_event_pool.pop_back();
      return e;
    }
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

LaunchTimer::LaunchTimer(int kind, double work, hipStream_t s) : kind_(kind), work_(work), s_(s) {
  if (kind < 0 || kind >= 32 || !(g_timing_mask.load(std::memory_order_relaxed) >> kind & 1u))
    return;
  e0_ = take_event();
  if (e0_ && hipEventRecord(e0_, s_) != hipSuccess) e0_ = nullptr;
}

LaunchTimer::~LaunchTimer() {
  if (!e0_) return;
  hipEvent_t e1 = take_event();
  if (!e1 || hipEventRecord(e1, s_) != hipSuccess) return;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timed.push_back(Timed{kind_, work_, e0_, e1});
}

// Streams marked as background (hi2x_stream_background): a short list, read on every
// launch that consults it, written rarely.
namespace {
std::mutex g_bg_mu;
std::vector<hipStream_t> g_bg;
}  // namespace

bool stream_background(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_bg_mu);
  for (hipStream_t b : g_bg)
    if (b == s) return true;
  return false;
}

}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_stream_background(void* stream, int background) {
  clear_error();
  const hipStream_t s = as_stream(stream);
  std::lock_guard<std::mutex> lk(g_bg_mu);
  auto it = std::find(g_bg.begin(), g_bg.end(), s);
  if (background && it == g_bg.end()) {
    HI2X_REQUIRE(g_bg.size() < 256, "stream_background: more than 256 background streams");
    g_bg.push_back(s);
  } else if (!background && it != g_bg.end()) {
    g_bg.erase(it);
  }
  return HI2X_OK;
}

extern "C" int hi2x_timing_enable(unsigned mask) {
  clear_error();
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (const Timed& t : g_timed) {  // forget earlier records (their events are reused)
    if (hipEventSynchronize(t.e1) != hipSuccess) {
      set_error("timing: event synchronisation failed");
      return HI2X_ELAUNCH;
    }
    g_event_pool.push_back(t.e0);
    g_event_pool.push_back(t.e1);
  }
  g_timed.clear();
  g_timing_mask.store(mask, std::memory_order_relaxed);
  return HI2X_OK;
}

extern "C" int hi2x_timing_query(int kind, int64_t* launches, double* ms, double* work) {
  clear_error();
  HI2X_REQUIRE(launches && ms && work, "timing_query: null output");
  std::lock_guard<std::mutex> lk(g_timing_mu);
  int64_t n = 0;
  double tot = 0.0, w = 0.0;
  for (const Timed& t : g_timed) {
    if (t.kind != kind) continue;
    float dt = 0.0f;
    HI2X_HIP(hipEventSynchronize(t.e1));
    HI2X_HIP(hipEventElapsedTime(&dt, t.e0, t.e1));
    ++n;
    tot += dt;
    w += t.work;
  }
  *launches = n;
  *ms = tot;
  *work = w;
  return HI2X_OK;
}

extern "C" int hi2x_version(void) { return 100; }

extern "C" const char* hi2x_last_error(void) { return hi2x::g_err; }
