// Error reporting, version and kernel-timer entry points of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "internal.h"

namespace bioemu {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(BIOEMU_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return BIOEMU_OK;
}

// ---------------------------------------------------------------------------
// Kernel timer: when enabled, every launch made through a KernelTimerScope is
// bracketed by two hipEvents recorded on the launch stream.  Events come from
// a pool that only grows, so steady-state timing allocates nothing.
// ---------------------------------------------------------------------------
namespace {

struct TimerRecord {
  int name_idx;
  hipEvent_t start, stop;
};

struct TimerState {
  std::mutex mu;
  bool enabled = false;
  std::vector<std::string> names;
  std::vector<TimerRecord> records;  // pending (not yet folded into totals)
  std::vector<hipEvent_t> pool;      // free events
  std::vector<int64_t> launches;
  std::vector<double> total_ms;
};

TimerState& timer() {
  static TimerState* t = new TimerState();  // never destroyed: events outlive static teardown
  return *t;
}

int name_index(TimerState& t, const char* name) {
  for (size_t i = 0; i < t.names.size(); ++i)
    if (t.names[i] == name) return (int)i;
  t.names.emplace_back(name);
  t.launches.push_back(0);
  t.total_ms.push_back(0.0);
  return (int)t.names.size() - 1;
}

hipEvent_t take_event(TimerState& t) {
  if (!t.pool.empty()) {
    hipEvent_t e = t.pool.back();
    t.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Folds every pending record into the totals (synchronises on its events).
int drain(TimerState& t) {
  for (const TimerRecord& r : t.records) {
    float ms = 0.f;
    if (hipEventSynchronize(r.stop) != hipSuccess || hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
      return set_error(BIOEMU_ERR_LAUNCH, "kernel timer: event query failed");
    t.launches[r.name_idx] += 1;
    t.total_ms[r.name_idx] += ms;
    t.pool.push_back(r.start);
    t.pool.push_back(r.stop);
  }
  t.records.clear();
  return BIOEMU_OK;
}

}  // namespace

KernelTimerScope::KernelTimerScope(const char* name, hipStream_t stream) : stream_(stream) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  if (!t.enabled) return;
  name_idx_ = name_index(t, name);
  start_ = take_event(t);
  stop_ = take_event(t);
  if (!start_ || !stop_) {
    name_idx_ = -1;
    return;
  }
  (void)hipEventRecord(start_, stream_);
}

KernelTimerScope::~KernelTimerScope() {
  if (name_idx_ < 0) return;
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  (void)hipEventRecord(stop_, stream_);
  t.records.push_back({name_idx_, start_, stop_});
}

}  // namespace bioemu

using namespace bioemu;

extern "C" const char* bioemu_version(void) { return "bioemu2_mi355x 0.2 gfx950"; }

extern "C" const char* bioemu_last_error(void) { return bioemu::g_last_error; }

extern "C" int bioemu_timer_enable(int on) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  t.enabled = on != 0;
  return BIOEMU_OK;
}

extern "C" int bioemu_timer_reset(void) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  int rc = drain(t);
  for (size_t i = 0; i < t.names.size(); ++i) {
    t.launches[i] = 0;
    t.total_ms[i] = 0.0;
  }
  return rc;
}

extern "C" int bioemu_timer_count(void) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  return (int)t.names.size();
}

extern "C" int bioemu_timer_query(int idx, char* name, size_t name_len, int64_t* launches,
                                  double* total_ms) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  int rc = drain(t);
  if (rc) return rc;
  if (idx < 0 || (size_t)idx >= t.names.size())
    return set_error(BIOEMU_ERR_INVALID_ARG, "kernel timer: index %d out of range", idx);
  if (name && name_len) {
    strncpy(name, t.names[idx].c_str(), name_len - 1);
    name[name_len - 1] = '\0';
  }
  if (launches) *launches = t.launches[idx];
  if (total_ms) *total_ms = t.total_ms[idx];
  return BIOEMU_OK;
}
