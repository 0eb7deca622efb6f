// Optional per-kernel timing with HIP events recorded on the launch stream around
// every kernel (enabled by the library's *_profile_enable entry point).  Used by
// bench.py to time the dominant kernel inside the timed region.  Each shared
// library that includes this header keeps its own records.  Not thread safe.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace lucid_prof {

struct Rec {
  const char* name;
  hipEvent_t a, b;
};

inline bool& enabled() {
  static bool on = false;
  return on;
}
// Optional filter: when not empty, only launches of the kernel with this name are timed
// (so that a timed region carries the events of one kernel, not two per launch).
inline std::string& only() {
  static std::string s;
  return s;
}
inline bool wanted(const char* name) { return enabled() && (only().empty() || only() == name); }
inline std::vector<Rec>& records() {
  static std::vector<Rec> r;
  return r;
}
inline std::vector<hipEvent_t>& pool() {
  static std::vector<hipEvent_t> p;
  return p;
}
inline std::map<std::string, std::pair<double, long>>& totals() {
  static std::map<std::string, std::pair<double, long>> t;
  return t;
}

inline hipEvent_t pool_event() {
  auto& p = pool();
  if (!p.empty()) {
    hipEvent_t e = p.back();
    p.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// folds recorded events into totals; returns the number of kernels or -1
inline int collect() {
  for (auto& r : records()) {
    if (hipEventSynchronize(r.b) != hipSuccess) return -1;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return -1;
    auto& t = totals()[r.name];
    t.first += ms;
    t.second += 1;
    pool().push_back(r.a);
    pool().push_back(r.b);
  }
  records().clear();
  return (int)totals().size();
}

inline int entry(int idx, char* name, int name_len, double* total_ms, long* count) {
  int i = 0;
  for (auto& kv : totals()) {
    if (i++ != idx) continue;
    if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", kv.first.c_str());
    if (total_ms) *total_ms = kv.second.first;
    if (count) *count = kv.second.second;
    return 0;
  }
  return 1;
}

inline void reset() {
  collect();
  totals().clear();
}

}  // namespace lucid_prof

// Launch KERNEL on ST with BLOCK threads (LUCID_TIMED_LAUNCH: 256); on failure return the
// status from the enclosing function (STATUS_FN(name) must yield an int, 0 = ok).
#define LUCID_TIMED_LAUNCH_B(STATUS_FN, NAME, KERNEL, GRID, BLOCK, ST, ...)\
  do {                                                                     \
    hipEvent_t ev_a = nullptr, ev_b = nullptr;                             \
    if (lucid_prof::wanted(NAME)) {                                        \
      ev_a = lucid_prof::pool_event();                                     \
      ev_b = lucid_prof::pool_event();                                     \
      if (!ev_a || !ev_b || hipEventRecord(ev_a, ST) != hipSuccess)        \
        ev_a = nullptr;                                                    \
    }                                                                      \
    hipLaunchKernelGGL(KERNEL, GRID, BLOCK, 0, ST, __VA_ARGS__);            \
    if (int rc_ = STATUS_FN(NAME)) return rc_;                             \
    if (ev_a && hipEventRecord(ev_b, ST) == hipSuccess)                    \
      lucid_prof::records().push_back(lucid_prof::Rec{NAME, ev_a, ev_b});  \
  } while (0)
#define LUCID_TIMED_LAUNCH(STATUS_FN, NAME, KERNEL, GRID, ST, ...) \
  LUCID_TIMED_LAUNCH_B(STATUS_FN, NAME, KERNEL, GRID, dim3(256), ST, __VA_ARGS__)
