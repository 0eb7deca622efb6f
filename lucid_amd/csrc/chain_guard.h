// Host side of the bounded chain waits (mfma.h: chain_wait_ticks, chain_error) for one
// library.  A word of pinned host memory, mapped into every device, receives the give-up
// flag of any chain wait; each chain entry point checks it first and reports an earlier
// give-up as LUCID_ECHAIN-style error (the launch that gave up produced invalid results).
// Per device, on its first chain call, the library writes the word's device address and
// the wait bound into its module globals.  The word is the only memory the library
// allocates (4 bytes of pinned host memory, once per process, on the first chain call).
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace chain_guard {

constexpr int kMaxDevices = 64;

struct State {
  std::mutex mu;
  int* host = nullptr;   // pinned, mapped
  int* dev = nullptr;    // its device address
  bool ready[kMaxDevices] = {};
  long long ticks[kMaxDevices] = {};
  double limit_s = 2.0;  // wait bound in seconds
};

inline State& state() {
  static State s;
  return s;
}

// Make the current device's module globals point at the flag and carry the bound.
// Returns 0 or a hipError_t; `what` names the failing call.
inline int setup(std::string* what) {
  State& s = state();
  std::lock_guard<std::mutex> lock(s.mu);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return *what = "hipGetDevice", (int)e;
  if (dev < 0 || dev >= kMaxDevices) return *what = "device index out of range", (int)hipErrorInvalidDevice;
  if (!s.host) {
    e = hipHostMalloc(reinterpret_cast<void**>(&s.host), sizeof(int), hipHostMallocMapped | hipHostMallocPortable);
    if (e != hipSuccess) return *what = "hipHostMalloc(chain flag)", (int)e;
    *s.host = 0;
    e = hipHostGetDevicePointer(reinterpret_cast<void**>(&s.dev), s.host, 0);
    if (e != hipSuccess) return *what = "hipHostGetDevicePointer(chain flag)", (int)e;
  }
  if (!s.ready[dev]) {
    int rate_khz = 0;
    e = hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess || rate_khz <= 0) rate_khz = 100000;  // the documented 100 MHz
    const long long ticks = (long long)(s.limit_s * 1000.0 * rate_khz);
    e = hipMemcpyToSymbol(HIP_SYMBOL(chain_error), &s.dev, sizeof(s.dev));
    if (e != hipSuccess) return *what = "hipMemcpyToSymbol(chain_error)", (int)e;
    e = hipMemcpyToSymbol(HIP_SYMBOL(chain_wait_ticks), &ticks, sizeof(ticks));
    if (e != hipSuccess) return *what = "hipMemcpyToSymbol(chain_wait_ticks)", (int)e;
    s.ticks[dev] = ticks;
    s.ready[dev] = true;
  }
  return 0;
}

// 1 if a chain wait gave up since the last check (and clear the flag), else 0.
inline int take_flag() {
  State& s = state();
  if (!s.host) return 0;
  const int f = __atomic_exchange_n(s.host, 0, __ATOMIC_ACQ_REL);
  return f != 0;
}

// New wait bound for every device (applied on each device's next chain call).
inline void set_limit(double seconds) {
  State& s = state();
  std::lock_guard<std::mutex> lock(s.mu);
  s.limit_s = seconds;
  for (bool& r : s.ready) r = false;
}

}  // namespace chain_guard
