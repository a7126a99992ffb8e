// Host-side helpers shared by the launchers: one-time set-up per device that
// is safe under concurrent callers.
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>

namespace moe {

constexpr int kMaxDevices = 64;

// Runs a set-up step (hipFuncSetAttribute, an occupancy query) once per device,
// the first time a launcher needs it on that device; concurrent first callers
// wait for the one running it. The step's result is kept and returned to every
// later caller on that device.
template <typename R>
struct PerDeviceOnce {
  std::once_flag flag[kMaxDevices];
  R value[kMaxDevices];

  template <typename F>
  bool get(F&& step, R& out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    std::call_once(flag[dev], [&] { value[dev] = step(); });
    out = value[dev];
    return true;
  }
};

}  // namespace moe
