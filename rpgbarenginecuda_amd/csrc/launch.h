// Kernel launch helper shared by the .hip translation units.
//
// Every operator launches through Launch(): on the engine stream, followed by
// CheckLaunch, and -- while launch profiling is on (ProfileStart) and the stream
// is not being captured -- through hipExtLaunchKernel with a start/stop event
// pair attached to the dispatch itself, so the measured interval is the
// kernel's execution, not the host's launch latency.
#ifndef RPG_AMD_LAUNCH_H_
#define RPG_AMD_LAUNCH_H_

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <tuple>

#include "hip_common.h"

namespace rpg {

// The same with `shmem` bytes of dynamic LDS.
template <typename... KArgs, typename... Args>
inline void LaunchShared(const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem,
                         Args... args) {
  static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count mismatch");
  const LaunchTiming* timing = NextLaunchTiming(name);
  if (timing == nullptr) {
    kernel<<<grid, block, shmem, EngineStream()>>>(static_cast<KArgs>(args)...);
  } else {
    std::tuple<KArgs...> values{static_cast<KArgs>(args)...};
    void* ptrs[sizeof...(KArgs)];
    std::apply(
        [&ptrs](auto&... v) {
          size_t i = 0;
          ((ptrs[i++] = static_cast<void*>(&v)), ...);
        },
        values);
    RPG_HIP_CHECK(hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, shmem, EngineStream(),
                                     timing->start, timing->stop, 0));
  }
  CheckLaunch(name);
}

template <typename... KArgs, typename... Args>
inline void Launch(const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block, Args... args) {
  LaunchShared(name, kernel, grid, block, 0, args...);
}

}  // namespace rpg

#endif  // RPG_AMD_LAUNCH_H_
