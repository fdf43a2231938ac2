// Device runtime glue for the hot-path operators: HIP error -> rpg::Error,
// device-memory RAII, the process-wide engine stream, and the fixed-address
// pos0 scalar that lets position-dependent kernels be captured into a HIP graph.
//
// Interface follows the reference's runtime layer so the engine code that calls
// the operators keeps its shape:
//   DeviceBuffer            src/cuda_common.h:75-98
//   EngineStream            src/cuda_common.h:116,      src/cuda_common.cu:153-156
//   ScopedEngineStream      src/cuda_common.h:128-137
//   EnsureCaptureStream /
//   CaptureStream           src/cuda_common.h:120-123,  src/cuda_common.cu:158-184
//   PosStagingPtr / StagePos0 / StagePos0Cached / StreamIsCapturing
//                           src/cuda_common.h:153-175,  src/cuda_common.cu:186-223
//   QueryDevice / DescribeDevice
//                           src/cuda_common.h:38-56
//
// Difference that matters for performance: the reference stages pos0 into device
// memory with an 8-byte H2D copy before every RoPE / KV-write launch and the
// kernels always read it back. Here the eager path passes pos0 by value (no copy,
// no extra dependent read) and only a launch that is being captured into a graph
// gets the staging address, which the graph replay loop fills with StagePos0.
#ifndef RPG_AMD_HIP_COMMON_H_
#define RPG_AMD_HIP_COMMON_H_

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "common.h"

namespace rpg {

// ---------------------------------------------------------------- device query

struct DeviceInfo {
  bool available = false;
  std::string name;      // marketing name, e.g. "AMD Instinct MI355X"
  std::string arch;      // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
  int cu_count = 0;
  int clock_khz = 0;
  size_t total_mem = 0;
  size_t free_mem = 0;
  int runtime_version = 0;
  std::string reason;    // why available == false (never empty in that case)
};

// Never throws: one use is telling a CPU-only host why there is no device.
DeviceInfo QueryDevice(int index = 0);
std::string DescribeDevice(const DeviceInfo& d);

// ---------------------------------------------------------------- errors

[[noreturn]] void ThrowHipError(hipError_t err, const char* expr, const char* file, int line);

#define RPG_HIP_CHECK(expr)                                       \
  do {                                                            \
    hipError_t _rpg_e = (expr);                                   \
    if (_rpg_e != hipSuccess) {                                   \
      ::rpg::ThrowHipError(_rpg_e, #expr, __FILE__, __LINE__);    \
    }                                                             \
  } while (0)

// Called right after every kernel launch: a bad launch configuration is
// reported at the operator that caused it, not at the next synchronisation.
void CheckLaunch(const char* what);

// Blocks for a 1-D grid, with the grid-size range checked on the host.
unsigned GridFor(int64_t n, int threads);

// ---------------------------------------------------------------- device memory

class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t bytes) { Alloc(bytes); }
  ~DeviceBuffer() { Free(); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept;
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;

  void Alloc(size_t bytes);
  void Free();
  void Upload(const void* src, size_t bytes);
  void Download(void* dst, size_t bytes) const;

  void* data() { return ptr_; }
  const void* data() const { return ptr_; }
  size_t size() const { return bytes_; }
  bool empty() const { return ptr_ == nullptr; }

  // Non-owning view of `bytes` device bytes at `p` (a slice of an allocation
  // someone else owns, e.g. the model's weight arena): Free() forgets it.
  static DeviceBuffer View(void* p, size_t bytes);

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
  bool owned_ = true;
};

// ---------------------------------------------------------------- engine stream

// Stream every operator launches on. nullptr (the null stream) unless a
// ScopedEngineStream is active.
hipStream_t EngineStream();

// Lazily created dedicated stream for graph capture (the null stream cannot be
// captured). Creation is attempted once; false means it failed.
bool EnsureCaptureStream();
hipStream_t CaptureStream();

// Routes EngineStream() to `s` for the lifetime of the object (restored on
// unwind, so a throwing operator inside a capture window cannot leave the
// process launching on a dead stream).
class ScopedEngineStream {
 public:
  explicit ScopedEngineStream(hipStream_t s);
  ~ScopedEngineStream();
  ScopedEngineStream(const ScopedEngineStream&) = delete;
  ScopedEngineStream& operator=(const ScopedEngineStream&) = delete;

 private:
  hipStream_t prev_;
};

// Process-wide engine stream setter used by the C ABI (rpg_ops_set_stream).
void SetEngineStream(hipStream_t s);

// ---------------------------------------------------------------- pos0 staging

// Fixed device address holding the current pos0 (allocated on first use, never
// freed: the process owns it until exit).
int64_t* PosStagingPtr();
// Writes pos into the staging scalar on the engine stream; skipped while the
// engine stream is capturing (a captured copy would read a dead stack slot).
void StagePos0(int64_t pos);
bool StreamIsCapturing();
// StagePos0 with a host-side cache of the value currently in device memory.
int64_t* StagePos0Cached(int64_t pos);

// What a position-dependent kernel receives: the value itself on the eager
// path (dev == nullptr), or the staging address while capturing.
struct Pos0Arg {
  int64_t value;
  const int64_t* dev;
};
Pos0Arg Pos0ForLaunch(int64_t pos0);

// ---------------------------------------------------------------- launch profiling
//
// Kernel-execution timing with HIP events attached to the dispatches
// (hipExtLaunchKernel). ProfileStart(n) creates n event pairs (allocation
// happens here, never during the timed launches); each launch while active
// takes the next pair, until n are used. ProfileReport synchronises on the last
// event and returns per-kernel counts and durations as JSON:
//   {"<kernel>": {"count": c, "avg_us": a, "min_us": m, "max_us": M, "total_us": t}, ...}
struct LaunchTiming {
  hipEvent_t start;
  hipEvent_t stop;
};
void ProfileStart(int max_launches);
void ProfileStop();
std::string ProfileReport();
// Event pair for the next launch of `kernel_name`, or nullptr when profiling
// is off, exhausted, or the engine stream is being captured.
const LaunchTiming* NextLaunchTiming(const char* kernel_name);

}  // namespace rpg

#endif  // RPG_AMD_HIP_COMMON_H_
