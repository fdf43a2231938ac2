// Host-side implementation of the device runtime glue (see hip_common.h).
#include "hip_common.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <climits>
#include <cstdio>
#include <string>
#include <utility>
#include <vector>

namespace rpg {

void ThrowHipError(hipError_t err, const char* expr, const char* file, int line) {
  Throw("%s:%d: %s returned %s (HIP error %d)", file, line, expr, hipGetErrorString(err), static_cast<int>(err));
}

void CheckLaunch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) Throw("%s: the kernel launch reported %s", what, hipGetErrorString(e));
}

unsigned GridFor(int64_t n, int threads) {
  const int64_t g = (n + threads - 1) / threads;
  RPG_CHECK(g > 0 && g <= 0x7FFFFFFF, "launch grid of %lld workgroups does not fit a grid dimension",
            static_cast<long long>(g));
  return static_cast<unsigned>(g);
}

// ---------------------------------------------------------------- device query

DeviceInfo QueryDevice(int index) {
  DeviceInfo d;
  auto fail = [&d](std::string why) {
    d.reason = std::move(why);
    return d;
  };
  int count = 0;
  if (const hipError_t e = hipGetDeviceCount(&count); e != hipSuccess) {
    return fail(std::string("the HIP runtime reports no usable GPU (") + hipGetErrorString(e) + ")");
  }
  if (count <= 0) return fail("the HIP runtime sees no GPU");
  if (index < 0 || index >= count) {
    return fail("GPU " + std::to_string(index) + " requested, visible GPUs are 0.." + std::to_string(count - 1));
  }
  hipDeviceProp_t p{};
  if (const hipError_t e = hipGetDeviceProperties(&p, index); e != hipSuccess) {
    return fail("cannot read the properties of GPU " + std::to_string(index) + " (" + hipGetErrorString(e) + ")");
  }
  d.available = true;
  d.name = p.name;
  d.arch = p.gcnArchName;
  d.cu_count = p.multiProcessorCount;
  d.clock_khz = p.clockRate;
  d.total_mem = p.totalGlobalMem;
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) == hipSuccess) {
    d.free_mem = free_b;
    if (total_b > 0) d.total_mem = total_b;
  }
  int rt = 0;
  if (hipRuntimeGetVersion(&rt) == hipSuccess) d.runtime_version = rt;
  return d;
}

std::string DescribeDevice(const DeviceInfo& d) {
  if (!d.available) return "no device: " + d.reason;
  char buf[384];
  std::snprintf(buf, sizeof(buf), "%s [%s], %d CUs @ %d MHz, %.1f GiB (%.1f GiB free), HIP runtime %d",
                d.name.c_str(), d.arch.c_str(), d.cu_count, d.clock_khz / 1000,
                static_cast<double>(d.total_mem) / 1073741824.0,
                static_cast<double>(d.free_mem) / 1073741824.0, d.runtime_version);
  return std::string(buf);
}

// ---------------------------------------------------------------- DeviceBuffer

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_), owned_(o.owned_) {
  o.ptr_ = nullptr;
  o.bytes_ = 0;
  o.owned_ = true;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
  if (this != &o) {
    Free();
    ptr_ = o.ptr_;
    bytes_ = o.bytes_;
    owned_ = o.owned_;
    o.ptr_ = nullptr;
    o.bytes_ = 0;
    o.owned_ = true;
  }
  return *this;
}

DeviceBuffer DeviceBuffer::View(void* p, size_t bytes) {
  DeviceBuffer b;
  b.ptr_ = p;
  b.bytes_ = bytes;
  b.owned_ = false;
  return b;
}

void DeviceBuffer::Alloc(size_t bytes) {
  RPG_CHECK(bytes > 0, "DeviceBuffer: refusing a zero-byte allocation");
  Free();
  RPG_HIP_CHECK(hipMalloc(&ptr_, bytes));
  bytes_ = bytes;
  owned_ = true;
}

void DeviceBuffer::Free() {
  if (ptr_ == nullptr) return;
  if (owned_) {
    // Destructors must not throw; a failing free only happens once the runtime
    // is already tearing down.
    const hipError_t e = hipFree(ptr_);
    if (e != hipSuccess) RPG_LOG_WARN("hipFree failed: %s", hipGetErrorString(e));
  }
  ptr_ = nullptr;
  bytes_ = 0;
  owned_ = true;
}

void DeviceBuffer::Upload(const void* src, size_t bytes) {
  RPG_CHECK(ptr_ != nullptr, "DeviceBuffer::Upload on an unallocated buffer");
  RPG_CHECK(bytes <= bytes_, "DeviceBuffer::Upload overflow: %llu bytes into %llu",
            static_cast<unsigned long long>(bytes), static_cast<unsigned long long>(bytes_));
  RPG_HIP_CHECK(hipMemcpy(ptr_, src, bytes, hipMemcpyHostToDevice));
}

void DeviceBuffer::Download(void* dst, size_t bytes) const {
  RPG_CHECK(ptr_ != nullptr, "DeviceBuffer::Download on an unallocated buffer");
  RPG_CHECK(bytes <= bytes_, "DeviceBuffer::Download overflow: %llu bytes from %llu",
            static_cast<unsigned long long>(bytes), static_cast<unsigned long long>(bytes_));
  RPG_HIP_CHECK(hipMemcpy(dst, ptr_, bytes, hipMemcpyDeviceToHost));
}

// ---------------------------------------------------------------- engine stream
//
// Process-lifetime objects, intentionally never released: their release would
// run from static destructors after the runtime may already be gone.
namespace {

int64_t* g_pos_staging = nullptr;
hipStream_t g_engine_stream = nullptr;
hipStream_t g_capture_stream = nullptr;
bool g_capture_tried = false;
// Value currently held by g_pos_staging, maintained only by StagePos0.
int64_t g_pos_last = INT64_MIN;

}  // namespace

hipStream_t EngineStream() { return g_engine_stream; }

void SetEngineStream(hipStream_t s) { g_engine_stream = s; }

bool EnsureCaptureStream() {
  if (g_capture_tried) return g_capture_stream != nullptr;
  g_capture_tried = true;
  // Blocking stream at the default priority: it stays ordered with the
  // synchronous copies that go through the null stream.
  if (hipStreamCreate(&g_capture_stream) != hipSuccess) {
    g_capture_stream = nullptr;
    return false;
  }
  return true;
}

hipStream_t CaptureStream() { return EnsureCaptureStream() ? g_capture_stream : nullptr; }

ScopedEngineStream::ScopedEngineStream(hipStream_t s) : prev_(g_engine_stream) { g_engine_stream = s; }

ScopedEngineStream::~ScopedEngineStream() { g_engine_stream = prev_; }

// ---------------------------------------------------------------- pos0 staging
//
// The staging scalar is one int64 of device memory at a fixed address. A
// captured launch reads that address on every replay; the host writes the
// position for the next replay through StagePos0. g_pos_last mirrors what the
// last completed-or-queued write put there, so StagePos0Cached can skip a copy
// of an unchanged value. Nothing is written while the engine stream captures:
// a captured host-to-device copy would keep reading the caller's (dead) stack
// slot on replay, and the address, not the value, is what the graph needs.

int64_t* PosStagingPtr() {
  if (g_pos_staging != nullptr) return g_pos_staging;
  void* p = nullptr;
  RPG_HIP_CHECK(hipMalloc(&p, sizeof(int64_t)));
  g_pos_staging = static_cast<int64_t*>(p);
  return g_pos_staging;
}

bool StreamIsCapturing() {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(EngineStream(), &st) != hipSuccess) {
    (void)hipGetLastError();  // a failed query counts as "not capturing"; the sticky error is cleared
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

namespace {

// Writes pos into the staging scalar unless capturing (or, with skip_same,
// unless it already holds pos). The source is pageable host memory, which the
// runtime copies out before the call returns.
int64_t* StagePos(int64_t pos, bool skip_same) {
  int64_t* dev = PosStagingPtr();
  if (StreamIsCapturing() || (skip_same && g_pos_last == pos)) return dev;
  RPG_HIP_CHECK(hipMemcpyAsync(dev, &pos, sizeof(pos), hipMemcpyHostToDevice, EngineStream()));
  g_pos_last = pos;
  return dev;
}

}  // namespace

void StagePos0(int64_t pos) { (void)StagePos(pos, false); }

int64_t* StagePos0Cached(int64_t pos) { return StagePos(pos, true); }

// ---------------------------------------------------------------- launch profiling

namespace {

struct ProfileState {
  std::vector<LaunchTiming> pairs;
  std::vector<const char*> names;  // kernel names are string literals
  size_t used = 0;
  bool active = false;
};

ProfileState& Prof() {
  static ProfileState s;  // never destroyed before the runtime: events are leaked at exit on purpose
  return s;
}

}  // namespace

void ProfileStart(int max_launches) {
  RPG_CHECK(max_launches > 0 && max_launches <= (1 << 20), "profile capacity %d out of range", max_launches);
  ProfileState& s = Prof();
  while (s.pairs.size() < static_cast<size_t>(max_launches)) {
    LaunchTiming t{};
    RPG_HIP_CHECK(hipEventCreate(&t.start));
    RPG_HIP_CHECK(hipEventCreate(&t.stop));
    s.pairs.push_back(t);
  }
  s.names.assign(static_cast<size_t>(max_launches), nullptr);
  s.used = 0;
  s.active = true;
}

void ProfileStop() { Prof().active = false; }

const LaunchTiming* NextLaunchTiming(const char* kernel_name) {
  ProfileState& s = Prof();
  if (!s.active || s.used >= s.names.size()) return nullptr;
  if (StreamIsCapturing()) return nullptr;
  s.names[s.used] = kernel_name;
  return &s.pairs[s.used++];
}

std::string ProfileReport() {
  ProfileState& s = Prof();
  struct Agg {
    int count = 0;
    double total = 0, mn = 1e30, mx = 0;
  };
  std::vector<std::pair<std::string, Agg>> aggs;
  if (s.used > 0) RPG_HIP_CHECK(hipEventSynchronize(s.pairs[s.used - 1].stop));
  for (size_t i = 0; i < s.used; ++i) {
    float ms = 0.f;
    RPG_HIP_CHECK(hipEventElapsedTime(&ms, s.pairs[i].start, s.pairs[i].stop));
    const double us = 1e3 * static_cast<double>(ms);
    auto it = std::find_if(aggs.begin(), aggs.end(), [&](const auto& a) { return a.first == s.names[i]; });
    if (it == aggs.end()) {
      aggs.emplace_back(s.names[i], Agg{});
      it = aggs.end() - 1;
    }
    Agg& a = it->second;
    ++a.count;
    a.total += us;
    a.mn = std::min(a.mn, us);
    a.mx = std::max(a.mx, us);
  }
  std::string out = "{";
  char buf[320];
  for (size_t i = 0; i < aggs.size(); ++i) {
    const Agg& a = aggs[i].second;
    std::snprintf(buf, sizeof(buf),
                  "%s\"%s\": {\"count\": %d, \"avg_us\": %.4f, \"min_us\": %.4f, \"max_us\": %.4f, \"total_us\": %.4f}",
                  i ? ", " : "", aggs[i].first.c_str(), a.count, a.total / a.count, a.mn, a.mx, a.total);
    out += buf;
  }
  return out + "}";
}

Pos0Arg Pos0ForLaunch(int64_t pos0) {
  if (StreamIsCapturing()) {
    // The staging scalar must already exist: allocating inside a capture is illegal.
    RPG_CHECK(g_pos_staging != nullptr,
              "pos0 staging scalar not allocated before graph capture; call PosStagingPtr() "
              "(rpg_ops_init) before beginning the capture");
    return Pos0Arg{pos0, g_pos_staging};
  }
  return Pos0Arg{pos0, nullptr};
}

}  // namespace rpg
