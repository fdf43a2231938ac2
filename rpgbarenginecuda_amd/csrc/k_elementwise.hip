// Element-wise operators: SwiGLU gate (silu(gate) * up), the residual add, and
// the streaming copy / read / fill probes used to calibrate bandwidth and HBM
// counters.
//
// Reference semantics:
//   SiluMul (src/kernels_gpu.cu:863-869): gate[i] = (v / (1.0f + expf(-v))) * up[i]
//   VecAdd  (src/kernels_gpu.cu:871-875): a[i] += b[i]
//
// MI355X mapping: pure streams (12 B per element). Measured at the prefill size
// (17.3 M elements, 28 rotated buffer sets): one float4 per operand per thread,
// 512-thread blocks and nontemporal loads/stores reach ~6.2 TB/s, against
// ~4.9 TB/s for four float4 per thread with plain accesses -- many small
// independent waves keep more of HBM's channels busy than deep per-lane unrolls.
// SwiGLU's output stores are device-scope write-through (dev::StoreDeviceThrough4),
// ~2% faster again in the layer's kernel order.
// A scalar tail (n % 4) is handled by the first threads of block 0; unaligned
// pointers take a grid-stride scalar kernel.
#include <hip/hip_runtime.h>

#include <cstring>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"

namespace rpg {
namespace {

using dev::LoadStream4;
using dev::StoreStream4;

constexpr int kBlock = 512;

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

using dev::SiluMul;

// kThrough: the output goes out through a buffer resource bounded to the block's
// own span of gate (kBlock float4 at most), with device-scope write-through stores;
// otherwise with nontemporal global stores. Write-through pays off on prefill-sized
// launches and costs latency on a few blocks (decode at n = 1: 2.2 against 1.9 us),
// so the launcher picks it by size.
template <bool kThrough>
__global__ __launch_bounds__(kBlock) void SiluMulKernel(float* gate, const float* __restrict__ up, int64_t n4,
                                                        int64_t n) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBlock;
  const int64_t i = first + threadIdx.x;
  if (i < n4) {
    const float4 g = LoadStream4(gate + 4 * i);
    const float4 u = LoadStream4(up + 4 * i);
    const float4 y = make_float4(SiluMul(g.x, u.x), SiluMul(g.y, u.y), SiluMul(g.z, u.z), SiluMul(g.w, u.w));
    if constexpr (kThrough) {
      const int64_t span = n4 - first < kBlock ? n4 - first : kBlock;
      dev::StoreDeviceThrough4(dev::OutResource(gate + 4 * first, static_cast<uint32_t>(16 * span)), 16u * threadIdx.x, y);
    } else {
      StoreStream4(gate + 4 * i, y);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const int64_t j = 4 * n4 + threadIdx.x;
    gate[j] = SiluMul(gate[j], up[j]);
  }
}

__global__ __launch_bounds__(kBlock) void VecAddKernel(float* a, const float* __restrict__ b, int64_t n4, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < n4) {
    const float4 x = LoadStream4(a + 4 * i);
    const float4 y = LoadStream4(b + 4 * i);
    StoreStream4(a + 4 * i, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const int64_t j = 4 * n4 + threadIdx.x;
    a[j] = a[j] + b[j];
  }
}

__global__ __launch_bounds__(kBlock) void SiluMulScalarKernel(float* gate, const float* up, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    gate[i] = SiluMul(gate[i], up[i]);
  }
}

__global__ __launch_bounds__(kBlock) void VecAddScalarKernel(float* a, const float* b, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) a[i] = a[i] + b[i];
}

// The copy probe stores device-scope write-through (sc1 | nt), the fastest of the
// store policies measured for a back-to-back stream copy on MI355X (82 / 92 /
// 207 MB: 14.34 / 15.76 / 32.37 us against 14.92 / 16.46 / 33.37 us with
// nontemporal global stores, 15.72 / 17.38 / 35.80 us with plain ones), so the
// same-size ceilings are the best copy, not the one the ops happen to use.
__global__ __launch_bounds__(kBlock) void StreamCopyKernel(const float* __restrict__ src, float* __restrict__ dst,
                                                           int64_t n16) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBlock;
  const int64_t i = first + threadIdx.x;
  if (i < n16) {
    const int64_t span = n16 - first < kBlock ? n16 - first : kBlock;
    dev::StoreDeviceThrough4(dev::OutResource(dst + 4 * first, static_cast<uint32_t>(16 * span)), 16u * threadIdx.x,
                             LoadStream4(src + 4 * i));
  }
}

// Write-only probe: 256-thread blocks measured faster than 512 for pure writes
// (23 MB: 5.1 vs 5.7 us; 368 MB: 6.9 vs 6.3 TB/s).
constexpr int kFillBlock = 256;

__global__ __launch_bounds__(kFillBlock) void StreamFillKernel(float* __restrict__ dst, int64_t n16, float value) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kFillBlock + threadIdx.x;
  if (i < n16) StoreStream4(dst + 4 * i, make_float4(value, value, value, value));
}

// Read-only probe: each thread reads kReadUnroll float4 (the workgroup's span is
// contiguous, lane-strided by the block so every load instruction covers whole
// lines) and folds their bits with XOR. The fold is stored only when it equals
// `key`, which the caller chooses so that it does not occur: the loads stay live
// and the kernel writes nothing (the sink is at most one word).
constexpr int kReadBlock = 256;
constexpr int kReadUnroll = 4;

__global__ __launch_bounds__(kReadBlock) void StreamReadKernel(const float* __restrict__ src, int64_t n16,
                                                               uint32_t key, uint32_t* __restrict__ sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kReadBlock * kReadUnroll) + threadIdx.x;
  uint32_t fold = 0;
#pragma unroll
  for (int u = 0; u < kReadUnroll; ++u) {
    const int64_t i = base + static_cast<int64_t>(u) * kReadBlock;
    if (i < n16) {
      const float4 v = LoadStream4(src + 4 * i);
      fold ^= __float_as_uint(v.x) ^ __float_as_uint(v.y) ^ __float_as_uint(v.z) ^ __float_as_uint(v.w);
    }
  }
  if (fold == key) sink[0] = fold;
}

// Write-through output stores from this many elements up (64 blocks of kBlock
// float4): below it the launch is latency-bound and the write-through
// acknowledgement only lengthens it.
constexpr int64_t kThroughMinElems = int64_t{64} * kBlock * 4;

// Blocks for the vector kernels: at least one, so block 0 exists for the tail.
unsigned VecGrid(int64_t n4) { return n4 > 0 ? GridFor(n4, kBlock) : 1u; }

unsigned ScalarGrid(int64_t n) {
  const int64_t blocks = (n + kBlock - 1) / kBlock;
  return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

}  // namespace

void GpuSiluMulInPlace(float* gate_dev, const float* up_dev, int64_t n) {
  if (n <= 0) return;
  RPG_CHECK(gate_dev != nullptr && up_dev != nullptr, "SiluMul got a null pointer");
  if (Aligned16(gate_dev) && Aligned16(up_dev)) {
    Launch("SiluMulKernel", n >= kThroughMinElems ? SiluMulKernel<true> : SiluMulKernel<false>, dim3(VecGrid(n / 4)),
           dim3(kBlock), gate_dev, up_dev, n / 4, n);
  } else {
    Launch("SiluMulScalarKernel", SiluMulScalarKernel, dim3(ScalarGrid(n)), dim3(kBlock), gate_dev, up_dev, n);
  }
}

void GpuVecAddInPlace(float* a_dev, const float* b_dev, int64_t n) {
  if (n <= 0) return;
  RPG_CHECK(a_dev != nullptr && b_dev != nullptr, "VecAdd got a null pointer");
  if (Aligned16(a_dev) && Aligned16(b_dev)) {
    Launch("VecAddKernel", VecAddKernel, dim3(VecGrid(n / 4)), dim3(kBlock), a_dev, b_dev, n / 4, n);
  } else {
    Launch("VecAddScalarKernel", VecAddScalarKernel, dim3(ScalarGrid(n)), dim3(kBlock), a_dev, b_dev, n);
  }
}

void GpuStreamCopy(const void* src, void* dst, int64_t bytes) {
  RPG_CHECK(bytes > 0 && bytes % 16 == 0, "stream copy size %lld must be a positive multiple of 16",
            static_cast<long long>(bytes));
  RPG_CHECK(Aligned16(src) && Aligned16(dst), "stream copy buffers must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  Launch("StreamCopyKernel", StreamCopyKernel, dim3(GridFor(n16, kBlock)), dim3(kBlock),
         static_cast<const float*>(src), static_cast<float*>(dst), n16);
}

void GpuStreamRead(const void* src, int64_t bytes, uint32_t key, uint32_t* sink) {
  RPG_CHECK(bytes > 0 && bytes % 16 == 0, "stream read size %lld must be a positive multiple of 16",
            static_cast<long long>(bytes));
  RPG_CHECK(Aligned16(src) && sink != nullptr, "stream read needs a 16-byte aligned source and a sink word");
  const int64_t n16 = bytes / 16;
  Launch("StreamReadKernel", StreamReadKernel, dim3(GridFor(n16, kReadBlock * kReadUnroll)), dim3(kReadBlock),
         static_cast<const float*>(src), n16, key, sink);
}

void GpuStreamFill(void* dst, int64_t bytes, uint32_t pattern) {
  RPG_CHECK(bytes > 0 && bytes % 16 == 0, "stream fill size %lld must be a positive multiple of 16",
            static_cast<long long>(bytes));
  RPG_CHECK(Aligned16(dst), "stream fill buffer must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  float value;
  std::memcpy(&value, &pattern, sizeof(value));
  Launch("StreamFillKernel", StreamFillKernel, dim3(GridFor(n16, kFillBlock)), dim3(kFillBlock),
         static_cast<float*>(dst), n16, value);
}

}  // namespace rpg
