// Element-wise operators: SwiGLU gate (silu(gate) * up), the residual add, and
// the streaming-copy probe used to calibrate bandwidth and HBM counters.
//
// Reference semantics:
//   SiluMul (src/kernels_gpu.cu:863-869): gate[i] = (v / (1.0f + expf(-v))) * up[i]
//   VecAdd  (src/kernels_gpu.cu:871-875): a[i] += b[i]
//
// MI355X mapping: pure streams (12 B per element), so each thread keeps kUnroll
// independent 128-bit loads per operand in flight; a block covers
// kBlock*kUnroll float4 with lane-contiguous addresses per load instruction.
// A scalar tail (n % 4) is handled by the first threads of block 0, and
// unaligned pointers take a grid-stride scalar kernel.
#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "kernels_gpu.h"

namespace rpg {
namespace {

using dev::Load4;
using dev::Store4;

constexpr int kBlock = 256;
constexpr int kUnroll = 4;

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__device__ __forceinline__ float Silu(float v) { return v / (1.0f + expf(-v)); }

struct SiluMulOp {
  __device__ __forceinline__ float operator()(float g, float u) const { return Silu(g) * u; }
};

struct AddOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};

// a[i] = op(a[i], b[i]) over n elements, a and b 16-byte aligned.
template <typename Op>
__global__ __launch_bounds__(kBlock) void BinaryVecKernel(float* a, const float* __restrict__ b, int64_t n4,
                                                          int64_t n, Op op) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
  float4 va[kUnroll];
  float4 vb[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * kBlock;
    if (i < n4) {
      va[u] = Load4(a + 4 * i);
      vb[u] = Load4(b + 4 * i);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * kBlock;
    if (i < n4) {
      Store4(a + 4 * i, make_float4(op(va[u].x, vb[u].x), op(va[u].y, vb[u].y), op(va[u].z, vb[u].z),
                                    op(va[u].w, vb[u].w)));
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const int64_t i = 4 * n4 + threadIdx.x;
    a[i] = op(a[i], b[i]);
  }
}

template <typename Op>
__global__ __launch_bounds__(kBlock) void BinaryScalarKernel(float* a, const float* b, int64_t n, Op op) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    a[i] = op(a[i], b[i]);
  }
}

template <typename Op>
void LaunchBinary(float* a, const float* b, int64_t n, Op op, const char* vec_name, const char* scalar_name) {
  if (Aligned16(a) && Aligned16(b)) {
    const int64_t n4 = n / 4;
    const int64_t per_block = static_cast<int64_t>(kBlock) * kUnroll;
    const int64_t blocks = n4 > 0 ? (n4 + per_block - 1) / per_block : 1;
    RPG_CHECK(blocks <= 0x7FFFFFFF, "grid dimension out of range: %lld", static_cast<long long>(blocks));
    BinaryVecKernel<Op><<<static_cast<unsigned>(blocks), kBlock, 0, EngineStream()>>>(a, b, n4, n, op);
    CheckLaunch(vec_name);
    return;
  }
  const int64_t blocks = (n + kBlock - 1) / kBlock;
  const unsigned grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
  BinaryScalarKernel<Op><<<grid, kBlock, 0, EngineStream()>>>(a, b, n, op);
  CheckLaunch(scalar_name);
}

__global__ __launch_bounds__(kBlock) void StreamCopyKernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                           int64_t n16) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
  float4 v[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * kBlock;
    if (i < n16) v[u] = src[i];
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + u * kBlock;
    if (i < n16) dst[i] = v[u];
  }
}

}  // namespace

void GpuSiluMulInPlace(float* gate_dev, const float* up_dev, int64_t n) {
  if (n <= 0) return;
  RPG_CHECK(gate_dev != nullptr && up_dev != nullptr, "SiluMul got a null pointer");
  LaunchBinary(gate_dev, up_dev, n, SiluMulOp{}, "SiluMulVecKernel", "SiluMulScalarKernel");
}

void GpuVecAddInPlace(float* a_dev, const float* b_dev, int64_t n) {
  if (n <= 0) return;
  RPG_CHECK(a_dev != nullptr && b_dev != nullptr, "VecAdd got a null pointer");
  LaunchBinary(a_dev, b_dev, n, AddOp{}, "VecAddVecKernel", "VecAddScalarKernel");
}

void GpuStreamCopy(const void* src, void* dst, int64_t bytes) {
  RPG_CHECK(bytes > 0 && bytes % 16 == 0, "stream copy size %lld must be a positive multiple of 16",
            static_cast<long long>(bytes));
  RPG_CHECK(Aligned16(src) && Aligned16(dst), "stream copy buffers must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  const int64_t per_block = static_cast<int64_t>(kBlock) * kUnroll;
  const int64_t blocks = (n16 + per_block - 1) / per_block;
  RPG_CHECK(blocks <= 0x7FFFFFFF, "grid dimension out of range: %lld", static_cast<long long>(blocks));
  StreamCopyKernel<<<static_cast<unsigned>(blocks), kBlock, 0, EngineStream()>>>(
      static_cast<const float4*>(src), static_cast<float4*>(dst), n16);
  CheckLaunch("StreamCopyKernel");
}

}  // namespace rpg
