// RMSNorm and fused residual-add + RMSNorm.
//
// Reference numerics (src/kernels_gpu.cu:564-591): per row, the sum of squares
// is accumulated in double, scale = (float)(1.0 / sqrt(ss / n + eps)), and
// out = x * scale * w in fp32. Only the order of the double summation differs
// here (lane-partial sums combined by a butterfly instead of a 128-thread
// strided sum and LDS tree); double rounding makes that invisible after the
// cast to fp32 in all but astronomically rare rows.
//
// MI355X mapping, all HBM-bound (about 0.5 flop/byte):
//   * hidden rows (n = 256*V, e.g. 2048 or 2560): one wave64 per row, each lane
//     holds V float4 (lane-contiguous 16-byte chunks, so every load instruction
//     covers 1 KiB of the row coalesced), a 6-step xor butterfly reduces in
//     registers; x is read exactly once from HBM, never re-read.
//   * head rows (n = 128): 16 lanes per row, lane L owning elements 4L..4L+3 and
//     64+4L..64+4L+3 (the layout the RoPE fusion needs), 4-step butterfly.
//   * anything else (odd n, unaligned rows): a 256-thread block per row, two
//     passes, the second pass re-reading the row from cache.
#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "kernels_gpu.h"

namespace rpg {
namespace {

using dev::AddSquares;
using dev::Load4;
using dev::RmsScale;
using dev::ScaleMul;
using dev::Store4;

constexpr int kBlock = 256;
constexpr int kMaxWaveChunks = 16;  // hidden rows up to 4096 floats stay in registers

// ---------------------------------------------------------------- one wave per row

template <int V>
__global__ __launch_bounds__(kBlock) void RmsNormWaveKernel(const float* x, const float* __restrict__ w,
                                                            int64_t n_rows, int64_t stride, float eps,
                                                            float* out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const float* xr = x + row * stride + 4 * lane;
  float4 v[V];
#pragma unroll
  for (int c = 0; c < V; ++c) v[c] = Load4(xr + 256 * c);
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < V; ++c) ss = AddSquares(ss, v[c]);
  ss = dev::WaveSum(ss);
  const float scale = RmsScale(ss, 256 * V, eps);
  const float* wr = w + 4 * lane;
  float* orow = out + row * stride + 4 * lane;
#pragma unroll
  for (int c = 0; c < V; ++c) Store4(orow + 256 * c, ScaleMul(v[c], scale, Load4(wr + 256 * c)));
}

template <int V>
__global__ __launch_bounds__(kBlock) void AddRmsNormWaveKernel(float* x, const float* __restrict__ d,
                                                               const float* __restrict__ w, int64_t n_rows,
                                                               float eps, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int64_t base = row * (256 * V) + 4 * lane;
  float4 v[V];
#pragma unroll
  for (int c = 0; c < V; ++c) {
    const float4 a = Load4(x + base + 256 * c);
    const float4 b = Load4(d + base + 256 * c);
    v[c] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
#pragma unroll
  for (int c = 0; c < V; ++c) Store4(x + base + 256 * c, v[c]);
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < V; ++c) ss = AddSquares(ss, v[c]);
  ss = dev::WaveSum(ss);
  const float scale = RmsScale(ss, 256 * V, eps);
  const float* wr = w + 4 * lane;
#pragma unroll
  for (int c = 0; c < V; ++c) Store4(out + base + 256 * c, ScaleMul(v[c], scale, Load4(wr + 256 * c)));
}

// ---------------------------------------------------------------- 16 lanes per 128-wide row

__global__ __launch_bounds__(kBlock) void RmsNormHeadKernel(const float* x, const float* __restrict__ w,
                                                            int64_t n_rows, int64_t stride, float eps,
                                                            float* out) {
  const int l = threadIdx.x & 15;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 16) + (threadIdx.x >> 4);
  if (row >= n_rows) return;
  const float* xr = x + row * stride;
  const float4 a = Load4(xr + 4 * l);
  const float4 b = Load4(xr + 64 + 4 * l);
  double ss = AddSquares(AddSquares(0.0, a), b);
  ss = dev::GroupSum<16>(ss);
  const float scale = RmsScale(ss, 128, eps);
  float* orow = out + row * stride;
  Store4(orow + 4 * l, ScaleMul(a, scale, Load4(w + 4 * l)));
  Store4(orow + 64 + 4 * l, ScaleMul(b, scale, Load4(w + 64 + 4 * l)));
}

// ---------------------------------------------------------------- generic fallback

// Block-wide double sum; all threads receive the result. Ends with a barrier
// after which every thread of the block has finished its reads of pass 1.
__device__ double BlockSum(double v) {
  __shared__ double part[kBlock / 64];
  v = dev::WaveSum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kBlock / 64; ++i) s += part[i];
  return s;
}

__global__ __launch_bounds__(kBlock) void RmsNormRowKernel(const float* x, const float* __restrict__ w, int64_t n,
                                                           int64_t stride, float eps, float* out) {
  const int64_t row = blockIdx.x;
  const float* xr = x + row * stride;
  double ss = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) {
    const double v = static_cast<double>(xr[i]);
    ss = fma(v, v, ss);
  }
  const float scale = RmsScale(BlockSum(ss), n, eps);
  float* orow = out + row * stride;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) orow[i] = (xr[i] * scale) * w[i];
}

__global__ __launch_bounds__(kBlock) void AddRmsNormRowKernel(float* x, const float* __restrict__ d,
                                                              const float* __restrict__ w, int64_t n, float eps,
                                                              float* __restrict__ out) {
  const int64_t row = blockIdx.x;
  float* xr = x + row * n;
  const float* dr = d + row * n;
  double ss = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) {
    const float s = xr[i] + dr[i];
    xr[i] = s;
    const double v = static_cast<double>(s);
    ss = fma(v, v, ss);
  }
  const float scale = RmsScale(BlockSum(ss), n, eps);
  float* orow = out + row * n;
  // Each thread re-reads only the elements it wrote itself in pass 1.
  for (int64_t i = threadIdx.x; i < n; i += kBlock) orow[i] = (xr[i] * scale) * w[i];
}

// ---------------------------------------------------------------- dispatch helpers

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <template <int> class Launcher, typename... Args>
bool DispatchChunks(int v, Args... args) {
  switch (v) {
#define RPG_CASE(N) \
  case N:           \
    Launcher<N>::Run(args...); \
    return true;
    RPG_CASE(1) RPG_CASE(2) RPG_CASE(3) RPG_CASE(4) RPG_CASE(5) RPG_CASE(6) RPG_CASE(7) RPG_CASE(8)
    RPG_CASE(9) RPG_CASE(10) RPG_CASE(11) RPG_CASE(12) RPG_CASE(13) RPG_CASE(14) RPG_CASE(15) RPG_CASE(16)
#undef RPG_CASE
    default:
      return false;
  }
}

template <int V>
struct RmsNormWaveLauncher {
  static void Run(const float* x, const float* w, int64_t n_rows, int64_t stride, float eps, float* out) {
    const unsigned grid = GridFor(n_rows, kBlock / 64);
    RmsNormWaveKernel<V><<<grid, kBlock, 0, EngineStream()>>>(x, w, n_rows, stride, eps, out);
  }
};

template <int V>
struct AddRmsNormWaveLauncher {
  static void Run(float* x, const float* d, const float* w, int64_t n_rows, float eps, float* out) {
    const unsigned grid = GridFor(n_rows, kBlock / 64);
    AddRmsNormWaveKernel<V><<<grid, kBlock, 0, EngineStream()>>>(x, d, w, n_rows, eps, out);
  }
};

}  // namespace

void GpuRmsNorm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, float eps,
                float* out) {
  RPG_CHECK(n > 0 && n_rows > 0 && stride >= n, "invalid RmsNorm arguments");
  RPG_CHECK(x != nullptr && w != nullptr && out != nullptr, "RmsNorm got a null pointer");
  const bool vec_ok = Aligned16(x) && Aligned16(w) && Aligned16(out) && stride % 4 == 0;
  if (vec_ok && n == 128) {
    RmsNormHeadKernel<<<GridFor(n_rows, kBlock / 16), kBlock, 0, EngineStream()>>>(x, w, n_rows, stride, eps,
                                                                                   out);
    CheckLaunch("RmsNormHeadKernel");
    return;
  }
  if (vec_ok && n % 256 == 0 && n / 256 <= kMaxWaveChunks &&
      DispatchChunks<RmsNormWaveLauncher>(static_cast<int>(n / 256), x, w, n_rows, stride, eps, out)) {
    CheckLaunch("RmsNormWaveKernel");
    return;
  }
  RPG_CHECK(n_rows <= 0x7FFFFFFF, "too many rows for RmsNorm: %lld", static_cast<long long>(n_rows));
  RmsNormRowKernel<<<static_cast<unsigned>(n_rows), kBlock, 0, EngineStream()>>>(x, w, n, stride, eps, out);
  CheckLaunch("RmsNormRowKernel");
}

void GpuAddRmsNorm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n, float eps, float* out) {
  RPG_CHECK(n > 0 && n_rows > 0, "invalid AddRmsNorm arguments");
  RPG_CHECK(x != nullptr && d != nullptr && w != nullptr && out != nullptr, "AddRmsNorm got a null pointer");
  RPG_CHECK(out != x && out != d, "AddRmsNorm: out must not alias x or d");
  const bool vec_ok = Aligned16(x) && Aligned16(d) && Aligned16(w) && Aligned16(out);
  if (vec_ok && n % 256 == 0 && n / 256 <= kMaxWaveChunks &&
      DispatchChunks<AddRmsNormWaveLauncher>(static_cast<int>(n / 256), x, d, w, n_rows, eps, out)) {
    CheckLaunch("AddRmsNormWaveKernel");
    return;
  }
  RPG_CHECK(n_rows <= 0x7FFFFFFF, "too many rows for AddRmsNorm: %lld", static_cast<long long>(n_rows));
  AddRmsNormRowKernel<<<static_cast<unsigned>(n_rows), kBlock, 0, EngineStream()>>>(x, d, w, n, eps, out);
  CheckLaunch("AddRmsNormRowKernel");
}

}  // namespace rpg
