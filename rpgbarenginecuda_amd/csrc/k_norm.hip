// RMSNorm and fused residual-add + RMSNorm.
//
// Reference numerics (src/kernels_gpu.cu:564-591): per row, the sum of squares
// is accumulated in double, scale = (float)(1.0 / sqrt(ss / n + eps)), and
// out = x * scale * w in fp32. Only the order of the double summation differs
// here (per-thread partials, a wave butterfly, then the two wave partials),
// which double rounding makes invisible after the cast to fp32 in all but
// astronomically rare rows.
//
// MI355X mapping, all HBM-bound (about 0.5 flop/byte):
//   * hidden rows with n % 512 == 0 (2048, 2560, ...): a 128-thread block (two
//     wave64) per row, thread t holding float4 chunks t, t+128, ... (U = n/512 of
//     them), so each load instruction of a wave covers 1 KiB of the row; the
//     activations stream with nontemporal hints, the weight row stays cached.
//     Measured at n = 2811 x 2048 over 28 rotated layers: 5.5 TB/s for the fused
//     add+norm vs 4.1 TB/s for a wave-per-row layout with plain accesses. The
//     fused add+norm with at least two rows per workgroup of a four-per-CU grid
//     runs persistent (AddRmsNormRowsKernel), the next row's loads in flight.
//   * rows with n % 256 == 0 otherwise: one wave64 per row, V = n/256 float4 per lane.
//   * head rows (n = 128): 8 lanes per row with the layout of head_row.h (the
//     one the RoPE fusion needs), 3-step butterfly, shared with the fused kernel.
//   * anything else (odd n, unaligned rows): a 256-thread block per row, two
//     passes, the second re-reading the row from cache.
#include <hip/hip_runtime.h>

#include <atomic>

#include "dev_util.h"
#include "head_row.h"
#include "kernels_gpu.h"
#include "launch.h"

namespace rpg {
namespace {

using dev::AddSquares;
using dev::Load4;
using dev::LoadStream4;
using dev::RmsScale;
using dev::ScaleMul;
using dev::Store4;
using dev::StoreStream4;

constexpr int kRowBlock = 128;   // threads per hidden row
constexpr int kMaxRowChunks = 8; // n up to 4096 in registers
constexpr int kBlock = 256;
constexpr int kMaxWaveChunks = 16;

// Sum over the two waves of a 128-thread block; every thread gets the total.
__device__ __forceinline__ double TwoWaveSum(double v) {
  __shared__ double part[kRowBlock / 64];
  v = dev::WaveSum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return part[0] + part[1];
}

// ---------------------------------------------------------------- 128 threads per row

template <int U>
__global__ __launch_bounds__(kRowBlock) void RmsNormRowBlockKernel(const float* x, const float* __restrict__ w,
                                                                   int64_t stride, float eps, float* out) {
  const int64_t row = blockIdx.x;
  const float* xr = x + row * stride + 4 * threadIdx.x;
  float4 v[U];
#pragma unroll
  for (int c = 0; c < U; ++c) v[c] = LoadStream4(xr + 4 * kRowBlock * c);
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < U; ++c) ss = AddSquares(ss, v[c]);
  const float scale = RmsScale(TwoWaveSum(ss), 4 * kRowBlock * U, eps);
  const float* wr = w + 4 * threadIdx.x;
  float* orow = out + row * stride + 4 * threadIdx.x;
#pragma unroll
  for (int c = 0; c < U; ++c) StoreStream4(orow + 4 * kRowBlock * c, ScaleMul(v[c], scale, Load4(wr + 4 * kRowBlock * c)));
}

template <int U>
__global__ __launch_bounds__(kRowBlock) void AddRmsNormRowBlockKernel(float* x, const float* __restrict__ d,
                                                                      const float* __restrict__ w, float eps,
                                                                      float* __restrict__ out) {
  constexpr int kN = 4 * kRowBlock * U;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kN + 4 * threadIdx.x;
  float4 v[U];
#pragma unroll
  for (int c = 0; c < U; ++c) {
    const float4 a = LoadStream4(x + base + 4 * kRowBlock * c);
    const float4 b = LoadStream4(d + base + 4 * kRowBlock * c);
    v[c] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
#pragma unroll
  for (int c = 0; c < U; ++c) StoreStream4(x + base + 4 * kRowBlock * c, v[c]);
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < U; ++c) ss = AddSquares(ss, v[c]);
  const float scale = RmsScale(TwoWaveSum(ss), kN, eps);
  const float* wr = w + 4 * threadIdx.x;
#pragma unroll
  for (int c = 0; c < U; ++c) {
    StoreStream4(out + base + 4 * kRowBlock * c, ScaleMul(v[c], scale, Load4(wr + 4 * kRowBlock * c)));
  }
}

// The same rows with a persistent grid of four workgroups per CU for prefill-sized
// launches: workgroup b takes rows b, b + G, ... (G = gridDim.x) and requests the
// next row's x and d before it stores and reduces the current one, so each
// workgroup's writes overlap its next reads; the weight row stays in registers.
// Every row goes through the same operations in the same order as in
// AddRmsNormRowBlockKernel (bit-identical). Measured in the prefill chain at
// n = 2811 (28 rotated layers): 16.03-16.05 against 16.26-16.27 us; grids that
// give the CUs unequal workgroup counts (896, 1152, 1408) took 17.3-17.7 us.
template <int U>
__global__ __launch_bounds__(kRowBlock) void AddRmsNormRowsKernel(float* x, const float* __restrict__ d,
                                                                  const float* __restrict__ w, int64_t n_rows,
                                                                  float eps, float* __restrict__ out) {
  constexpr int kN = 4 * kRowBlock * U;
  // wave partials, alternating between two slots: a wave writes slot p of row i + 2
  // only after the barrier of row i + 1, which the other wave reaches after it has
  // read slot p of row i
  __shared__ double part[2][kRowBlock / 64];
  const int tid = threadIdx.x;
  float4 wv[U], a[U], b[U];
#pragma unroll
  for (int c = 0; c < U; ++c) wv[c] = Load4(w + 4 * tid + 4 * kRowBlock * c);
  int64_t row = blockIdx.x;  // < n_rows: the grid never exceeds the rows
#pragma unroll
  for (int c = 0; c < U; ++c) {
    a[c] = LoadStream4(x + row * kN + 4 * tid + 4 * kRowBlock * c);
    b[c] = LoadStream4(d + row * kN + 4 * tid + 4 * kRowBlock * c);
  }
  int slot = 0;
  for (; row < n_rows; row += gridDim.x) {
    float4 v[U];
#pragma unroll
    for (int c = 0; c < U; ++c) v[c] = make_float4(a[c].x + b[c].x, a[c].y + b[c].y, a[c].z + b[c].z, a[c].w + b[c].w);
    const int64_t next = row + gridDim.x;
    if (next < n_rows) {  // uniform over the workgroup
#pragma unroll
      for (int c = 0; c < U; ++c) {
        a[c] = LoadStream4(x + next * kN + 4 * tid + 4 * kRowBlock * c);
        b[c] = LoadStream4(d + next * kN + 4 * tid + 4 * kRowBlock * c);
      }
    }
    const int64_t base = row * kN + 4 * tid;
#pragma unroll
    for (int c = 0; c < U; ++c) StoreStream4(x + base + 4 * kRowBlock * c, v[c]);
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < U; ++c) ss = AddSquares(ss, v[c]);
    ss = dev::WaveSum(ss);
    if ((tid & 63) == 0) part[slot][tid >> 6] = ss;
    __syncthreads();
    const float scale = RmsScale(part[slot][0] + part[slot][1], kN, eps);
    slot ^= 1;
#pragma unroll
    for (int c = 0; c < U; ++c) StoreStream4(out + base + 4 * kRowBlock * c, ScaleMul(v[c], scale, wv[c]));
  }
}

// ---------------------------------------------------------------- one wave per row

template <int V>
__global__ __launch_bounds__(kBlock) void RmsNormWaveKernel(const float* x, const float* __restrict__ w,
                                                            int64_t n_rows, int64_t stride, float eps, float* out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const float* xr = x + row * stride + 4 * lane;
  float4 v[V];
#pragma unroll
  for (int c = 0; c < V; ++c) v[c] = LoadStream4(xr + 256 * c);
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < V; ++c) ss = AddSquares(ss, v[c]);
  ss = dev::WaveSum(ss);
  const float scale = RmsScale(ss, 256 * V, eps);
  const float* wr = w + 4 * lane;
  float* orow = out + row * stride + 4 * lane;
#pragma unroll
  for (int c = 0; c < V; ++c) StoreStream4(orow + 256 * c, ScaleMul(v[c], scale, Load4(wr + 256 * c)));
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
    const float4 a = LoadStream4(x + base + 256 * c);
    const float4 b = LoadStream4(d + base + 256 * c);
    v[c] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
#pragma unroll
  for (int c = 0; c < V; ++c) StoreStream4(x + base + 256 * c, v[c]);
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < V; ++c) ss = AddSquares(ss, v[c]);
  ss = dev::WaveSum(ss);
  const float scale = RmsScale(ss, 256 * V, eps);
  const float* wr = w + 4 * lane;
#pragma unroll
  for (int c = 0; c < V; ++c) StoreStream4(out + base + 256 * c, ScaleMul(v[c], scale, Load4(wr + 256 * c)));
}

// ---------------------------------------------------------------- 8 lanes per 128-wide row

// Per-head q/k norm (n = 128): the same row routine as the fused q/k kernel.
__global__ __launch_bounds__(kBlock) void RmsNormHeadKernel(const float* x, const float* __restrict__ w,
                                                            int64_t n_rows, int64_t stride, float eps, float* out) {
  const int l = threadIdx.x % dev::kHeadLanes;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / dev::kHeadLanes) + threadIdx.x / dev::kHeadLanes;
  if (row >= n_rows) return;
  dev::HeadRow r = dev::LoadHeadRowStream(x + row * stride, l);
  dev::NormHeadRow(r, dev::LoadHeadVec(w, l), eps);
  dev::StoreHeadRowStream(out + row * stride, l, r);
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
  // Each thread re-reads and overwrites only the elements it read in pass 1.
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
  for (int64_t i = threadIdx.x; i < n; i += kBlock) orow[i] = (xr[i] * scale) * w[i];
}

// ---------------------------------------------------------------- dispatch

bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Runs Launcher<v> for a runtime v in [N, kMax]; false if v is out of range.
template <template <int> class Launcher, int kMax, int N = 1, typename... Args>
bool DispatchChunks(int v, Args... args) {
  if constexpr (N > kMax) {
    return false;
  } else {
    if (v == N) {
      Launcher<N>::Run(args...);
      return true;
    }
    return DispatchChunks<Launcher, kMax, N + 1>(v, args...);
  }
}

template <int U>
struct RmsNormRowBlockLauncher {
  static void Run(const float* x, const float* w, int64_t n_rows, int64_t stride, float eps, float* out) {
    RPG_CHECK(n_rows <= 0x7FFFFFFF, "too many rows: %lld", static_cast<long long>(n_rows));
    Launch("RmsNormRowBlockKernel", RmsNormRowBlockKernel<U>, dim3(static_cast<unsigned>(n_rows)), dim3(kRowBlock), x,
           w, stride, eps, out);
  }
};

// Compute units of the current device, queried once per device.
int CurrentDeviceCUs() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // 0: not queried yet
  int dev = 0;
  RPG_HIP_CHECK(hipGetDevice(&dev));
  int cus = dev >= 0 && dev < kMaxDevices ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (cus == 0) {
    RPG_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    RPG_CHECK(cus > 0, "device %d reports %d compute units", dev, cus);
    if (dev >= 0 && dev < kMaxDevices) cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// AddRmsNormRowsKernel takes launches with at least two rows per workgroup of its
// grid (four workgroups per CU); smaller ones run one workgroup per row.
constexpr int kRowsBlocksPerCu = 4;
constexpr int64_t kRowsMinRows = 2048;  // smaller launches skip the CU query (MI355X: 2 x 4 x 256 = 2048)

template <int U>
struct AddRmsNormRowBlockLauncher {
  static void Run(float* x, const float* d, const float* w, int64_t n_rows, float eps, float* out) {
    RPG_CHECK(n_rows <= 0x7FFFFFFF, "too many rows: %lld", static_cast<long long>(n_rows));
    if (n_rows >= kRowsMinRows) {
      const int64_t grid = int64_t{kRowsBlocksPerCu} * CurrentDeviceCUs();
      if (n_rows >= 2 * grid) {
        Launch("AddRmsNormRowsKernel", AddRmsNormRowsKernel<U>, dim3(static_cast<unsigned>(grid)), dim3(kRowBlock), x,
               d, w, n_rows, eps, out);
        return;
      }
    }
    Launch("AddRmsNormRowBlockKernel", AddRmsNormRowBlockKernel<U>, dim3(static_cast<unsigned>(n_rows)),
           dim3(kRowBlock), x, d, w, eps, out);
  }
};

template <int V>
struct RmsNormWaveLauncher {
  static void Run(const float* x, const float* w, int64_t n_rows, int64_t stride, float eps, float* out) {
    Launch("RmsNormWaveKernel", RmsNormWaveKernel<V>, dim3(GridFor(n_rows, kBlock / 64)), dim3(kBlock), x, w, n_rows,
           stride, eps, out);
  }
};

template <int V>
struct AddRmsNormWaveLauncher {
  static void Run(float* x, const float* d, const float* w, int64_t n_rows, float eps, float* out) {
    Launch("AddRmsNormWaveKernel", AddRmsNormWaveKernel<V>, dim3(GridFor(n_rows, kBlock / 64)), dim3(kBlock), x, d,
           w, n_rows, eps, out);
  }
};

}  // namespace

void GpuRmsNorm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, float eps,
                float* out) {
  RPG_CHECK(n > 0 && n_rows > 0 && stride >= n, "RMSNorm: n and n_rows have to be positive and stride at least n");
  RPG_CHECK(x != nullptr && w != nullptr && out != nullptr, "RmsNorm got a null pointer");
  const bool vec_ok = Aligned16(x) && Aligned16(w) && Aligned16(out) && stride % 4 == 0;
  if (vec_ok && n == 128) {
    Launch("RmsNormHeadKernel", RmsNormHeadKernel, dim3(GridFor(n_rows, kBlock / dev::kHeadLanes)), dim3(kBlock), x,
           w, n_rows,
           stride, eps, out);
    return;
  }
  if (vec_ok && n % 512 == 0 &&
      DispatchChunks<RmsNormRowBlockLauncher, kMaxRowChunks>(static_cast<int>(n / 512), x, w, n_rows, stride, eps,
                                                             out)) {
    return;
  }
  if (vec_ok && n % 256 == 0 &&
      DispatchChunks<RmsNormWaveLauncher, kMaxWaveChunks>(static_cast<int>(n / 256), x, w, n_rows, stride, eps,
                                                          out)) {
    return;
  }
  RPG_CHECK(n_rows <= 0x7FFFFFFF, "too many rows for RmsNorm: %lld", static_cast<long long>(n_rows));
  Launch("RmsNormRowKernel", RmsNormRowKernel, dim3(static_cast<unsigned>(n_rows)), dim3(kBlock), x, w, n, stride, eps,
         out);
}

void GpuAddRmsNorm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n, float eps, float* out) {
  RPG_CHECK(n > 0 && n_rows > 0, "invalid AddRmsNorm arguments");
  RPG_CHECK(x != nullptr && d != nullptr && w != nullptr && out != nullptr, "AddRmsNorm got a null pointer");
  RPG_CHECK(out != x && out != d, "AddRmsNorm: out must not alias x or d");
  const bool vec_ok = Aligned16(x) && Aligned16(d) && Aligned16(w) && Aligned16(out);
  if (vec_ok && n % 512 == 0 &&
      DispatchChunks<AddRmsNormRowBlockLauncher, kMaxRowChunks>(static_cast<int>(n / 512), x, d, w, n_rows, eps,
                                                                out)) {
    return;
  }
  if (vec_ok && n % 256 == 0 &&
      DispatchChunks<AddRmsNormWaveLauncher, kMaxWaveChunks>(static_cast<int>(n / 256), x, d, w, n_rows, eps, out)) {
    return;
  }
  RPG_CHECK(n_rows <= 0x7FFFFFFF, "too many rows for AddRmsNorm: %lld", static_cast<long long>(n_rows));
  Launch("AddRmsNormRowKernel", AddRmsNormRowKernel, dim3(static_cast<unsigned>(n_rows)), dim3(kBlock), x, d, w, n,
         eps, out);
}

}  // namespace rpg
