// Device helpers shared by the hot-path kernels (included only by .hip files).
//
// Everything here is written for CDNA4 wave64: reductions run over the 64 lanes
// of a wavefront (or over an aligned 16-lane group of it) with cross-lane
// shuffles, never through LDS, and all activation traffic moves as 128-bit
// float4 loads/stores.
#ifndef RPG_AMD_DEV_UTIL_H_
#define RPG_AMD_DEV_UTIL_H_

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rpg {
namespace dev {

constexpr int kWave = 64;

// ---------------------------------------------------------------- reductions

// Sum over all 64 lanes of the wave; every lane receives the total.
__device__ __forceinline__ double WaveSum(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over the aligned group of W lanes (W a power of two <= 64) that contains
// the calling lane; every lane of the group receives the group total.
template <int W>
__device__ __forceinline__ double GroupSum(double v) {
#pragma unroll
  for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, W);
  return v;
}

// Sum of squares of a float4, accumulated into a double. Each product of two
// fp32 values is exact in double, so the fma only rounds the running sum.
__device__ __forceinline__ double AddSquares(double acc, float4 v) {
  acc = fma(static_cast<double>(v.x), static_cast<double>(v.x), acc);
  acc = fma(static_cast<double>(v.y), static_cast<double>(v.y), acc);
  acc = fma(static_cast<double>(v.z), static_cast<double>(v.z), acc);
  acc = fma(static_cast<double>(v.w), static_cast<double>(v.w), acc);
  return acc;
}

// RMSNorm scale from the double sum of squares: float(1 / sqrt(ss/n + eps)),
// every step in double as in the reference (src/kernels_gpu.cu:584-585).
__device__ __forceinline__ float RmsScale(double ss, int64_t n, float eps) {
  const double mean = ss / static_cast<double>(n);
  return static_cast<float>(1.0 / sqrt(mean + static_cast<double>(eps)));
}

// The same scale for 128-element head rows, with 1/sqrt computed as the hardware
// reciprocal square root (v_rsq_f64) refined by two Newton-Raphson steps in
// double: accurate to a few double ulps, so the value cast to fp32 equals the
// correctly rounded one except when the exact result lies within ~2^-50 of an
// fp32 rounding boundary. It replaces a double sqrt and a double division (about
// 30 fp64 instructions per row), which at 24 head rows per token is a visible
// share of the fused q/k kernel's issue slots. ss/128 is exact (power of two).
__device__ __forceinline__ float HeadRmsScale(double ss, float eps) {
  const double x = ss * (1.0 / 128.0) + static_cast<double>(eps);
  double y = __builtin_amdgcn_rsq(x);
  y = y * (1.5 - 0.5 * x * y * y);
  y = y * (1.5 - 0.5 * x * y * y);
  return static_cast<float>(__builtin_isinf(x) ? 0.0 : y);  // 1/sqrt(inf) = 0, as the division would give
}

// (v * scale) * w per component, left to right as the reference writes
// `xr[i] * scale * w[i]` (src/kernels_gpu.cu:589).
__device__ __forceinline__ float4 ScaleMul(float4 v, float scale, float4 w) {
  return make_float4((v.x * scale) * w.x, (v.y * scale) * w.y, (v.z * scale) * w.z, (v.w * scale) * w.w);
}

// ---------------------------------------------------------------- fp16

// Exact binary16 -> binary32 from the bit pattern, independent of the f16
// denormal mode: Inf/NaN keep their payload shifted into the fp32 mantissa,
// normals are re-biased (+112 in the exponent), and subnormals/zero are
// mag * 2^-24, which is exact in fp32.
__device__ __forceinline__ float HalfBitsToFloat(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t mag = h & 0x7FFFu;
  uint32_t bits;
  if (mag >= 0x7C00u) {
    bits = 0x7F800000u | ((mag & 0x3FFu) << 13);
  } else if (mag >= 0x0400u) {
    bits = (mag << 13) + 0x38000000u;
  } else {
    bits = __float_as_uint(static_cast<float>(mag) * 0x1p-24f);
  }
  return __uint_as_float(sign | bits);
}

// fp32 -> binary16 bits with IEEE round-to-nearest-even (the hardware convert
// under the default round mode; f16 denormals are preserved by the default
// kernel mode, and |x| >= 65520 becomes Inf).
__device__ __forceinline__ uint32_t FloatToHalfBits(float f) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
}

__device__ __forceinline__ uint2 PackHalf4(float4 v) {
  uint2 r;
  r.x = FloatToHalfBits(v.x) | (FloatToHalfBits(v.y) << 16);
  r.y = FloatToHalfBits(v.z) | (FloatToHalfBits(v.w) << 16);
  return r;
}

// ---------------------------------------------------------------- memory

__device__ __forceinline__ float4 Load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void Store4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// Streaming (nontemporal) 128-bit accesses for activation tensors that are
// touched exactly once per launch: the loads and stores carry the nontemporal
// cache hint, so the stream does not evict reused lines (weights, RoPE rows)
// and leaves less dirty data in L2 at the end of the kernel. Measured on
// MI355X at the prefill sizes: +10-25% effective bandwidth over plain accesses.
typedef float F32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int U32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float4 LoadStream4(const float* p) {
  const F32x4 v = __builtin_nontemporal_load(reinterpret_cast<const F32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void StoreStream4(float* p, float4 v) {
  const F32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<F32x4*>(p));
}
// Four fp16 values packed in a uint2, stored with the nontemporal hint.
__device__ __forceinline__ void StoreStreamHalf4(uint16_t* p, uint2 v) {
  const U32x2 w = {v.x, v.y};
  __builtin_nontemporal_store(w, reinterpret_cast<U32x2*>(p));
}

// Write-through output stores for write-dominated kernels (the embedding
// gathers): a raw buffer store with the cache-policy bits sc0 | sc1 | nt, i.e.
// system-scope write-through with the streaming hint, so the written lines are
// not left dirty in the XCDs' L2s for the end-of-kernel release to flush.
// Measured on MI355X: a 23 MB fill 4.45 us against 5.5-5.9 us with plain or
// nontemporal global stores; the Q4_K and Q6_K gathers at n = 2811 0.2-0.4 us
// faster. Every
// store instruction of a wave must cover whole 128-byte lines: with partial
// lines the write-through path is several times slower. The buffer resource
// bounds every store to `bytes` from `base` (out-of-range stores are dropped).
typedef unsigned int U32x4 __attribute__((ext_vector_type(4)));
constexpr int kStoreThroughPolicy = 1 | 2 | 16;  // sc0 | nt | sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t OutResource(void* base, uint32_t bytes) {
  // 0x00020000: raw (untyped) buffer, 32-bit data format, as for gfx9 CDNA parts.
  return __builtin_amdgcn_make_buffer_rsrc(base, static_cast<short>(0), static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void StoreThrough4(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, float4 v) {
  const U32x4 w = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(w, rs, static_cast<int>(byte_off), 0, kStoreThroughPolicy);
}

// The device-scope form (sc1 | nt): the store is made coherent across the XCDs, so
// it also writes through the XCD's L2, with the streaming hint. Used by SwiGLU's
// output (207 MB at n = 2811): measured on MI355X in the layer's kernel order
// (add + RMSNorm, q/k, SwiGLU over 28 rotated layers) 32.3-32.5 us against
// 33.0-33.2 us with nontemporal global stores, and the add + RMSNorm launched after
// it 0.05-0.1 us faster. Same whole-line rule as StoreThrough4.
constexpr int kStoreDeviceThroughPolicy = 2 | 16;  // nt | sc1

// 16-byte buffer stores with an explicit cache policy (sc0 = 1, nt = 2, sc1 = 16).
template <int kPolicy>
__device__ __forceinline__ void StoreBuf4(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, float4 v) {
  const U32x4 w = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(w, rs, static_cast<int>(byte_off), 0, kPolicy);
}
template <int kPolicy>
__device__ __forceinline__ void StoreBufU4(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, uint4 v) {
  const U32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, rs, static_cast<int>(byte_off), 0, kPolicy);
}

template <int kPolicy>
__device__ __forceinline__ void StoreBufU2(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, uint2 v) {
  const U32x2 w = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(w, rs, static_cast<int>(byte_off), 0, kPolicy);
}

// 8-byte buffer load with an explicit cache policy; with sc1 (16) the load is
// device-coherent: it returns what a device-scope store from another XCD left,
// not a stale line of this XCD's L2.
template <int kPolicy>
__device__ __forceinline__ uint2 LoadBufU2(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off) {
  const U32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<int>(byte_off), 0, kPolicy);
  return make_uint2(v.x, v.y);
}
constexpr int kLoadDevicePolicy = 16;  // sc1
template <int kPolicy>
__device__ __forceinline__ float4 LoadBuf4(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off) {
  const U32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(byte_off), 0, kPolicy);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
template <int kPolicy>
__device__ __forceinline__ float LoadBuf1(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(byte_off), 0, kPolicy));
}

__device__ __forceinline__ void StoreDeviceThrough4(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, float4 v) {
  StoreBuf4<kStoreDeviceThroughPolicy>(rs, byte_off, v);
}

// No cache-policy bits: an ordinary write-back store, for buffer stores that want
// the default policy (the fp16 KV-cache rows of the fused q/k kernel; the
// streaming hint on those scattered 256-byte rows made the kernel ~5% slower).
constexpr int kStorePlainPolicy = 0;

// SwiGLU element (src/kernels_gpu.cu:868): silu(g) * u = (g / (1 + e^-g)) * u,
// IEEE division. Shared by SiluMulKernel and the gate / up matvec that applies
// it to its two row totals, so both produce the same bits.
__device__ __forceinline__ float SiluMul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

}  // namespace dev
}  // namespace rpg

#endif  // RPG_AMD_DEV_UTIL_H_
