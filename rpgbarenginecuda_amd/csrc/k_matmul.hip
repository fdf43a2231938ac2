// Quantised matrix x fp32 activations: OUT[t][r] = sum_e W[r][e] * X[t][e]
// (reference GpuMatMulQuant, src/kernels_gpu.h:42-49; kernels src/kernels_gpu.cu:166-560).
//
// Numerics: every weight is dequantised bit-exactly as the reference CPU dequant
// does it (quant_dev.h), then accumulated in fp32 with fused multiply-adds. The
// reference sums in fp32 too (per-thread partial sums in a thread-strided order,
// then a shared-memory tree), so no fp32 implementation agrees with it bit for
// bit unless it copies that order; parity is instead held to a bound on the
// fp32 summation error against the exact (double) dot product.
//
// MI355X mapping (all of it HBM-bound at decode: 0.5625 / 0.8203 weight bytes per
// multiply-add for Q4_K / Q6_K):
//   * one wave64 per R output rows; the 64 lanes form 8 groups of 8, group c
//     taking super-blocks c, c + 8, c + 16, ... of the row, so each load
//     instruction of a wave reads 8 whole blocks (1152 / 1680 contiguous bytes
//     per row at cols = 2048);
//   * Q4_K lane s of a group reads the 16-byte block header and 16 bytes of qs
//     (sub-block pair g = s / 2, half hh = s % 2): 32 weights, elements
//     64g + 16hh + i (low nibbles) and 64g + 32 + 16hh + i (high nibbles);
//   * Q6_K lane s reads 8 bytes each of ql (two runs) and qh at l = 8(s % 4) in
//     half h = s / 4: 32 weights, elements 128h + 32q + l + i. Q6_K blocks are
//     only 2-byte aligned, so these come from aligned dwords and a byte shift;
//   * the activations a lane needs (32 floats per token) are loaded once per
//     block and reused for all R rows of the wave; each row's weights are
//     dequantised once and reused for all T tokens of the tile;
//   * the lane partial sums are combined by a 6-step butterfly; lane 0 stores.
// Rows with cols beyond what the loop covers, F32 matrices and unaligned
// matrices take a per-element generic kernel.
#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"
#include "quant_dev.h"

namespace rpg {
namespace {

using dev::ByteOf;
using dev::HalfBitsToFloat;
using dev::ScaleMinK4;

constexpr int kMmBlock = 256;        // 4 waves per workgroup
constexpr int kWavesPerBlock = kMmBlock / 64;
constexpr int kGroupLanes = 8;       // lanes sharing one super-block
constexpr int kGroups = 64 / kGroupLanes;

bool Aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

__device__ __forceinline__ float WaveSumF(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// 8 bytes at a 2-byte aligned address, from aligned dwords (a Q6_K block starts
// at a multiple of 210 bytes). The third dword is read only when the address is
// not 4-byte aligned, so no byte past p + 9 is ever touched.
__device__ __forceinline__ uint2 Load8Align2(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~static_cast<uintptr_t>(3));
  const bool odd = (a & 3) != 0;
  const uint32_t w0 = base[0];
  const uint32_t w1 = base[1];
  const uint32_t w2 = base[odd ? 2 : 1];
  return odd ? make_uint2(__builtin_amdgcn_alignbyte(w1, w0, 2), __builtin_amdgcn_alignbyte(w2, w1, 2))
             : make_uint2(w0, w1);
}

// ---------------------------------------------------------------- per-lane block decode

// The lane's 32 activations of one token for the block starting at column col0.
template <uint32_t kType>
__device__ __forceinline__ void LoadLaneX(const float* __restrict__ xt, int64_t col0, int s, float (&xv)[32]) {
  if (kType == kGgmlQ4_K) {
    const int g = s >> 1;
    const int hh = s & 1;
    const float* lo = xt + col0 + 64 * g + 16 * hh;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 a = *reinterpret_cast<const float4*>(lo + 4 * k);
      const float4 b = *reinterpret_cast<const float4*>(lo + 32 + 4 * k);
      xv[4 * k] = a.x; xv[4 * k + 1] = a.y; xv[4 * k + 2] = a.z; xv[4 * k + 3] = a.w;
      xv[16 + 4 * k] = b.x; xv[16 + 4 * k + 1] = b.y; xv[16 + 4 * k + 2] = b.z; xv[16 + 4 * k + 3] = b.w;
    }
  } else {
    const int h = s >> 2;
    const int lq = 8 * (s & 3);
    const float* base = xt + col0 + 128 * h + lq;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 a = *reinterpret_cast<const float4*>(base + 32 * q);
      const float4 b = *reinterpret_cast<const float4*>(base + 32 * q + 4);
      xv[8 * q] = a.x; xv[8 * q + 1] = a.y; xv[8 * q + 2] = a.z; xv[8 * q + 3] = a.w;
      xv[8 * q + 4] = b.x; xv[8 * q + 5] = b.y; xv[8 * q + 6] = b.z; xv[8 * q + 7] = b.w;
    }
  }
}

// Raw bytes a lane needs from one block (loads only; decoded later so that the
// loads of all rows are in flight together).
struct LaneBytes {
  uint4 a;  // Q4_K: header (d, dmin, scales); Q6_K: ql run 0 (x, y), ql run 1 (z, w)
  uint4 b;  // Q4_K: 16 qs bytes;              Q6_K: qh (x, y), scales of the half (z, w)
  uint32_t d6;  // Q6_K: d (f16 bits)
};

template <uint32_t kType>
__device__ __forceinline__ LaneBytes LoadLaneBytes(const uint8_t* __restrict__ blk, int s) {
  LaneBytes r;
  if (kType == kGgmlQ4_K) {
    const int g = s >> 1;
    const int hh = s & 1;
    r.a = *reinterpret_cast<const uint4*>(blk);
    r.b = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g + 16 * hh);
    r.d6 = 0;
  } else {
    const int h = s >> 2;
    const int lq = 8 * (s & 3);
    const uint2 ql0 = Load8Align2(blk + 64 * h + lq);
    const uint2 ql1 = Load8Align2(blk + 64 * h + 32 + lq);
    const uint2 qh = Load8Align2(blk + 128 + 32 * h + lq);
    const uint2 sc = Load8Align2(blk + 192 + 8 * h);
    r.a = make_uint4(ql0.x, ql0.y, ql1.x, ql1.y);
    r.b = make_uint4(qh.x, qh.y, sc.x, sc.y);
    r.d6 = *reinterpret_cast<const uint16_t*>(blk + 208);
  }
  return r;
}

// The lane's 32 weights, in the same order as LoadLaneX's activations.
template <uint32_t kType>
__device__ __forceinline__ void DecodeLane(const LaneBytes& r, int s, float (&wv)[32]) {
  if (kType == kGgmlQ4_K) {
    const int g = s >> 1;
    const float d = HalfBitsToFloat(r.a.x & 0xFFFFu);
    const float dmin = HalfBitsToFloat(r.a.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    ScaleMinK4(2 * g, r.a.y, r.a.z, r.a.w, &sc0, &m0);
    ScaleMinK4(2 * g + 1, r.a.y, r.a.z, r.a.w, &sc1, &m1);
    const float d1 = d * static_cast<float>(sc0);
    const float n1 = dmin * static_cast<float>(m0);
    const float d2 = d * static_cast<float>(sc1);
    const float n2 = dmin * static_cast<float>(m1);
    const uint32_t qw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t byte = ByteOf(qw[i >> 2], i & 3);
      wv[i] = d1 * static_cast<float>(byte & 0x0Fu) - n1;
      wv[16 + i] = d2 * static_cast<float>(byte >> 4) - n2;
    }
  } else {
    const int is = (s & 3) >> 1;  // (l >> 4) for l = 8(s % 4) .. +7
    const float d = HalfBitsToFloat(r.d6);
    const uint32_t ql[2][2] = {{r.a.x, r.a.y}, {r.a.z, r.a.w}};
    const uint32_t qh[2] = {r.b.x, r.b.y};
    const uint32_t scw[2] = {r.b.z, r.b.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int si = is + 2 * q;
      const int8_t sc = static_cast<int8_t>(ByteOf(scw[si >> 2], si & 3));
      const float ds = d * static_cast<float>(sc);
      const int shift = q < 2 ? 0 : 4;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t nib = (ByteOf(ql[q & 1][i >> 2], i & 3) >> shift) & 0x0Fu;
        const uint32_t hi2 = (ByteOf(qh[i >> 2], i & 3) >> (2 * q)) & 3u;
        wv[8 * q + i] = ds * static_cast<float>(static_cast<int>(nib | (hi2 << 4)) - 32);
      }
    }
  }
}

template <uint32_t kType>
struct BlockBytesOf;
template <>
struct BlockBytesOf<kGgmlQ4_K> {
  static constexpr int64_t value = kQ4KBlockBytes;
};
template <>
struct BlockBytesOf<kGgmlQ6_K> {
  static constexpr int64_t value = kQ6KBlockBytes;
};

// ---------------------------------------------------------------- kernels

// R rows per wave, T tokens per tile (blockIdx.y). For T == 1 the activations
// stay in registers across the R rows; for T > 1 each row's weights are decoded
// once and the activations of each token are loaded in turn.
template <uint32_t kType, int R, int T>
__global__ __launch_bounds__(kMmBlock) void MatMulQuantKernel(const uint8_t* __restrict__ w, int64_t rows,
                                                              int64_t row_bytes, int32_t nb,
                                                              const float* __restrict__ x, int64_t cols,
                                                              int64_t n_tokens, float* __restrict__ out) {
  constexpr int64_t kBB = BlockBytesOf<kType>::value;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6)) * R;
  if (r0 >= rows) return;  // uniform over the wave
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * T;
  const int c = lane / kGroupLanes;
  const int s = lane % kGroupLanes;
  const int nt = static_cast<int>(n_tokens - t0 < T ? n_tokens - t0 : T);

  float acc[R][T];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;

  for (int b = c; b < nb; b += kGroups) {
    const int64_t col0 = static_cast<int64_t>(b) * kQK_K;
    LaneBytes lb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = r0 + r < rows ? r0 + r : rows - 1;  // clamped: the load stays in bounds
      lb[r] = LoadLaneBytes<kType>(w + row * row_bytes + b * kBB, s);
    }
    if (T == 1) {
      float xv[32];
      LoadLaneX<kType>(x + t0 * cols, col0, s, xv);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float wv[32];
        DecodeLane<kType>(lb[r], s, wv);
#pragma unroll
        for (int i = 0; i < 32; ++i) acc[r][0] = __builtin_fmaf(wv[i], xv[i], acc[r][0]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float wv[32];
        DecodeLane<kType>(lb[r], s, wv);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (t < nt) {
            float xv[32];
            LoadLaneX<kType>(x + (t0 + t) * cols, col0, s, xv);
#pragma unroll
            for (int i = 0; i < 32; ++i) acc[r][t] = __builtin_fmaf(wv[i], xv[i], acc[r][t]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float v = WaveSumF(acc[r][t]);
      if (lane == 0 && r0 + r < rows && t < nt) out[(t0 + t) * rows + r0 + r] = v;
    }
  }
}

// Any type, any alignment: one wave per (row, token), lanes strided over the
// columns, per-element byte-wise decode; fp32 FMA accumulation and the same
// butterfly.
__global__ __launch_bounds__(kMmBlock) void MatMulGenericKernel(uint32_t type, const uint8_t* __restrict__ w,
                                                                int64_t rows, int64_t row_bytes, int32_t block_elems,
                                                                int32_t block_bytes, const float* __restrict__ x,
                                                                int64_t cols, int64_t n_tokens,
                                                                float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (unit >= rows * n_tokens) return;
  const int64_t t = unit / rows;
  const int64_t r = unit - t * rows;
  const uint8_t* row = w + r * row_bytes;
  const float* xt = x + t * cols;
  float acc = 0.0f;
  for (int64_t e = lane; e < cols; e += 64) {
    const int64_t bi = e / block_elems;
    const float wv = dev::DeqElemAny(type, row + bi * block_bytes, static_cast<int>(e - bi * block_elems));
    acc = __builtin_fmaf(wv, xt[e], acc);
  }
  acc = WaveSumF(acc);
  if (lane == 0) out[t * rows + r] = acc;
}

template <uint32_t kType, int R, int T>
void LaunchQuant(const char* name, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                 int64_t cols, int64_t n_tokens, float* out) {
  const int64_t waves = (rows + R - 1) / R;
  const int64_t tiles = (n_tokens + T - 1) / T;
  RPG_CHECK(tiles <= 65535, "too many token tiles: %lld", static_cast<long long>(tiles));
  Launch(name, MatMulQuantKernel<kType, R, T>, dim3(GridFor(waves, kWavesPerBlock), static_cast<unsigned>(tiles)),
         dim3(kMmBlock), w, rows, row_bytes, nb, x, cols, n_tokens, out);
}

// Rows per wave: enough waves to cover the chip first (a wave per row below
// 8192 rows), then 2 or 4 rows so each lane's activations serve several rows.
template <uint32_t kType>
void LaunchByShape(const char* name, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                   int64_t cols, int64_t n_tokens, float* out) {
  if (n_tokens == 1) {
    if (rows >= 32768) return LaunchQuant<kType, 4, 1>(name, w, rows, row_bytes, nb, x, cols, n_tokens, out);
    if (rows >= 8192) return LaunchQuant<kType, 2, 1>(name, w, rows, row_bytes, nb, x, cols, n_tokens, out);
    return LaunchQuant<kType, 1, 1>(name, w, rows, row_bytes, nb, x, cols, n_tokens, out);
  }
  if (n_tokens <= 2) return LaunchQuant<kType, 1, 2>(name, w, rows, row_bytes, nb, x, cols, n_tokens, out);
  if (n_tokens <= 4) return LaunchQuant<kType, 1, 4>(name, w, rows, row_bytes, nb, x, cols, n_tokens, out);
  return LaunchQuant<kType, 1, 8>(name, w, rows, row_bytes, nb, x, cols, n_tokens, out);
}

}  // namespace

void GpuMatMulQuantRaw(uint32_t type, const uint8_t* w_dev, int64_t rows, int64_t cols, const float* x_dev,
                       int64_t n_tokens, float* out_dev) {
  RPG_CHECK(rows > 0 && cols > 0, "invalid MatMulQuant shape [%lld, %lld]", static_cast<long long>(rows),
            static_cast<long long>(cols));
  RPG_CHECK(n_tokens > 0, "n_tokens must be positive");
  const BlockShape bs = DeviceBlockShape(type);
  RPG_CHECK(cols % bs.elems == 0, "dot length %lld is not a multiple of the block size %d",
            static_cast<long long>(cols), bs.elems);
  RPG_CHECK(w_dev != nullptr && x_dev != nullptr && out_dev != nullptr, "MatMulQuant got a null pointer");
  const int64_t row_bytes = TypeRowBytes(type, cols);
  const bool x_ok = Aligned(x_dev, 16) && cols % 4 == 0;
  const int64_t nb = cols / kQK_K;
  if (type == kGgmlQ4_K && x_ok && Aligned(w_dev, 16) && nb <= 0x7FFFFFFF) {
    LaunchByShape<kGgmlQ4_K>("MatMulQ4KKernel", w_dev, rows, row_bytes, static_cast<int32_t>(nb), x_dev, cols,
                             n_tokens, out_dev);
    return;
  }
  if (type == kGgmlQ6_K && x_ok && Aligned(w_dev, 2) && nb <= 0x7FFFFFFF) {
    LaunchByShape<kGgmlQ6_K>("MatMulQ6KKernel", w_dev, rows, row_bytes, static_cast<int32_t>(nb), x_dev, cols,
                             n_tokens, out_dev);
    return;
  }
  const int64_t units = rows * n_tokens;
  Launch("MatMulGenericKernel", MatMulGenericKernel, dim3(GridFor(units, kWavesPerBlock)), dim3(kMmBlock), type,
         w_dev, rows, row_bytes, bs.elems, bs.bytes, x_dev, cols, n_tokens, out_dev);
}

void GpuMatMulQuant(const GpuTensor& w, const float* X_dev, int64_t n_tokens, float* OUT_dev) {
  RPG_CHECK(w.matrix, "GpuMatMulQuant got a non-matrix tensor (%s)", w.type_name());
  RPG_CHECK(w.valid(), "GpuMatMulQuant got an empty tensor");
  RPG_CHECK(w.buf.size() == static_cast<size_t>(w.rows * w.row_bytes()),
            "tensor byte count does not match the [%lld, %lld] shape", static_cast<long long>(w.rows),
            static_cast<long long>(w.cols));
  GpuMatMulQuantRaw(w.type, static_cast<const uint8_t*>(w.buf.data()), w.rows, w.cols, X_dev, n_tokens, OUT_dev);
}

}  // namespace rpg
