// Q4_K / Q6_K row dequantisation and the token_embd row-dequant gather.
//
// Values are bit-identical to the reference CPU dequant (src/quant.cc:252-279
// DeqQ4_K, :321-354 DeqQ6_K, :159-167 GetScaleMinK4; f16 from src/dtypes.h:21-47):
//   Q4_K: y = (d*sc)*q - (dmin*m)     (three separately rounded fp32 ops)
//   Q6_K: y = (d*sc)*q                (two separately rounded fp32 ops)
// The library is compiled with -ffp-contract=off, so no multiply-subtract is
// fused; signed zeros follow from the same op order (e.g. sc < 0, q = 0 -> -0).
//
// MI355X mapping: the unit of work is one 256-element super-block.
//   Q4_K: 32 lanes per block. Lane j (g = j/8, kq = j%8) loads the 16-byte block
//     header (d, dmin, 12 scale bytes; one 128-bit load, broadcast in cache) and
//     one 32-bit word of qs (the 32 lanes cover all 128 qs bytes coalesced); the
//     low nibbles give elements 64g+4kq..+3, the high nibbles 64g+32+4kq..+3.
//     The two (scale, min) pairs are unpacked once per lane, in registers.
//   Q6_K: 16 lanes per block. Lane j (half = j/8, kq = j%8) loads 4 bytes of each
//     of ql[half*64 + 4kq], ql[half*64 + 32 + 4kq], qh[half*32 + 4kq], the 8 scales
//     of its half and d, and produces 16 elements: four float4 at
//     half*128 + 32*quarter + 4kq. Q6_K blocks are 210 bytes, so a block start is
//     only 2-byte aligned; loads are 16-bit.
// Every lane ends with float4 stores, so a wave writes 2 KiB (Q4_K) or 4 KiB (Q6_K)
// of fp32 as full 128-byte lines. The one-workgroup-per-token gathers store them
// write-through (dev::StoreThrough4, measured faster for these write-dominated
// kernels: Q4_K 4.5-4.8 vs 4.9-5.7 us, Q6_K 4.75-5.0 vs 4.95-5.25 us at n = 2811);
// the flat block kernel keeps nontemporal global stores.
#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"
#include "quant_dev.h"

namespace rpg {
namespace {

using dev::ByteOf;
using dev::DeqElemAny;
using dev::HalfBitsToFloat;
using dev::ScaleMinK4;
using dev::StoreStream4;

constexpr int kBlock = 256;

bool Aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Output policies of the decoders: put(e, v) stores the float4 of elements
// e..e+3 of the block's 256 outputs.
struct StreamOut {  // nontemporal global stores at out
  float* out;
  __device__ void operator()(int e, float4 v) const { StoreStream4(out + e, v); }
};
struct ThroughOut {  // write-through buffer stores at byte offset off of the resource
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off;
  __device__ void operator()(int e, float4 v) const { dev::StoreThrough4(rs, off + 4u * static_cast<uint32_t>(e), v); }
};

// One lane's share (8 elements) of a Q4_K block; blk must be 16-byte aligned.
template <typename Put>
__device__ __forceinline__ void DecodeQ4KLane(const uint8_t* blk, int j, const Put& put) {
  const int g = j >> 3;
  const int kq = j & 7;
  const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
  const uint32_t qw = *reinterpret_cast<const uint32_t*>(blk + 16 + 32 * g + 4 * kq);
  const float d = HalfBitsToFloat(hdr.x & 0xFFFFu);
  const float dmin = HalfBitsToFloat(hdr.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  ScaleMinK4(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
  ScaleMinK4(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
  const float d1 = d * static_cast<float>(sc0);
  const float n1 = dmin * static_cast<float>(m0);
  const float d2 = d * static_cast<float>(sc1);
  const float n2 = dmin * static_cast<float>(m1);
  float lo[4], hi[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    lo[b] = d1 * static_cast<float>((qw >> (8 * b)) & 0xFu) - n1;
    hi[b] = d2 * static_cast<float>((qw >> (8 * b + 4)) & 0xFu) - n2;
  }
  put(64 * g + 4 * kq, make_float4(lo[0], lo[1], lo[2], lo[3]));
  put(64 * g + 32 + 4 * kq, make_float4(hi[0], hi[1], hi[2], hi[3]));
}

// 4 (8) bytes at a 2-byte aligned address as one dword (dwordx2) load: the
// device runs in unaligned-access mode, which the compiler assumes for amdhsa.
__device__ __forceinline__ uint32_t Load4Bytes2Aligned(const uint8_t* p) {
  uint32_t w;
  __builtin_memcpy(&w, __builtin_assume_aligned(p, 2), 4);
  return w;
}
__device__ __forceinline__ uint2 Load8Bytes2Aligned(const uint8_t* p) {
  uint2 w;
  __builtin_memcpy(&w, __builtin_assume_aligned(p, 2), 8);
  return w;
}

// One lane's share (16 elements) of a Q6_K block; blk must be 2-byte aligned.
template <typename Put>
__device__ __forceinline__ void DecodeQ6KLane(const uint8_t* blk, int j, const Put& put) {
  const int half = j >> 3;
  const int kq = j & 7;
  const uint32_t ql0 = Load4Bytes2Aligned(blk + 64 * half + 4 * kq);
  const uint32_t ql1 = Load4Bytes2Aligned(blk + 64 * half + 32 + 4 * kq);
  const uint32_t qh = Load4Bytes2Aligned(blk + 128 + 32 * half + 4 * kq);
  const uint2 scw = Load8Bytes2Aligned(blk + 192 + 8 * half);  // scales 0..3 / 4..7 of this half
  const uint32_t sc_lo = scw.x;
  const uint32_t sc_hi = scw.y;
  const float d = HalfBitsToFloat(*reinterpret_cast<const uint16_t*>(blk + 208));
  const int is = kq >> 2;  // (l >> 4) for l = 4kq..4kq+3
#pragma unroll
  for (int quarter = 0; quarter < 4; ++quarter) {
    const int si = is + 2 * quarter;  // 0..7 within the half
    const int8_t sc = static_cast<int8_t>(ByteOf(si < 4 ? sc_lo : sc_hi, si & 3));
    const float ds = d * static_cast<float>(sc);
    const uint32_t qlw = (quarter & 1) ? ql1 : ql0;
    const int nib_shift = quarter < 2 ? 0 : 4;
    float y[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t nib = (qlw >> (8 * b + nib_shift)) & 0xFu;
      const uint32_t hi2 = (ByteOf(qh, b) >> (2 * quarter)) & 3u;
      const int q = static_cast<int>(nib | (hi2 << 4)) - 32;
      y[b] = ds * static_cast<float>(q);
    }
    put(128 * half + 32 * quarter + 4 * kq, make_float4(y[0], y[1], y[2], y[3]));
  }
}

template <uint32_t kType>
struct QuantTraits;
template <>
struct QuantTraits<kGgmlQ4_K> {
  static constexpr int kLanes = 32;
  static constexpr int kWaveTok = 2;           // token gathers: GatherWaveKernel, 2 tokens per workgroup
  static constexpr bool kStoreThrough = true;  // measured faster at n = 2811 (~4.6 vs ~5.0 us)
  static constexpr bool kVectorId = false;     // token id through a scalar load (GatherRowsKernel)
  static constexpr int64_t kBytes = kQ4KBlockBytes;
  template <typename Put>
  __device__ static void Decode(const uint8_t* blk, int j, const Put& put) { DecodeQ4KLane(blk, j, put); }
  // +0 in every element this lane would decode (same store pattern: whole lines).
  template <typename Put>
  __device__ static void Zero(int j, const Put& put) {
    const int g = j >> 3;
    const int kq = j & 7;
    put(64 * g + 4 * kq, make_float4(0.f, 0.f, 0.f, 0.f));
    put(64 * g + 32 + 4 * kq, make_float4(0.f, 0.f, 0.f, 0.f));
  }
};
template <>
struct QuantTraits<kGgmlQ6_K> {
  static constexpr int kLanes = 16;
  static constexpr int kWaveTok = 0;           // token gathers: GatherRowsKernel
  static constexpr bool kStoreThrough = true;  // ~0.2 us faster at n = 2811 with launches queued back to back
  static constexpr bool kVectorId = true;      // token id through a vector load (GatherRowsKernel)
  static constexpr int64_t kBytes = kQ6KBlockBytes;
  template <typename Put>
  __device__ static void Decode(const uint8_t* blk, int j, const Put& put) { DecodeQ6KLane(blk, j, put); }
  template <typename Put>
  __device__ static void Zero(int j, const Put& put) {
#pragma unroll
    for (int quarter = 0; quarter < 4; ++quarter) {
      put(128 * (j >> 3) + 32 * quarter + 4 * (j & 7), make_float4(0.f, 0.f, 0.f, 0.f));
    }
  }
};

// Gather: unit = (token t, block b). toks == nullptr means "dequantise row 0 of
// the table", which is how GpuDequantRow reuses the kernel.
template <uint32_t kType>
__global__ __launch_bounds__(kBlock) void GatherBlocksKernel(const uint8_t* __restrict__ emb, int64_t rows,
                                                             int64_t row_bytes, int32_t nb,
                                                             const int32_t* __restrict__ toks, int64_t n_units,
                                                             float* __restrict__ x) {
  using T = QuantTraits<kType>;
  constexpr int kUnits = kBlock / T::kLanes;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * kUnits + threadIdx.x / T::kLanes;
  const int j = threadIdx.x % T::kLanes;
  if (unit >= n_units) return;
  const int64_t t = unit / nb;
  const int32_t b = static_cast<int32_t>(unit - t * nb);
  float* out = x + (t * nb + b) * kQK_K;
  const int64_t tok = toks != nullptr ? static_cast<int64_t>(toks[t]) : 0;
  if (tok < 0 || tok >= rows) {
    T::Zero(j, StreamOut{out});
    return;
  }
  T::Decode(emb + tok * row_bytes + b * T::kBytes, j, StreamOut{out});
}

// Gather with one workgroup per token: nb * kLanes threads, the token id is a
// uniform (scalar) load and the row address is uniform, so each lane's block
// loads depend on one scalar load instead of a per-lane id load.
template <uint32_t kType>
__global__ __launch_bounds__(1024) void GatherRowsKernel(const uint8_t* __restrict__ emb, int64_t rows,
                                                         int64_t row_bytes, const int32_t* __restrict__ toks,
                                                         float* __restrict__ x) {
  using T = QuantTraits<kType>;
  // The kernel arguments are fetched in one batch (the empty asm takes them as
  // scalar inputs and emits nothing), so the row loads wait for the id's round trip
  // only. Where the asm sits decides how the compiler loads the token id: ahead of
  // the id load it becomes a vector load (then readfirstlane), after it a scalar
  // load. Measured at n = 2811 over three processes each: Q4_K 4.56-4.69 us with
  // the scalar id against 4.85-5.07 us with the vector one; Q6_K 4.62-4.76 us with
  // the vector id against 4.82-4.84 us with the scalar one.
  if constexpr (T::kVectorId) asm volatile("" ::"s"(emb), "s"(rows), "s"(row_bytes), "s"(toks), "s"(x));
  const int64_t t = blockIdx.x;
  const int32_t b = static_cast<int32_t>(threadIdx.x / T::kLanes);
  const int j = threadIdx.x % T::kLanes;
  const int64_t nb = blockDim.x / T::kLanes;
  const int64_t tok = static_cast<int64_t>(toks[t]);
  if constexpr (!T::kVectorId) asm volatile("" ::"s"(emb), "s"(rows), "s"(row_bytes), "s"(x), "s"(tok));
  const bool valid = tok >= 0 && tok < rows;
  const uint8_t* blk = emb + (valid ? tok : 0) * row_bytes + b * T::kBytes;
  if constexpr (T::kStoreThrough) {
    // The token's output row through a buffer resource bounded to that row, so
    // the offsets stay 32-bit at any token count.
    const uint32_t row_out_bytes = static_cast<uint32_t>(nb * kQK_K * sizeof(float));
    const ThroughOut put{dev::OutResource(x + t * nb * kQK_K, row_out_bytes),
                         static_cast<uint32_t>(b) * static_cast<uint32_t>(kQK_K * sizeof(float))};
    if (valid) {
      T::Decode(blk, j, put);
    } else {
      T::Zero(j, put);
    }
  } else {
    const StreamOut put{x + (t * nb + b) * kQK_K};
    if (valid) {
      T::Decode(blk, j, put);
    } else {
      T::Zero(j, put);
    }
  }
}

// Gather with one wave per token (kTok tokens per workgroup): 8 lanes per
// super-block, lane kq covering the elements 4kq..4kq+3 of every 32-element
// sub-block, so each store instruction of the block's 8 lanes writes one whole
// 128-byte line. A lane issues all of its block's loads before it decodes and
// stores. Rows wider than 8 blocks loop (lane block b, b + 8, ...). Workgroups
// hold kTok waves, so 2811 tokens are 2811 waves: every token's id load and row
// loads are in flight at once on 256 CUs, where one workgroup of 8 x 32 lanes
// per token leaves a second round of workgroups waiting for a slot.
__device__ __forceinline__ void DecodeQ4KLane8(const uint8_t* blk, int kq, const ThroughOut& put) {
  const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
  uint32_t qw[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) qw[g] = *reinterpret_cast<const uint32_t*>(blk + 16 + 32 * g + 4 * kq);
  const float d = HalfBitsToFloat(hdr.x & 0xFFFFu);
  const float dmin = HalfBitsToFloat(hdr.x >> 16);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t sc0, m0, sc1, m1;
    ScaleMinK4(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
    ScaleMinK4(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
    const float d1 = d * static_cast<float>(sc0);
    const float n1 = dmin * static_cast<float>(m0);
    const float d2 = d * static_cast<float>(sc1);
    const float n2 = dmin * static_cast<float>(m1);
    float lo[4], hi[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      lo[b] = d1 * static_cast<float>((qw[g] >> (8 * b)) & 0xFu) - n1;
      hi[b] = d2 * static_cast<float>((qw[g] >> (8 * b + 4)) & 0xFu) - n2;
    }
    put(64 * g + 4 * kq, make_float4(lo[0], lo[1], lo[2], lo[3]));
    put(64 * g + 32 + 4 * kq, make_float4(hi[0], hi[1], hi[2], hi[3]));
  }
}

__device__ __forceinline__ void DecodeQ6KLane8(const uint8_t* blk, int kq, const ThroughOut& put) {
  uint32_t ql0[2], ql1[2], qh[2], sc_lo[2], sc_hi[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    ql0[half] = Load4Bytes2Aligned(blk + 64 * half + 4 * kq);
    ql1[half] = Load4Bytes2Aligned(blk + 64 * half + 32 + 4 * kq);
    qh[half] = Load4Bytes2Aligned(blk + 128 + 32 * half + 4 * kq);
    const uint2 scw = Load8Bytes2Aligned(blk + 192 + 8 * half);
    sc_lo[half] = scw.x;
    sc_hi[half] = scw.y;
  }
  const float d = HalfBitsToFloat(*reinterpret_cast<const uint16_t*>(blk + 208));
  const int is = kq >> 2;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int quarter = 0; quarter < 4; ++quarter) {
      const int si = is + 2 * quarter;
      const int8_t sc = static_cast<int8_t>(ByteOf(si < 4 ? sc_lo[half] : sc_hi[half], si & 3));
      const float ds = d * static_cast<float>(sc);
      const uint32_t qlw = (quarter & 1) ? ql1[half] : ql0[half];
      const int nib_shift = quarter < 2 ? 0 : 4;
      float y[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t nib = (qlw >> (8 * b + nib_shift)) & 0xFu;
        const uint32_t hi2 = (ByteOf(qh[half], b) >> (2 * quarter)) & 3u;
        const int q = static_cast<int>(nib | (hi2 << 4)) - 32;
        y[b] = ds * static_cast<float>(q);
      }
      put(128 * half + 32 * quarter + 4 * kq, make_float4(y[0], y[1], y[2], y[3]));
    }
  }
}

template <uint32_t kType, int kTok>
__global__ __launch_bounds__(64 * kTok) void GatherWaveKernel(const uint8_t* __restrict__ emb, int64_t rows,
                                                              int64_t row_bytes, int32_t nb,
                                                              const int32_t* __restrict__ toks, int64_t seq,
                                                              float* __restrict__ x) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTok + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= seq) return;  // no barriers below
  const int64_t tok = static_cast<int64_t>(toks[t]);
  const bool valid = tok >= 0 && tok < rows;
  const uint8_t* row = emb + (valid ? tok : 0) * row_bytes;
  const uint32_t row_out_bytes = static_cast<uint32_t>(nb) * static_cast<uint32_t>(kQK_K * sizeof(float));
  const __amdgpu_buffer_rsrc_t rs = dev::OutResource(x + t * nb * kQK_K, row_out_bytes);
  const int kq = lane & 7;
  for (int32_t b = lane >> 3; b < nb; b += 8) {
    const ThroughOut put{rs, static_cast<uint32_t>(b) * static_cast<uint32_t>(kQK_K * sizeof(float))};
    if (!valid) {
#pragma unroll
      for (int i = 0; i < 8; ++i) put(32 * i + 4 * kq, make_float4(0.f, 0.f, 0.f, 0.f));
    } else if constexpr (kType == kGgmlQ4_K) {
      DecodeQ4KLane8(row + b * kQ4KBlockBytes, kq, put);
    } else {
      DecodeQ6KLane8(row + b * kQ6KBlockBytes, kq, put);
    }
  }
}

// F32 tables: rows are plain floats; one float4 per thread.
__global__ __launch_bounds__(kBlock) void GatherF32Kernel(const float* __restrict__ emb, int64_t rows, int64_t cols,
                                                          const int32_t* __restrict__ toks, int64_t total4,
                                                          float* __restrict__ x) {
  const int64_t i4 = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i4 >= total4) return;
  const int64_t i = 4 * i4;
  const int64_t t = i / cols;
  const int64_t e = i - t * cols;
  const int64_t tok = toks != nullptr ? static_cast<int64_t>(toks[t]) : 0;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tok >= 0 && tok < rows) v = dev::Load4(emb + tok * cols + e);
  StoreStream4(x + i, v);
}

__global__ __launch_bounds__(kBlock) void GatherElemKernel(uint32_t type, const uint8_t* __restrict__ emb,
                                                           int64_t rows, int64_t cols, int64_t row_bytes,
                                                           int32_t block_elems, int32_t block_bytes,
                                                           const int32_t* __restrict__ toks, int64_t total,
                                                           float* __restrict__ x) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= total) return;
  const int64_t t = i / cols;
  const int64_t e = i - t * cols;
  const int64_t tok = toks != nullptr ? static_cast<int64_t>(toks[t]) : 0;
  if (tok < 0 || tok >= rows) {
    x[i] = 0.0f;
    return;
  }
  const int64_t bi = e / block_elems;
  x[i] = DeqElemAny(type, emb + tok * row_bytes + bi * block_bytes, static_cast<int>(e - bi * block_elems));
}

__global__ __launch_bounds__(kBlock) void F16SweepKernel(float* out) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i < 65536) out[i] = HalfBitsToFloat(static_cast<uint32_t>(i));
}

// GatherWaveKernel for the token gathers of type kType when its traits ask for it.
template <uint32_t kType>
bool LaunchGatherWave(const uint8_t* emb, int64_t rows, int64_t row_bytes, int64_t nb, const int32_t* toks,
                      int64_t seq, float* x, const char* name) {
  constexpr int kTok = QuantTraits<kType>::kWaveTok;
  if constexpr (kTok == 0) {
    return false;
  } else {
    RPG_CHECK(seq <= 0x7FFFFFFFLL * kTok, "too many tokens: %lld", static_cast<long long>(seq));
    RPG_CHECK(nb <= 0xFFFFFFFFLL / (kQK_K * sizeof(float)), "row of %lld blocks is too wide for one output resource",
              static_cast<long long>(nb));
    Launch(name, GatherWaveKernel<kType, kTok>, dim3(static_cast<unsigned>((seq + kTok - 1) / kTok)), dim3(64 * kTok),
           emb, rows, row_bytes, static_cast<int32_t>(nb), toks, seq, x);
    return true;
  }
}

// Shared launcher for the gather and the single-row dequant (toks == nullptr,
// rows == 1, seq == 1, cols == n_elems).
void LaunchGather(uint32_t type, const uint8_t* emb, int64_t rows, int64_t cols, const int32_t* toks, int64_t seq,
                  float* x) {
  const BlockShape bs = DeviceBlockShape(type);
  RPG_CHECK(cols > 0 && cols % bs.elems == 0, "row width %lld is not a multiple of the %s block size %d",
            static_cast<long long>(cols), TypeName(type), bs.elems);
  const int64_t row_bytes = TypeRowBytes(type, cols);
  if (seq <= 0) return;
  const int64_t total = seq * cols;
  const int64_t nb64 = cols / kQK_K;
  if (toks != nullptr && type == kGgmlQ4_K && Aligned(emb, 16) && Aligned(x, 16) &&
      LaunchGatherWave<kGgmlQ4_K>(emb, rows, row_bytes, nb64, toks, seq, x, "GatherQ4KKernel")) {
    return;
  }
  if (toks != nullptr && type == kGgmlQ6_K && Aligned(emb, 2) && Aligned(x, 16) &&
      LaunchGatherWave<kGgmlQ6_K>(emb, rows, row_bytes, nb64, toks, seq, x, "GatherQ6KKernel")) {
    return;
  }
  if (toks != nullptr && type == kGgmlQ4_K && nb64 * 32 <= 1024 && Aligned(emb, 16) && Aligned(x, 16)) {
    RPG_CHECK(seq <= 0x7FFFFFFF, "too many tokens: %lld", static_cast<long long>(seq));
    Launch("GatherQ4KKernel", GatherRowsKernel<kGgmlQ4_K>, dim3(static_cast<unsigned>(seq)),
           dim3(static_cast<unsigned>(nb64 * 32)), emb, rows, row_bytes, toks, x);
    return;
  }
  if (toks != nullptr && type == kGgmlQ6_K && nb64 * 16 <= 1024 && Aligned(emb, 2) && Aligned(x, 16)) {
    RPG_CHECK(seq <= 0x7FFFFFFF, "too many tokens: %lld", static_cast<long long>(seq));
    Launch("GatherQ6KKernel", GatherRowsKernel<kGgmlQ6_K>, dim3(static_cast<unsigned>(seq)),
           dim3(static_cast<unsigned>(nb64 * 16)), emb, rows, row_bytes, toks, x);
    return;
  }
  if (type == kGgmlQ4_K && Aligned(emb, 16) && Aligned(x, 16)) {
    const int32_t nb = static_cast<int32_t>(cols / kQK_K);
    const int64_t units = seq * nb;
    Launch("GatherBlocksQ4KKernel", GatherBlocksKernel<kGgmlQ4_K>, dim3(GridFor(units, kBlock / 32)), dim3(kBlock), emb,
           rows, row_bytes, nb, toks, units, x);
    return;
  }
  if (type == kGgmlQ6_K && Aligned(emb, 2) && Aligned(x, 16)) {
    const int32_t nb = static_cast<int32_t>(cols / kQK_K);
    const int64_t units = seq * nb;
    Launch("GatherBlocksQ6KKernel", GatherBlocksKernel<kGgmlQ6_K>, dim3(GridFor(units, kBlock / 16)), dim3(kBlock), emb,
           rows, row_bytes, nb, toks, units, x);
    return;
  }
  if (type == kGgmlF32 && cols % 4 == 0 && Aligned(emb, 16) && Aligned(x, 16)) {
    const int64_t total4 = total / 4;
    Launch("GatherF32Kernel", GatherF32Kernel, dim3(GridFor(total4, kBlock)), dim3(kBlock),
           reinterpret_cast<const float*>(emb), rows, cols, toks, total4, x);
    return;
  }
  Launch("GatherElemKernel", GatherElemKernel, dim3(GridFor(total, kBlock)), dim3(kBlock), type, emb, rows, cols,
         row_bytes, bs.elems, bs.bytes, toks, total, x);
}

}  // namespace

void GpuDequantRow(uint32_t type, const uint8_t* src_dev, int64_t n_elems, float* dst_dev) {
  const BlockShape bs = DeviceBlockShape(type);
  RPG_CHECK(n_elems > 0 && n_elems % bs.elems == 0, "dequant: %lld elements do not fill whole blocks of %d",
            static_cast<long long>(n_elems), bs.elems);
  RPG_CHECK(src_dev != nullptr && dst_dev != nullptr, "DequantRow got a null pointer");
  LaunchGather(type, src_dev, 1, n_elems, nullptr, 1, dst_dev);
}

void GpuEmbeddingLookupRaw(uint32_t type, const uint8_t* emb_dev, int64_t rows, int64_t cols, const int32_t* toks_dev,
                           int64_t seq, float* x_dev) {
  RPG_CHECK(rows > 0 && cols > 0 && seq >= 0, "invalid EmbeddingLookup arguments");
  if (seq == 0) return;
  RPG_CHECK(emb_dev != nullptr && toks_dev != nullptr && x_dev != nullptr, "EmbeddingLookup got a null pointer");
  LaunchGather(type, emb_dev, rows, cols, toks_dev, seq, x_dev);
}

void GpuEmbeddingLookup(const GpuTensor& emb, const int32_t* toks_dev, int64_t seq, float* x_dev) {
  RPG_CHECK(emb.valid(), "EmbeddingLookup got an empty tensor");
  RPG_CHECK(emb.buf.size() >= static_cast<size_t>(emb.rows * emb.row_bytes()),
            "embedding buffer is smaller than its [%lld, %lld] shape", static_cast<long long>(emb.rows),
            static_cast<long long>(emb.cols));
  GpuEmbeddingLookupRaw(emb.type, static_cast<const uint8_t*>(emb.buf.data()), emb.rows, emb.cols, toks_dev, seq,
                        x_dev);
}

void GpuF16Sweep(float* out_dev) {
  RPG_CHECK(out_dev != nullptr, "F16Sweep got a null pointer");
  Launch("F16SweepKernel", F16SweepKernel, dim3(65536 / kBlock), dim3(kBlock), out_dev);
}

}  // namespace rpg
