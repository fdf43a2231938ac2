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

#include <atomic>

#include <cfloat>
#include <climits>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"
#include "matmul_mfma.h"
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
// Waves per workgroup of the one-token decode kernel (MatVecQuantKernel).
constexpr int kDecWaves = 4;
constexpr int kDecBlock = 64 * kDecWaves;

bool Aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

__device__ __forceinline__ float WaveSumF(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float WaveMaxF(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// 8 bytes starting `sh` (0 or 2) bytes into the 12-byte window w0..w2.
__device__ __forceinline__ uint2 Window8(uint3 w, uint32_t sh) {
  return make_uint2(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(w.z, w.y, sh));
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

// Q6_K blocks start at multiples of 210 bytes, so a block base is only 2-byte
// aligned. Each 8-byte field is read as the three aligned dwords around it
// (one dwordx3 load from the 4-aligned base ab = blk - sh) and byte-aligned.
// Every window lies inside the block except up to 2 bytes before its start,
// which share an aligned dword (hence a page) with the block's first bytes, so
// no window can touch memory outside pages the tensor occupies.
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
    const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(blk) & 3u);
    const uint8_t* ab = blk - sh;
    const uint3 f0 = *reinterpret_cast<const uint3*>(ab + 64 * h + lq);
    const uint3 f1 = *reinterpret_cast<const uint3*>(ab + 64 * h + 32 + lq);
    const uint3 fh = *reinterpret_cast<const uint3*>(ab + 128 + 32 * h + lq);
    // scales: dwords at ab + 192 + 8h, + 4, and + 8 (sh == 2) or + 4 again (sh == 0),
    // so the window never passes byte 209 of the block; the third address is
    // arithmetic, not a select, so all loads stay unconditional.
    const uint8_t* sp = ab + 192 + 8 * h;
    const uint3 fs = make_uint3(*reinterpret_cast<const uint32_t*>(sp), *reinterpret_cast<const uint32_t*>(sp + 4),
                                *reinterpret_cast<const uint32_t*>(sp + 4 + 2 * sh));
    const uint2 ql0 = Window8(f0, sh);
    const uint2 ql1 = Window8(f1, sh);
    const uint2 qh = Window8(fh, sh);
    const uint2 sc = Window8(fs, sh);
    r.a = make_uint4(ql0.x, ql0.y, ql1.x, ql1.y);
    r.b = make_uint4(qh.x, qh.y, sc.x, sc.y);
    r.d6 = *reinterpret_cast<const uint16_t*>(blk + 208);
  }
  return r;
}

// Byte k of a word as an exact float (v_cvt_f32_ubyte{0..3}).
__device__ __forceinline__ float UByteF(uint32_t w, int k) { return static_cast<float>((w >> (8 * k)) & 0xFFu); }

// The four bytes of a word whose bytes are all below 16 (4-bit quants), as the
// exact floats q * 2^-9, two per instruction (v_cvt_pk_f32_fp8): gfx950 reads a
// byte as an OCP FP8 E4M3 value, whose subnormals are m * 2^-9 (m = 0..7) and
// whose smallest binade is (8 + m) * 2^-9, so every byte 0..15 is q * 2^-9
// (checked on the device for all sixteen). The caller scales the block factor by
// 2^9 instead, which is exact, so each product and sum is the unscaled one times
// 2^-9: the same roundings, hence the same bits, as with q itself, except where
// a partial sum would fall below 2^-126 (activations of magnitude < ~2^-117).
typedef float F32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void NibblesF(uint32_t w, float (&f)[4]) {
  const F32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const F32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  f[0] = a.x;
  f[1] = a.y;
  f[2] = b.x;
  f[3] = b.y;
}
constexpr float kNibbleScale = 512.0f;  // 2^9: undoes NibblesF's factor

// Hides a packed-quant word's known-zero bits from the optimiser, which would
// otherwise extract each field with a bit-field extract and then convert it (two
// instructions per weight) instead of converting the byte directly (one). Emits
// no instruction.
__device__ __forceinline__ uint32_t Opaque(uint32_t w) {
  __asm__("" : "+v"(w));
  return w;
}

// The lane's 32 weights, in the same order as LoadLaneX's activations.
//
// Bit-exact with the reference's separately rounded ops, with one fused
// multiply-add per weight: d and dmin are fp16 values (11 significant bits), the
// 6-bit scale / min and the 4- or 6-bit quants are small integers, so
//   Q4_K: d * sc and dmin * m need <= 17 bits, (d * sc) * q <= 21 bits: all exact
//         in fp32, and fma(d * sc, q, -(dmin * m)) rounds once, exactly where
//         fl(fl(d * sc) * q) - fl(dmin * m) does;
//   Q6_K: d * sc needs <= 18 bits and (d * sc) * (q - 32) <= 24 bits: exact, and
//         fma(d * sc, q, -32 * (d * sc)) equals it (32 * ds is exact too).
// Infinities, NaNs and signed zeros come out the same way in both forms.
template <uint32_t kType>
__device__ __forceinline__ void DecodeLane(const LaneBytes& r, int s, float (&wv)[32]) {
  if (kType == kGgmlQ4_K) {
    const int g = s >> 1;
    const float d = HalfBitsToFloat(r.a.x & 0xFFFFu);
    const float dmin = HalfBitsToFloat(r.a.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    ScaleMinK4(2 * g, r.a.y, r.a.z, r.a.w, &sc0, &m0);
    ScaleMinK4(2 * g + 1, r.a.y, r.a.z, r.a.w, &sc1, &m1);
    // (d * sc * 2^9) * (q * 2^-9) is the exact d * sc * q inside the fma
    const float d1 = (d * static_cast<float>(sc0)) * kNibbleScale;
    const float n1 = -(dmin * static_cast<float>(m0));
    const float d2 = (d * static_cast<float>(sc1)) * kNibbleScale;
    const float n2 = -(dmin * static_cast<float>(m1));
    const uint32_t qw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float lo[4], hi[4];
      NibblesF(qw[k] & 0x0F0F0F0Fu, lo);
      NibblesF((qw[k] >> 4) & 0x0F0F0F0Fu, hi);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wv[4 * k + j] = __builtin_fmaf(d1, lo[j], n1);
        wv[16 + 4 * k + j] = __builtin_fmaf(d2, hi[j], n2);
      }
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
      const float off = -32.0f * ds;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        // the 6-bit quants of 4 consecutive elements, one per byte
        const uint32_t nib = ((q < 2 ? ql[q & 1][k] : ql[q & 1][k] >> 4)) & 0x0F0F0F0Fu;
        const uint32_t hi2 = (2 * q >= 4 ? qh[k] >> (2 * q - 4) : qh[k] << (4 - 2 * q)) & 0x30303030u;
        const uint32_t q6 = Opaque(nib | hi2);
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[8 * q + 4 * k + j] = __builtin_fmaf(ds, UByteF(q6, j), off);
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

// A lane's field offsets inside a row (bytes from the row's first byte), for rows
// that start at a multiple of 4 bytes (Q4_K rows always do; Q6_K rows when the
// matrix base and the row size are multiples of 4). They do not change from row
// to row, so each load is the row's wave-uniform address plus a 32-bit lane offset
// and an immediate: no per-row address arithmetic on the vector unit.
struct LaneOffs {
  uint32_t a;   // Q4_K: the block header; Q6_K: the aligned dword before ql run 0 (run 1 at +32)
  uint32_t b;   // Q4_K: the lane's 16 qs bytes; Q6_K: the aligned dword before the qh run
  uint32_t c;   // Q6_K: the first scale dword (the second at +4)
  uint32_t c3;  // Q6_K: the third scale dword (+4 again when the block is 4-aligned)
  uint32_t d;   // Q6_K: d
  uint32_t sh;  // Q6_K: the block's byte offset inside its aligned dword (0 or 2)
};

template <uint32_t kType>
__device__ __forceinline__ LaneOffs MakeLaneOffs(uint32_t blk_off, int s) {
  LaneOffs o;
  if (kType == kGgmlQ4_K) {
    o.a = blk_off;
    o.b = blk_off + 16 + 32 * (s >> 1) + 16 * (s & 1);
    o.c = o.c3 = o.d = o.sh = 0;
  } else {
    const uint32_t h = static_cast<uint32_t>(s >> 2);
    const uint32_t lq = 8u * static_cast<uint32_t>(s & 3);
    o.sh = blk_off & 3u;
    const uint32_t ab = blk_off - o.sh;
    o.a = ab + 64 * h + lq;
    o.b = ab + 128 + 32 * h + lq;
    o.c = ab + 192 + 8 * h;
    o.c3 = o.c + 4 + 2 * o.sh;
    o.d = blk_off + 208;
  }
  return o;
}

// LoadLaneBytes for rows that start at a multiple of 4 bytes, through a buffer
// resource on the matrix (wave-uniform), the row's byte offset in a scalar
// register and the lane's row-invariant offsets: same bytes, same windows.
typedef unsigned int LbU32x3 __attribute__((ext_vector_type(3)));
typedef unsigned int LbU32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int LbU32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t MatrixResource(const uint8_t* base) {
  // 0x00020000: raw (untyped) buffer, 32-bit data format; no record limit (the
  // row offsets stay below 2^31, and every field read lies inside its block's
  // aligned dwords).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), static_cast<short>(0), -1, 0x00020000);
}

template <uint32_t kType>
__device__ __forceinline__ LaneBytes LoadLaneBytesBuf(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, const LaneOffs& o) {
  LaneBytes r;
  if (kType == kGgmlQ4_K) {
    const LbU32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(o.a), static_cast<int>(row_off), 0);
    const LbU32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(o.b), static_cast<int>(row_off), 0);
    r.a = make_uint4(a.x, a.y, a.z, a.w);
    r.b = make_uint4(b.x, b.y, b.z, b.w);
    r.d6 = 0;
  } else {
    const LbU32x3 f0 = __builtin_amdgcn_raw_buffer_load_b96(rs, static_cast<int>(o.a), static_cast<int>(row_off), 0);
    const LbU32x3 f1 = __builtin_amdgcn_raw_buffer_load_b96(rs, static_cast<int>(o.a + 32), static_cast<int>(row_off), 0);
    const LbU32x3 fh = __builtin_amdgcn_raw_buffer_load_b96(rs, static_cast<int>(o.b), static_cast<int>(row_off), 0);
    const LbU32x2 s01 = __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<int>(o.c), static_cast<int>(row_off), 0);
    const uint32_t s2 = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(o.c3), static_cast<int>(row_off), 0);
    const uint16_t d = __builtin_amdgcn_raw_buffer_load_b16(rs, static_cast<int>(o.d), static_cast<int>(row_off), 0);
    const uint2 ql0 = Window8(make_uint3(f0.x, f0.y, f0.z), o.sh);
    const uint2 ql1 = Window8(make_uint3(f1.x, f1.y, f1.z), o.sh);
    const uint2 qh = Window8(make_uint3(fh.x, fh.y, fh.z), o.sh);
    const uint2 sc = Window8(make_uint3(s01.x, s01.y, s2), o.sh);
    r.a = make_uint4(ql0.x, ql0.y, ql1.x, ql1.y);
    r.b = make_uint4(qh.x, qh.y, sc.x, sc.y);
    r.d6 = d;
  }
  return r;
}

// ---------------------------------------------------------------- decode (one token)
//
// One token, rows of at most 16 super-blocks (cols <= 4096: every Qwen3-1.7B /
// 4B matrix except ffn_down): persistent waves. Each lane loads its 32 (or 64)
// activations once and keeps them in registers, then the wave walks rows
// wave, wave + W, ... (W = all waves of the grid), RI rows per step, with the
// next step's weight bytes in flight while the current ones are decoded.
//
// Per-weight work is one byte-to-float conversion and one fused multiply-add:
//   Q6_K: the 6-bit quant q becomes the signed byte 4(q - 32) = ((q << 2) ^ 0x80)
//         (converted exactly with a sign-extending byte select), and a group of 8
//         weights sharing a scale contributes (d * sc / 4) * sum_i 4(q_i - 32) x_i.
//         d * sc / 4 is exact, so this differs from summing the dequantised
//         weights w_i = d * sc * (q_i - 32) (also exact) only in rounding order.
//   Q4_K: w_i = d1 q_i - m1 per sub-block, so a lane's 16 weights of one
//         sub-block contribute d1 * sum_i q_i x_i - m1 * sum_i x_i, with the
//         activation sums taken once per kernel. The two products can partly
//         cancel, so the error bound of this form is in terms of
//         sum_i (|d1 q_i| + |m1|) |x_i| rather than sum_i |w_i x_i|.
// The RI row sums are then reduced together: two cross-half exchanges leave each
// 16-lane row of the wave with one of the RI rows, and DPP steps finish the sum.

__device__ __forceinline__ float DppAdd(float v, int ctrl_sel) {
  int m;
  switch (ctrl_sel) {
    case 0: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
    case 1: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad_perm 2,3,0,1
    case 2: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false); break; // row_mirror
  }
  return v + __int_as_float(m);
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the total.
__device__ __forceinline__ float RowSum16(float v) {
  v = DppAdd(v, 0);
  v = DppAdd(v, 1);
  v = DppAdd(v, 2);
  return DppAdd(v, 3);
}

// Reduces RI (1, 2 or 4) per-lane values over the wave. Afterwards lane l holds
// the total of row (l >> 4) & (RI - 1) (for RI == 1: every lane holds row 0).
template <int RI>
__device__ __forceinline__ float ReduceRows(const float (&v)[RI], int lane) {
  if (RI == 1) {
    float a = RowSum16(v[0]);
    a += __shfl_xor(a, 16, 64);
    return a + __shfl_xor(a, 32, 64);
  } else if (RI == 2) {
    const bool hi = (lane & 16) != 0;
    float a = (hi ? v[1] : v[0]) + __shfl_xor(hi ? v[0] : v[1], 16, 64);
    a += __shfl_xor(a, 32, 64);
    return RowSum16(a);
  } else {
    const bool b5 = (lane & 32) != 0;
    const bool b4 = (lane & 16) != 0;
    // lanes with bit 5 set keep rows 2, 3; the others rows 0, 1
    const float k0 = b5 ? v[2] : v[0];
    const float k1 = b5 ? v[3] : v[1];
    const float s0 = b5 ? v[0] : v[2];
    const float s1 = b5 ? v[1] : v[3];
    const float n0 = k0 + __shfl_xor(s0, 32, 64);
    const float n1 = k1 + __shfl_xor(s1, 32, 64);
    // bit 4 picks one of the two
    const float a = (b4 ? n1 : n0) + __shfl_xor(b4 ? n0 : n1, 16, 64);
    return RowSum16(a);
  }
}

// Row index (0..RI-1) whose total lane `lane` holds after ReduceRows.
template <int RI>
__device__ __forceinline__ int ReducedRow(int lane) {
  return RI == 1 ? 0 : (RI == 2 ? (lane >> 4) & 1 : (((lane >> 5) & 1) << 1) | ((lane >> 4) & 1));
}

// Signed byte k of a word as an exact float (sign-extending byte select).
__device__ __forceinline__ float SByteF(uint32_t w, int k) {
  return static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(w >> (8 * k))));
}

// Lane contribution of one block for one row, given resident activations.
// sx: Q4_K only, the lane's activation sums (low-nibble run, high-nibble run).
template <uint32_t kType>
__device__ __forceinline__ float BlockDot(const LaneBytes& r, int s, const float (&xv)[32], const float (&sx)[2]) {
  if (kType == kGgmlQ4_K) {
    const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.a.x & 0xFFFFu)));
    const float dmin = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.a.x >> 16)));
    // Lane s of the block's 8 lanes decodes sub-block s's scale and min and forms
    // its two factors; lane s needs sub-blocks 2 (s >> 1) and 2 (s >> 1) + 1,
    // which lanes s & ~1 and s | 1 of its quad hold (DPP quad_perm [0,0,2,2] and
    // [1,1,3,3]). Same factors, same bits, as decoding both here. The 8 lanes of
    // a block take the same branches, so their quads are whole.
    uint32_t scs, ms;
    ScaleMinK4(s, r.a.y, r.a.z, r.a.w, &scs, &ms);
    const float fa = (d * kNibbleScale) * static_cast<float>(scs);
    const float fb = -(dmin * static_cast<float>(ms));
    const float a0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(fa), 0xA0, 0xF, 0xF, false));
    const float b0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(fb), 0xA0, 0xF, 0xF, false));
    const float a1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(fa), 0xF5, 0xF, 0xF, false));
    const float b1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(fb), 0xF5, 0xF, 0xF, false));
    const uint32_t qw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    float slo = 0.0f, shi = 0.0f;  // 2^-9 sum(q x) of the two runs
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float lo[4], hi[4];
      NibblesF(qw[k] & 0x0F0F0F0Fu, lo);
      NibblesF((qw[k] >> 4) & 0x0F0F0F0Fu, hi);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        slo = __builtin_fmaf(lo[j], xv[4 * k + j], slo);
        shi = __builtin_fmaf(hi[j], xv[16 + 4 * k + j], shi);
      }
    }
    float acc = a0 * slo;
    acc = __builtin_fmaf(b0, sx[0], acc);
    acc = __builtin_fmaf(a1, shi, acc);
    return __builtin_fmaf(b1, sx[1], acc);
  } else {
    // Bytes 4(q6 - 32) = (q6 << 2) ^ 0x80 as signed int8, q6 = nib | h << 4, built
    // in place: bits 2-5 the low nibble (ql shifted by 2 either way), bits 6-7 the
    // 2-bit high part h (qh shifted so that field q lands there), the ^ 0x80
    // applied to all of qh once (it flips the top bit of every 2-bit field). The
    // group factor d * sc / 4 = (d / 4) * sc is exact either way.
    const int is = (s & 3) >> 1;
    const float d4 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.d6))) * 0.25f;
    const uint32_t ql[2][2] = {{r.a.x, r.a.y}, {r.a.z, r.a.w}};
    const uint32_t qhx[2] = {r.b.x ^ 0xAAAAAAAAu, r.b.y ^ 0xAAAAAAAAu};
    // scale is + 2 q of the half's eight: byte 2 (q & 1) of scs[q >> 1]
    const uint32_t scs[2] = {r.b.z >> (8 * is), r.b.w >> (8 * is)};
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float dsc = d4 * SByteF(scs[q >> 1], 2 * (q & 1));
      float part = 0.0f;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint32_t lo = q < 2 ? ql[q & 1][k] << 2 : ql[q & 1][k] >> 2;
        const uint32_t hi = qhx[k] << (6 - 2 * q);
        const uint32_t b = Opaque((lo & 0x3C3C3C3Cu) | (hi & 0xC0C0C0C0u));
#pragma unroll
        for (int j = 0; j < 4; ++j) part = __builtin_fmaf(SByteF(b, j), xv[8 * q + 4 * k + j], part);
      }
      acc = __builtin_fmaf(dsc, part, acc);
    }
    return acc;
  }
}

// Sums of each lane's two 16-activation runs (Q4_K's low- and high-nibble runs).
__device__ __forceinline__ void RunSums(const float (&xv)[32], float (&sx)[2]) {
  float a = 0.0f, z = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    a += xv[i];
    z += xv[16 + i];
  }
  sx[0] = a;
  sx[1] = z;
}

// Up to kMaxSegs matrices of one type and width decoded as one row space: rows
// [end[i-1], end[i]) are matrix i (w[i], out[i]); unused ends are INT64_MAX. A
// single matrix is one segment.
constexpr int kMaxSegs = 4;
struct MatSegs {
  const uint8_t* w[kMaxSegs];
  float* out[kMaxSegs];
  int64_t end[kMaxSegs];
  uint32_t b_mask;      // segments of the kernel's second type (bit i: segment i)
  int64_t row_bytes_b;  // row bytes of those segments
};

// Residual + RMSNorm in front of a one-token matvec: the activations a wave
// holds are h = RMSNorm(x + d) * w instead of x. d == nullptr: h = RMSNorm(x) * w.
// x_out != nullptr: the first workgroup also writes x + d there (the updated residual
// stream; it must not alias x or d, which other waves are still reading).
struct NormPrologue {
  const float* d;
  const float* w;
  float* x_out;
  float eps;
};

// The first three segment ends clamped to 32 bits (the launcher keeps every row
// index below 2^31), so the per-row segment lookup compares in scalar registers:
// the scalar unit has no ordered 64-bit compare, and 64-bit ones run on the
// vector unit.
struct SegEnds32 {
  int32_t e[3];
};
__device__ __forceinline__ SegEnds32 Ends32(const MatSegs& sg) {
  SegEnds32 r;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.e[i] = static_cast<int32_t>(sg.end[i] < INT32_MAX ? sg.end[i] : INT32_MAX);
  return r;
}
// Segment of global row r (uniform over the wave, so scalar).
__device__ __forceinline__ int SegOf(const SegEnds32& se, int64_t r) {
  const int32_t r32 = static_cast<int32_t>(r);
  return (r32 >= se.e[0]) + (r32 >= se.e[1]) + (r32 >= se.e[2]);
}

// a[i] through selects over constant indices. Indexing the kernel-argument
// arrays with a runtime i makes the compiler issue one more scalar load that
// waits for i; with constant indices every field is fetched in the kernel's first
// batch of argument loads, so the first weight load waits on one round trip
// instead of a chain of four or five.
template <typename T>
__device__ __forceinline__ T PickSeg(const T (&a)[kMaxSegs], int i) {
  static_assert(kMaxSegs == 4, "PickSeg selects among four segments");
  return i == 0 ? a[0] : i == 1 ? a[1] : i == 2 ? a[2] : a[3];
}
// First global row of segment i (0 for the first segment).
__device__ __forceinline__ int64_t SegFirst(const MatSegs& sg, int i) {
  return i == 0 ? 0 : i == 1 ? sg.end[0] : i == 2 ? sg.end[1] : sg.end[2];
}

// Each lane keeps the activations of its NX block groups in registers (rows of
// up to 8 * NX blocks; used for NX == 1). Rows run over all segments; a row
// group of RI rows never straddles two (segment sizes are multiples of RI).
// kPaired (RI == 2): the layer's gate / up pair. Virtual rows 2p and 2p + 1 are
// row p of w[0] (gate) and of w[1] (up), and out[0][p] = silu(gate) * up, the
// SwiGLU formed from the two row totals (each total the same bits as an
// unpaired launch computes for that row).
// kTypeB != kType: segments in sg.b_mask are matrices of kTypeB (a layer's
// Q6_K attn_v beside its Q4_K q / k in Q4_K_M files). Each lane then holds its
// activations in both types' lane orders, and a row pair takes the path of its
// segment's type (uniform over the wave): every row the same bits as a launch
// of its own type.
// kNorm (rows of at most kGroups blocks): x is the residual stream and each
// workgroup forms h = RMSNorm(x + nrm.d) * nrm.w itself, the GpuAddRmsNorm
// maths (double sum of squares, float(1 / sqrt(ss / n + eps)), then
// (v * scale) * w), before the dot products; the sum of squares is taken in
// another order than GpuAddRmsNorm's, so the scale can differ from it in the
// last bit of the double sum.
// kAl4: every row of every segment starts at a multiple of 4 bytes and lies below
// 2^31 bytes from its segment's base (checked by the launcher), so the weight
// loads take the buffer form of LoadLaneBytesBuf.
template <uint32_t kType, int NX, int RI, bool kPaired = false, uint32_t kTypeB = kType, bool kNorm = false,
          bool kAl4 = false>
__global__ __launch_bounds__(kDecBlock) void MatVecQuantKernel(MatSegs sg, int64_t rows, int64_t row_bytes, int32_t nb,
                                                              const float* __restrict__ x, NormPrologue nrm) {
  static_assert(!kNorm || NX == 1, "the norm prologue needs the whole row in one wave");
  constexpr int64_t kBB = BlockBytesOf<kType>::value;
  constexpr bool kMixed = kTypeB != kType;
  constexpr int64_t kBBB = BlockBytesOf<kTypeB>::value;
  const int lane = threadIdx.x & 63;
  const int c = lane / kGroupLanes;
  const int s = lane % kGroupLanes;
  // Every kernel argument the first activation and weight loads depend on, fetched
  // in one batch: the empty asm takes them as scalar inputs (it emits nothing), so
  // the compiler issues their loads together at entry instead of one at a time
  // next to each use, where each waited for the one before (4-5 serial scalar
  // round trips before the first weight load).
  asm volatile("" ::"s"(sg.w[0]), "s"(sg.w[1]), "s"(sg.w[2]), "s"(sg.w[3]), "s"(sg.end[0]), "s"(sg.end[1]),
               "s"(sg.end[2]), "s"(rows), "s"(row_bytes), "s"(nb), "s"(x));

  const SegEnds32 se = Ends32(sg);
  // Row bookkeeping is uniform over the wave: keep it in scalar registers.
  // (32-bit: the launcher keeps rows + stride below 2^31, and the scalar unit
  // compares 32-bit values only.)
  const int32_t nrows = static_cast<int32_t>(rows);
  const int32_t stride = static_cast<int32_t>(gridDim.x) * kDecWaves * RI;
  int32_t r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * kDecWaves + (threadIdx.x >> 6))) * RI;
  // No early exit for waves past the last row: a branch here would keep the
  // compiler from fetching the remaining kernel arguments in the first batch. Such
  // waves load the last row's bytes (the load below clamps the row) and skip the
  // row loop.

  float xv[NX][32];
  float sx[NX][2];
  int64_t lane_off[NX];  // byte offset of this lane's block inside a row (clamped to the last block)
  float xvb[kMixed ? NX : 1][32];  // the same activations in kTypeB's lane order
  float sxb[kMixed ? NX : 1][2];
  int64_t lane_off_b[kMixed ? NX : 1];
  LaneOffs offs[NX];
  LaneOffs offs_b[kMixed ? NX : 1];
  if (kNorm) {
    // The workgroup forms h once: each thread takes 4-float slices of the row,
    // the sum of squares meets in LDS (waves added in a fixed order), and h is
    // staged in LDS, from where each wave reads its lanes' elements.
    __shared__ float hs[kGroups * kQK_K];
    __shared__ double part[kDecWaves];
    static_assert(kGroups * kQK_K <= 8 * kDecBlock, "two float4 per thread cover the row");
    const int n = nb * kQK_K;  // <= kGroups * kQK_K
    float4 v[2], wv[2];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 4 * static_cast<int>(threadIdx.x) + 4 * kDecBlock * j;
      if (i < n) {
        v[j] = dev::Load4(x + i);
        if (nrm.d != nullptr) {
          const float4 dd = dev::Load4(nrm.d + i);
          v[j] = make_float4(v[j].x + dd.x, v[j].y + dd.y, v[j].z + dd.z, v[j].w + dd.w);
        }
        wv[j] = dev::Load4(nrm.w + i);
        ss = dev::AddSquares(ss, v[j]);
        if (nrm.x_out != nullptr && blockIdx.x == 0) dev::Store4(nrm.x_out + i, v[j]);
      }
    }
    ss = dev::WaveSum(ss);
    if (lane == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    double total = part[0];
#pragma unroll
    for (int q = 1; q < kDecWaves; ++q) total += part[q];
    const float scale = dev::RmsScale(total, n, nrm.eps);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 4 * static_cast<int>(threadIdx.x) + 4 * kDecBlock * j;
      if (i < n) dev::Store4(hs + i, dev::ScaleMul(v[j], scale, wv[j]));
    }
    __syncthreads();
    const bool live = c < nb;
    lane_off[0] = static_cast<int64_t>(live ? c : nb - 1) * kBB;
    if (live) {
      LoadLaneX<kType>(hs, static_cast<int64_t>(c) * kQK_K, s, xv[0]);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) xv[0][i] = 0.0f;
    }
    RunSums(xv[0], sx[0]);
    if (kMixed) {
      lane_off_b[0] = static_cast<int64_t>(live ? c : nb - 1) * kBBB;
      if (live) {
        LoadLaneX<kTypeB>(hs, static_cast<int64_t>(c) * kQK_K, s, xvb[0]);
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) xvb[0][i] = 0.0f;
      }
      RunSums(xvb[0], sxb[0]);
    }
    if (r0 >= nrows) return;  // after the workgroup's barriers
  }
#pragma unroll
  for (int it = 0; it < (kNorm ? 0 : NX); ++it) {
    const int b = c + kGroups * it;
    lane_off[it] = static_cast<int64_t>(b < nb ? b : nb - 1) * kBB;
    if (b < nb) {
      LoadLaneX<kType>(x, static_cast<int64_t>(b) * kQK_K, s, xv[it]);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) xv[it][i] = 0.0f;
    }
    RunSums(xv[it], sx[it]);
    if (kMixed) {
      lane_off_b[it] = static_cast<int64_t>(b < nb ? b : nb - 1) * kBBB;
      if (b < nb) {
        LoadLaneX<kTypeB>(x, static_cast<int64_t>(b) * kQK_K, s, xvb[it]);
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) xvb[it][i] = 0.0f;
      }
      RunSums(xvb[it], sxb[it]);
    }
  }

#pragma unroll
  for (int it = 0; it < NX; ++it) {
    offs[it] = MakeLaneOffs<kType>(static_cast<uint32_t>(lane_off[it]), s);
    if (kMixed) offs_b[it] = MakeLaneOffs<kTypeB>(static_cast<uint32_t>(lane_off_b[it]), s);
  }

  // Rows past the end are clamped to the last row (loads stay in bounds; results are dropped).
  auto load = [&](int32_t base_row, LaneBytes (&lb)[RI][NX]) {
    if (kPaired) {
      const int64_t p = (base_row < nrows ? base_row : nrows - 2) >> 1;
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        if (kAl4) {
          const __amdgpu_buffer_rsrc_t rs = MatrixResource(sg.w[r]);
          const uint32_t ro = static_cast<uint32_t>(p * row_bytes);
#pragma unroll
          for (int it = 0; it < NX; ++it) lb[r][it] = LoadLaneBytesBuf<kType>(rs, ro, offs[it]);
        } else {
          const uint8_t* rp = sg.w[r] + p * row_bytes;
#pragma unroll
          for (int it = 0; it < NX; ++it) lb[r][it] = LoadLaneBytes<kType>(rp + lane_off[it], s);
        }
      }
      return;
    }
    // base_row is clamped before the segment lookup: past the last row the lookup
    // would name an unused (null) segment, and the row offset from its first row
    // would be negative.
    const int32_t br = base_row < nrows ? base_row : nrows - 1;
    const int sgi = SegOf(se, br);
    const uint8_t* wseg = PickSeg(sg.w, sgi);
    const int64_t first = SegFirst(sg, sgi);
    if (kMixed && ((sg.b_mask >> sgi) & 1u)) {
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        const int64_t row = br + r < nrows ? br + r : nrows - 1;
        if (kAl4) {
          const uint32_t ro = static_cast<uint32_t>((row - first) * sg.row_bytes_b);
#pragma unroll
          for (int it = 0; it < NX; ++it) lb[r][it] = LoadLaneBytesBuf<kTypeB>(MatrixResource(wseg), ro, offs_b[it]);
        } else {
          const uint8_t* rp = wseg + (row - first) * sg.row_bytes_b;
#pragma unroll
          for (int it = 0; it < NX; ++it) lb[r][it] = LoadLaneBytes<kTypeB>(rp + lane_off_b[it], s);
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      const int64_t row = br + r < nrows ? br + r : nrows - 1;
      if (kAl4) {
        const uint32_t ro = static_cast<uint32_t>((row - first) * row_bytes);
#pragma unroll
        for (int it = 0; it < NX; ++it) lb[r][it] = LoadLaneBytesBuf<kType>(MatrixResource(wseg), ro, offs[it]);
      } else {
        const uint8_t* rp = wseg + (row - first) * row_bytes;
#pragma unroll
        for (int it = 0; it < NX; ++it) lb[r][it] = LoadLaneBytes<kType>(rp + lane_off[it], s);
      }
    }
  };

  // One row step on bytes already loaded.
  auto step = [&](const LaneBytes (&cur)[RI][NX], int32_t rs) {
    float acc[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) acc[r] = 0.0f;
    const bool row_b = kMixed && ((sg.b_mask >> SegOf(se, rs)) & 1u);
#pragma unroll
    for (int it = 0; it < NX; ++it) {
      if (c + kGroups * it < nb) {
        if (row_b) {
#pragma unroll
          for (int r = 0; r < RI; ++r) acc[r] += BlockDot<kTypeB>(cur[r][it], s, xvb[it], sxb[it]);
        } else {
#pragma unroll
          for (int r = 0; r < RI; ++r) acc[r] += BlockDot<kType>(cur[r][it], s, xv[it], sx[it]);
        }
      }
    }
    const float total = ReduceRows<RI>(acc, lane);
    if (kPaired) {
      // lanes 0 and 16 hold the gate and up totals of pair rs / 2
      const float g = __shfl(total, 0, 64);
      const float u = __shfl(total, 16, 64);
      if (lane == 0) sg.out[0][rs >> 1] = dev::SiluMul(g, u);
    } else {
      const int rr = ReducedRow<RI>(lane);
      const int sgi = SegOf(se, rs);
      const int64_t first = SegFirst(sg, sgi);
      if ((lane & 15) == 0 && lane < 16 * RI && rs + rr < nrows) PickSeg(sg.out, sgi)[rs - first + rr] = total;
    }
  };
  if constexpr (kMixed) {
    // Two register sets used in turn, so no loaded byte is copied: with both
    // types' decode paths in the loop, the copy of the next step's bytes cost
    // more than the second set (q / k / v of a Q4_K_M layer: 5.5 -> 4.9 us; the
    // single-type kernels measured slower this way).
    LaneBytes ba[RI][NX], bb[RI][NX];
    load(r0, ba);
    while (r0 < nrows) {
      const int32_t r1 = r0 + stride;
      if (r1 < nrows) load(r1, bb);
      step(ba, r0);
      if (r1 >= nrows) break;
      r0 = r1 + stride;
      if (r0 < nrows) load(r0, ba);
      step(bb, r1);
    }
  } else {
    LaneBytes cur[RI][NX];
    load(r0, cur);
    for (; r0 < nrows; r0 += stride) {
      LaneBytes nxt[RI][NX];
      load(r0 + stride < nrows ? r0 + stride : r0, nxt);
      step(cur, r0);
#pragma unroll
      for (int r = 0; r < RI; ++r)
#pragma unroll
        for (int it = 0; it < NX; ++it) cur[r][it] = nxt[r][it];
    }
  }
}

// Wide rows (9 to 64 blocks; e.g. ffn_down, 4B projections): the WS waves of a
// workgroup share RI rows, wave q taking the block groups q, q + WS, ... (a
// group is 8 consecutive blocks, one per lane group), so a matrix with few rows
// still fills the chip. Each wave keeps the activations of its NXW groups in
// registers and reduces its partial sums; the WS partials of a row meet in LDS
// and wave 0 adds them in wave order, so results are deterministic.
template <uint32_t kType, int WS, int NXW, int RI, bool kAl4 = false>
__global__ __launch_bounds__(64 * WS) void MatVecSplitKernel(const uint8_t* __restrict__ w, int64_t rows,
                                                             int64_t row_bytes, int32_t nb,
                                                             const float* __restrict__ x, float* __restrict__ out) {
  constexpr int64_t kBB = BlockBytesOf<kType>::value;
  __shared__ float part[WS][RI];
  const int lane = threadIdx.x & 63;
  const int q = threadIdx.x >> 6;
  const int c = lane / kGroupLanes;
  const int s = lane % kGroupLanes;
  // The kernel arguments in one batch at entry (see MatVecQuantKernel).
  asm volatile("" ::"s"(w), "s"(rows), "s"(row_bytes), "s"(nb), "s"(x), "s"(out));
  const int64_t stride = static_cast<int64_t>(gridDim.x) * RI;
  int64_t r0 = static_cast<int64_t>(blockIdx.x) * RI;  // uniform over the workgroup

  float xv[NXW][32];
  float sx[NXW][2];
  int64_t lane_off[NXW];
  bool valid[NXW];
#pragma unroll
  for (int it = 0; it < NXW; ++it) {
    const int b = c + kGroups * (q + WS * it);
    valid[it] = b < nb;
    lane_off[it] = static_cast<int64_t>(valid[it] ? b : nb - 1) * kBB;
    if (valid[it]) {
      LoadLaneX<kType>(x, static_cast<int64_t>(b) * kQK_K, s, xv[it]);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) xv[it][i] = 0.0f;
    }
    RunSums(xv[it], sx[it]);
  }

  LaneOffs offs[NXW];
#pragma unroll
  for (int it = 0; it < NXW; ++it) offs[it] = MakeLaneOffs<kType>(static_cast<uint32_t>(lane_off[it]), s);

  auto load = [&](int64_t base_row, LaneBytes (&lb)[RI][NXW]) {
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      const int64_t row = base_row + r < rows ? base_row + r : rows - 1;
      if (kAl4) {
        const uint32_t ro = static_cast<uint32_t>(row * row_bytes);
#pragma unroll
        for (int it = 0; it < NXW; ++it) lb[r][it] = LoadLaneBytesBuf<kType>(MatrixResource(w), ro, offs[it]);
      } else {
        const uint8_t* rp = w + row * row_bytes;
#pragma unroll
        for (int it = 0; it < NXW; ++it) lb[r][it] = LoadLaneBytes<kType>(rp + lane_off[it], s);
      }
    }
  };

  LaneBytes cur[RI][NXW];
  load(r0 < rows ? r0 : 0, cur);
  for (; r0 < rows; r0 += stride) {
    LaneBytes nxt[RI][NXW];
    load(r0 + stride < rows ? r0 + stride : r0, nxt);
    float acc[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int it = 0; it < NXW; ++it) {
      if (valid[it]) {
#pragma unroll
        for (int r = 0; r < RI; ++r) acc[r] += BlockDot<kType>(cur[r][it], s, xv[it], sx[it]);
      }
    }
    const float total = ReduceRows<RI>(acc, lane);
    const int rr = ReducedRow<RI>(lane);
    if ((lane & 15) == 0 && lane < 16 * RI) part[q][rr] = total;
    __syncthreads();
    if (q == 0 && lane < RI && r0 + lane < rows) {
      float v = part[0][lane];
#pragma unroll
      for (int k = 1; k < WS; ++k) v += part[k][lane];
      out[r0 + lane] = v;
    }
    __syncthreads();  // part is rewritten by the next row step
#pragma unroll
    for (int r = 0; r < RI; ++r)
#pragma unroll
      for (int it = 0; it < NXW; ++it) cur[r][it] = nxt[r][it];
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

// Decode: persistent waves, 2 rows per step (4 for Q4_K matrices of 32768 rows
// or more), at most kDecodeWaves waves (16 per CU).
constexpr int64_t kDecodeWaves = 4096;

// Whether every row of the launch starts at a multiple of 4 bytes and below 2^31
// bytes from its segment's base (the buffer-load form of the decode kernels).
bool RowsAligned4(const MatSegs& sg, int32_t n_seg, int64_t row_bytes, bool paired) {
  const int64_t lim = int64_t(1) << 31;
  if (paired) {
    const int64_t pairs = sg.end[0] / 2;
    return (row_bytes & 3) == 0 && (reinterpret_cast<uintptr_t>(sg.w[0]) & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(sg.w[1]) & 3) == 0 && pairs * row_bytes < lim;
  }
  for (int32_t i = 0; i < n_seg; ++i) {
    const int64_t rb = ((sg.b_mask >> i) & 1u) ? sg.row_bytes_b : row_bytes;
    const int64_t first = i == 0 ? 0 : sg.end[i - 1];
    if ((rb & 3) != 0 || (reinterpret_cast<uintptr_t>(sg.w[i]) & 3) != 0 || (sg.end[i] - first) * rb >= lim) {
      return false;
    }
  }
  return true;
}

// nrm != nullptr: the launch forms the norm itself (x is then the residual
// stream); nrm->x_out is cleared afterwards, so a group of launches writes the
// updated residual once.
template <uint32_t kType, int RI, bool kPaired = false, uint32_t kTypeB = kType>
void LaunchDecodeSegs(const char* name, const MatSegs& sg, int32_t n_seg, int64_t row_bytes, int32_t nb,
                      const float* x, NormPrologue* nrm = nullptr) {
  const int64_t rows = sg.end[n_seg - 1];
  RPG_CHECK(rows < (int64_t(1) << 31) - kDecodeWaves * RI, "too many rows for one decode launch: %lld",
            static_cast<long long>(rows));
  const int64_t need = (rows + kDecWaves * RI - 1) / (kDecWaves * RI);
  const int64_t cap = kDecodeWaves / kDecWaves;
  const unsigned grid = static_cast<unsigned>(need < cap ? need : cap);
  if (RowsAligned4(sg, n_seg, row_bytes, kPaired)) {
    if (nrm != nullptr) {
      Launch(name, MatVecQuantKernel<kType, 1, RI, kPaired, kTypeB, true, true>, dim3(grid), dim3(kDecBlock), sg,
             rows, row_bytes, nb, x, *nrm);
      nrm->x_out = nullptr;
      return;
    }
    Launch(name, MatVecQuantKernel<kType, 1, RI, kPaired, kTypeB, false, true>, dim3(grid), dim3(kDecBlock), sg, rows,
           row_bytes, nb, x, NormPrologue{});
    return;
  }
  if (nrm != nullptr) {
    Launch(name, MatVecQuantKernel<kType, 1, RI, kPaired, kTypeB, true>, dim3(grid), dim3(kDecBlock), sg, rows,
           row_bytes, nb, x, *nrm);
    nrm->x_out = nullptr;
    return;
  }
  Launch(name, MatVecQuantKernel<kType, 1, RI, kPaired, kTypeB>, dim3(grid), dim3(kDecBlock), sg, rows, row_bytes, nb,
         x, NormPrologue{});
}

MatSegs OneSeg(const uint8_t* w, int64_t rows, float* out) {
  MatSegs sg{};
  for (int i = 0; i < kMaxSegs; ++i) sg.end[i] = INT64_MAX;
  sg.w[0] = w;
  sg.out[0] = out;
  sg.end[0] = rows;
  return sg;
}

template <uint32_t kType, int RI>
void LaunchDecode(const char* name, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                  float* out) {
  LaunchDecodeSegs<kType, RI>(name, OneSeg(w, rows, out), 1, row_bytes, nb, x);
}

// Split decode: at most max_grid workgroups (rows are visited with a stride);
// measured best at 4096 for one block group per wave, 1024 for two.
template <uint32_t kType, int WS, int NXW, int RI>
void LaunchSplit(const char* name, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                 float* out) {
  const int64_t max_grid = NXW == 1 ? 4096 : 1024;
  const int64_t need = (rows + RI - 1) / RI;
  const unsigned grid = static_cast<unsigned>(need < max_grid ? need : max_grid);
  if (RowsAligned4(OneSeg(w, rows, out), 1, row_bytes, false)) {
    Launch(name, MatVecSplitKernel<kType, WS, NXW, RI, true>, dim3(grid), dim3(64 * WS), w, rows, row_bytes, nb, x,
           out);
    return;
  }
  Launch(name, MatVecSplitKernel<kType, WS, NXW, RI>, dim3(grid), dim3(64 * WS), w, rows, row_bytes, nb, x, out);
}

// Rows per wave: enough waves to cover the chip first (a wave per row below
// 8192 rows), then 2 or 4 rows so each lane's activations serve several rows.
template <uint32_t kType>
void LaunchByShape(const char* name, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                   int64_t cols, int64_t n_tokens, float* out) {
  const char* dname = kType == kGgmlQ4_K ? "MatVecQ4KKernel" : "MatVecQ6KKernel";
  const char* sname = kType == kGgmlQ4_K ? "MatVecSplitQ4KKernel" : "MatVecSplitQ6KKernel";
  if (n_tokens == 1 && nb <= kGroups) {
    if (kType == kGgmlQ4_K && rows >= 32768) return LaunchDecode<kType, 4>(dname, w, rows, row_bytes, nb, x, out);
    return LaunchDecode<kType, 2>(dname, w, rows, row_bytes, nb, x, out);
  }
  if (n_tokens == 1 && nb <= 2 * kGroups) return LaunchSplit<kType, 2, 1, 2>(sname, w, rows, row_bytes, nb, x, out);
  if (n_tokens == 1 && nb <= 3 * kGroups) return LaunchSplit<kType, 3, 1, 2>(sname, w, rows, row_bytes, nb, x, out);
  if (n_tokens == 1 && nb <= 4 * kGroups) return LaunchSplit<kType, 4, 1, 2>(sname, w, rows, row_bytes, nb, x, out);
  if (n_tokens == 1 && nb <= 8 * kGroups) return LaunchSplit<kType, 4, 2, 1>(sname, w, rows, row_bytes, nb, x, out);
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

// Token counts from which the matrix-core GEMM replaces the tiled kernel
// (measured on Qwen3-1.7B matrices: at 16 tokens 26 us vs 50 us for 6144 x 2048
// Q4_K, 362 us vs 622 us for the 151936-row lm_head, but 22 us vs 19 us for
// 2048 x 2048; from 32 tokens it wins for every shape).
constexpr int64_t kMfmaMinTokens = 32;
constexpr int64_t kMfmaMinTokensWide = 16;  // matrices of at least kMfmaWideRows rows
constexpr int64_t kMfmaWideRows = 4096;

namespace {

// The matrix-core GEMM takes Q4_K / Q6_K matrices with enough tokens, 16-byte
// aligned activations and rows at the alignment its quant loads assume.
bool MfmaEligible(uint32_t type, const uint8_t* w_dev, const float* x_dev, int64_t rows, int64_t cols,
                  int64_t n_tokens) {
  const bool enough = n_tokens >= kMfmaMinTokens || (n_tokens >= kMfmaMinTokensWide && rows >= kMfmaWideRows);
  return (type == kGgmlQ4_K || type == kGgmlQ6_K) && enough && Aligned(x_dev, 16) && cols % kQK_K == 0 &&
         Aligned(w_dev, type == kGgmlQ4_K ? 16 : 2) && cols / kQK_K <= 0x7FFFFFFF;
}

}  // namespace

namespace {

// GpuSetForceGenericMatMul: while set, every matmul entry point runs
// MatMulGenericKernel (per-element decode, one wave per output) so the
// specialised kernels can be checked against it on the same inputs.
std::atomic<bool> g_force_generic{false};

}  // namespace

void GpuSetForceGenericMatMul(bool force) { g_force_generic.store(force); }

bool GpuForceGenericMatMul() { return g_force_generic.load(); }

void GpuMatMulQuantRaw(uint32_t type, const uint8_t* w_dev, int64_t rows, int64_t cols, const float* x_dev,
                       int64_t n_tokens, float* out_dev) {
  RPG_CHECK(rows > 0 && cols > 0, "invalid MatMulQuant shape [%lld, %lld]", static_cast<long long>(rows),
            static_cast<long long>(cols));
  RPG_CHECK(n_tokens > 0, "matmul: no tokens (n_tokens <= 0)");
  const BlockShape bs = DeviceBlockShape(type);
  RPG_CHECK(cols % bs.elems == 0, "matmul: %lld columns do not fill whole blocks of %d",
            static_cast<long long>(cols), bs.elems);
  RPG_CHECK(w_dev != nullptr && x_dev != nullptr && out_dev != nullptr, "MatMulQuant got a null pointer");
  const int64_t row_bytes = TypeRowBytes(type, cols);
  const bool x_ok = Aligned(x_dev, 16) && cols % 4 == 0;
  const int64_t nb = cols / kQK_K;
  const bool generic = g_force_generic.load();
  if (!generic && MfmaEligible(type, w_dev, x_dev, rows, cols, n_tokens)) {
    LaunchMatMulMfma(type, w_dev, rows, row_bytes, static_cast<int32_t>(nb), x_dev, cols, n_tokens, out_dev);
    return;
  }
  if (!generic && type == kGgmlQ4_K && x_ok && Aligned(w_dev, 16) && nb <= 0x7FFFFFFF) {
    LaunchByShape<kGgmlQ4_K>("MatMulQ4KKernel", w_dev, rows, row_bytes, static_cast<int32_t>(nb), x_dev, cols,
                             n_tokens, out_dev);
    return;
  }
  if (!generic && type == kGgmlQ6_K && x_ok && Aligned(w_dev, 2) && nb <= 0x7FFFFFFF) {
    LaunchByShape<kGgmlQ6_K>("MatMulQ6KKernel", w_dev, rows, row_bytes, static_cast<int32_t>(nb), x_dev, cols,
                             n_tokens, out_dev);
    return;
  }
  const int64_t units = rows * n_tokens;
  Launch("MatMulGenericKernel", MatMulGenericKernel, dim3(GridFor(units, kWavesPerBlock)), dim3(kMmBlock), type,
         w_dev, rows, row_bytes, bs.elems, bs.bytes, x_dev, cols, n_tokens, out_dev);
}

namespace {

// Whether every matrix of a group runs on the one-token decode kernels (Q4_K /
// Q6_K rows of at most kGroups blocks at their load alignment).
bool DecodeEligible(const GpuTensor* const* ws, int32_t n_mats, const float* x_dev, int64_t n_tokens) {
  const int64_t cols = ws[0]->cols;
  if (n_tokens != 1 || !Aligned(x_dev, 16) || cols % kQK_K != 0 || cols / kQK_K > kGroups) return false;
  for (int32_t k = 0; k < n_mats; ++k) {
    const bool q4 = ws[k]->type == kGgmlQ4_K, q6 = ws[k]->type == kGgmlQ6_K;
    if (!(q4 || q6) || !Aligned(ws[k]->buf.data(), q4 ? 16 : 2)) return false;
  }
  return true;
}

// The one-token launches of an eligible group: Q4_K and Q6_K together in one
// launch when no Q4_K matrix needs its own 4-rows-per-wave shape; otherwise one
// launch per run of consecutive same-type matrices, and matrices with odd rows
// or the 4-rows shape each on their own (the kernel of a single matrix, so every
// output is bit-identical to its GpuMatMulQuant). nrm: see LaunchDecodeSegs.
void DecodeGroup(const GpuTensor* const* ws, int32_t n_mats, const float* x_dev, float* const* outs,
                 NormPrologue* nrm) {
  const int64_t cols = ws[0]->cols;
  const int32_t nb = static_cast<int32_t>(cols / kQK_K);
  if (n_mats > 1 && n_mats <= kMaxSegs) {
    bool even = true, any4 = false, any6 = false;
    int64_t total4 = 0;
    for (int32_t k = 0; k < n_mats; ++k) {
      const bool q4 = ws[k]->type == kGgmlQ4_K;
      even = even && ws[k]->rows % 2 == 0;
      any4 = any4 || q4;
      any6 = any6 || !q4;
      if (q4) total4 += ws[k]->rows;
    }
    if (even && any4 && any6 && total4 < 32768) {
      MatSegs sg{};
      for (int k = 0; k < kMaxSegs; ++k) sg.end[k] = INT64_MAX;
      int64_t end = 0;
      for (int32_t k = 0; k < n_mats; ++k) {
        sg.w[k] = static_cast<const uint8_t*>(ws[k]->buf.data());
        sg.out[k] = outs[k];
        end += ws[k]->rows;
        sg.end[k] = end;
        if (ws[k]->type == kGgmlQ6_K) sg.b_mask |= 1u << k;
      }
      sg.row_bytes_b = TypeRowBytes(kGgmlQ6_K, cols);
      LaunchDecodeSegs<kGgmlQ4_K, 2, false, kGgmlQ6_K>(nrm ? "NormMatVecQ4KQ6KKernel" : "MatVecQ4KQ6KKernel", sg,
                                                       n_mats, TypeRowBytes(kGgmlQ4_K, cols), nb, x_dev, nrm);
      return;
    }
  }
  int32_t i = 0;
  while (i < n_mats) {
    const uint32_t type = ws[i]->type;
    const bool q4 = type == kGgmlQ4_K;
    const int64_t row_bytes = TypeRowBytes(type, cols);
    int32_t j = i + 1;
    while (j < n_mats && j - i < kMaxSegs && ws[j]->type == type) ++j;
    int64_t total = 0;
    bool fuse = j - i > 1;
    for (int32_t k = i; k < j && fuse; ++k) {
      fuse = ws[k]->rows % 2 == 0;
      total += ws[k]->rows;
    }
    fuse = fuse && !(q4 && total >= 32768);  // the 4-rows-per-wave shape stays per matrix
    const int32_t n_launch = fuse ? 1 : j - i;
    for (int32_t l = 0; l < n_launch; ++l) {
      const int32_t first = i + l, last = fuse ? j : i + l + 1;
      MatSegs sg{};
      for (int s = 0; s < kMaxSegs; ++s) sg.end[s] = INT64_MAX;
      int64_t end = 0;
      for (int32_t k = first; k < last; ++k) {
        sg.w[k - first] = static_cast<const uint8_t*>(ws[k]->buf.data());
        sg.out[k - first] = outs[k];
        end += ws[k]->rows;
        sg.end[k - first] = end;
      }
      if (q4 && end >= 32768) {  // a single matrix (a run that large is not fused)
        LaunchDecodeSegs<kGgmlQ4_K, 4>(nrm ? "NormMatVecQ4KKernel" : "MatVecQ4KKernel", sg, 1, row_bytes, nb, x_dev,
                                       nrm);
      } else if (q4) {
        LaunchDecodeSegs<kGgmlQ4_K, 2>(nrm ? "NormMatVecQ4KKernel" : "MatVecQ4KKernel", sg, last - first, row_bytes,
                                       nb, x_dev, nrm);
      } else {
        LaunchDecodeSegs<kGgmlQ6_K, 2>(nrm ? "NormMatVecQ6KKernel" : "MatVecQ6KKernel", sg, last - first, row_bytes,
                                       nb, x_dev, nrm);
      }
    }
    i = j;
  }
}

// The gate / up pair of GpuMatMulQuantSwiGLU on the paired one-token kernel.
bool SwiGLUDecodeEligible(const GpuTensor& w_gate, const GpuTensor& w_up, const float* x_dev, int64_t n_tokens) {
  const int64_t cols = w_gate.cols;
  const uint32_t type = w_gate.type;
  const bool q4 = type == kGgmlQ4_K, q6 = type == kGgmlQ6_K;
  return n_tokens == 1 && w_up.type == type && (q4 || q6) && Aligned(x_dev, 16) && cols % kQK_K == 0 &&
         cols / kQK_K <= kGroups && Aligned(w_gate.buf.data(), q4 ? 16 : 2) && Aligned(w_up.buf.data(), q4 ? 16 : 2) &&
         w_gate.buf.size() == static_cast<size_t>(w_gate.rows * w_gate.row_bytes()) &&
         w_up.buf.size() == static_cast<size_t>(w_up.rows * w_up.row_bytes());
}

void DecodeSwiGLU(const GpuTensor& w_gate, const GpuTensor& w_up, const float* x_dev, float* gate_dev,
                  NormPrologue* nrm) {
  MatSegs sg{};
  for (int i = 0; i < kMaxSegs; ++i) sg.end[i] = INT64_MAX;
  sg.w[0] = static_cast<const uint8_t*>(w_gate.buf.data());
  sg.w[1] = static_cast<const uint8_t*>(w_up.buf.data());
  sg.out[0] = gate_dev;
  sg.end[0] = 2 * w_gate.rows;  // virtual rows: (gate p, up p) pairs
  const int32_t nb = static_cast<int32_t>(w_gate.cols / kQK_K);
  const int64_t row_bytes = TypeRowBytes(w_gate.type, w_gate.cols);
  if (w_gate.type == kGgmlQ4_K) {
    LaunchDecodeSegs<kGgmlQ4_K, 2, true>(nrm ? "NormMatVecSwiGLUQ4KKernel" : "MatVecSwiGLUQ4KKernel", sg, 1,
                                         row_bytes, nb, x_dev, nrm);
  } else {
    LaunchDecodeSegs<kGgmlQ6_K, 2, true>(nrm ? "NormMatVecSwiGLUQ6KKernel" : "MatVecSwiGLUQ6KKernel", sg, 1,
                                         row_bytes, nb, x_dev, nrm);
  }
}

void CheckGroup(const GpuTensor* const* ws, int32_t n_mats, float* const* outs) {
  RPG_CHECK(ws != nullptr && outs != nullptr && n_mats > 0, "GpuMatMulQuantGroup needs at least one matrix");
  for (int32_t i = 0; i < n_mats; ++i) {
    RPG_CHECK(ws[i] != nullptr && outs[i] != nullptr, "GpuMatMulQuantGroup got a null matrix or output");
    RPG_CHECK(ws[i]->matrix && ws[i]->valid(), "GpuMatMulQuantGroup got a non-matrix or empty tensor");
    RPG_CHECK(ws[i]->cols == ws[0]->cols, "GpuMatMulQuantGroup matrices must share their width (%lld vs %lld)",
              static_cast<long long>(ws[i]->cols), static_cast<long long>(ws[0]->cols));
    RPG_CHECK(ws[i]->buf.size() == static_cast<size_t>(ws[i]->rows * ws[i]->row_bytes()),
              "tensor byte count does not match the [%lld, %lld] shape", static_cast<long long>(ws[i]->rows),
              static_cast<long long>(ws[i]->cols));
  }
}

// The norm prologue of a fused call, or false when the call has no fused form.
bool MakeNorm(const GpuNormIn& in, int64_t cols, NormPrologue* nrm) {
  RPG_CHECK(in.x != nullptr && in.w != nullptr, "norm-fused matmul needs x and the norm weights");
  RPG_CHECK(in.x_out == nullptr || (in.x_out != in.x && in.x_out != in.d),
            "norm-fused matmul: x_out must not alias x or d (other waves are still reading them)");
  if (!Aligned(in.w, 16) || (in.d != nullptr && !Aligned(in.d, 16)) ||
      (in.x_out != nullptr && !Aligned(in.x_out, 16)) || cols % kQK_K != 0 || cols / kQK_K > kGroups) {
    return false;
  }
  *nrm = NormPrologue{in.d, in.w, in.x_out, in.eps};
  return true;
}

}  // namespace

void GpuMatMulQuantGroup(const GpuTensor* const* ws, int32_t n_mats, const float* x_dev, int64_t n_tokens,
                         float* const* outs) {
  CheckGroup(ws, n_mats, outs);
  const int64_t cols = ws[0]->cols;
  if (g_force_generic.load()) {
    for (int32_t i = 0; i < n_mats; ++i) GpuMatMulQuant(*ws[i], x_dev, n_tokens, outs[i]);
    return;
  }
  // Prefill: the activations are split once for all the matrices (each output
  // bit-identical to its own GpuMatMulQuant call, which splits the same way).
  bool mfma = true;
  for (int32_t i = 0; i < n_mats && mfma; ++i) {
    mfma = MfmaEligible(ws[i]->type, static_cast<const uint8_t*>(ws[i]->buf.data()), x_dev, ws[i]->rows, cols,
                        n_tokens);
  }
  if (mfma) {
    const SplitActivations sa = SplitForMfma(x_dev, n_tokens, cols);
    for (int32_t i = 0; i < n_mats; ++i) {
      LaunchMatMulMfmaSplit(ws[i]->type, static_cast<const uint8_t*>(ws[i]->buf.data()), ws[i]->rows,
                            ws[i]->row_bytes(), static_cast<int32_t>(cols / kQK_K), sa, outs[i]);
    }
    return;
  }
  if (DecodeEligible(ws, n_mats, x_dev, n_tokens)) {
    DecodeGroup(ws, n_mats, x_dev, outs, nullptr);
    return;
  }
  for (int32_t i = 0; i < n_mats; ++i) GpuMatMulQuant(*ws[i], x_dev, n_tokens, outs[i]);
}

void GpuMatMulQuantSwiGLU(const GpuTensor& w_gate, const GpuTensor& w_up, const float* x_dev, int64_t n_tokens,
                          float* gate_dev, float* up_dev) {
  RPG_CHECK(w_gate.matrix && w_gate.valid() && w_up.matrix && w_up.valid(),
            "GpuMatMulQuantSwiGLU got a non-matrix or empty tensor");
  RPG_CHECK(w_gate.rows == w_up.rows && w_gate.cols == w_up.cols,
            "gate [%lld, %lld] and up [%lld, %lld] must have the same shape", static_cast<long long>(w_gate.rows),
            static_cast<long long>(w_gate.cols), static_cast<long long>(w_up.rows), static_cast<long long>(w_up.cols));
  RPG_CHECK(n_tokens > 0, "matmul: no tokens (n_tokens <= 0)");
  RPG_CHECK(x_dev != nullptr && gate_dev != nullptr && up_dev != nullptr, "GpuMatMulQuantSwiGLU got a null pointer");
  if (!g_force_generic.load() && SwiGLUDecodeEligible(w_gate, w_up, x_dev, n_tokens)) {
    DecodeSwiGLU(w_gate, w_up, x_dev, gate_dev, nullptr);
    return;
  }
  const GpuTensor* mats[2] = {&w_gate, &w_up};
  float* outs[2] = {gate_dev, up_dev};
  GpuMatMulQuantGroup(mats, 2, x_dev, n_tokens, outs);
  GpuSiluMulInPlace(gate_dev, up_dev, n_tokens * w_gate.rows);
}

bool GpuNormMatMulQuantGroup(const GpuNormIn& in, const GpuTensor* const* ws, int32_t n_mats, float* const* outs) {
  CheckGroup(ws, n_mats, outs);
  NormPrologue nrm;
  if (g_force_generic.load() || !MakeNorm(in, ws[0]->cols, &nrm) || !DecodeEligible(ws, n_mats, in.x, 1)) {
    return false;
  }
  DecodeGroup(ws, n_mats, in.x, outs, &nrm);
  return true;
}

bool GpuNormMatMulQuantSwiGLU(const GpuNormIn& in, const GpuTensor& w_gate, const GpuTensor& w_up, float* gate_dev,
                              float* up_dev) {
  RPG_CHECK(w_gate.matrix && w_gate.valid() && w_up.matrix && w_up.valid(),
            "GpuNormMatMulQuantSwiGLU got a non-matrix or empty tensor");
  RPG_CHECK(w_gate.rows == w_up.rows && w_gate.cols == w_up.cols, "gate and up must have the same shape");
  RPG_CHECK(gate_dev != nullptr && up_dev != nullptr, "GpuNormMatMulQuantSwiGLU got a null output");
  NormPrologue nrm;
  if (g_force_generic.load() || !MakeNorm(in, w_gate.cols, &nrm) || !SwiGLUDecodeEligible(w_gate, w_up, in.x, 1)) {
    return false;
  }
  DecodeSwiGLU(w_gate, w_up, in.x, gate_dev, &nrm);
  return true;
}

void GpuMatMulQuant(const GpuTensor& w, const float* X_dev, int64_t n_tokens, float* OUT_dev) {
  RPG_CHECK(w.matrix, "GpuMatMulQuant: the %s weight tensor is not a 2-D matrix", w.type_name());
  RPG_CHECK(w.valid(), "GpuMatMulQuant got an empty tensor");
  RPG_CHECK(w.buf.size() == static_cast<size_t>(w.rows * w.row_bytes()),
            "tensor byte count does not match the [%lld, %lld] shape", static_cast<long long>(w.rows),
            static_cast<long long>(w.cols));
  GpuMatMulQuantRaw(w.type, static_cast<const uint8_t*>(w.buf.data()), w.rows, w.cols, X_dev, n_tokens, OUT_dev);
}

}  // namespace rpg
