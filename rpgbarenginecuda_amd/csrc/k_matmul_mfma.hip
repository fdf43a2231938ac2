// Prefill GEMM for the quantised matmul on the fp16 matrix cores of gfx950:
// OUT[t][r] = sum_e W[r][e] * X[t][e] for n_tokens large enough to fill a tile.
//
// Operands (every product the matrix core forms is exact; it accumulates in fp32):
//   * activations: per token t a power of two s_t brings max |x_t| into
//     [2^13, 2^14); x s_t is split into two fp16 terms hi + lo (round to
//     nearest, then the rest), which reproduce x to ~2^-22 |x|. The pre-pass
//     (SplitActivationsKernel) does this once per input; the result is divided
//     by s_t at the end (exact);
//   * Q4_K weights: the matrix core sees sc_j * q (6-bit scale times 4-bit quant,
//     at most 945, exact in fp16), so a whole 256-element block accumulates in
//     one register set and the block scale d is applied once per block; the min
//     term dmin * sum_j m_j * sum(x over sub-block j) is one more 16-deep MFMA
//     step per block, over the token's 8 run sums (fp32 sums of x, times s_t 2^-6,
//     split in two fp16 terms) against m_j 2^6 (exact);
//   * Q6_K weights: sc * (q - 32) can need 12 significant bits, so it is fed as
//     two exact operands, (sc with its low bit cleared) * (q - 32) (an even
//     integer of magnitude <= 4096) and (sc & 1) * (q - 32); d once per block.
// Exact operand values are built from the quant bytes with a byte permute
// against 0x64 (the fp16 bits of 1024 + q) and one packed fp16 fma or add.
//
// Tiling: a 256-thread workgroup computes 128 tokens x 128 weight rows; wave
// (wm, wn) owns tokens 64 wm + [0, 64) and rows 64 wn + [0, 64) as 2 x 2 tiles
// of v_mfma_f32_32x32x16_f16 (A = activations [token][k], B = weights [k][row],
// so each lane's outputs for one register are 32 consecutive rows of one token:
// coalesced stores). The K loop walks 64-column chunks: each thread stages 32
// columns of one token's activation planes and decodes 32 weights of one row
// into LDS, then the waves run the chunk's MFMAs from LDS only, while the next
// chunk's global loads (held in registers, branch-free) are in flight. The LDS
// image is kept under 80 KB and the registers under 256 so that two
// workgroups share a CU and cover each other's barriers and LDS latency.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"
#include "matmul_mfma.h"
#include "quant_dev.h"

namespace rpg {
namespace {

using dev::ByteOf;
using dev::ScaleMinK4;

typedef _Float16 F16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 H2 __attribute__((ext_vector_type(2)));
typedef float F32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileT = 128;       // tokens per workgroup
constexpr int kTileR = 128;       // weight rows per workgroup
constexpr int kChunk = 64;        // K columns staged per step
constexpr int kPad = 8;           // fp16 padding per staged row (breaks LDS bank conflicts)
constexpr int kRowStride = kChunk + kPad;
constexpr int kThreads = 256;
constexpr int kPlanes = 2;        // fp16 terms per activation
constexpr int kSumShift = 6;      // run sums stored times 2^-6, m_j times 2^6
constexpr uint32_t kMagic = 0x64646464u;  // byte 0x64 above a quant byte q: fp16 bits of 1024 + q

__device__ __forceinline__ float HalfF(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// fp16 pairs (1024 + q0, 1024 + q1) and (1024 + q2, 1024 + q3) of the four bytes of w.
__device__ __forceinline__ H2 MagicLo(uint32_t w) { return __builtin_bit_cast(H2, __builtin_amdgcn_perm(kMagic, w, 0x04010400u)); }
__device__ __forceinline__ H2 MagicHi(uint32_t w) { return __builtin_bit_cast(H2, __builtin_amdgcn_perm(kMagic, w, 0x04030402u)); }

__device__ __forceinline__ F16x8 Join(H2 a, H2 b, H2 c, H2 d) {
  F16x8 v;
  v[0] = a[0]; v[1] = a[1]; v[2] = b[0]; v[3] = b[1];
  v[4] = c[0]; v[5] = c[1]; v[6] = d[0]; v[7] = d[1];
  return v;
}

// sc * q for eight nibble bytes (q in 0..15, sc in 0..63): (1024 + q) sc - 1024 sc
// in one fused step, exact.
__device__ __forceinline__ F16x8 ScaledQ4(uint2 q, _Float16 sc) {
  const H2 s2 = {sc, sc};
  const _Float16 o = static_cast<_Float16>(-1024.0f) * sc;
  const H2 o2 = {o, o};
  return Join(__builtin_elementwise_fma(MagicLo(q.x), s2, o2), __builtin_elementwise_fma(MagicHi(q.x), s2, o2),
              __builtin_elementwise_fma(MagicLo(q.y), s2, o2), __builtin_elementwise_fma(MagicHi(q.y), s2, o2));
}

// q - 32 for eight 6-bit quant bytes, exact.
__device__ __forceinline__ F16x8 CenteredQ6(uint2 q) {
  const _Float16 c = static_cast<_Float16>(-1056.0f);
  const H2 c2 = {c, c};
  return Join(MagicLo(q.x) + c2, MagicHi(q.x) + c2, MagicLo(q.y) + c2, MagicHi(q.y) + c2);
}

// 32 bytes at a 2-byte aligned address, from nine aligned dwords (Q6_K rows
// are 210-byte blocks; the dwords around the field stay inside the tensor's pages).
__device__ __forceinline__ void Load32Aligned2(const uint8_t* p, uint32_t out[8]) {
  const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint32_t* a = reinterpret_cast<const uint32_t*>(p - sh);
  uint32_t w[9];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = a[i];
  w[8] = sh != 0 ? a[8] : 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

// Raw weight bytes one staging thread decodes per chunk: row `row`, 32 of the
// chunk's 64 columns (half hf).
//   Q4_K: hdr = d | dmin | 12 scale bytes of the block; q[0..3] = qs bytes
//         32 kc + 16 hf .. + 15 (low nibbles: sub-block 2 kc, columns 16 hf + i;
//         high nibbles: sub-block 2 kc + 1, columns 32 + 16 hf + i).
//   Q6_K: hdr.x = d, hdr.y = the two scales of the 16-groups of these 32 columns;
//         q[0..7] = ql bytes, q[8..15] = qh bytes of quarter 2 (kc & 1) + hf.
struct StageRaw {
  uint4 hdr;
  uint32_t q[16];
};

__device__ __forceinline__ StageRaw FetchStageQ4K(const uint8_t* __restrict__ blk, int kc, int hf) {
  StageRaw r;
  r.hdr = *reinterpret_cast<const uint4*>(blk);
  const uint4 v = *reinterpret_cast<const uint4*>(blk + 16 + 32 * kc + 16 * hf);
  r.q[0] = v.x; r.q[1] = v.y; r.q[2] = v.z; r.q[3] = v.w;
#pragma unroll
  for (int i = 4; i < 16; ++i) r.q[i] = 0u;
  return r;
}

__device__ __forceinline__ StageRaw FetchStageQ6K(const uint8_t* __restrict__ blk, int kc, int hf) {
  StageRaw r;
  const int half = kc >> 1;
  const int quarter = 2 * (kc & 1) + hf;
  const uint8_t* sc = blk + 192 + 4 * kc + 2 * hf;  // 2-byte aligned: one aligned dword holds both
  const uint32_t scw = *reinterpret_cast<const uint32_t*>(sc - (reinterpret_cast<uintptr_t>(sc) & 3u));
  const uint32_t scs = (reinterpret_cast<uintptr_t>(sc) & 2u) ? (scw >> 16) : (scw & 0xFFFFu);
  r.hdr = make_uint4(*reinterpret_cast<const uint16_t*>(blk + 208), scs, 0u, 0u);
  Load32Aligned2(blk + 64 * half + 32 * (quarter & 1), r.q);
  Load32Aligned2(blk + 128 + 32 * half, r.q + 8);
  return r;
}

// Activation pre-pass: one workgroup per token row, 8 consecutive columns
// per thread and step (four threads per 32-column run). kU > 0: the row has at
// most kU * 8 * kThreads columns and each thread keeps its kU steps in
// registers between the max pass and the split pass; kU == 0 reads the row
// twice (any width). Both give the same bits.
struct SplitArgs {
  const float* x;
  int64_t cols;
  int64_t plane_elems;
  int64_t sum_elems;
  _Float16* planes;
  _Float16* sum_planes;
  float* inv_scale;
};

template <int kU>
__device__ __forceinline__ void SplitRow(const SplitArgs& a, int64_t t) {
  const float* __restrict__ x = a.x;
  const int64_t cols = a.cols;
  const int64_t plane_elems = a.plane_elems;
  const int64_t sum_elems = a.sum_elems;
  _Float16* __restrict__ planes = a.planes;
  _Float16* __restrict__ sum_planes = a.sum_planes;
  constexpr int kSteps = kU > 0 ? kU : 1;
  constexpr int64_t kStride = 8 * kThreads;
  __shared__ float red[kThreads / 64];
  const float* row = x + t * cols;
  const int64_t runs = cols / 32;
  const int tid = threadIdx.x;
  float4 held[kSteps][2];
  float mx = 0.0f;
  auto absmax8 = [](float m, const float4& f0, const float4& f1) {
    m = fmaxf(m, fmaxf(fmaxf(fabsf(f0.x), fabsf(f0.y)), fmaxf(fabsf(f0.z), fabsf(f0.w))));
    return fmaxf(m, fmaxf(fmaxf(fabsf(f1.x), fabsf(f1.y)), fmaxf(fabsf(f1.z), fabsf(f1.w))));
  };
  if (kU > 0) {
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int64_t e = 8 * tid + kStride * u;
      held[u][0] = make_float4(0.f, 0.f, 0.f, 0.f);
      held[u][1] = held[u][0];
      if (e < cols) {
        held[u][0] = *reinterpret_cast<const float4*>(row + e);
        held[u][1] = *reinterpret_cast<const float4*>(row + e + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) mx = absmax8(mx, held[u][0], held[u][1]);
  } else {
    for (int64_t e = 8 * tid; e < cols; e += kStride) {
      mx = absmax8(mx, *reinterpret_cast<const float4*>(row + e), *reinterpret_cast<const float4*>(row + e + 4));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // s = 2^e with max |x| s in [2^13, 2^14); 1 for an all-zero or non-finite row
  int e = 0;
  if (mx > 0.0f && mx <= 3.4e38f) {
    int ex;
    (void)frexpf(mx, &ex);  // mx = f 2^ex, f in [0.5, 1)
    e = 14 - ex;
    e = e < -120 ? -120 : (e > 120 ? 120 : e);
  }
  const float s = ldexpf(1.0f, e);
  const float ss = ldexpf(1.0f, e - kSumShift);
  if (tid == 0) a.inv_scale[t] = ldexpf(1.0f, -e);
  // cols is a multiple of 32, so every group of four lanes walks whole runs
  // together and the shuffles below stay inside a run
  auto split8 = [&](int64_t c, const float4& f0, const float4& f1) {
    const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
    F16x8 hi, lo;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sum += v[j];
      const float y = v[j] * s;
      const _Float16 a = static_cast<_Float16>(y);
      hi[j] = a;
      lo[j] = static_cast<_Float16>(y - static_cast<float>(a));
    }
    *reinterpret_cast<F16x8*>(planes + t * cols + c) = hi;
    *reinterpret_cast<F16x8*>(planes + plane_elems + t * cols + c) = lo;
    // run sum: the four 8-column partial sums, pairwise
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if ((tid & 3) == 0) {
      const float ys = sum * ss;
      const _Float16 a = static_cast<_Float16>(ys);
      const int64_t si = t * runs + c / 32;
      sum_planes[si] = a;
      sum_planes[sum_elems + si] = static_cast<_Float16>(ys - static_cast<float>(a));
    }
  };
  if (kU > 0) {
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int64_t c = 8 * tid + kStride * u;
      if (c < cols) split8(c, held[u][0], held[u][1]);
    }
  } else {
    for (int64_t c = 8 * tid; c < cols; c += kStride) {
      split8(c, *reinterpret_cast<const float4*>(row + c), *reinterpret_cast<const float4*>(row + c + 4));
    }
  }
}

template <int kU>
__global__ __launch_bounds__(kThreads) void SplitActivationsKernel(SplitArgs a) {
  SplitRow<kU>(a, blockIdx.x);
}

// LDS image of the workgroup's operands: two buffers of activation planes
// and decoded weights, plus the per-block values used at each block's end.
template <int kWOps>
struct GemmLds {
  _Float16 xs[kPlanes][kTileT][kRowStride];
  _Float16 ws[kWOps][kTileR][kRowStride];
  _Float16 ss[kWOps == 1 ? kPlanes : 1][kTileT][8];  // Q4_K: the block's run sums of each token
  _Float16 sm[kWOps == 1 ? kTileR : 1][8];           // Q4_K: m_j 2^6 of each row
  float sd[kTileR][2];                               // d, dmin of each row's block
};

// One chunk's global loads, held in registers until the chunk is staged.
struct ChunkLoads {
  uint4 x[kPlanes][4];
  uint4 sum;
  StageRaw raw;
};

// Branch-free: a token past n_tokens reads token 0 (a valid address) and the
// value is replaced by zero.
template <bool kQ4>
__device__ __forceinline__ void FetchChunk(ChunkLoads& f, int c, const _Float16* st_src, const _Float16* st_sum,
                                           int64_t plane_elems, bool st_ok, const uint8_t* st_w, int st_hf) {
  constexpr int64_t kBB = kQ4 ? kQ4KBlockBytes : kQ6KBlockBytes;
  const uint32_t keep = st_ok ? 0xFFFFFFFFu : 0u;
#pragma unroll
  for (int p = 0; p < kPlanes; ++p)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 v = *reinterpret_cast<const uint4*>(st_src + p * plane_elems + kChunk * c + 8 * g);
      f.x[p][g] = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
    }
  if (kQ4) {
    const uint4 v = *reinterpret_cast<const uint4*>(st_sum + 8 * (c >> 2));
    f.sum = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
  }
  const uint8_t* blk = st_w + (c >> 2) * kBB;
  f.raw = kQ4 ? FetchStageQ4K(blk, c & 3, st_hf) : FetchStageQ6K(blk, c & 3, st_hf);
}

// Chunk c (held in f) -> LDS.
template <bool kQ4, int kWOps>
__device__ __forceinline__ void StageChunk(GemmLds<kWOps>& L, const ChunkLoads& f, int c, int st_i, int st_hf) {
  const int kc = c & 3;
#pragma unroll
  for (int p = 0; p < kPlanes; ++p)
#pragma unroll
    for (int g = 0; g < 4; ++g) *reinterpret_cast<uint4*>(&L.xs[p][st_i][32 * st_hf + 8 * g]) = f.x[p][g];
  const StageRaw& raw = f.raw;
  if (kQ4) {
    const uint32_t s0 = raw.hdr.y, s1 = raw.hdr.z, s2 = raw.hdr.w;
    uint32_t scl, ml, sch, mh;
    ScaleMinK4(2 * kc, s0, s1, s2, &scl, &ml);
    ScaleMinK4(2 * kc + 1, s0, s1, s2, &sch, &mh);
    const _Float16 fl = static_cast<_Float16>(static_cast<float>(scl));
    const _Float16 fh = static_cast<_Float16>(static_cast<float>(sch));
#pragma unroll
    for (int g = 0; g < 2; ++g) {  // low nibbles: sub-block 2 kc; high: 2 kc + 1
      const uint32_t bx = raw.q[2 * g], by = raw.q[2 * g + 1];
      *reinterpret_cast<F16x8*>(&L.ws[0][st_i][16 * st_hf + 8 * g]) =
          ScaledQ4(make_uint2(bx & 0x0F0F0F0Fu, by & 0x0F0F0F0Fu), fl);
      *reinterpret_cast<F16x8*>(&L.ws[0][st_i][32 + 16 * st_hf + 8 * g]) =
          ScaledQ4(make_uint2((bx >> 4) & 0x0F0F0F0Fu, (by >> 4) & 0x0F0F0F0Fu), fh);
    }
    if (kc == 3) {  // used by this chunk's block end only
      *reinterpret_cast<uint4*>(&L.ss[st_hf][st_i][0]) = f.sum;
      if (st_hf == 0) {
        F16x8 mv;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          uint32_t scj, mj;
          ScaleMinK4(j, s0, s1, s2, &scj, &mj);
          mv[j] = static_cast<_Float16>(static_cast<float>(mj << kSumShift));
        }
        *reinterpret_cast<F16x8*>(&L.sm[st_i][0]) = mv;
        L.sd[st_i][0] = HalfF(raw.hdr.x & 0xFFFFu);
        L.sd[st_i][1] = HalfF(raw.hdr.x >> 16);
      }
    }
  } else {
    const int quarter = 2 * (kc & 1) + st_hf;
    const int nshift = quarter < 2 ? 0 : 4;
#pragma unroll
    for (int g = 0; g < 4; ++g) {  // columns 32 st_hf + 8 g .. + 7: 16-group g / 2
      const uint32_t lx = raw.q[2 * g], ly = raw.q[2 * g + 1];
      const uint32_t hx = raw.q[8 + 2 * g], hy = raw.q[8 + 2 * g + 1];
      const uint2 q = make_uint2(((lx >> nshift) & 0x0F0F0F0Fu) | (((hx >> (2 * quarter)) & 0x03030303u) << 4),
                                 ((ly >> nshift) & 0x0F0F0F0Fu) | (((hy >> (2 * quarter)) & 0x03030303u) << 4));
      const F16x8 qc = CenteredQ6(q);
      const int sc = static_cast<int8_t>(ByteOf(raw.hdr.y, g >> 1));
      const _Float16 se = static_cast<_Float16>(static_cast<float>(sc & ~1));
      const _Float16 so = static_cast<_Float16>(static_cast<float>(sc & 1));
      *reinterpret_cast<F16x8*>(&L.ws[0][st_i][32 * st_hf + 8 * g]) = qc * se;
      *reinterpret_cast<F16x8*>(&L.ws[kWOps - 1][st_i][32 * st_hf + 8 * g]) = qc * so;
    }
    if (kc == 3 && st_hf == 0) L.sd[st_i][0] = HalfF(raw.hdr.x & 0xFFFFu);
  }
}

// Chunk c on the matrix cores, one 16-deep K-step at a time (the other
// workgroup on the CU covers the LDS latency); at a block's end the block
// scale (and for Q4_K the min term) moves part into acc.
template <bool kQ4, int kWOps>
__device__ __forceinline__ void ComputeChunk(const GemmLds<kWOps>& L, int c, int wm, int wn, int li, int h,
                                             F32x16 (&acc)[2][2], F32x16 (&part)[2][2]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int kcol = 16 * ks + 8 * h;
    F16x8 af[2][kPlanes], bf[2][kWOps];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int o = 0; o < kWOps; ++o)
        bf[nt][o] = *reinterpret_cast<const F16x8*>(&L.ws[o][64 * wn + 32 * nt + li][kcol]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int p = 0; p < kPlanes; ++p)
        af[mt][p] = *reinterpret_cast<const F16x8*>(&L.xs[p][64 * wm + 32 * mt + li][kcol]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int p = 0; p < kPlanes; ++p)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int o = 0; o < kWOps; ++o)
            part[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mt][p], bf[nt][o], part[mt][nt], 0, 0, 0);
  }
  if ((c & 3) != 3) return;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const float d = L.sd[64 * wn + 32 * nt + li][0];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[mt][nt][i] = __builtin_fmaf(d, part[mt][nt][i], acc[mt][nt][i]);
        part[mt][nt][i] = 0.0f;
      }
  }
  if (!kQ4) return;
  F16x8 bm[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const F16x8 v = *reinterpret_cast<const F16x8*>(&L.sm[64 * wn + 32 * nt + li][0]);
    const F16x8 z = {};
    bm[nt] = h == 0 ? v : z;  // k 8..15 carry zero weights
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) {
      const F16x8 a = *reinterpret_cast<const F16x8*>(&L.ss[p][64 * wm + 32 * mt + li][0]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        part[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bm[nt], part[mt][nt], 0, 0, 0);
    }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const float dmin = L.sd[64 * wn + 32 * nt + li][1];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[mt][nt][i] = __builtin_fmaf(-dmin, part[mt][nt][i], acc[mt][nt][i]);
        part[mt][nt][i] = 0.0f;
      }
  }
}

// Blocks [z bps, min(nb, (z + 1) bps)) of K for z = blockIdx.z; with one
// split (partial == nullptr) the result goes to out, otherwise the K-slice's
// partial tile to partial[z] for MatMulSplitReduceKernel.
// kPP (grids of at most kPingPongTiles tiles): one 512-thread workgroup per CU
// in two roles. Waves 4-7 only fetch and stage (their loads run three chunks
// ahead in four register sets) and waves 0-3 only run the MFMAs, from two LDS
// buffers that alternate every chunk, so each SIMD pairs a staging wave with
// a matrix-core wave; one barrier per chunk. With few tiles this covers the
// load latency that the second workgroup of the kPP == false shape cannot
// (measured 5-33% faster up to 128 tiles); with many tiles two independent
// workgroups per CU are faster. Same chunks, same order: the same bits.
constexpr int kGemmThreadsPP = 2 * kThreads;
constexpr int64_t kPingPongTiles = 128;

template <uint32_t kType, bool kPP>
__global__ __launch_bounds__(kPP ? kGemmThreadsPP : kThreads, kPP ? 1 : 2) void MatMulMfmaKernel(const uint8_t* __restrict__ w, int64_t rows,
                                                             int64_t row_bytes, int32_t nb,
                                                             const _Float16* __restrict__ planes,
                                                             const _Float16* __restrict__ sum_planes,
                                                             int64_t sum_stride,
                                                             const float* __restrict__ inv_scale, int64_t cols,
                                                             int64_t n_tokens, int32_t blocks_per_split,
                                                             float* __restrict__ out, float* __restrict__ partial) {
  constexpr bool kQ4 = kType == kGgmlQ4_K;
  constexpr int kWOps = kQ4 ? 1 : 2;  // weight operands per column (Q6_K: even and odd scale parts)
  __shared__ __attribute__((aligned(16))) GemmLds<kWOps> L2[kPP ? 2 : 1];

  const bool producer = kPP && threadIdx.x >= kThreads;
  const int tid = producer ? threadIdx.x - kThreads : threadIdx.x;  // index within the role
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int li = lane & 31;  // A: token row / B: weight row inside a 32-tile
  const int h = lane >> 5;   // which 8 of the 16 K of a step
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kTileT;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTileR;

  F32x16 acc[2][2], part[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[mt][nt][i] = 0.0f;
        part[mt][nt][i] = 0.0f;
      }

  // staging map: thread -> (tile row st_i, 32-column half st_hf of the chunk):
  // activations of token t0 + st_i, weights of row r0 + st_i (both clamped to
  // valid rows; an activation past n_tokens is zeroed)
  const int st_i = tid >> 1;
  const int st_hf = tid & 1;
  const int64_t st_t = t0 + st_i;
  const bool st_ok = st_t < n_tokens;
  const int64_t st_tc = st_ok ? st_t : 0;
  const int64_t runs = cols / 32;
  const int64_t plane_elems = n_tokens * cols;
  const int b0 = static_cast<int>(blockIdx.z) * blocks_per_split;  // first block of this K-slice
  const int n_blk = nb - b0 < blocks_per_split ? nb - b0 : blocks_per_split;
  const _Float16* st_src = planes + st_tc * cols + 32 * st_hf + static_cast<int64_t>(kQK_K) * b0;
  const _Float16* st_sum = sum_planes + st_hf * sum_stride + st_tc * runs + 8 * b0;
  const int64_t st_r = r0 + st_i;
  const uint8_t* st_w = w + (st_r < rows ? st_r : rows - 1) * row_bytes + static_cast<int64_t>(b0) * (kQ4 ? kQ4KBlockBytes : kQ6KBlockBytes);

  const int n_chunks = 4 * n_blk;
  if constexpr (kPP) {
    // n_chunks is a multiple of 4: producers and consumers pass the same
    // 1 + n_chunks barriers; chunk j is staged into L2[j & 1] between
    // barriers j and j + 1, and computed between barriers j + 1 and j + 2.
    if (producer) {
#define RPG_FETCH(f, j) FetchChunk<kQ4>(f, j, st_src, st_sum, plane_elems, st_ok, st_w, st_hf)
      ChunkLoads f0, f1, f2, f3;
      RPG_FETCH(f0, 0);
      RPG_FETCH(f1, 1);
      RPG_FETCH(f2, 2);
      RPG_FETCH(f3, 3);
      StageChunk<kQ4, kWOps>(L2[0], f0, 0, st_i, st_hf);
      if (4 < n_chunks) RPG_FETCH(f0, 4);
      __syncthreads();
      for (int c = 0; c < n_chunks; c += 4) {
        StageChunk<kQ4, kWOps>(L2[1], f1, c + 1, st_i, st_hf);
        if (c + 5 < n_chunks) RPG_FETCH(f1, c + 5);
        __syncthreads();
        StageChunk<kQ4, kWOps>(L2[0], f2, c + 2, st_i, st_hf);
        if (c + 6 < n_chunks) RPG_FETCH(f2, c + 6);
        __syncthreads();
        StageChunk<kQ4, kWOps>(L2[1], f3, c + 3, st_i, st_hf);
        if (c + 7 < n_chunks) RPG_FETCH(f3, c + 7);
        __syncthreads();
        if (c + 4 < n_chunks) {
          StageChunk<kQ4, kWOps>(L2[0], f0, c + 4, st_i, st_hf);
          if (c + 8 < n_chunks) RPG_FETCH(f0, c + 8);
        }
        __syncthreads();
      }
#undef RPG_FETCH
      return;
    }
    __syncthreads();
    for (int c = 0; c < n_chunks; c += 4) {
      ComputeChunk<kQ4, kWOps>(L2[0], c, wm, wn, li, h, acc, part);
      __syncthreads();
      ComputeChunk<kQ4, kWOps>(L2[1], c + 1, wm, wn, li, h, acc, part);
      __syncthreads();
      ComputeChunk<kQ4, kWOps>(L2[0], c + 2, wm, wn, li, h, acc, part);
      __syncthreads();
      ComputeChunk<kQ4, kWOps>(L2[1], c + 3, wm, wn, li, h, acc, part);
      __syncthreads();
    }
  } else {
    ChunkLoads f;
    FetchChunk<kQ4>(f, 0, st_src, st_sum, plane_elems, st_ok, st_w, st_hf);
    for (int c = 0; c < n_chunks; ++c) {
      if (c > 0) __syncthreads();  // every wave is done with chunk c - 1's operands
      StageChunk<kQ4, kWOps>(L2[0], f, c, st_i, st_hf);
      __syncthreads();
      if (c + 1 < n_chunks) FetchChunk<kQ4>(f, c + 1, st_src, st_sum, plane_elems, st_ok, st_w, st_hf);
      ComputeChunk<kQ4, kWOps>(L2[0], c, wm, wn, li, h, acc, part);
    }
  }

  // D[i][j]: j = lane % 32 (weight row), i = (r % 4) + 8 (r / 4) + 4 (lane / 32) (token)
  float* dst = partial != nullptr ? partial + static_cast<int64_t>(blockIdx.z) * n_tokens * rows : out;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t tok = t0 + 64 * wm + 32 * mt + (i & 3) + 8 * (i >> 2) + 4 * h;
      if (tok >= n_tokens) continue;
      const float inv = inv_scale[tok];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int64_t row = r0 + 64 * wn + 32 * nt + li;
        if (row < rows) dst[tok * rows + row] = acc[mt][nt][i] * inv;
      }
    }
  }
}

// out[e] = sum over z = 0 .. splits - 1 of partial[z][e], in that order.
__global__ __launch_bounds__(kThreads) void MatMulSplitReduceKernel(const float* __restrict__ partial, int64_t elems,
                                                                     int32_t splits, float* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= elems) return;
  float v = partial[e];
  for (int32_t z = 1; z < splits; ++z) v += partial[z * elems + e];
  out[e] = v;
}

// ---------------------------------------------------------------- large grids: pre-decoded weight planes
//
// For grids of many tiles the weights are decoded once per call instead of
// once per token tile: DecodeWeightPlanesKernel writes fp16 operand planes
// ([ops][rows][cols], K contiguous) and, per (row, block), (d, dmin) and
// m_j 2^6. Q4_K: the exact sc_j q of StageChunk. Q6_K: w = sc (q - 32) as
// hi = w rounded to fp16 and lo = w - hi (exact; lo is nonzero only for
// |w| > 2048, where it is +-1); the matrix cores form x_hi w_hi, x_lo w_hi and
// x_hi w_lo and leave out x_lo w_lo, which is below 2^-22 |x w| (|x_lo| <=
// 2^-11 |x|, |w_lo| <= 2^-11 |w|): three products instead of the four of the
// even / odd scale split. MatMulMfmaPlanesKernel streams both operands
// through LDS unchanged. Its workgroup is 8 waves (2 x 4) over 128
// tokens x kPTileR rows, each wave 64 tokens x 32 kPNT rows; two LDS buffers
// alternate every 64-column chunk, the next chunk's LDS writes and global loads
// are issued after the first of its four K-steps, and the block-end values are
// loaded at the block's first chunk, so one barrier per chunk is the only
// synchronisation. For Q4_K the MFMAs, block scales and min terms of each
// accumulator run in the order of MatMulMfmaKernel (the same bits for tiles
// that are not split along K).
typedef uint32_t U32x4 __attribute__((ext_vector_type(4)));

constexpr int kPThreads = 512;
constexpr int kPStage = 2 * kTileT * kRowStride;  // fp16 elements of one buffer's activation part

template <uint32_t kType>
struct PlanesCfg {
  static constexpr bool kQ4 = kType == kGgmlQ4_K;
  static constexpr int kOps = kQ4 ? 1 : 2;   // weight operands per column
  static constexpr int kNT = kQ4 ? 2 : 1;    // 32-row MFMA tiles per wave
  static constexpr int kTileR = 4 * 32 * kNT;
  static constexpr int kBufHalfs = kPStage + kOps * kTileR * kRowStride;
};

// One thread per (row, block, 32-column run j = 2 kc + hf): the 32 operands
// StageChunk<kQ4> builds for chunk kc, half hf, at the same chunk columns.
struct PlanesArgs {
  const uint8_t* w;
  int64_t rows;
  int64_t row_bytes;
  int32_t nb;
  _Float16* planes;
  float2* dd;
  U32x4* mm;
};

template <uint32_t kType>
__device__ __forceinline__ void DecodeWeightUnit(const PlanesArgs& a, int64_t u) {
  const uint8_t* __restrict__ w = a.w;
  const int64_t rows = a.rows;
  const int64_t row_bytes = a.row_bytes;
  const int32_t nb = a.nb;
  _Float16* __restrict__ planes = a.planes;
  float2* __restrict__ dd = a.dd;
  U32x4* __restrict__ mm = a.mm;
  constexpr bool kQ4 = kType == kGgmlQ4_K;
  constexpr int64_t kBB = kQ4 ? kQ4KBlockBytes : kQ6KBlockBytes;
  if (u >= rows * nb * 8) return;
  const int j = static_cast<int>(u & 7);
  const int64_t rb = u >> 3;  // row * nb + block
  const int64_t r = rb / nb;
  const int b = static_cast<int>(rb - r * nb);
  const int kc = j >> 1, hf = j & 1;
  const int64_t cols = static_cast<int64_t>(nb) * kQK_K;
  const uint8_t* blk = w + r * row_bytes + b * kBB;
  _Float16* dst = planes + r * cols + static_cast<int64_t>(kQK_K) * b + kChunk * kc;
  const StageRaw raw = kQ4 ? FetchStageQ4K(blk, kc, hf) : FetchStageQ6K(blk, kc, hf);
  if (kQ4) {
    const uint32_t s0 = raw.hdr.y, s1 = raw.hdr.z, s2 = raw.hdr.w;
    uint32_t scl, ml, sch, mh;
    ScaleMinK4(2 * kc, s0, s1, s2, &scl, &ml);
    ScaleMinK4(2 * kc + 1, s0, s1, s2, &sch, &mh);
    const _Float16 fl = static_cast<_Float16>(static_cast<float>(scl));
    const _Float16 fh = static_cast<_Float16>(static_cast<float>(sch));
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const uint32_t bx = raw.q[2 * g], by = raw.q[2 * g + 1];
      *reinterpret_cast<F16x8*>(dst + 16 * hf + 8 * g) = ScaledQ4(make_uint2(bx & 0x0F0F0F0Fu, by & 0x0F0F0F0Fu), fl);
      *reinterpret_cast<F16x8*>(dst + 32 + 16 * hf + 8 * g) =
          ScaledQ4(make_uint2((bx >> 4) & 0x0F0F0F0Fu, (by >> 4) & 0x0F0F0F0Fu), fh);
    }
    if (j == 0) {
      F16x8 mv;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t sci, mi;
        ScaleMinK4(i, s0, s1, s2, &sci, &mi);
        mv[i] = static_cast<_Float16>(static_cast<float>(mi << kSumShift));
      }
      mm[rb] = __builtin_bit_cast(U32x4, mv);
      dd[rb] = make_float2(HalfF(raw.hdr.x & 0xFFFFu), HalfF(raw.hdr.x >> 16));
    }
  } else {
    const int64_t plane = rows * cols;
    const int quarter = 2 * (kc & 1) + hf;
    const int nshift = quarter < 2 ? 0 : 4;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t lx = raw.q[2 * g], ly = raw.q[2 * g + 1];
      const uint32_t hx = raw.q[8 + 2 * g], hy = raw.q[8 + 2 * g + 1];
      const uint2 q = make_uint2(((lx >> nshift) & 0x0F0F0F0Fu) | (((hx >> (2 * quarter)) & 0x03030303u) << 4),
                                 ((ly >> nshift) & 0x0F0F0F0Fu) | (((hy >> (2 * quarter)) & 0x03030303u) << 4));
      const F16x8 qc = CenteredQ6(q);
      const float sc = static_cast<float>(static_cast<int8_t>(ByteOf(raw.hdr.y, g >> 1)));
      // w = sc (q - 32), |w| <= 4096, exact in fp32; hi = w rounded to fp16
      // (exact unless |w| > 2048 and odd), lo = w - hi in {-1, 0, 1}
      F16x8 wh, wl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float wf = static_cast<float>(qc[i]) * sc;
        const _Float16 a = static_cast<_Float16>(wf);
        wh[i] = a;
        wl[i] = static_cast<_Float16>(wf - static_cast<float>(a));
      }
      *reinterpret_cast<F16x8*>(dst + 32 * hf + 8 * g) = wh;
      *reinterpret_cast<F16x8*>(dst + plane + 32 * hf + 8 * g) = wl;
    }
    if (j == 0) dd[rb] = make_float2(HalfF(raw.hdr.x & 0xFFFFu), 0.0f);
  }
}

template <uint32_t kType>
__global__ __launch_bounds__(kThreads) void DecodeWeightPlanesKernel(PlanesArgs a) {
  DecodeWeightUnit<kType>(a, static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x);
}

// The activation split and a matrix's weight decode in one launch: workgroups
// below n_split split token row blockIdx.x, the others decode weights, so the
// two independent passes share the chip instead of following each other.
template <uint32_t kType, int kU>
__global__ __launch_bounds__(kThreads) void PrepareKernel(SplitArgs sa, int32_t n_split, PlanesArgs pa) {
  if (static_cast<int32_t>(blockIdx.x) < n_split) {
    SplitRow<kU>(sa, blockIdx.x);
    return;
  }
  DecodeWeightUnit<kType>(pa, (static_cast<int64_t>(blockIdx.x) - n_split) * kThreads + threadIdx.x);
}

// Tiles are numbered row tile fastest (tile = token tile * row_tiles + row
// tile). Workgroup g < dp_tiles computes tile g over all of K, straight to
// out. The others split the remaining tiles along K: g - dp_tiles =
// (tile - dp_tiles) * splits + slice, slice covering blocks [slice bps,
// min(nb, (slice + 1) bps)); each writes its 128 x kTileR partial tile (times
// 1 / s_t, zero for tokens past n_tokens) to partial[g - dp_tiles], and
// MatMulPlanesReduceKernel sums the slices in order. With a 1-D grid the
// split workgroups are dispatched last, after the whole rounds.
template <uint32_t kType>
__global__ __launch_bounds__(kPThreads, 1) void MatMulMfmaPlanesKernel(
    const _Float16* __restrict__ wplanes, const float2* __restrict__ dd, const U32x4* __restrict__ mm, int64_t rows,
    int32_t nb, const _Float16* __restrict__ planes, const _Float16* __restrict__ sum_planes, int64_t sum_stride,
    const float* __restrict__ inv_scale, int64_t n_tokens, int32_t row_tiles, int32_t dp_tiles, int32_t splits,
    int32_t bps, float* __restrict__ out, int64_t ldo, float* __restrict__ partial) {
  using C = PlanesCfg<kType>;
  constexpr bool kQ4 = C::kQ4;
  constexpr int kOps = C::kOps;
  constexpr int kNT = C::kNT;
  __shared__ __attribute__((aligned(16))) _Float16 lds[2 * C::kBufHalfs];
  __shared__ float2 be_d[C::kTileR];                       // (d, dmin) of each row
  __shared__ U32x4 be_m[kQ4 ? C::kTileR : 1];              // Q4_K: m_j 2^6 of each row
  __shared__ U32x4 be_s[kQ4 ? kPlanes : 1][kQ4 ? kTileT : 1];  // Q4_K: run sums of each token
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2;  // 64-token half of the tile
  const int wn = wave & 3;   // 32 kNT-row quarter of the tile
  const int li = lane & 31;
  const int h = lane >> 5;
  const int g = static_cast<int>(blockIdx.x);
  const bool split = g >= dp_tiles;
  const int tile = split ? dp_tiles + (g - dp_tiles) / splits : g;
  const int slice = split ? (g - dp_tiles) % splits : 0;
  const int64_t t0 = static_cast<int64_t>(tile / row_tiles) * kTileT;
  const int64_t r0 = static_cast<int64_t>(tile % row_tiles) * C::kTileR;
  const int64_t cols = static_cast<int64_t>(nb) * kQK_K;
  const int64_t runs = cols / 32;
  const int64_t plane_elems = n_tokens * cols;
  const int b0 = split ? slice * bps : 0;
  const int n_blk = split ? (nb - b0 < bps ? nb - b0 : bps) : nb;
  const int n_chunks = 4 * n_blk;

  F32x16 acc[2][kNT], part[2][kNT];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[mt][nt][i] = 0.0f;
        part[mt][nt][i] = 0.0f;
      }

  // staging map: 16-byte piece j of thread tid is row (tid >> 3) + 64 j' of
  // its operand, segment tid & 7 of the chunk. Activations: j = 0..3 ->
  // plane j >> 1, token rows 64 (j & 1) + tid >> 3 (clamped; a token past
  // n_tokens reads a valid row whose outputs are never stored). Weights:
  // j = 0..3 -> operand j / (4 / kOps), rows 64 (j % (4 / kOps)) + tid >> 3
  // (clamped to the last row likewise).
  // element offsets are 32-bit: the launcher checks that both operand
  // images hold fewer than 2^31 elements
  const int seg = tid & 7;
  const int row8 = tid >> 3;
  const int icols = static_cast<int>(cols);
  U32x4 ra[4], rb[4];
  int aoff[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    int64_t t = t0 + 64 * k + row8;
    t = t < n_tokens ? t : n_tokens - 1;
    aoff[k] = static_cast<int>(t) * icols + kQK_K * b0 + 8 * seg;
  }
  constexpr int kRowsPerOp = 4 / kOps;  // 64-row groups per operand
  int boff[kRowsPerOp];
#pragma unroll
  for (int k = 0; k < kRowsPerOp; ++k) {
    int64_t r = r0 + 64 * k + row8;
    r = r < rows ? r : rows - 1;
    boff[k] = static_cast<int>(r) * icols + kQK_K * b0 + 8 * seg;
  }
  const int iplane = static_cast<int>(plane_elems);
  const int wplane = static_cast<int>(rows * cols);
  const int lds_a = row8 * kRowStride + 8 * seg;
  const int lds_b = kPStage + row8 * kRowStride + 8 * seg;

#define RPG_PLANES_LOAD(c)                                                                                  \
  do {                                                                                                      \
    const int off_ = (c) * kChunk;                                                                          \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) ra[j] =                                                   \
        *reinterpret_cast<const U32x4*>(planes + (aoff[j & 1] + (j >> 1) * iplane + off_));                 \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) rb[j] =                                                   \
        *reinterpret_cast<const U32x4*>(wplanes + (boff[j % kRowsPerOp] + (j / kRowsPerOp) * wplane + off_)); \
  } while (0)
#define RPG_PLANES_STAGE(buf)                                                                               \
  do {                                                                                                      \
    _Float16* base_ = lds + (buf) * C::kBufHalfs;                                                           \
    _Pragma("unroll") for (int j = 0; j < 4; ++j)                                                           \
        *reinterpret_cast<U32x4*>(base_ + lds_a + ((j >> 1) * kTileT + 64 * (j & 1)) * kRowStride) = ra[j]; \
    _Pragma("unroll") for (int j = 0; j < 4; ++j)                                                           \
        *reinterpret_cast<U32x4*>(base_ + lds_b +                                                           \
                                  ((j / kRowsPerOp) * C::kTileR + 64 * (j % kRowsPerOp)) * kRowStride) = rb[j]; \
  } while (0)

  // Block-end values of the tile, through LDS (registers are the scarce
  // resource): per row (d, dmin) and m_j 2^6, per token and plane the
  // block's 8 run sums (Q4_K). Thread tid fetches piece tid (and 512 + tid):
  //   Q4_K: pieces 0..255 m of row tid; 256..511 run sums of plane (q - 256)
  //         / 128, token (q - 256) % 128; 512..639 (d, dmin) of rows 2 (q -
  //         512) and + 1.
  //   Q6_K: pieces 0..63 (d, 0) of rows 2 q and + 1.
  // Rows and tokens are clamped like the operand loads.
  const int be_tok = static_cast<int>(t0 + (tid & 127) < n_tokens ? t0 + (tid & 127) : n_tokens - 1);
  const int be_row = static_cast<int>(r0 + (tid & 255) < rows ? r0 + (tid & 255) : rows - 1);
  const int be_row2a = static_cast<int>(r0 + 2 * tid < rows ? r0 + 2 * tid : rows - 1);
  const int be_row2b = static_cast<int>(r0 + 2 * tid + 1 < rows ? r0 + 2 * tid + 1 : rows - 1);
  constexpr int kDPairs = C::kTileR / 2;
  U32x4 be_v;
  float2 be_d0, be_d1;
  auto fetch_block_end = [&](int blk) {
    if (kQ4) {
      if (tid < 256) be_v = mm[be_row * nb + blk];
      else be_v = *reinterpret_cast<const U32x4*>(sum_planes + ((tid - 256) >> 7) * sum_stride +
                                                  (be_tok * static_cast<int>(runs) + 8 * blk));
    }
    if (tid < kDPairs) {
      be_d0 = dd[be_row2a * nb + blk];
      be_d1 = dd[be_row2b * nb + blk];
    }
  };
  auto store_block_end = [&]() {
    if (kQ4) {
      if (tid < 256) be_m[tid] = be_v;
      else be_s[(tid - 256) >> 7][tid & 127] = be_v;
    }
    if (tid < kDPairs) {
      be_d[2 * tid] = be_d0;
      be_d[2 * tid + 1] = be_d1;
    }
  };

  // first: the block's first K-step, whose first product per accumulator
  // starts from zero (an exact sum, so no zeroing pass at the block end)
  auto k_step = [&](int buf, int ks, bool first) {
    const _Float16* xs = lds + buf * C::kBufHalfs;
    const _Float16* ws = xs + kPStage;
    const int kcol = 16 * ks + 8 * h;
    F16x8 af[2][kPlanes], bf[kNT][kOps];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int o = 0; o < kOps; ++o)
        bf[nt][o] = *reinterpret_cast<const F16x8*>(ws + (o * C::kTileR + 32 * kNT * wn + 32 * nt + li) * kRowStride + kcol);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int p = 0; p < kPlanes; ++p)
        af[mt][p] = *reinterpret_cast<const F16x8*>(xs + (p * kTileT + 64 * wm + 32 * mt + li) * kRowStride + kcol);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int p = 0; p < kPlanes; ++p)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int o = 0; o < kOps; ++o) {
            if (p == 1 && o == 1) continue;  // Q6_K x_lo w_lo: below 2^-22 |x w|, not formed
            const F32x16 zero = {};
            part[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mt][p], bf[nt][o],
                                                                  first && p == 0 && o == 0 ? zero : part[mt][nt], 0, 0, 0);
          }
  };

  // the next block's first K-step overwrites part (its products start from zero)
  auto block_end = [&]() {
    float2 bd[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) bd[nt] = be_d[32 * kNT * wn + 32 * nt + li];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const float d = bd[nt].x;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][nt][i] = __builtin_fmaf(d, part[mt][nt][i], acc[mt][nt][i]);
    }
    if (!kQ4) return;
    F16x8 bmf[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const F16x8 z = {};
      bmf[nt] = h == 0 ? __builtin_bit_cast(F16x8, be_m[32 * kNT * wn + 32 * nt + li]) : z;  // k 8..15: zero weights
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int p = 0; p < kPlanes; ++p) {
        const F16x8 a = __builtin_bit_cast(F16x8, be_s[p][64 * wm + 32 * mt + li]);
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
          const F32x16 zero = {};
          part[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bmf[nt], p == 0 ? zero : part[mt][nt], 0, 0, 0);
        }
      }
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const float dmin = bd[nt].y;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][nt][i] = __builtin_fmaf(-dmin, part[mt][nt][i], acc[mt][nt][i]);
    }
  };

  // The loads and LDS writes are unconditional (the last chunks re-stage the
  // final chunk into the idle buffer): registers filled under a condition that
  // spans iterations end up in scratch memory.
  const int last = n_chunks - 1;
  fetch_block_end(b0);
  RPG_PLANES_LOAD(0);
  RPG_PLANES_STAGE(0);
  RPG_PLANES_LOAD(last > 0 ? 1 : 0);
  store_block_end();
  __syncthreads();
  for (int blk = 0; blk < n_blk; ++blk) {
    // A block's end values are fetched at its first chunk, ahead of that
    // chunk's staging loads (so the wait before the next LDS writes never
    // waits for a load issued after them), and stored to LDS before the
    // chunk's barrier; the previous block's end read them three barriers
    // earlier.
    if (blk > 0) fetch_block_end(b0 + blk);
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {  // chunk 4 blk + kc, in LDS buffer kc & 1
      const int c = 4 * blk + kc;
      k_step(kc & 1, 0, kc == 0);
      RPG_PLANES_STAGE((kc & 1) ^ 1);
      RPG_PLANES_LOAD(c + 2 < last ? c + 2 : last);
      k_step(kc & 1, 1, false);
      k_step(kc & 1, 2, false);
      k_step(kc & 1, 3, false);
      if (kc == 0 && blk > 0) store_block_end();
      if (kc == 3) block_end();
      __syncthreads();
    }
  }
#undef RPG_PLANES_LOAD
#undef RPG_PLANES_STAGE

  if (split) {
    float* dst = partial + static_cast<int64_t>(g - dp_tiles) * kTileT * C::kTileR;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int lt = 64 * wm + 32 * mt + (i & 3) + 8 * (i >> 2) + 4 * h;
        const int64_t tok = t0 + lt;
        const float inv = tok < n_tokens ? inv_scale[tok] : 0.0f;
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) dst[lt * C::kTileR + 32 * kNT * wn + 32 * nt + li] = acc[mt][nt][i] * inv;
      }
    }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t tok = t0 + 64 * wm + 32 * mt + (i & 3) + 8 * (i >> 2) + 4 * h;
      if (tok >= n_tokens) continue;
      const float inv = inv_scale[tok];
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        const int64_t row = r0 + 32 * kNT * wn + 32 * nt + li;
        if (row < rows) out[tok * ldo + row] = acc[mt][nt][i] * inv;
      }
    }
  }
}

// out = the sum over slices, in order, of the split tiles' partial tiles.
template <int kTileRows>
__global__ __launch_bounds__(kThreads) void MatMulPlanesReduceKernel(const float* __restrict__ partial,
                                                                      int64_t split_tiles, int32_t splits,
                                                                      int32_t row_tiles, int32_t dp_tiles,
                                                                      int64_t n_tokens, int64_t rows,
                                                                      float* __restrict__ out, int64_t ldo) {
  constexpr int64_t kTileElems = static_cast<int64_t>(kTileT) * kTileRows;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= split_tiles * kTileElems) return;
  const int64_t st = e / kTileElems;
  const int64_t le = e - st * kTileElems;
  const int64_t tile = dp_tiles + st;
  const int64_t tok = (tile / row_tiles) * kTileT + le / kTileRows;
  const int64_t row = (tile % row_tiles) * kTileRows + le % kTileRows;
  if (tok >= n_tokens || row >= rows) return;
  const float* p = partial + st * splits * kTileElems + le;
  float v = p[0];
  for (int32_t z = 1; z < splits; ++z) v += p[z * kTileElems];
  out[tok * ldo + row] = v;
}

}  // namespace

namespace {

// ---------------------------------------------------------------- split-activation buffer
//
// Grow-only, library-owned. An outgrown buffer is retired, not freed: a graph
// captured earlier keeps its address (growth during a capture is refused).
// Never freed at exit (a destructor running after the HIP runtime has shut down
// can hang).
struct SplitBuffer {
  std::mutex mu;
  void* ptr = nullptr;
  size_t bytes = 0;
};
SplitBuffer& Splits() {
  static SplitBuffer* b = new SplitBuffer();
  return *b;
}

void* EnsureSplitBuffer(size_t bytes) {
  SplitBuffer& b = Splits();
  std::lock_guard<std::mutex> lock(b.mu);
  if (b.bytes < bytes) {
    RPG_CHECK(!StreamIsCapturing(),
              "the prefill matmul needs a %zu-byte activation buffer (have %zu), which cannot be allocated during "
              "graph capture; run the same shape once before capturing",
              bytes, b.bytes);
    const size_t grow = bytes > 2 * b.bytes ? bytes : 2 * b.bytes;
    void* p = nullptr;
    RPG_HIP_CHECK(hipMalloc(&p, grow));
    b.ptr = p;  // the previous buffer stays allocated (see above)
    b.bytes = grow;
  }
  return b.ptr;
}

SplitBuffer& PartialTiles() {
  static SplitBuffer* b = new SplitBuffer();
  return *b;
}

// Grow-only buffer of the K-slices' partial tiles (same policy as the split buffer).
void* EnsurePartialTiles(size_t bytes) {
  SplitBuffer& b = PartialTiles();
  std::lock_guard<std::mutex> lock(b.mu);
  if (b.bytes < bytes) {
    RPG_CHECK(!StreamIsCapturing(),
              "the prefill matmul needs a %zu-byte partial-tile buffer (have %zu), which cannot be allocated during "
              "graph capture; run the same shape once before capturing",
              bytes, b.bytes);
    const size_t grow = bytes > 2 * b.bytes ? bytes : 2 * b.bytes;
    void* p = nullptr;
    RPG_HIP_CHECK(hipMalloc(&p, grow));
    b.ptr = p;  // the previous buffer stays allocated
    b.bytes = grow;
  }
  return b.ptr;
}

SplitBuffer& WeightPlanes() {
  static SplitBuffer* b = new SplitBuffer();
  return *b;
}

// Grow-only buffer of the decoded weight planes: an outgrown buffer is retired,
// not freed, as for the split buffer, and it grows at least twofold, so a
// forward's growing matrix shapes retire few buffers (the largest request is one
// 64 MB slice of planes plus its block values).
void* EnsureWeightPlanes(size_t bytes) {
  SplitBuffer& b = WeightPlanes();
  std::lock_guard<std::mutex> lock(b.mu);
  if (b.bytes < bytes) {
    RPG_CHECK(!StreamIsCapturing(),
              "the prefill matmul needs a %zu-byte weight-plane buffer (have %zu), which cannot be allocated during "
              "graph capture; run the same shape once before capturing",
              bytes, b.bytes);
    const size_t grow = bytes > 2 * b.bytes ? bytes : 2 * b.bytes;
    void* p = nullptr;
    RPG_HIP_CHECK(hipMalloc(&p, grow));
    b.ptr = p;  // the previous buffer stays allocated
    b.bytes = grow;
  }
  return b.ptr;
}

// Decoded planes are used for grids of many tiles (from kPlanesMinTokens
// tokens). A matrix whose planes exceed kPlanesMaxBytes (a 151936-row output
// projection) is decoded and multiplied in row slices that fit, each writing
// its columns of OUT.
constexpr int64_t kPlanesMinTokens = 512;
constexpr size_t kPlanesMaxBytes = size_t{64} << 20;

// OUT[:, 0 : rows) with row stride ldo for the `rows` weight rows at w.
SplitArgs SplitArgsOf(const SplitActivations& sa) {
  return SplitArgs{sa.x, sa.cols, sa.n_tokens * sa.cols, sa.sum_stride, static_cast<_Float16*>(sa.planes),
                   static_cast<_Float16*>(sa.sums), sa.inv_scale};
}

// Register steps per thread of the split (a row of up to 5 steps, 10240
// columns, stays in registers between its two passes; 0: wider rows).
int SplitSteps(int64_t cols) {
  const int64_t steps = (cols + 8 * kThreads - 1) / (8 * kThreads);
  return steps <= 5 ? static_cast<int>(steps) : 0;
}

// Launches a pending split on its own.
void LaunchPendingSplit(const SplitActivations& sa) {
  if (!sa.pending) return;
  sa.pending = false;
  const SplitArgs a = SplitArgsOf(sa);
  const dim3 grid(static_cast<unsigned>(sa.n_tokens)), block(kThreads);
  switch (SplitSteps(sa.cols)) {
    case 1: Launch("SplitActivationsKernel", SplitActivationsKernel<1>, grid, block, a); break;
    case 2: Launch("SplitActivationsKernel", SplitActivationsKernel<2>, grid, block, a); break;
    case 3: Launch("SplitActivationsKernel", SplitActivationsKernel<3>, grid, block, a); break;
    case 4: Launch("SplitActivationsKernel", SplitActivationsKernel<4>, grid, block, a); break;
    case 5: Launch("SplitActivationsKernel", SplitActivationsKernel<5>, grid, block, a); break;
    default: Launch("SplitActivationsKernel", SplitActivationsKernel<0>, grid, block, a); break;
  }
}

// The weight decode of one row slice, with a pending split in the same launch.
template <uint32_t kType>
void LaunchDecode(const PlanesArgs& pa, const SplitActivations& sa) {
  const int64_t units = pa.rows * pa.nb * 8;
  const unsigned decode_wgs = GridFor(units, kThreads);
  if (!sa.pending) {
    Launch(kType == kGgmlQ4_K ? "DecodeWeightPlanesQ4KKernel" : "DecodeWeightPlanesQ6KKernel",
           DecodeWeightPlanesKernel<kType>, dim3(decode_wgs), dim3(kThreads), pa);
    return;
  }
  sa.pending = false;
  const SplitArgs a = SplitArgsOf(sa);
  RPG_CHECK(sa.n_tokens + static_cast<int64_t>(decode_wgs) <= 0x7FFFFFFF, "split + decode grid too large");
  const int32_t n_split = static_cast<int32_t>(sa.n_tokens);
  const dim3 grid(static_cast<unsigned>(sa.n_tokens + decode_wgs)), block(kThreads);
  const char* name = kType == kGgmlQ4_K ? "PrepareQ4KKernel" : "PrepareQ6KKernel";
  switch (SplitSteps(sa.cols)) {
    case 1: Launch(name, PrepareKernel<kType, 1>, grid, block, a, n_split, pa); break;
    case 2: Launch(name, PrepareKernel<kType, 2>, grid, block, a, n_split, pa); break;
    case 3: Launch(name, PrepareKernel<kType, 3>, grid, block, a, n_split, pa); break;
    case 4: Launch(name, PrepareKernel<kType, 4>, grid, block, a, n_split, pa); break;
    case 5: Launch(name, PrepareKernel<kType, 5>, grid, block, a, n_split, pa); break;
    default: Launch(name, PrepareKernel<kType, 0>, grid, block, a, n_split, pa); break;
  }
}

template <uint32_t kType>
void LaunchPlanesRows(const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const SplitActivations& sa,
                      float* out, int64_t ldo) {
  using C = PlanesCfg<kType>;
  const int64_t cols = static_cast<int64_t>(nb) * kQK_K;
  const size_t plane_bytes = static_cast<size_t>(C::kOps) * rows * cols * sizeof(_Float16);
  const size_t dd_off = (plane_bytes + 255) / 256 * 256;
  const size_t mm_off = dd_off + (static_cast<size_t>(rows) * nb * sizeof(float2) + 255) / 256 * 256;
  const size_t bytes = mm_off + static_cast<size_t>(rows) * nb * sizeof(U32x4);
  uint8_t* base = static_cast<uint8_t*>(EnsureWeightPlanes(bytes));
  _Float16* wplanes = reinterpret_cast<_Float16*>(base);
  float2* dd = reinterpret_cast<float2*>(base + dd_off);
  U32x4* mm = reinterpret_cast<U32x4*>(base + mm_off);
  LaunchDecode<kType>(PlanesArgs{w, rows, row_bytes, nb, wplanes, dd, mm}, sa);

  const int64_t gy = (sa.n_tokens + kTileT - 1) / kTileT;
  const int64_t gx = (rows + C::kTileR - 1) / C::kTileR;
  const int64_t tiles = gx * gy;
  RPG_CHECK(tiles * 8 <= 0x7FFFFFFF, "matmul grid too large: %lld tiles", static_cast<long long>(tiles));
  // One workgroup per CU, so a grid runs in rounds of kCUs workgroups. Plans:
  // whole rounds of tiles unsplit and the tiles left over split along K to
  // fill the last round (dp = the whole rounds), or every tile split alike
  // (dp = 0). Each is priced as rounds x blocks per workgroup x the time of
  // one block of one tile, plus the reduce (slices + 1 passes over the split
  // tiles at ~4 TB/s); the cheapest wins.
  constexpr int64_t kCUs = 256;
  constexpr double kBlockUs = C::kQ4 ? 10.0 : 6.6;  // measured, 2811 tokens
  const double tile_bytes = 4.0 * kTileT * C::kTileR;
  int64_t best_dp = tiles;
  int32_t best_splits = 1, best_bps = nb;
  double best = 0.0;
  for (int plan = 0; plan < 2; ++plan) {
    const int64_t dp = plan == 0 ? tiles / kCUs * kCUs : 0;
    const int64_t rest = tiles - dp;
    for (int32_t s = 1; s <= nb && s <= 16; ++s) {
      const int32_t b = (nb + s - 1) / s;
      const int32_t slices = (nb + b - 1) / b;
      if (rest == 0 && slices > 1) break;
      const int64_t rounds_rest = (rest * slices + kCUs - 1) / kCUs;
      const double us = static_cast<double>(dp / kCUs) * nb * kBlockUs + static_cast<double>(rounds_rest) * b * kBlockUs +
                        (slices > 1 ? (slices + 1) * static_cast<double>(rest) * tile_bytes / 4e6 : 0.0);
      if (best == 0.0 || us < best) {
        best = us;
        best_dp = slices > 1 ? dp : tiles;
        best_splits = slices;
        best_bps = b;
      }
    }
  }
  const int64_t split_tiles = tiles - best_dp;
  float* partial = nullptr;
  if (split_tiles > 0) {
    partial = static_cast<float*>(EnsurePartialTiles(static_cast<size_t>(split_tiles) * best_splits * kTileT *
                                                     C::kTileR * sizeof(float)));
  }
  const int64_t wgs = best_dp + split_tiles * best_splits;
  Launch(kType == kGgmlQ4_K ? "MatMulMfmaQ4KPlanesKernel" : "MatMulMfmaQ6KPlanesKernel", MatMulMfmaPlanesKernel<kType>,
         dim3(static_cast<unsigned>(wgs)), dim3(kPThreads), static_cast<const _Float16*>(wplanes),
         static_cast<const float2*>(dd), static_cast<const U32x4*>(mm), rows, nb,
         static_cast<const _Float16*>(sa.planes), static_cast<const _Float16*>(sa.sums), sa.sum_stride, sa.inv_scale,
         sa.n_tokens, static_cast<int32_t>(gx), static_cast<int32_t>(best_dp), best_splits, best_bps, out, ldo, partial);
  if (split_tiles > 0) {
    const int64_t elems = split_tiles * kTileT * C::kTileR;
    Launch("MatMulPlanesReduceKernel", MatMulPlanesReduceKernel<C::kTileR>, dim3(GridFor(elems, kThreads)),
           dim3(kThreads), static_cast<const float*>(partial), split_tiles, best_splits, static_cast<int32_t>(gx),
           static_cast<int32_t>(best_dp), sa.n_tokens, rows, out, ldo);
  }
}

template <uint32_t kType>
void LaunchPlanes(const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const SplitActivations& sa,
                  float* out) {
  using C = PlanesCfg<kType>;
  const int64_t row_plane_bytes = static_cast<int64_t>(C::kOps) * nb * kQK_K * sizeof(_Float16);
  int64_t slice = static_cast<int64_t>(kPlanesMaxBytes) / row_plane_bytes / C::kTileR * C::kTileR;
  if (slice < C::kTileR) slice = C::kTileR;
  for (int64_t r = 0; r < rows; r += slice) {
    const int64_t n = rows - r < slice ? rows - r : slice;
    LaunchPlanesRows<kType>(w + r * row_bytes, n, row_bytes, nb, sa, out + r, rows);
  }
}

}  // namespace

SplitActivations SplitForMfma(const float* x, int64_t n_tokens, int64_t cols) {
  RPG_CHECK(n_tokens > 0 && cols > 0 && cols % 32 == 0, "invalid activation split [%lld, %lld]",
            static_cast<long long>(n_tokens), static_cast<long long>(cols));
  RPG_CHECK(n_tokens <= 0x7FFFFFFF, "too many tokens for the activation split: %lld", static_cast<long long>(n_tokens));
  const int64_t elems = n_tokens * cols;
  const int64_t sum_elems = elems / 32;
  const size_t plane_bytes = static_cast<size_t>(elems) * sizeof(_Float16);
  const size_t sum_bytes = (static_cast<size_t>(sum_elems) * sizeof(_Float16) + 255) / 256 * 256;
  const size_t bytes = kPlanes * plane_bytes + kPlanes * sum_bytes + static_cast<size_t>(n_tokens) * sizeof(float);
  uint8_t* base = static_cast<uint8_t*>(EnsureSplitBuffer(bytes));
  SplitActivations sa;
  sa.planes = base;
  sa.sums = base + kPlanes * plane_bytes;
  sa.inv_scale = reinterpret_cast<float*>(base + kPlanes * plane_bytes + kPlanes * sum_bytes);
  sa.sum_stride = static_cast<int64_t>(sum_bytes / sizeof(_Float16));
  sa.n_tokens = n_tokens;
  sa.cols = cols;
  sa.x = x;
  sa.pending = true;
  return sa;
}

// Launched by GpuMatMulQuantRaw / GpuMatMulQuantGroup for Q4_K / Q6_K with
// enough tokens; the caller has checked the type, the alignment (Q4_K 16 bytes,
// Q6_K 2 bytes) and cols % 256 == 0, and split the activations. When the output
// tiles cannot give every CU a workgroup, K is divided
// into slices of whole blocks whose partial tiles are summed afterwards in a
// fixed order (deterministic). Between one and two workgroups per CU the
// extra pass costs more than the second workgroup slot gains.
void LaunchMatMulMfmaSplit(uint32_t type, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb,
                           const SplitActivations& sa, float* out) {
  const int64_t gy = (sa.n_tokens + kTileT - 1) / kTileT;
  const int64_t gx = (rows + kTileR - 1) / kTileR;
  RPG_CHECK(gy <= 65535 && gx <= 0x7FFFFFFF, "matmul grid too large: %lld x %lld", static_cast<long long>(gx),
            static_cast<long long>(gy));
  RPG_CHECK(static_cast<int64_t>(nb) * kQK_K == sa.cols, "split activations have %lld columns, the matrix %lld",
            static_cast<long long>(sa.cols), static_cast<long long>(nb) * kQK_K);
  // (the planes kernel indexes both operand images with 32-bit offsets;
  // the weight slices stay within kPlanesMaxBytes)
  if (sa.n_tokens >= kPlanesMinTokens && kPlanes * sa.n_tokens * sa.cols < (int64_t{1} << 31)) {
    if (type == kGgmlQ4_K) {
      LaunchPlanes<kGgmlQ4_K>(w, rows, row_bytes, nb, sa, out);
    } else {
      LaunchPlanes<kGgmlQ6_K>(w, rows, row_bytes, nb, sa, out);
    }
    return;
  }
  LaunchPendingSplit(sa);
  constexpr int64_t kFill = 256;
  const int64_t tiles = gx * gy;
  int64_t want = tiles >= kFill ? 1 : (kFill + tiles - 1) / tiles;
  if (want > nb) want = nb;
  const int32_t bps = static_cast<int32_t>((nb + want - 1) / want);
  const int32_t splits = static_cast<int32_t>((nb + bps - 1) / bps);
  float* partial = nullptr;
  const int64_t elems = sa.n_tokens * rows;
  if (splits > 1) partial = static_cast<float*>(EnsurePartialTiles(static_cast<size_t>(splits) * elems * sizeof(float)));
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(splits));
  const _Float16* planes = static_cast<const _Float16*>(sa.planes);
  const _Float16* sums = static_cast<const _Float16*>(sa.sums);
  // wide matrices (more than 16 row tiles) only while the token tiles are
  // mostly empty: ffn_gate measured 14% faster at 130 tokens, 9% slower at 256
  const bool pp = tiles <= kPingPongTiles && (gx <= 16 || sa.n_tokens <= 160);
  const dim3 block(pp ? kGemmThreadsPP : kThreads);
  if (type == kGgmlQ4_K) {
    Launch(pp ? "MatMulMfmaQ4KPingPongKernel" : "MatMulMfmaQ4KKernel",
           pp ? MatMulMfmaKernel<kGgmlQ4_K, true> : MatMulMfmaKernel<kGgmlQ4_K, false>, grid, block, w, rows,
           row_bytes, nb, planes, sums, sa.sum_stride, sa.inv_scale, sa.cols, sa.n_tokens, bps, out, partial);
  } else {
    Launch(pp ? "MatMulMfmaQ6KPingPongKernel" : "MatMulMfmaQ6KKernel",
           pp ? MatMulMfmaKernel<kGgmlQ6_K, true> : MatMulMfmaKernel<kGgmlQ6_K, false>, grid, block, w, rows,
           row_bytes, nb, planes, sums, sa.sum_stride, sa.inv_scale, sa.cols, sa.n_tokens, bps, out, partial);
  }
  if (splits > 1) {
    Launch("MatMulSplitReduceKernel", MatMulSplitReduceKernel, dim3(GridFor(elems, kThreads)), dim3(kThreads),
           static_cast<const float*>(partial), elems, splits, out);
  }
}

void LaunchMatMulMfma(uint32_t type, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                      int64_t cols, int64_t n_tokens, float* out) {
  LaunchMatMulMfmaSplit(type, w, rows, row_bytes, nb, SplitForMfma(x, n_tokens, cols), out);
}

}  // namespace rpg
