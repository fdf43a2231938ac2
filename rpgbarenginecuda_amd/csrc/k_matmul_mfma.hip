// Prefill GEMM for the quantised matmul on the bf16 matrix cores of gfx950:
// OUT[t][r] = sum_e W[r][e] * X[t][e] for n_tokens large enough to fill a tile.
//
// Exactness of the operands:
//   * weights: the MFMA sees only the integer quants (Q4_K: q in 0..15; Q6_K:
//     q - 32 in -32..31), exact in bf16; the block scales are applied afterwards
//     in fp32, per sub-block (Q4_K, 32 elements: d1 * sum(q x) - m1 * sum(x)) or
//     per 16-element group (Q6_K: d * sc * sum((q - 32) x)), with d1 = d * sc,
//     m1 = dmin * m and d * sc exact in fp32 (11-bit fp16 times a 6/8-bit integer);
//   * activations: each fp32 x is split into three bf16 terms h + m + l (each the
//     round-to-nearest of what is left), which reproduce x to within 2^-27 |x|;
//     the three products with the same quant are accumulated by the matrix core
//     in fp32, like the fp32 fused multiply-adds of the other kernels.
// The activation run sums of Q4_K are summed in fp32 from the unsplit x.
//
// Tiling: a 256-thread workgroup computes 128 tokens x 128 weight rows; wave
// (wm, wn) owns tokens 64 wm + [0, 64) and rows 64 wn + [0, 64) as 2 x 2 tiles
// of v_mfma_f32_32x32x16_bf16 (A = activations [token][k], B = quants [k][row],
// so each lane's outputs for one register are 32 consecutive rows of one token:
// coalesced stores). The K loop walks 64-column chunks: the workgroup stages the
// chunk's activations as three bf16 planes plus the per-(token, sub-block) run
// sums in LDS, while each lane fetches the quant bytes its B operands need for
// the chunk straight from global memory.
#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"
#include "quant_dev.h"

namespace rpg {
namespace {

using dev::ByteOf;
using dev::ScaleMinK4;

typedef __bf16 Bf16x8 __attribute__((ext_vector_type(8)));
typedef float F32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileT = 128;       // tokens per workgroup
constexpr int kTileR = 128;       // weight rows per workgroup
constexpr int kChunk = 64;        // K columns staged per step
constexpr int kPad = 8;           // bf16 padding per staged row (breaks LDS bank conflicts)
constexpr int kRowStride = kChunk + kPad;
constexpr int kThreads = 256;

__device__ __forceinline__ float HalfF(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// Hides a packed-quant word's known-zero bits from the optimiser so bytes are
// converted directly (v_cvt_f32_ubyte{0..3}) instead of extracted first. Emits
// no instruction.
__device__ __forceinline__ uint32_t Opaque(uint32_t w) {
  __asm__("" : "+v"(w));
  return w;
}

// Eight exact integers (as bytes, unsigned or signed) -> eight bf16 lanes.
__device__ __forceinline__ Bf16x8 BytesToBf16U(uint32_t lo, uint32_t hi) {
  lo = Opaque(lo);
  hi = Opaque(hi);
  Bf16x8 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = static_cast<__bf16>(static_cast<float>((lo >> (8 * j)) & 0xFFu));
    v[4 + j] = static_cast<__bf16>(static_cast<float>((hi >> (8 * j)) & 0xFFu));
  }
  return v;
}
__device__ __forceinline__ Bf16x8 BytesToBf16S(uint32_t lo, uint32_t hi) {
  Bf16x8 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = static_cast<__bf16>(static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(lo >> (8 * j)))));
    v[4 + j] = static_cast<__bf16>(static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(hi >> (8 * j)))));
  }
  return v;
}

// 8 bytes starting `sh` (0 or 2) bytes into three aligned dwords.
__device__ __forceinline__ uint2 Window8x(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t sh) {
  return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// 8 bytes at a 2-byte aligned address (see the Q6_K note in k_matmul.hip: the
// aligned dwords around a field never leave the pages the tensor occupies).
__device__ __forceinline__ uint2 Load8Aligned2(const uint8_t* p) {
  const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint32_t* a = reinterpret_cast<const uint32_t*>(p - sh);
  return Window8x(a[0], a[1], a[1 + (sh >> 1)], sh);
}

// The per-chunk quant bytes and scales one lane needs for one weight row.
// Q4_K: q8[ks] = the 8 quants (as nibble bytes) for K-step ks; scale/min of the
// chunk's two sub-blocks. Q6_K: q8[ks] = the 8 signed quants (q - 32) for K-step
// ks; ds[ks] = d * sc of the group K-step ks falls in.
struct ChunkQuants {
  uint2 q8[4];
  float sc[4];   // Q4_K: d1 of sub-block 0, 1 in [0], [1]; Q6_K: d * sc per K-step
  float mn[2];   // Q4_K: m1 of sub-block 0, 1
};

// Q4_K chunk kc (0..3) of block blk; lane half h selects k = 8h .. 8h + 7 of
// each 16-wide K-step. Sub-block of K-step ks: 2 kc + ks / 2.
__device__ __forceinline__ ChunkQuants LoadChunkQ4K(const uint8_t* __restrict__ blk, int kc, int h) {
  ChunkQuants c;
  const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
  const float d = HalfF(hdr.x & 0xFFFFu);
  const float dmin = HalfF(hdr.x >> 16);
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    uint32_t sc, m;
    ScaleMinK4(2 * kc + s2, hdr.y, hdr.z, hdr.w, &sc, &m);
    c.sc[s2] = d * static_cast<float>(sc);
    c.mn[s2] = dmin * static_cast<float>(m);
  }
  c.sc[2] = c.sc[3] = 0.0f;
  // elements of sub-block j live in qs[32 (j / 2) + l], nibble j & 1; both
  // sub-blocks of a chunk share the same 32 qs bytes (j = 2kc, 2kc + 1).
  const uint8_t* qs = blk + 16 + 32 * kc;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const uint2 raw = *reinterpret_cast<const uint2*>(qs + 16 * (ks & 1) + 8 * h);
    const int shift = (ks >> 1) * 4;  // K-steps 0, 1: low nibbles (sub-block 2kc); 2, 3: high
    c.q8[ks] = make_uint2((raw.x >> shift) & 0x0F0F0F0Fu, (raw.y >> shift) & 0x0F0F0F0Fu);
  }
  return c;
}

// Q6_K chunk kc (0..3) of block blk (2-byte aligned): elements 64 kc + [0, 64)
// = half kc / 2, quarters 2 (kc % 2) and 2 (kc % 2) + 1.
__device__ __forceinline__ ChunkQuants LoadChunkQ6K(const uint8_t* __restrict__ blk, int kc, int h) {
  ChunkQuants c;
  const int half = kc >> 1;
  const int q0 = 2 * (kc & 1);
  const float d = HalfF(*reinterpret_cast<const uint16_t*>(blk + 208));
  const uint2 scw = Load8Aligned2(blk + 192 + 8 * half);
  uint2 qh[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) qh[r] = Load8Aligned2(blk + 128 + 32 * half + 16 * r + 8 * h);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int quarter = q0 + (ks >> 1);
    const int lq = 16 * (ks & 1) + 8 * h;  // element index inside the 32-run of the quarter
    const uint2 ql = Load8Aligned2(blk + 64 * half + 32 * (quarter & 1) + lq);
    const int nshift = quarter < 2 ? 0 : 4;
    const uint2 hb = qh[ks & 1];
    uint32_t w[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t qlw = k == 0 ? ql.x : ql.y;
      const uint32_t qhw = k == 0 ? hb.x : hb.y;
      const uint32_t nib = (qlw >> nshift) & 0x0F0F0F0Fu;
      const uint32_t hi2 = ((qhw >> (2 * quarter)) & 0x03030303u) << 4;
      w[k] = (nib | hi2) ^ 0x20202020u;  // 6-bit q - 32, two's complement in 6 bits
      // sign-extend each 6-bit field to a byte: bit 5 -> bits 6, 7
      w[k] |= ((w[k] & 0x20202020u) >> 5) * 0xC0u;
    }
    c.q8[ks] = make_uint2(w[0], w[1]);
    const int si = (lq >> 4) + 2 * quarter;  // index inside the half's 8 scales
    const int8_t sc = static_cast<int8_t>(ByteOf(si < 4 ? scw.x : scw.y, si & 3));
    c.sc[ks] = d * static_cast<float>(sc);
  }
  c.mn[0] = c.mn[1] = 0.0f;
  return c;
}

template <uint32_t kType>
__global__ __launch_bounds__(kThreads) void MatMulMfmaKernel(const uint8_t* __restrict__ w, int64_t rows,
                                                             int64_t row_bytes, int32_t nb,
                                                             const float* __restrict__ x, int64_t cols,
                                                             int64_t n_tokens, float* __restrict__ out) {
  constexpr int64_t kBB = kType == kGgmlQ4_K ? kQ4KBlockBytes : kQ6KBlockBytes;
  __shared__ __attribute__((aligned(16))) __bf16 xs[3][kTileT][kRowStride];
  __shared__ float xsum[kTileT][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int li = lane & 31;  // A: token row / B: weight row inside a 32-tile
  const int h = lane >> 5;   // which 8 of the 16 K of a step
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kTileT;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTileR;

  // the two weight rows of this lane (clamped: loads stay in bounds, results dropped)
  const uint8_t* wrow[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int64_t r = r0 + 64 * wn + 32 * nt + li;
    wrow[nt] = w + (r < rows ? r : rows - 1) * row_bytes;
  }

  F32x16 acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][nt][i] = 0.0f;

  // staging map: thread -> (token tok, sub-block half sh of the chunk: 32 columns)
  const int st_tok = tid >> 1;
  const int st_half = tid & 1;
  const int64_t st_t = t0 + st_tok;

  for (int b = 0; b < nb; ++b) {
    for (int kc = 0; kc < 4; ++kc) {
      // this chunk's quants for both weight rows (in flight during the staging)
      ChunkQuants cq[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        cq[nt] = kType == kGgmlQ4_K ? LoadChunkQ4K(wrow[nt] + b * kBB, kc, h) : LoadChunkQ6K(wrow[nt] + b * kBB, kc, h);

      // stage 128 tokens x 64 columns: three bf16 planes and fp32 run sums
      {
        float v[32];
        if (st_t < n_tokens) {
          const float* src = x + st_t * cols + static_cast<int64_t>(b) * kQK_K + kChunk * kc + 32 * st_half;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float4 f = *reinterpret_cast<const float4*>(src + 4 * i);
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 32; ++i) v[i] = 0.0f;
        }
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) s += v[i];
        xsum[st_tok][st_half] = s;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          Bf16x8 ph, pm, pl;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float xv = v[8 * g + j];
            const __bf16 bh = static_cast<__bf16>(xv);
            const float r1 = xv - static_cast<float>(bh);
            const __bf16 bm = static_cast<__bf16>(r1);
            const float r2 = r1 - static_cast<float>(bm);
            ph[j] = bh;
            pm[j] = bm;
            pl[j] = static_cast<__bf16>(r2);
          }
          const int col = 32 * st_half + 8 * g;
          *reinterpret_cast<Bf16x8*>(&xs[0][st_tok][col]) = ph;
          *reinterpret_cast<Bf16x8*>(&xs[1][st_tok][col]) = pm;
          *reinterpret_cast<Bf16x8*>(&xs[2][st_tok][col]) = pl;
        }
      }
      __syncthreads();

      if (kType == kGgmlQ4_K) {
        // two sub-blocks per chunk, two K-steps each
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          F32x16 part[2][2];
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
              for (int i = 0; i < 16; ++i) part[mt][nt][i] = 0.0f;
#pragma unroll
          for (int k2 = 0; k2 < 2; ++k2) {
            const int ks = 2 * sb + k2;
            Bf16x8 bq[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) bq[nt] = BytesToBf16U(cq[nt].q8[ks].x, cq[nt].q8[ks].y);
            const int kcol = 16 * (ks & 1) + 32 * sb + 8 * h;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
              const int tok = 64 * wm + 32 * mt + li;
#pragma unroll
              for (int p = 0; p < 3; ++p) {
                const Bf16x8 a = *reinterpret_cast<const Bf16x8*>(&xs[p][tok][kcol]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                  part[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq[nt], part[mt][nt], 0, 0, 0);
              }
            }
          }
          // acc += d1 * part - m1 * sum(x over the sub-block), per (token, row)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int tok = 64 * wm + 32 * mt + (i & 3) + 8 * (i >> 2) + 4 * h;
              const float sx = xsum[tok][sb];
#pragma unroll
              for (int nt = 0; nt < 2; ++nt) {
                float a = __builtin_fmaf(cq[nt].sc[sb], part[mt][nt][i], acc[mt][nt][i]);
                acc[mt][nt][i] = __builtin_fmaf(-cq[nt].mn[sb], sx, a);
              }
            }
          }
        }
      } else {
        // one scale group per K-step
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          F32x16 part[2][2];
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
              for (int i = 0; i < 16; ++i) part[mt][nt][i] = 0.0f;
          Bf16x8 bq[2];
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) bq[nt] = BytesToBf16S(cq[nt].q8[ks].x, cq[nt].q8[ks].y);
          const int kcol = 16 * ks + 8 * h;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            const int tok = 64 * wm + 32 * mt + li;
#pragma unroll
            for (int p = 0; p < 3; ++p) {
              const Bf16x8 a = *reinterpret_cast<const Bf16x8*>(&xs[p][tok][kcol]);
#pragma unroll
              for (int nt = 0; nt < 2; ++nt)
                part[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq[nt], part[mt][nt], 0, 0, 0);
            }
          }
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
              for (int i = 0; i < 16; ++i)
                acc[mt][nt][i] = __builtin_fmaf(cq[nt].sc[ks], part[mt][nt][i], acc[mt][nt][i]);
        }
      }
      __syncthreads();  // the next chunk overwrites xs / xsum
    }
  }

  // D[i][j]: j = lane % 32 (weight row), i = (r % 4) + 8 (r / 4) + 4 (lane / 32) (token)
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int64_t row = r0 + 64 * wn + 32 * nt + li;
      if (row >= rows) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t tok = t0 + 64 * wm + 32 * mt + (i & 3) + 8 * (i >> 2) + 4 * h;
        if (tok < n_tokens) out[tok * rows + row] = acc[mt][nt][i];
      }
    }
  }
}

}  // namespace

// Launched by GpuMatMulQuantRaw for Q4_K / Q6_K with enough tokens; the caller
// has checked the type, the alignment (Q4_K 16 bytes, Q6_K 2 bytes, x 16 bytes)
// and cols % 256 == 0.
void LaunchMatMulMfma(uint32_t type, const uint8_t* w, int64_t rows, int64_t row_bytes, int32_t nb, const float* x,
                      int64_t cols, int64_t n_tokens, float* out) {
  const int64_t gy = (n_tokens + kTileT - 1) / kTileT;
  const int64_t gx = (rows + kTileR - 1) / kTileR;
  RPG_CHECK(gy <= 65535 && gx <= 0x7FFFFFFF, "matmul grid too large: %lld x %lld", static_cast<long long>(gx),
            static_cast<long long>(gy));
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  if (type == kGgmlQ4_K) {
    Launch("MatMulMfmaQ4KKernel", MatMulMfmaKernel<kGgmlQ4_K>, grid, dim3(kThreads), w, rows, row_bytes, nb, x, cols,
           n_tokens, out);
  } else {
    Launch("MatMulMfmaQ6KKernel", MatMulMfmaKernel<kGgmlQ6_K>, grid, dim3(kThreads), w, rows, row_bytes, nb, x, cols,
           n_tokens, out);
  }
}

}  // namespace rpg
