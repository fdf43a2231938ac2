// Device-side helpers for the ggml Q4_K / Q6_K block formats, shared by the
// dequant / gather kernels and the quantised matmul.
//
// Block layouts (src/quant.cc:29-45, restated in src/quant_gpu.cuh:50-179):
//   Q4_K, 144 bytes / 256 elements: d f16 | dmin f16 | scales[12] | qs[128]
//     element 64g + l (l < 32) is the low nibble of qs[32g + l], element 64g + 32 + l
//     the high nibble; sub-block j = e / 32 has 6-bit (sc, m) from GetScaleMinK4.
//     y = (d * sc) * q - (dmin * m), three separately rounded fp32 ops.
//   Q6_K, 210 bytes / 256 elements: ql[128] | qh[64] | sc[16] int8 | d f16
//     element 128h + 32q + l: nibble of ql[64h + l + 32(q & 1)] (low for q < 2),
//     high bits (qh[32h + l] >> 2q) & 3, scale sc[8h + l/16 + 2q];
//     y = (d * sc) * (q6 - 32), two separately rounded fp32 ops.
// Everything that includes this header is compiled with -ffp-contract=off, so
// the dequantised values are bit-identical to the reference CPU dequant.
#ifndef RPG_AMD_QUANT_DEV_H_
#define RPG_AMD_QUANT_DEV_H_

#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "quant_types.h"

namespace rpg {
namespace dev {

__device__ __forceinline__ uint32_t ByteOf(uint32_t word, int i) { return (word >> (8 * i)) & 0xFFu; }

// 6-bit (scale, min) of sub-block j (0..7) from the 12 packed bytes
// (GetScaleMinK4, src/quant.cc:159-167):
//   j < 4:  sc = q[j] & 63,                          m = q[j + 4] & 63
//   j >= 4: sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4),
//           m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4)
// With k = j & 3 both forms read byte k of each of the three words, so both are
// computed and one is selected: no branch on j, which is lane-dependent in the
// kernels and would otherwise split the wave.
__device__ __forceinline__ void ScaleMinK4(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t* sc, uint32_t* m) {
  const int k = j & 3;
  const uint32_t b0 = ByteOf(s0, k);
  const uint32_t b1 = ByteOf(s1, k);
  const uint32_t b2 = ByteOf(s2, k);
  const uint32_t hi_sc = (b2 & 0x0Fu) | ((b0 >> 6) << 4);
  const uint32_t hi_m = (b2 >> 4) | ((b1 >> 6) << 4);
  *sc = j < 4 ? (b0 & 63u) : hi_sc;
  *m = j < 4 ? (b1 & 63u) : hi_m;
}

// Element e of one quantised block (or of an F32 row) with byte loads only, so
// any alignment works: the fallback of the gather and of the matmul.
__device__ __forceinline__ float DeqElemAny(uint32_t type, const uint8_t* blk, int e) {
  if (type == kGgmlF32) {
    const uint32_t u = static_cast<uint32_t>(blk[4 * e]) | (static_cast<uint32_t>(blk[4 * e + 1]) << 8) |
                       (static_cast<uint32_t>(blk[4 * e + 2]) << 16) | (static_cast<uint32_t>(blk[4 * e + 3]) << 24);
    return __uint_as_float(u);
  }
  if (type == kGgmlQ4_K) {
    const int sub = e >> 5;
    const int l = e & 31;
    const int g = sub >> 1;
    const uint8_t qb = blk[16 + 32 * g + l];
    const uint32_t raw = (sub & 1) ? (qb >> 4) : (qb & 0x0Fu);
    const uint8_t* s = blk + 4;
    uint32_t sc, m;
    if (sub < 4) {
      sc = s[sub] & 63u;
      m = s[sub + 4] & 63u;
    } else {
      sc = (s[sub + 4] & 0x0Fu) | ((s[sub - 4] >> 6) << 4);
      m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
    }
    const float d = HalfBitsToFloat(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
    const float dmin = HalfBitsToFloat(static_cast<uint32_t>(blk[2]) | (static_cast<uint32_t>(blk[3]) << 8));
    const float d1 = d * static_cast<float>(sc);
    const float m1 = dmin * static_cast<float>(m);
    return d1 * static_cast<float>(raw) - m1;
  }
  // Q6_K
  const int half = e >> 7;
  const int r = e & 127;
  const int quarter = r >> 5;
  const int l = r & 31;
  const uint8_t qlb = blk[64 * half + l + ((quarter & 1) ? 32 : 0)];
  const uint32_t nib = quarter < 2 ? (qlb & 0x0Fu) : (qlb >> 4);
  const uint32_t hi2 = (blk[128 + 32 * half + l] >> (2 * quarter)) & 3u;
  const int q = static_cast<int>(nib | (hi2 << 4)) - 32;
  const int8_t sc = static_cast<int8_t>(blk[192 + 8 * half + (l >> 4) + 2 * quarter]);
  const float d = HalfBitsToFloat(static_cast<uint32_t>(blk[208]) | (static_cast<uint32_t>(blk[209]) << 8));
  return (d * static_cast<float>(sc)) * static_cast<float>(q);
}

}  // namespace dev
}  // namespace rpg

#endif  // RPG_AMD_QUANT_DEV_H_
