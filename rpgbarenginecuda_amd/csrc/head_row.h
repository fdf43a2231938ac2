// One 128-element attention head row spread over 8 lanes of a wave64.
//
// Lane l (0..7) owns the float4 chunks at elements 4l and 32+4l of the first
// half (a[0], a[1]) and the same offsets + 64 in the second half (b[0], b[1]).
// Both members of every NeoX RoPE pair (i, i+64) therefore sit in the same lane,
// and the row's sum of squares is a 3-step butterfly inside the aligned 8-lane
// group. Measured on MI355X for the fused q/k kernel at n = 2811: 8 lanes with
// 4 float4 each beat 16 lanes with 2 (more loads in flight per lane, half the
// waves, half the per-row scalar work) and 4 or 2 lanes (too few waves).
//
// The standalone head RMSNorm, the standalone RoPE and the fused q/k kernel all
// use these routines, so the fused and unfused paths give identical bits.
#ifndef RPG_AMD_HEAD_ROW_H_
#define RPG_AMD_HEAD_ROW_H_

#include "dev_util.h"

namespace rpg {
namespace dev {

constexpr int kHeadLanes = 8;

struct HeadRow {
  float4 a[2];  // first half: elements 4l.. and 32+4l..
  float4 b[2];  // second half: the same offsets + 64
};

__device__ __forceinline__ int HeadOffset(int l, int c) { return 4 * l + 32 * c; }

__device__ __forceinline__ HeadRow LoadHeadRowStream(const float* p, int l) {
  HeadRow r;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    r.a[c] = LoadStream4(p + HeadOffset(l, c));
    r.b[c] = LoadStream4(p + 64 + HeadOffset(l, c));
  }
  return r;
}

__device__ __forceinline__ void StoreHeadRowStream(float* p, int l, const HeadRow& r) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    StoreStream4(p + HeadOffset(l, c), r.a[c]);
    StoreStream4(p + 64 + HeadOffset(l, c), r.b[c]);
  }
}

// The same fp32 row through a buffer resource: `off` is the byte offset of the
// row's first element in rs, and every store carries the cache policy kPolicy.
template <int kPolicy>
__device__ __forceinline__ void StoreHeadRowBuf(__amdgpu_buffer_rsrc_t rs, uint32_t off, int l, const HeadRow& r) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    StoreBuf4<kPolicy>(rs, off + 4u * HeadOffset(l, c), r.a[c]);
    StoreBuf4<kPolicy>(rs, off + 4u * (64 + HeadOffset(l, c)), r.b[c]);
  }
}

// Swap one dword between the lanes of each even/odd pair (DPP quad_perm [1,0,3,2]).
__device__ __forceinline__ uint32_t SwapLanePair(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xF, 0xF, false));
}

// fp16 (IEEE round-to-nearest-even) copy of the row with 16-byte stores. Lane l
// holds the packed halves of chunks l and 8+l of each half row; lanes 2m and 2m+1
// swap one packed chunk so the even lane writes elements 8m..8m+7 (its chunk 2m
// and the odd lane's 2m+1) and the odd lane 32+8m..32+8m+7. Each store instruction
// then covers whole 128-byte lines. Both lanes of a pair must be active (the
// callers' conditions are uniform over the 8 lanes of a row). Plain stores:
// nontemporal ones measured no faster for these scattered 256-byte cache rows.
template <typename Put>
__device__ __forceinline__ void HeadRowHalfChunks(int l, const HeadRow& r, const Put& put) {
  const bool odd = (l & 1) != 0;
  const int e0 = odd ? 32 + 8 * (l >> 1) : 8 * (l >> 1);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const uint2 c0 = PackHalf4(s == 0 ? r.a[0] : r.b[0]);
    const uint2 c1 = PackHalf4(s == 0 ? r.a[1] : r.b[1]);
    const uint2 send = odd ? c0 : c1;
    const uint2 recv = make_uint2(SwapLanePair(send.x), SwapLanePair(send.y));
    put(e0 + 64 * s, odd ? make_uint4(recv.x, recv.y, c1.x, c1.y) : make_uint4(c0.x, c0.y, recv.x, recv.y));
  }
}

__device__ __forceinline__ void StoreHeadRowHalf(uint16_t* p, int l, const HeadRow& r) {
  HeadRowHalfChunks(l, r, [p](int e, uint4 v) { *reinterpret_cast<uint4*>(p + e) = v; });
}

// The same fp16 row through a buffer resource (`off` = byte offset of the row in rs),
// every store with the cache policy kPolicy.
template <int kPolicy>
__device__ __forceinline__ void StoreHeadRowHalfBuf(__amdgpu_buffer_rsrc_t rs, uint32_t off, int l, const HeadRow& r) {
  HeadRowHalfChunks(l, r, [rs, off](int e, uint4 v) { StoreBufU4<kPolicy>(rs, off + 2u * e, v); });
}

// Per-lane share of a 128-element vector read from cache (weights, RoPE rows).
// Issued right after the activation loads so their latency overlaps with HBM's.
__device__ __forceinline__ HeadRow LoadHeadVec(const float* __restrict__ p, int l) {
  HeadRow r;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    r.a[c] = Load4(p + HeadOffset(l, c));
    r.b[c] = Load4(p + 64 + HeadOffset(l, c));
  }
  return r;
}

// RMSNorm of the row with weight w (the lane's share, from LoadHeadVec): sum of
// squares in double (order a0, b0, a1, b1 per lane, then the 8-lane butterfly),
// HeadRmsScale, then (x*scale)*w.
__device__ __forceinline__ void NormHeadRow(HeadRow& r, const HeadRow& w, float eps) {
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < 2; ++c) ss = AddSquares(AddSquares(ss, r.a[c]), r.b[c]);
  ss = GroupSum<kHeadLanes>(ss);
  const float scale = HeadRmsScale(ss, eps);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    r.a[c] = ScaleMul(r.a[c], scale, w.a[c]);
    r.b[c] = ScaleMul(r.b[c], scale, w.b[c]);
  }
}

// NeoX rotation with a RoPE table row held as cos = t.a (elements 0..63) and
// sin = t.b (64..127): x_i <- a*c - b*s, x_{i+64} <- b*c + a*s, each product
// rounded separately. With apply == false the row is left as it is.
__device__ __forceinline__ void RotateHeadRow(HeadRow& r, const HeadRow& t, bool apply) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float4 co = t.a[c];
    const float4 si = t.b[c];
    const float4 a = r.a[c];
    const float4 b = r.b[c];
    const float4 ra = make_float4(a.x * co.x - b.x * si.x, a.y * co.y - b.y * si.y, a.z * co.z - b.z * si.z,
                                  a.w * co.w - b.w * si.w);
    const float4 rb = make_float4(b.x * co.x + a.x * si.x, b.y * co.y + a.y * si.y, b.z * co.z + a.z * si.z,
                                  b.w * co.w + a.w * si.w);
    r.a[c] = apply ? ra : a;
    r.b[c] = apply ? rb : b;
  }
}

}  // namespace dev
}  // namespace rpg

#endif  // RPG_AMD_HEAD_ROW_H_
