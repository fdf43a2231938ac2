// Causal attention over the fp16 KV cache (reference GpuAttentionFromCache,
// src/kernels_gpu.h:113-128; kernel src/kernels_gpu.cu:737-823).
//
// Semantics (per token t at absolute position pos = pos0 + t, query head h,
// kv head h / (n_heads / n_kv_heads)): scores s_j = (q . k_j) / sqrt(d) over the
// cached positions j in [0, pos], p = softmax(s), out = sum_j p_j v_j, with k and
// v the fp16 cache rows converted exactly to fp32.
//
// MI355X mapping (flash-decoding with an online softmax; the reference instead
// keeps one block per (t, h) with every score in shared memory):
//   * one wave64 per (t, h, key chunk); keys are taken 64 at a time, lane l
//     scoring key l of the block (its 256-byte K row against q broadcast from
//     LDS), then the wave keeps a running max m, a running sum l of
//     exp(s - m) and a running output o (lane l owns dims 2l, 2l + 1), rescaled
//     when the max grows;
//   * the no-cache path (GpuCausalAttention, fp32 k / v rows of the segment)
//     runs the per-query-head kernel on fp32 rows;
//   * decode and short prefills with a GQA group of 1, 2 or 4 use one wave per
//     (token, kv head, chunk) for the whole group (AttnDecodeGroupKernel), other
//     shapes one wave per query head (AttnChunkKernel);
//   * prefill (many (t, h) pairs) uses a single chunk per pair and writes the
//     normalised output directly; decode (few pairs) splits the keys into up to
//     kMaxChunks (kMaxGroupChunks for the grouped decode kernel) chunks so the
//     whole chip streams the cache, each chunk storing
//     (m, l, o) to a partials buffer that a second kernel merges;
//   * the partials buffer is library-owned and grows on demand;
//     GpuAttentionWarmupShmem(max positions) sizes it before a graph capture,
//     where allocating is not allowed.
// Under graph capture pos0 comes from the staging scalar, so chunk ranges are
// laid out for the position budget (sh_positions) and checked against the
// actual position inside the kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <utility>
#include <vector>

#include "dev_util.h"
#include "head_row.h"
#include "kernels_gpu.h"
#include "launch.h"

namespace rpg {
namespace {

constexpr int kD = 128;          // head_dim of the fast path
constexpr int kBlockThreads = 256;
constexpr int kWaves = kBlockThreads / 64;
constexpr int kMaxChunks = 64;
// The grouped decode kernel splits the keys finer: up to 128 chunks of 32 keys,
// one 32-key slab per wave at the decode positions that fill the chip.
constexpr int kMaxGroupChunks = 128;
constexpr int kPartFloats = kD + 4;  // o[128], m, l, 2 unused: 16-byte aligned rows for the float4 accesses
constexpr int64_t kFaMinTokens = 64;  // prefill calls with at least this many tokens run on the matrix cores
constexpr int64_t kFaMaxPartialFloats = int64_t{64} << 20;  // 256 MiB of prefill key-chunk partials at most

__device__ __forceinline__ int64_t ReadPos0(int64_t value, const int64_t* dev) { return dev != nullptr ? *dev : value; }

// Chunks of chunk_len keys that hold keys 0..pos: a graph captured for a
// position budget launches n_chunks chunks, but only these carry keys at the
// live position; with one live chunk its wave writes the final output and the
// merge has nothing to do.
__device__ __forceinline__ int32_t LiveChunks(int64_t pos, int64_t chunk_len, int32_t n_chunks) {
  const int64_t live = pos / chunk_len + 1;
  return live < n_chunks ? static_cast<int32_t>(live) : n_chunks;
}
// The same count through a 32-bit division when pos and chunk_len fit (every
// real position): the 64-bit division is a long vector-unit sequence in front
// of the first K / V load.
__device__ __forceinline__ int32_t LiveChunks32(int64_t pos, int64_t chunk_len, int32_t n_chunks) {
  if (pos < 0 || pos > INT32_MAX || chunk_len > INT32_MAX) return LiveChunks(pos, chunk_len, n_chunks);
  const uint32_t live = static_cast<uint32_t>(pos) / static_cast<uint32_t>(chunk_len) + 1u;
  return live < static_cast<uint32_t>(n_chunks) ? static_cast<int32_t>(live) : n_chunks;
}

// Wave reductions: DPP inside each 16-lane row (lane pairs xor 1, xor 2, then
// mirrored halves and rows, which pair every lane with a partner of the other
// half), then two cross-row exchanges.
__device__ __forceinline__ float DppMov(float v, int ctrl_sel) {
  int m;
  switch (ctrl_sel) {
    case 0: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
    case 1: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad_perm 2,3,0,1
    case 2: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false); break; // row_mirror
  }
  return __int_as_float(m);
}
// Across the four rows (every lane of each row holding its row's value): row 1
// takes row 0's value and row 3 row 2's (row_bcast:15, rows 1 and 3 written),
// then rows 2 and 3 take row 1's (row_bcast:31), so lane 63 ends with
// op(op(r3, r2), op(r1, r0)), which it hands to the whole wave as a scalar. With
// a commutative op that is the value the xor-16 / xor-32 exchange forms, and it
// takes two DPP moves instead of two LDS permutes. Every lane must be active.
template <typename Op>
__device__ __forceinline__ float AcrossRows(float v, float identity, Op op) {
  const int id = __float_as_int(identity);
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x142, 0xA, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x143, 0xC, 0xF, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float WaveMax(float v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) v = fmaxf(v, DppMov(v, k));
  return AcrossRows(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float WaveSumF(float v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) v += DppMov(v, k);
  return AcrossRows(v, 0.0f, [](float a, float b) { return a + b; });
}
// Lane 2 i of the caller's 16-lane row, broadcast to the whole row (row_newbcast).
__device__ __forceinline__ float RowLane2i(float v, int i) {
  int m;
  switch (i) {
    case 0: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150, 0xF, 0xF, false); break;
    case 1: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x152, 0xF, 0xF, false); break;
    case 2: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x154, 0xF, 0xF, false); break;
    case 3: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x156, 0xF, 0xF, false); break;
    case 4: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x158, 0xF, 0xF, false); break;
    case 5: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x15A, 0xF, 0xF, false); break;
    case 6: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x15C, 0xF, 0xF, false); break;
    default: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x15E, 0xF, 0xF, false); break;
  }
  return __int_as_float(m);
}

__device__ __forceinline__ float HalfToF(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// Key / value rows: the fp16 cache ([kv head][position][d], 16-bit bits) or
// fp32 rows of the current segment ([token][kv head][d], the no-cache path).
// Load8 converts elements 8 i .. 8 i + 7 of a row, Load2 elements 2 l, 2 l + 1.
__device__ __forceinline__ void Load8(const uint16_t* row, int i, float f[8]) {
  const uint4 w = reinterpret_cast<const uint4*>(row)[i];
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = HalfToF(wd[k] & 0xFFFFu);
    f[2 * k + 1] = HalfToF(wd[k] >> 16);
  }
}
__device__ __forceinline__ void Load8(const float* row, int i, float f[8]) {
  const float4 a = reinterpret_cast<const float4*>(row)[2 * i];
  const float4 b = reinterpret_cast<const float4*>(row)[2 * i + 1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ float2 Load2(const uint16_t* row, int lane) {
  const uint32_t w = reinterpret_cast<const uint32_t*>(row)[lane];
  return make_float2(HalfToF(w & 0xFFFFu), HalfToF(w >> 16));
}
__device__ __forceinline__ float2 Load2(const float* row, int lane) {
  return reinterpret_cast<const float2*>(row)[lane];
}

// One wave per (t, h, chunk). part == nullptr: a single chunk, the output is
// written normalised; otherwise (m, l, o) of the chunk go to part. Row s of kv
// head kh starts at kh * head_stride + s * pos_stride elements; positions at or
// past max_seq are never read.
template <typename KV>
__global__ __launch_bounds__(kBlockThreads) void AttnChunkKernel(
    const float* __restrict__ q, const KV* __restrict__ kc, const KV* __restrict__ vc, int64_t head_stride,
    int64_t pos_stride, int64_t max_seq, int32_t n_heads, int32_t group, float scale, int64_t pos0_val,
    const int64_t* __restrict__ pos0_dev, int64_t seq, int32_t n_chunks, int64_t chunk_len, float* __restrict__ out,
    float* __restrict__ part) {
  __shared__ float qs[kWaves][kD];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * kWaves + wv;
  const int64_t total = seq * n_heads * n_chunks;
  const bool active = unit < total;
  const int64_t th = active ? unit / n_chunks : 0;
  const int32_t c = active ? static_cast<int32_t>(unit - th * n_chunks) : 0;
  const int64_t t = th / n_heads;
  const int32_t h = static_cast<int32_t>(th - t * n_heads);
  const int32_t kh = h / group;
  const int64_t pos = ReadPos0(pos0_val, pos0_dev) + t;

  // q of (t, h), staged unscaled: the scale multiplies the finished dot
  // product, as in the reference.
  const float* qt = q + (t * n_heads + h) * kD;
  if (active) {
    qs[wv][2 * lane] = qt[2 * lane];
    qs[wv][2 * lane + 1] = qt[2 * lane + 1];
  }
  __syncthreads();
  if (!active) return;
  const int32_t live = LiveChunks(pos, chunk_len, n_chunks);
  if (c >= live) return;  // no key of this chunk is visible at this position
  if (live == 1) part = nullptr;

  const int64_t lo = static_cast<int64_t>(c) * chunk_len;
  int64_t hi = lo + chunk_len;
  if (hi > pos + 1) hi = pos + 1;
  if (hi > max_seq) hi = max_seq;  // only reachable through a replayed graph with a bad staged pos0

  const KV* kb = kc + static_cast<int64_t>(kh) * head_stride;
  const KV* vb = vc + static_cast<int64_t>(kh) * head_stride;
  float m = -INFINITY;
  float l = 0.0f;
  float o0 = 0.0f, o1 = 0.0f;

  for (int64_t base = lo; base < hi; base += 64) {
    const int64_t s = base + lane;
    const bool valid = s < hi;
    // score of key s: its row against q
    float sc = -INFINITY;
    if (valid) {
      const KV* kr = kb + s * pos_stride;
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four interleaved partial sums: a 32-deep chain
#pragma unroll
      for (int i = 0; i < kD / 8; ++i) {
        float f[8];
        Load8(kr, i, f);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[k] = __builtin_fmaf(qs[wv][8 * i + 2 * k], f[2 * k], acc[k]);
          acc[k] = __builtin_fmaf(qs[wv][8 * i + 2 * k + 1], f[2 * k + 1], acc[k]);
        }
      }
      sc = ((acc[0] + acc[1]) + (acc[2] + acc[3])) * scale;
    }
    const float bm = WaveMax(sc);
    const float mn = fmaxf(m, bm);
    const float corr = expf(m - mn);  // exp(-inf) = 0 on the first block
    const float p = valid ? expf(sc - mn) : 0.0f;
    l = l * corr + WaveSumF(p);
    o0 *= corr;
    o1 *= corr;
    m = mn;
    // o += sum_j p_j v_j over the block: lane l reads dims 2l, 2l + 1 of each v
    // row (one row per wave load); 16 rows are requested before any is used so
    // their latencies overlap.
    const int64_t nk = hi - base < 64 ? hi - base : 64;
    const KV* vr = vb + base * pos_stride;
    for (int j0 = 0; j0 < 64; j0 += 16) {
      if (j0 >= nk) break;
      float2 vv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = j0 + i < nk ? j0 + i : static_cast<int>(nk) - 1;  // clamped: stays in the block
        vv[i] = Load2(vr + static_cast<int64_t>(j) * pos_stride, lane);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // p of a key past the block's end is 0 (invalid lanes), so the clamped
        // duplicate rows add nothing
        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j0 + i));
        o0 = __builtin_fmaf(pj, vv[i].x, o0);
        o1 = __builtin_fmaf(pj, vv[i].y, o1);
      }
    }
  }

  if (part == nullptr) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float* ot = out + (t * n_heads + h) * kD;
    ot[2 * lane] = o0 * inv;
    ot[2 * lane + 1] = o1 * inv;
  } else {
    float* pp = part + unit * kPartFloats;
    pp[2 * lane] = o0;
    pp[2 * lane + 1] = o1;
    if (lane == 0) {
      pp[kD] = m;
      pp[kD + 1] = l;
    }
  }
}

// One workgroup per (t, h) merges its n_chunks partials (n_chunks <= 128) into
// out: M = max m_c, L = sum l_c e^(m_c - M), out = sum o_c e^(m_c - M) / L. Every
// wave forms M and L itself (lane c holds chunks c and c + 64, summed in the same
// order in each wave); the chunks' outputs are split over the waves in groups of
// 16 (wave w takes groups w, w + 4, ...; lane l owns dims 2l, 2l + 1), so the
// workgroup's loads are in flight together, and the waves' sums meet in LDS,
// added in wave order. (A merge by the last chunk to arrive would save this
// launch, but its device-scope release fence writes the whole L2 back once per
// chunk, which costs more.)
__global__ __launch_bounds__(kBlockThreads) void AttnMergeKernel(const float* __restrict__ part, int64_t pairs,
                                                                  int32_t n_chunks, int32_t n_heads, int64_t chunk_len,
                                                                  int64_t pos0_val, const int64_t* __restrict__ pos0_dev,
                                                                  float* __restrict__ out) {
  __shared__ float2 osum[kWaves][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t th = blockIdx.x;
  if (th >= pairs) return;  // uniform over the workgroup
  const int32_t live = LiveChunks(ReadPos0(pos0_val, pos0_dev) + th / n_heads, chunk_len, n_chunks);
  if (live == 1) return;  // the chunk kernel wrote the output (uniform over the workgroup)
  const float* pp = part + th * n_chunks * kPartFloats;
  const bool has0 = lane < live;
  const bool has1 = lane + 64 < live;
  const float m0 = has0 ? pp[lane * kPartFloats + kD] : -INFINITY;
  const float l0 = has0 ? pp[lane * kPartFloats + kD + 1] : 0.0f;
  const float m1 = has1 ? pp[(lane + 64) * kPartFloats + kD] : -INFINITY;
  const float l1 = has1 ? pp[(lane + 64) * kPartFloats + kD + 1] : 0.0f;
  const float mx = WaveMax(fmaxf(m0, m1));
  const float f0 = m0 == -INFINITY ? 0.0f : expf(m0 - mx);
  const float f1 = m1 == -INFINITY ? 0.0f : expf(m1 - mx);
  const float L = WaveSumF(l0 * f0 + l1 * f1);
  float o0 = 0.0f, o1 = 0.0f;
  for (int c0 = 16 * w; c0 < live; c0 += 16 * kWaves) {
    float2 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = c0 + i < live ? c0 + i : live - 1;  // clamped: its weight is used only if c0 + i < live
      v[i] = *reinterpret_cast<const float2*>(pp + c * kPartFloats + 2 * lane);
    }
    const float fset = c0 < 64 ? f0 : f1;  // a group of 16 lies in one set
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float fc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fset), (c0 + i) & 63));
      if (c0 + i < live) {
        o0 = __builtin_fmaf(v[i].x, fc, o0);
        o1 = __builtin_fmaf(v[i].y, fc, o1);
      }
    }
  }
  osum[w][lane] = make_float2(o0, o1);
  __syncthreads();
  if (w != 0) return;
  float2 acc = osum[0][lane];
#pragma unroll
  for (int q = 1; q < kWaves; ++q) {
    acc.x += osum[q][lane].x;
    acc.y += osum[q][lane].y;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  out[th * kD + 2 * lane] = acc.x * inv;
  out[th * kD + 2 * lane + 1] = acc.y * inv;
}

// The merge of prefill key chunks (many pairs, few chunks): 32 threads per
// (t, h), 4 dims each; the partials' maxima are in log2 units, so the chunk
// weights are 2^(m_c - M); weights and normaliser are summed in chunk order.
__global__ __launch_bounds__(kBlockThreads) void AttnMergeRowsKernel(const float* __restrict__ part, int64_t pairs,
                                                                      int32_t n_chunks, int32_t n_heads,
                                                                      int64_t chunk_len, int64_t pos0_val,
                                                                      const int64_t* __restrict__ pos0_dev,
                                                                      float* __restrict__ out) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kBlockThreads + threadIdx.x;
  const int64_t th = u / (kD / 4);
  if (th >= pairs) return;
  const int dq = static_cast<int>(u - th * (kD / 4));
  const int32_t live = LiveChunks(ReadPos0(pos0_val, pos0_dev) + th / n_heads, chunk_len, n_chunks);
  if (live == 1) return;  // the prefill kernel wrote the output
  const float* pp = part + th * n_chunks * kPartFloats;
  float mx = -INFINITY;
  for (int32_t c = 0; c < live; ++c) mx = fmaxf(mx, pp[c * kPartFloats + kD]);
  float L = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int32_t c = 0; c < live; ++c) {
    const float mc = pp[c * kPartFloats + kD];
    const float f = mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc - mx);
    L = __builtin_fmaf(pp[c * kPartFloats + kD + 1], f, L);
    const float4 v = *reinterpret_cast<const float4*>(pp + c * kPartFloats + 4 * dq);
    acc.x = __builtin_fmaf(v.x, f, acc.x);
    acc.y = __builtin_fmaf(v.y, f, acc.y);
    acc.z = __builtin_fmaf(v.z, f, acc.z);
    acc.w = __builtin_fmaf(v.w, f, acc.w);
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  *reinterpret_cast<float4*>(out + th * kD + 4 * dq) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

// ---------------------------------------------------------------- decode, one wave per kv head
//
// One wave per (token, kv head, key chunk) serves all G query heads of the GQA
// group, so each K/V row is read once. Keys go 32 at a time: lane l covers dims
// 8 (l % 16) .. + 7 of key base + 4 i + l / 16 (i = 0..7), so one load
// instruction reads four whole 256-byte rows. The 8 partial dot products a lane
// holds per head are reduced over its 16-lane row by a transposing butterfly
// (xor 8, 4, 2, then 1): afterwards lanes 2i and 2i + 1 of row r both hold the
// score of key base + 4 i + r. The online softmax then runs over the wave (each
// key counted once), and V rows are accumulated with the probability of key
// base + 4 i + r taken from lane 16 r + 2 i; the four rows' partial outputs are
// summed at the end.
//
// kPrep (one token): q, k and v arrive as the projections' raw rows and the
// wave first does what QkNormRopeKvKernel does for its kv head, with the same
// routines on the same 8-lane head layout (so the same bits): 8-lane group g
// < G takes query head kh G + g, group G the k row, group G + 1 the v row;
// q and k get the per-head RMSNorm and the RoPE rotation at pos, k and v are
// rounded to fp16. The wave of the chunk that holds pos stores the new K / V
// rows into the cache and uses them for that key straight from LDS (the store
// need not be visible to its own loads); the other chunks never read key pos.
// Waves (chunks) per workgroup of the one-launch decode, and so at most
// kMaxGroupChunks / kFusedWaves workgroups per (token, kv head) pair.
constexpr int kFusedWaves = 4;  // 8 measured slower: 10.1 against 8.9 us at 512 positions
constexpr int kMaxFusedGroups = kMaxGroupChunks / kFusedWaves;
// uint32 slots between two (token, kv head) pairs' arrival counters: one counter
// per 256 bytes. Packed counters (8 pairs in one 32-byte line) serialized the
// pairs' atomics on one line: 13.8 against 11.7 us at 4096 positions.
constexpr int kCounterStride = 64;

// The merge of the fused grouped decode (AttnDecodeGroupKernel<G, kPrep, true>),
// reached by every wave of a workgroup with at least two live chunks per pair.
// Partials are rows of kPartFloats: o[128], m, l.
template <int G, int kW>
__device__ __forceinline__ void FusedMerge(float (*wpart)[4][G][kPartFloats], int* last_flag, const float (&m)[G],
                                           const float (&l)[G], const float (&o)[G][8], int lane, int wave, int r,
                                           int rho, int64_t t, int32_t kh, int32_t n_heads, int32_t n_kv_heads,
                                           int32_t n_groups, int32_t live_groups, int32_t grp,
                                           float* __restrict__ out, float* __restrict__ part,
                                           uint32_t* __restrict__ cnt) {
  // 1. the workgroup's chunks, in chunk order: wave w's (m, l) and its four
  // rows' partial o (each row r summed over keys 4 i + r; the rows' sum is taken
  // here instead of by cross-row exchanges) to LDS, then wave hh < G merges head hh
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    *reinterpret_cast<float4*>(&wpart[wave][r][hh][8 * rho]) = make_float4(o[hh][0], o[hh][1], o[hh][2], o[hh][3]);
    *reinterpret_cast<float4*>(&wpart[wave][r][hh][8 * rho + 4]) = make_float4(o[hh][4], o[hh][5], o[hh][6], o[hh][7]);
    if (lane == 0) {
      wpart[wave][0][hh][kD] = m[hh];
      wpart[wave][0][hh][kD + 1] = l[hh];
    }
  }
  __syncthreads();
  const int hh = wave;
  const int64_t th = t * n_heads + static_cast<int64_t>(kh) * G + hh;
  if (hh < G) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kW; ++w) mx = fmaxf(mx, wpart[w][0][hh][kD]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const float mw = wpart[w][0][hh][kD];
      const float f = mw == -INFINITY ? 0.0f : expf(mw - mx);
      L = __builtin_fmaf(wpart[w][0][hh][kD + 1], f, L);
      float2 v[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) v[rr] = *reinterpret_cast<const float2*>(&wpart[w][rr][hh][2 * lane]);
      o0 = __builtin_fmaf((v[0].x + v[1].x) + (v[2].x + v[3].x), f, o0);
      o1 = __builtin_fmaf((v[0].y + v[1].y) + (v[2].y + v[3].y), f, o1);
    }
    if (live_groups == 1) {  // one workgroup holds every live chunk: the output directly
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      *reinterpret_cast<float2*>(out + th * kD + 2 * lane) = make_float2(o0 * inv, o1 * inv);
      return;
    }
    const __amdgpu_buffer_rsrc_t rs =
        dev::OutResource(part + (th * n_groups + grp) * kPartFloats, kPartFloats * sizeof(float));
    dev::StoreBufU2<dev::kStoreDeviceThroughPolicy>(rs, 8u * lane, make_uint2(__float_as_uint(o0), __float_as_uint(o1)));
    if (lane == 0) {
      dev::StoreBufU2<dev::kStoreDeviceThroughPolicy>(rs, 4u * kD, make_uint2(__float_as_uint(mx), __float_as_uint(L)));
    }
    // The stores are device-scope write-through: once they are acknowledged they
    // are visible to every XCD, so waiting for them stands in for an agent-scope
    // release fence (whose L2 write-back, one per workgroup, cost more than the
    // separate merge launch). The clobber keeps the compiler from moving memory
    // accesses across the wait.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if (live_groups == 1) return;  // uniform over the workgroup
  // 2. count the workgroup in; the last of the pair's live workgroups merges them all
  __syncthreads();
  uint32_t* counter = cnt + (t * n_kv_heads + kh) * kCounterStride;
  if (threadIdx.x == 0) {
    const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last_flag = before == static_cast<uint32_t>(live_groups - 1);
  }
  __syncthreads();
  if (!*last_flag) return;  // uniform over the workgroup
  if (hh < G) {
    // Device-coherent (sc1) loads of the partials, issued after the barrier that
    // follows the counter's atomic: every other workgroup's stores were
    // acknowledged before its atomic. Lane i < live_groups holds group i's (m, l);
    // every lane then walks the groups for its two dims.
    const __amdgpu_buffer_rsrc_t rs = dev::OutResource(part + th * n_groups * kPartFloats,
                                                       static_cast<uint32_t>(live_groups) * kPartFloats * sizeof(float));
    auto load2 = [&](int g, int off) {
      const uint2 u = dev::LoadBufU2<dev::kLoadDevicePolicy>(rs, 4u * static_cast<uint32_t>(g * kPartFloats + off));
      return make_float2(__uint_as_float(u.x), __uint_as_float(u.y));
    };
    const bool has = lane < live_groups;
    const float2 ml = has ? load2(lane, kD) : make_float2(-INFINITY, 0.0f);
    const float mx = WaveMax(ml.x);
    const float f = ml.x == -INFINITY ? 0.0f : expf(ml.x - mx);
    const float L = WaveSumF(ml.y * f);
    // every group's rows requested at once (one memory round trip), then summed in group order
    static_assert(kMaxGroupChunks / kW <= kMaxFusedGroups, "a pair has at most kMaxFusedGroups workgroups");
    float2 v[kMaxFusedGroups];
#pragma unroll
    for (int g = 0; g < kMaxFusedGroups; ++g) {
      if (g < live_groups) v[g] = load2(g, 2 * lane);  // uniform
    }
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int g = 0; g < kMaxFusedGroups; ++g) {
      if (g < live_groups) {
        const float fg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), g));
        o0 = __builtin_fmaf(v[g].x, fg, o0);
        o1 = __builtin_fmaf(v[g].y, fg, o1);
      }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    *reinterpret_cast<float2*>(out + th * kD + 2 * lane) = make_float2(o0 * inv, o1 * inv);
  }
  // every workgroup of the pair has counted in: ready for the next call
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct DecodePrep {
  const float* k;
  const float* v;
  const float* q_norm;
  const float* k_norm;
  const float* tab;
  int64_t rope_rows;
  float eps;
  uint16_t* k_store;
  uint16_t* v_store;
};

// kFused: one launch also merges. A workgroup takes kFusedWaves consecutive chunks of
// one (token, kv head); its waves' (m, l, o) meet in LDS and the workgroup stores
// one partial per query head; the workgroup whose vector atomic on the pair's
// counter (cnt[(t * n_kv_heads + kh) * kCounterStride]) arrives last merges the
// partials of all the pair's workgroups into out and puts the counter back to
// zero for the next call. With one live workgroup per pair there are no partials
// (part may be null) and that workgroup writes out directly.
// The partials go out device-scope write-through and are acknowledged before the
// atomic; the merging workgroup reads them with device-coherent loads. No wave
// waits on another workgroup: the first workgroups to finish just leave.
template <int G, bool kPrep = false, bool kFused = false>
__global__ __launch_bounds__(kFused ? 64 * kFusedWaves : kBlockThreads) void AttnDecodeGroupKernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t max_seq,
    int32_t n_heads, int32_t n_kv_heads, float scale, int64_t pos0_val, const int64_t* __restrict__ pos0_dev,
    int64_t seq, int32_t n_chunks, int64_t chunk_len, float* __restrict__ out, float* __restrict__ part,
    DecodePrep prep, uint32_t* __restrict__ cnt) {
  static_assert(!kPrep || G + 2 <= 8, "q heads, k and v: one 8-lane group each");
  constexpr int kW = kFused ? kFusedWaves : kWaves;  // waves per workgroup
  static_assert(!kFused || G <= kW, "the fused merge gives each query head of the group one wave");
  struct PrepLds {
    float q[G][kD];
    uint16_t k[kD];
    uint16_t v[kD];
  };
  __shared__ __attribute__((aligned(16))) PrepLds prep_lds[kPrep ? kW : 1];
  __shared__ __attribute__((aligned(16))) float wpart[kFused ? kW : 1][kFused ? 4 : 1][kFused ? G : 1][kPartFloats];
  __shared__ int last_flag;
  // Every kernel argument the first K / V loads depend on, fetched in one batch:
  // the empty asm takes them as scalar inputs (it emits nothing), so their loads
  // are issued together at entry instead of next to each use, where each waited
  // for the one before (five serial scalar round trips ahead of the first load).
  asm volatile("" ::"s"(kc), "s"(vc), "s"(max_seq), "s"(n_kv_heads), "s"(pos0_val), "s"(pos0_dev), "s"(seq),
               "s"(n_chunks), "s"(chunk_len), "s"(q), "s"(n_heads));
  const int lane = threadIdx.x & 63;
  // in a scalar register: the chunk, its key range and the merge's buffer
  // descriptors derive from it, and a vector wave index would put each buffer
  // access of the merge in a loop over the distinct descriptors
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int32_t n_groups = kFused ? (n_chunks + kW - 1) / kW : 1;
  int64_t tk;
  int32_t c;
  if constexpr (kFused) {
    // 32-bit: the grid is below 2^32 workgroups and n_groups positive
    const uint32_t tk32 = blockIdx.x / static_cast<uint32_t>(n_groups);
    tk = tk32;
    if (tk >= seq * n_kv_heads) return;  // uniform over the workgroup
    c = static_cast<int32_t>(blockIdx.x - tk32 * static_cast<uint32_t>(n_groups)) * kW + wave;
  } else {
    const int64_t unit = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    if (unit >= seq * n_kv_heads * n_chunks) return;  // no barriers below
    tk = unit / n_chunks;
    c = static_cast<int32_t>(unit - tk * n_chunks);
  }
  // tk < 2^32 in both forms (the unfused grid is also below 2^32 / kWaves workgroups)
  const int64_t t = static_cast<uint32_t>(tk) / static_cast<uint32_t>(n_kv_heads);
  const int32_t kh = static_cast<int32_t>(tk - t * n_kv_heads);
  const int64_t pos = ReadPos0(pos0_val, pos0_dev) + t;
  const int32_t live = LiveChunks32(pos, chunk_len, n_chunks);
  const int32_t live_groups = kFused ? (live + kW - 1) / kW : 0;
  if (kFused && c / kW >= live_groups) return;  // the whole workgroup: no visible key (uniform)
  // kFused: a wave past the live chunks keeps m = -inf, l = 0, o = 0 and joins the barriers
  const bool dead = c >= live;
  if (!kFused && dead) return;  // no key of this chunk is visible at this position
  if (live == 1) part = nullptr;
  const int64_t lo = dead ? 0 : static_cast<int64_t>(c) * chunk_len;
  int64_t hi = dead ? 0 : lo + chunk_len;
  if (hi > pos + 1) hi = pos + 1;
  if (hi > max_seq) hi = max_seq;  // only reachable through a replayed graph with a bad staged pos0
  const int rho = lane & 15;
  const int r = lane >> 4;
  const bool writer = kPrep && c == live - 1;  // the chunk that holds key pos
  // A slab of 32 keys through buffer resources on the chunk's rows [lo, hi) of
  // K and V: a row at or past hi reads as zeros (the resource's bound), so no row
  // index is clamped; such keys get probability 0. The lane's offset inside a
  // slab (row 4 i + r, bytes 16 rho..) is fixed, the slab's first row a scalar
  // offset. With kPipe the next slab's rows are loaded while this one is scored
  // (G <= 2: the second set of 16 registers per row fits), and the first slab is
  // requested before anything else.
  const int64_t head_row0 = static_cast<int64_t>(kh) * max_seq + lo;
  const uint32_t chunk_bytes = static_cast<uint32_t>(hi - lo) * (kD * 2);
  const __amdgpu_buffer_rsrc_t krs = dev::OutResource(const_cast<uint16_t*>(kc + head_row0 * kD), chunk_bytes);
  const __amdgpu_buffer_rsrc_t vrs = dev::OutResource(const_cast<uint16_t*>(vc + head_row0 * kD), chunk_bytes);
  const uint32_t lane_off = static_cast<uint32_t>(r) * (kD * 2) + 16u * static_cast<uint32_t>(rho);
  constexpr bool kPipe = G <= 2;
  auto load_slab = [&](int64_t base, uint4 (&kw)[8], uint4 (&vw)[8]) {
    const int so = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(base - lo) * (kD * 2)));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int vo = static_cast<int>(lane_off + static_cast<uint32_t>(i) * (4 * kD * 2));
      const dev::U32x4 a = __builtin_amdgcn_raw_buffer_load_b128(krs, vo, so, 0);
      const dev::U32x4 b = __builtin_amdgcn_raw_buffer_load_b128(vrs, vo, so, 0);
      kw[i] = make_uint4(a.x, a.y, a.z, a.w);
      vw[i] = make_uint4(b.x, b.y, b.z, b.w);
    }
  };
  uint4 kw[8], vw[8];
  if (kPipe && !dead) load_slab(lo, kw, vw);

  float qv[G][8];
  uint4 knew = make_uint4(0u, 0u, 0u, 0u), vnew = make_uint4(0u, 0u, 0u, 0u);
  if (kPrep) {  // a dead wave (kFused) runs it too and stores nothing: writer is false there
    PrepLds& P = prep_lds[threadIdx.x >> 6];
    const int g = lane >> 3;
    const int hl = lane & 7;
    const bool is_q = g < G, is_k = g == G, is_v = g > G;
    const float* src = is_q ? q + (t * n_heads + kh * G + g) * kD
                            : (is_k ? prep.k : prep.v) + (t * n_kv_heads + kh) * kD;
    const bool rope_ok = pos >= 0 && pos < prep.rope_rows;
    dev::HeadRow row = dev::LoadHeadVec(src, hl);
    const dev::HeadRow trig = dev::LoadHeadVec(prep.tab + (rope_ok ? pos : 0) * kD, hl);
    const dev::HeadRow w = dev::LoadHeadVec(is_q ? prep.q_norm : prep.k_norm, hl);
    if (!is_v) {  // uniform over each 8-lane group
      dev::NormHeadRow(row, w, prep.eps);
      dev::RotateHeadRow(row, trig, rope_ok);
    }
    if (is_q) {
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        *reinterpret_cast<float4*>(&P.q[g][dev::HeadOffset(hl, cc)]) = row.a[cc];
        *reinterpret_cast<float4*>(&P.q[g][64 + dev::HeadOffset(hl, cc)]) = row.b[cc];
      }
    } else if (g <= G + 1) {
      uint16_t* dst = is_k ? P.k : P.v;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        *reinterpret_cast<uint2*>(&dst[dev::HeadOffset(hl, cc)]) = dev::PackHalf4(row.a[cc]);
        *reinterpret_cast<uint2*>(&dst[64 + dev::HeadOffset(hl, cc)]) = dev::PackHalf4(row.b[cc]);
      }
      if (writer && pos >= 0 && pos < max_seq) {
        uint16_t* cache = (is_k ? prep.k_store : prep.v_store) + (static_cast<int64_t>(kh) * max_seq + pos) * kD;
        dev::StoreHeadRowHalf(cache, hl, row);
      }
    }
    // the wave's own LDS writes, read back by other lanes of the same wave
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      const float4 a = *reinterpret_cast<const float4*>(&P.q[hh][8 * rho]);
      const float4 b = *reinterpret_cast<const float4*>(&P.q[hh][8 * rho + 4]);
      qv[hh][0] = a.x; qv[hh][1] = a.y; qv[hh][2] = a.z; qv[hh][3] = a.w;
      qv[hh][4] = b.x; qv[hh][5] = b.y; qv[hh][6] = b.z; qv[hh][7] = b.w;
    }
    knew = *reinterpret_cast<const uint4*>(&P.k[8 * rho]);
    vnew = *reinterpret_cast<const uint4*>(&P.v[8 * rho]);
  } else {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      const float* qr = q + (t * n_heads + kh * G + hh) * kD + 8 * rho;
      const float4 a = *reinterpret_cast<const float4*>(qr);
      const float4 b = *reinterpret_cast<const float4*>(qr + 4);
      qv[hh][0] = a.x; qv[hh][1] = a.y; qv[hh][2] = a.z; qv[hh][3] = a.w;
      qv[hh][4] = b.x; qv[hh][5] = b.y; qv[hh][6] = b.z; qv[hh][7] = b.w;
    }
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[hh][j] = 0.0f;
  }

  // One slab: scores, online softmax, P.V. first: the chunk's first slab, where
  // m is -inf and o is zero, so o needs no rescale (l * corr is 0 there too).
  auto slab = [&](uint4 (&kw)[8], const uint4 (&vw)[8], int64_t base, bool first) {
    if (writer) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (base + 4 * i + r == pos) {  // the row this launch stores: from LDS, not the cache
          kw[i] = knew;
        }
      }
    }
    const int64_t skey = base + 4 * (rho >> 1) + r;  // the key whose score this lane ends with
    const bool valid = skey < hi;
    float p[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      float sp[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t wd[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
        float a0 = qv[hh][0] * HalfToF(wd[0] & 0xFFFFu);
        float a1 = qv[hh][1] * HalfToF(wd[0] >> 16);
        a0 = __builtin_fmaf(qv[hh][2], HalfToF(wd[1] & 0xFFFFu), a0);
        a1 = __builtin_fmaf(qv[hh][3], HalfToF(wd[1] >> 16), a1);
        a0 = __builtin_fmaf(qv[hh][4], HalfToF(wd[2] & 0xFFFFu), a0);
        a1 = __builtin_fmaf(qv[hh][5], HalfToF(wd[2] >> 16), a1);
        a0 = __builtin_fmaf(qv[hh][6], HalfToF(wd[3] & 0xFFFFu), a0);
        a1 = __builtin_fmaf(qv[hh][7], HalfToF(wd[3] >> 16), a1);
        sp[i] = a0 + a1;
      }
      // Transposing butterfly over the 16-lane row, in DPP moves. The partners
      // are rho ^ 15 (row mirror), rho ^ 7 (half-row mirror), rho ^ 2, rho ^ 1:
      // each differs from rho in the bit that step splits on (3, 2, 1, 0), so
      // the lane with that bit set keeps the upper half of the values and its
      // partner the lower half, and the lane sets a value has gathered stay
      // cosets of {0, 15}, {0, 7, 8, 15}, ... in rho's bits: disjoint, all 16
      // lanes at the end. Lane rho ends with key 4 (rho >> 1) + r.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool up = rho & 8;
        const float mine = up ? sp[j + 4] : sp[j];
        const float other = up ? sp[j] : sp[j + 4];
        sp[j] = mine + DppMov(other, 3);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bool up = rho & 4;
        const float mine = up ? sp[j + 2] : sp[j];
        const float other = up ? sp[j] : sp[j + 2];
        sp[j] = mine + DppMov(other, 2);
      }
      {
        const bool up = rho & 2;
        const float mine = up ? sp[1] : sp[0];
        const float other = up ? sp[0] : sp[1];
        sp[0] = mine + DppMov(other, 1);
      }
      sp[0] += DppMov(sp[0], 0);
      const float sc = valid ? sp[0] * scale : -INFINITY;
      const float bm = WaveMax(sc);
      const float mn = fmaxf(m[hh], bm);
      const float corr = mn == -INFINITY ? 1.0f : expf(m[hh] - mn);
      p[hh] = valid ? expf(sc - mn) : 0.0f;
      l[hh] = l[hh] * corr + WaveSumF((rho & 1) ? 0.0f : p[hh]);  // each key once
      m[hh] = mn;
      if (!first) {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[hh][j] *= corr;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t wd[4] = {vw[i].x, vw[i].y, vw[i].z, vw[i].w};
      if (writer && base + 4 * i + r == pos) {
        wd[0] = vnew.x; wd[1] = vnew.y; wd[2] = vnew.z; wd[3] = vnew.w;
      }
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        const float pi = RowLane2i(p[hh], i);  // probability of key base + 4 i + r (lane 2 i of row r)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          o[hh][2 * k] = __builtin_fmaf(pi, HalfToF(wd[k] & 0xFFFFu), o[hh][2 * k]);
          o[hh][2 * k + 1] = __builtin_fmaf(pi, HalfToF(wd[k] >> 16), o[hh][2 * k + 1]);
        }
      }
    }
  };
  if (kPipe) {
    // ping-pong between the two register sets, so no loaded row is copied
    uint4 kn[8], vn[8];
    for (int64_t base = lo; base < hi; base += 64) {
      const bool more = base + 32 < hi;  // uniform
      if (more) load_slab(base + 32, kn, vn);
      __builtin_amdgcn_sched_barrier(0);  // keep the next slab's loads ahead of this slab's scores
      slab(kw, vw, base, base == lo);
      if (!more) break;
      if (base + 64 < hi) load_slab(base + 64, kw, vw);
      __builtin_amdgcn_sched_barrier(0);
      slab(kn, vn, base + 32, false);
    }
  } else {
    for (int64_t base = lo; base < hi; base += 32) {
      load_slab(base, kw, vw);
      slab(kw, vw, base, base == lo);
    }
  }

  if constexpr (kFused) {
    if (live > 1) return FusedMerge<G, kW>(wpart, &last_flag, m, l, o, lane, wave, r, rho, t, kh, n_heads,
                                            n_kv_heads, n_groups, live_groups, c / kW, out, part, cnt);
    // one live chunk: its wave writes the output (the other waves are dead)
    if (dead) return;
  }
  // the four rows' partial outputs
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[hh][j] += __shfl_xor(o[hh][j], 16, 64);
      o[hh][j] += __shfl_xor(o[hh][j], 32, 64);
    }
  }
  if (r != 0) return;
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    const int64_t th = t * n_heads + kh * G + hh;
    float* dst;
    float f = 1.0f;
    if (part == nullptr) {
      dst = out + th * kD;
      f = l[hh] > 0.0f ? 1.0f / l[hh] : 0.0f;
    } else {
      float* pp = part + (th * n_chunks + c) * kPartFloats;
      dst = pp;
      if (rho == 0) {
        pp[kD] = m[hh];
        pp[kD + 1] = l[hh];
      }
    }
    *reinterpret_cast<float4*>(dst + 8 * rho) = make_float4(o[hh][0] * f, o[hh][1] * f, o[hh][2] * f, o[hh][3] * f);
    *reinterpret_cast<float4*>(dst + 8 * rho + 4) = make_float4(o[hh][4] * f, o[hh][5] * f, o[hh][6] * f, o[hh][7] * f);
  }
}

// ---------------------------------------------------------------- prefill on the matrix cores
//
// Flash attention with v_mfma_f32_32x32x16_f16. One workgroup = one query head
// and 128 consecutive tokens, 4 waves of 32 tokens; keys in blocks of 64 staged
// in LDS as [key][dim] rows (16-byte writes) and shared by the waves; the V^T
// fragments of the P.V step come out of the V rows through the transposing
// LDS read (ds_read_b64_tr_b16).
// Per wave and block:
//   S^T (64 keys x 32 queries) = K . Q^T    2 key tiles x 8 dim steps x 2 terms
//   O^T (128 dims x 32 queries) += V^T . P^T  4 dim tiles x 4 key steps x 2 terms
// Computing the transposes puts one query in each lane column: lane l owns query
// l % 32 (its running max, sum and rescale are lane values; lanes l and l + 32
// hold the two halves of the keys), and the S^T accumulator registers 0-7 / 8-15
// are already the B operand of the P.V step for the keys they hold, provided
// the V^T fragments follow the same key order.
// Exact operands: K and V are fp16 cache values. q (fp32) is scaled per row by
// 2^e (max |q| into [64, 128)) and split into two fp16 terms h + m that
// reproduce it to ~2^-23 relative (a score error ~65x inside the fp32
// dot-product bound the tests hold it to); the probabilities p in [0, 1] are split into
// two fp16 terms (to ~2^-22, plus an absolute 2^-25 below fp16's normal range).
// The matrix core forms exact products and accumulates in fp32; the score is
// rescaled by scale * 2^-e. Non-finite q gives NaN rows.
typedef _Float16 F16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 F16x4 __attribute__((ext_vector_type(4)));
typedef float F32x16 __attribute__((ext_vector_type(16)));

constexpr int kFaTokens = 128;    // tokens (of one head) per workgroup
constexpr int kFaKeys = 64;       // keys per LDS block
constexpr float kFaLazyLog2 = 8;  // the running max moves when a block's max exceeds it by more (log2 units)
constexpr int kFaOrderMax = 1024; // (token tile, key chunk) pairs an ordered launch can list
constexpr int kFaKStride = 136;   // halves per K row in LDS (128 + 8: conflict-free 16-byte reads)
constexpr int kFaCounterStride = 16;       // uint32 slots between two (tile, head) arrival counters (64 bytes)
constexpr int64_t kFaCounterSlots = 8192;  // (tile, head) counters per half (allocating / no-allocation)
constexpr int kFaFusedMaxChunks = 4;       // key chunks the fused merge takes (more: a separate merge launch)
constexpr int64_t kFaPartBlock = kFaTokens * (kD + 2);  // fused-merge partial floats per (tile, head, chunk)
constexpr int kFaVStride = 160;   // halves per V row in LDS (128 + 32: conflict-free transposing reads)

// ds_read_b64_tr_b16: in each 16-lane group, lane j receives element j % 4 of
// the 8 bytes addressed by lanes j / 4, 4 + j / 4, 8 + j / 4, 12 + j / 4.
typedef short S16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ F16x4 VTr(const _Float16* lds_ptr) {
  typedef __attribute__((address_space(3))) S16x4 LdsS16x4;
  const S16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (LdsS16x4*)((__attribute__((address_space(3))) _Float16*)(lds_ptr)));
  return __builtin_bit_cast(F16x4, v);
}

// x as two fp16 terms, *h = fp16(x) and *l = fp16(x - h) (the difference is
// exact in fp32). Each remainder is one mixed-precision FMA, h * -1 + x with h
// read as fp16 and the exact result rounded straight to fp16 into one half of
// the packed pair: the same bits as converting h back, subtracting and
// converting, in one instruction instead of three. (Written out because the
// compiler folds a multiply by -1 into a subtraction and then needs the
// conversions.)
__device__ __forceinline__ uint32_t RemainderPair(uint32_t hpair, float x0, float x1) {
  uint32_t d;
  asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %1, -1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(d)
      : "v"(hpair), "v"(x0), "v"(x1));
  return d;
}
__device__ __forceinline__ void SplitPair(const float (&x)[8], F16x8* h, F16x8* l) {
#pragma unroll
  for (int j = 0; j < 8; ++j) (*h)[j] = static_cast<_Float16>(x[j]);
  typedef unsigned int U32x4v __attribute__((ext_vector_type(4)));
  const U32x4v hw = __builtin_bit_cast(U32x4v, *h);
  U32x4v lw;
#pragma unroll
  for (int k = 0; k < 4; ++k) lw[k] = RemainderPair(hw[k], x[2 * k], x[2 * k + 1]);
  *l = __builtin_bit_cast(F16x8, lw);
}

__device__ __forceinline__ F16x8 SplitTerm(float (&x)[8]) {
  // x <- x - fp16(x), returning fp16(x) (round to nearest even; the difference is exact in fp32)
  F16x8 h;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    h[j] = static_cast<_Float16>(x[j]);
    x[j] -= static_cast<float>(h[j]);
  }
  return h;
}

// Dispatch order of the prefill workgroups. Workgroup g takes query head g %
// n_heads of pair g / n_heads; with n > 0, pair i is (token tile e[i] >> 6, key
// chunk e[i] & 63), the pairs sorted by their key blocks, most first, so the
// longest workgroups start first and the short ones fill the gaps at the end
// (longest-processing-time order). With n == 0 (more pairs than the table
// holds) pair i is (tiles - 1 - i / n_chunks, i % n_chunks): last tile first.
struct FaOrder {
  int32_t n;
  uint16_t e[kFaOrderMax];
};

// Key chunks: the workgroup of (token tile, key chunk c, head) takes keys
// [c chunk_len, (c + 1) chunk_len) of the tile's causal range, so the long tiles
// at the end of a prompt spread over several workgroups. A token whose keys all
// lie in chunk 0 (LiveChunks == 1) gets its normalised output from chunk 0; the
// others get an unnormalised partial (o, m, l) per live chunk in `part`, laid
// out as the decode partials ([token][head][chunk]), which AttnMergeRowsKernel
// combines.
__global__ __launch_bounds__(256, 2) void AttnPrefillMfmaKernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t max_seq,
    int32_t n_heads, int32_t group, float scale, int64_t pos0_val, const int64_t* __restrict__ pos0_dev, int64_t seq,
    int32_t n_chunks, int64_t chunk_len, int32_t tiles, float* __restrict__ out, float* __restrict__ part,
    FaOrder order, uint32_t* __restrict__ cnt) {
  __shared__ __attribute__((aligned(16))) _Float16 ks[kFaKeys * kFaKStride];
  __shared__ __attribute__((aligned(16))) _Float16 vs[kFaKeys * kFaVStride];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int hf = lane >> 5;    // which half of the keys / dims this lane holds
  const int col = lane & 31;   // the lane's query within the wave
  const int32_t pair = static_cast<int32_t>(blockIdx.x) / n_heads;
  // Slot i of the pair's n_heads workgroups takes kv head i % n_kv and query head
  // (i % n_kv) group + i / n_kv of it: the heads sharing a kv head sit n_kv
  // slots apart. Workgroups go to the XCDs in turn (id mod 8), so with 8 kv heads
  // (every Qwen3 shape here) all heads of a kv head, in every tile, run on one
  // XCD and read its K / V rows through one L2 instead of `group` of them.
  const int slot = static_cast<int>(blockIdx.x) - pair * n_heads;
  const int n_kv = n_heads / group;
  const int kh = slot % n_kv;
  const int h = kh * group + slot / n_kv;
  int32_t chunk, tile;
  if (order.n > 0) {
    const uint32_t entry = order.e[pair];
    chunk = static_cast<int32_t>(entry & 63u);
    tile = static_cast<int32_t>(entry >> 6);
  } else {
    tile = tiles - 1 - pair / n_chunks;
    chunk = pair - (tiles - 1 - tile) * n_chunks;
  }
  const int64_t t0 = static_cast<int64_t>(tile) * kFaTokens;
  const int64_t pos0 = ReadPos0(pos0_val, pos0_dev);
  const int64_t tq = t0 + 32 * wv + col;
  const bool qvalid = tq < seq;
  const int64_t qpos = pos0 + tq;

  // ---- q row: this lane holds dims 16 s + 8 hf + j (s = 0..7), the partner lane the rest
  float qv[8][8];
  const float* qrow = q + (tq * n_heads + h) * kD;
  float amax = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (qvalid) {
      a = *reinterpret_cast<const float4*>(qrow + 16 * s + 8 * hf);
      b = *reinterpret_cast<const float4*>(qrow + 16 * s + 8 * hf + 4);
    }
    qv[s][0] = a.x; qv[s][1] = a.y; qv[s][2] = a.z; qv[s][3] = a.w;
    qv[s][4] = b.x; qv[s][5] = b.y; qv[s][6] = b.z; qv[s][7] = b.w;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(qv[s][j]));
  }
  amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
  int e = 0;
  if (amax > 0.0f && amax <= 3.0e38f) e = 6 - ilogbf(amax);  // max |q| * 2^e in [64, 128)
  // Scores are kept in log2 units, so each exponential is one v_exp_f32:
  // p = 2^(s2 - m2) = e^(s - m). The score scale (1 / sqrt(d) times log2(e))
  // is applied to q before the split (one fp32 rounding, ~2^-24, under the
  // split's ~2^-23): q 2^e scale log2(e) lies in [8, 17), well inside fp16's
  // range for both terms. The matrix cores return s2 2^e, and the exponent
  // s2 - m2 is formed as fma(s2 2^e, 2^-e, -m2), exact scaling and one rounding.
  const float qmul = ldexpf(scale * 1.44269504088896340736f, e);
  const float sinv = ldexpf(1.0f, -e);
  F16x8 qb[2][8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
#pragma unroll
    for (int j = 0; j < 8; ++j) qv[s][j] *= qmul;
    qb[0][s] = SplitTerm(qv[s]);
    qb[1][s] = SplitTerm(qv[s]);
  }

  F32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = F32x16{};
  float m = -INFINITY, l = 0.0f;

  const int64_t t_last = (t0 + kFaTokens < seq ? t0 + kFaTokens : seq) - 1;
  const int64_t last_key = pos0 + t_last;                                   // the workgroup's causal limit
  const int64_t wave_last = pos0 + (t0 + 32 * wv + 31 < seq ? t0 + 32 * wv + 31 : seq - 1);
  const int64_t wave_first = pos0 + t0 + 32 * wv;   // the wave's first query position
  const bool wave_full = t0 + 32 * wv + 31 < seq;   // all 32 queries of the wave are tokens
  const uint16_t* kbase = kc + static_cast<int64_t>(kh) * max_seq * kD;
  const uint16_t* vbase = vc + static_cast<int64_t>(kh) * max_seq * kD;
  const int64_t klo = static_cast<int64_t>(chunk) * chunk_len;
  if (klo > last_key) return;  // no key of this chunk is visible to the tile (uniform: before any barrier)
  const int64_t kend = klo + chunk_len;

  for (int64_t kb = klo; kb <= last_key && kb < kend; kb += kFaKeys) {
    __syncthreads();  // the previous block is consumed
    {
      // thread t: key t / 4, dims 32 (t % 4) .. + 31 of K and V
      const int key = threadIdx.x >> 2;
      const int part = threadIdx.x & 3;
      // rows past the causal limit repeat the last visible row: their scores are
      // masked, so p = 0 meets finite values
      const int64_t j = kb + key < last_key ? kb + key : last_key;
      uint4 kw[4], vw[4];
      const uint4* kr = reinterpret_cast<const uint4*>(kbase + j * kD + 32 * part);
      const uint4* vr = reinterpret_cast<const uint4*>(vbase + j * kD + 32 * part);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kw[i] = kr[i];
        vw[i] = vr[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&ks[key * kFaKStride + 32 * part + 8 * i]) = kw[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&vs[key * kFaVStride + 32 * part + 8 * i]) = vw[i];
    }
    __syncthreads();
    if (kb > wave_last) continue;  // every query of this wave is before the block (uniform per wave)

    // ---- S^T = K . Q^T (the smallest term first)
    F32x16 st[2] = {F32x16{}, F32x16{}};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const F16x8 a = *reinterpret_cast<const F16x8*>(&ks[(32 * mt + col) * kFaKStride + 16 * s + 8 * hf]);
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[1][s], st[mt], 0, 0, 0);
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[0][s], st[mt], 0, 0, 0);
      }
    }

    // ---- online softmax: register r of tile mt is key kb + 32 mt + (r % 4) + 8 (r / 4) + 4 hf;
    // the causal test on the key's offset in the block (32-bit)
    // (a block wholly below every query of the wave, all of them valid, needs no mask)
    float bmax = -INFINITY;
    if (kb + kFaKeys - 1 <= wave_first && wave_full) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) bmax = fmaxf(bmax, st[mt][r]);
    } else {
      const int64_t rel64 = qvalid ? qpos - kb : -1;
      const int32_t rel = static_cast<int32_t>(rel64 < 64 ? rel64 : 64);  // offsets <= rel are visible
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int32_t off = 32 * mt + (r & 3) + 8 * (r >> 2) + 4 * hf;
          const float sc = off <= rel ? st[mt][r] : -INFINITY;
          st[mt][r] = sc;
          bmax = fmaxf(bmax, sc);
        }
      }
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64)) * sinv;  // exact: a power of two
    // The running max m moves only when a block's max exceeds it by more than
    // kFaLazyLog2, so p <= 2^kFaLazyLog2 and most blocks rescale nothing (o and
    // l are relative to whatever m is; the final o / l does not depend on it).
    const float mn = bmax > m + kFaLazyLog2 ? bmax : m;
    // 2^(-inf) = 0: masked scores give p = 0 once the row has a finite max;
    // before that (mn = -inf) the block contributes nothing
    const float base = mn == -INFINITY ? 0.0f : mn;
    if (__builtin_amdgcn_ballot_w64(mn != m) != 0) {  // some row of the wave moved
      const float corr = __builtin_amdgcn_exp2f(m - base);  // 1 where m stays; 0 on a row's first live block
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= corr;
    }
    float psum = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][r], sinv, -base));
        st[mt][r] = p;
        psum += p;
      }
    }
    psum += __shfl_xor(psum, 32, 64);
    l += psum;
    m = mn;

    // ---- O^T += V^T . P^T: key step ks takes registers 8 (ks % 2) .. + 7 of tile ks / 2
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2) {
      const int mt = ks2 >> 1;
      const int rb = 8 * (ks2 & 1);
      float pr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pr[j] = st[mt][rb + j];
      F16x8 ph, pl;
      SplitPair(pr, &ph, &pl);
      const int koff = 32 * mt + 16 * (ks2 & 1) + 4 * hf;  // keys koff + 0..3 and koff + 8..11
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        // V^T fragment of dim 32 dt + col from V rows by transposing reads: in
        // each 16-lane group, lane j points at key koff + j / 4 (resp. + 8),
        // dims 32 dt + 16 (col / 16) + 4 (j % 4) .. + 3, and receives dim
        // 32 dt + col of keys koff .. koff + 3 (resp. koff + 8 .. + 11)
        const int gj = lane & 15;
        const int vd = 32 * dt + (col & 16) + 4 * (gj & 3);
        const F16x4 lo = VTr(&vs[(koff + (gj >> 2)) * kFaVStride + vd]);
        const F16x4 hi = VTr(&vs[(koff + 8 + (gj >> 2)) * kFaVStride + vd]);
        const F16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pl, o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ph, o[dt], 0, 0, 0);
      }
    }
  }

  // ---- out[tq][h][dim]: register r of tile dt is dim 32 dt + (r % 4) + 8 (r / 4) + 4 hf
  // A chunk past the query's live chunks saw none of its keys and writes
  // nothing: in particular, for a query whose keys all lie in chunk 0, only
  // chunk 0 writes its output (another chunk would overwrite it with zeros).
  const int32_t live = qvalid ? LiveChunks(qpos, chunk_len, n_chunks) : 0;
  if (chunk < live && live == 1) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float* orow = out + (tq * n_heads + h) * kD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 v = make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                                     o[dt][4 * g + 3] * inv);
        *reinterpret_cast<float4*>(orow + 32 * dt + 8 * g + 4 * hf) = v;
      }
    }
  }
  if (cnt == nullptr) {
    // partials for AttnMergeRowsKernel: rows [token][head][chunk] of kPartFloats
    if (chunk < live && live > 1) {
      float* pp = part + ((tq * n_heads + h) * n_chunks + chunk) * kPartFloats;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 v = make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
          *reinterpret_cast<float4*>(pp + 32 * dt + 8 * g + 4 * hf) = v;
        }
      }
      if (hf == 0) {
        pp[kD] = m;
        pp[kD + 1] = l;
      }
    }
    return;
  }
  // ---- fused merge: partials in blocks of kFaPartBlock floats per (tile, head,
  // chunk), laid out [float4 q4 = 8 dt + 2 g + hf][token of the tile] and then
  // (m, l) per token, so each store instruction writes 32 consecutive tokens'
  // 16 bytes: whole 128-byte lines, as the device-scope write-through stores need
  // (partial lines make them several times slower). Offsets stay below 2^31 (the
  // launcher caps the partials at kFaMaxPartialFloats).
  const __amdgpu_buffer_rsrc_t prs = dev::OutResource(part, static_cast<uint32_t>(kFaMaxPartialFloats * 4));
  const int tloc = 32 * wv + col;
  auto block_of = [&](int32_t c) -> uint32_t {
    return static_cast<uint32_t>(((static_cast<int64_t>(tile) * n_heads + h) * n_chunks + c) * kFaPartBlock) * 4u;
  };
  if (chunk < live && live > 1) {
    const uint32_t blk = block_of(chunk);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 v = make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
        dev::StoreBuf4<dev::kStoreDeviceThroughPolicy>(prs, blk + 16u * ((8 * dt + 2 * g + hf) * kFaTokens + tloc), v);
      }
    }
    if (hf == 0) {
      dev::StoreBufU2<dev::kStoreDeviceThroughPolicy>(prs, blk + 4u * (kFaTokens * kD) + 8u * tloc,
                                                      make_uint2(__float_as_uint(m), __float_as_uint(l)));
    }
  }
  const int32_t tile_live = LiveChunks(last_key, chunk_len, n_chunks);  // the workgroups of this (tile, head)
  if (tile_live == 1) return;  // uniform: no partials in this tile
  // Wait for this thread's partial stores to be acknowledged (device-scope
  // write-through: visible to every XCD), then count the workgroup in. The
  // clobber keeps the compiler from moving memory accesses across the wait.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __shared__ int last_flag;
  __syncthreads();
  uint32_t* counter = cnt + (static_cast<int64_t>(tile) * n_heads + h) * kFaCounterStride;
  if (threadIdx.x == 0) {
    const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = before == static_cast<uint32_t>(tile_live - 1);
  }
  __syncthreads();
  if (!last_flag) return;  // uniform
  // The last workgroup of the (tile, head) merges: each lane its own query's
  // chunks, AttnMergeRowsKernel's arithmetic (chunk maxima, then the weights and
  // normaliser summed in chunk order), with this workgroup's own chunk from its
  // registers (the very values it stored) and the others' partials through
  // device-coherent (sc1) loads issued after the barrier that follows the atomic,
  // one chunk's 64 values at a time.
  if (qvalid && live > 1) {
    float mc[kFaFusedMaxChunks], lc[kFaFusedMaxChunks];
#pragma unroll
    for (int c = 0; c < kFaFusedMaxChunks; ++c) {
      mc[c] = -INFINITY;
      lc[c] = 0.0f;
      if (c < live && c != chunk) {
        const uint2 u = dev::LoadBufU2<dev::kLoadDevicePolicy>(prs, block_of(c) + 4u * (kFaTokens * kD) + 8u * tloc);
        mc[c] = __uint_as_float(u.x);
        lc[c] = __uint_as_float(u.y);
      } else if (c == chunk) {
        mc[c] = m;
        lc[c] = l;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < kFaFusedMaxChunks; ++c) {
      if (c < live) mx = fmaxf(mx, mc[c]);
    }
    float L = 0.0f;
    F32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = F32x16{};
#pragma unroll
    for (int c = 0; c < kFaFusedMaxChunks; ++c) {
      if (c < live) {
        const float f = mc[c] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mc[c] - mx);
        L = __builtin_fmaf(lc[c], f, L);
        if (c == chunk) {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[dt][r] = __builtin_fmaf(o[dt][r], f, acc[dt][r]);
        } else {
          const uint32_t blk = block_of(c);
          float4 v[4][4];
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g)
              v[dt][g] = dev::LoadBuf4<dev::kLoadDevicePolicy>(prs, blk + 16u * ((8 * dt + 2 * g + hf) * kFaTokens + tloc));
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              acc[dt][4 * g] = __builtin_fmaf(v[dt][g].x, f, acc[dt][4 * g]);
              acc[dt][4 * g + 1] = __builtin_fmaf(v[dt][g].y, f, acc[dt][4 * g + 1]);
              acc[dt][4 * g + 2] = __builtin_fmaf(v[dt][g].z, f, acc[dt][4 * g + 2]);
              acc[dt][4 * g + 3] = __builtin_fmaf(v[dt][g].w, f, acc[dt][4 * g + 3]);
            }
        }
      }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    float* orow = out + (tq * n_heads + h) * kD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 v = make_float4(acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv, acc[dt][4 * g + 2] * inv,
                                     acc[dt][4 * g + 3] * inv);
        *reinterpret_cast<float4*>(orow + 32 * dt + 8 * g + 4 * hf) = v;
      }
    }
  }
  // every workgroup of the (tile, head) has counted in: ready for the next call
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- partials buffer

// Grow-only device buffer for the chunk partials. A buffer that is outgrown is
// retired, not freed: a HIP graph captured earlier keeps its address and may
// still replay (the sizes involved are a few MiB). Deliberately never freed at
// exit (a destructor running after the HIP runtime has shut down can hang).
constexpr int64_t kMaxSplitPairs = 1024;

struct PartialsBuffer {
  std::mutex mu;
  float* ptr = nullptr;
  size_t floats = 0;
};
PartialsBuffer& Partials() {
  static PartialsBuffer* b = new PartialsBuffer();
  return *b;
}

float* EnsurePartials(size_t floats) {
  PartialsBuffer& b = Partials();
  std::lock_guard<std::mutex> lock(b.mu);
  if (b.floats < floats) {
    RPG_CHECK(!StreamIsCapturing(),
              "attention needs a %zu-float partials buffer (have %zu), which cannot be allocated during graph "
              "capture; call GpuAttentionWarmupShmem(max positions) before capturing",
              floats, b.floats);
    const size_t grow = floats > 2 * b.floats ? floats : 2 * b.floats;  // geometric: few retired buffers
    float* p = nullptr;
    RPG_HIP_CHECK(hipMalloc(&p, grow * sizeof(float)));
    b.ptr = p;  // the previous buffer stays allocated (see above)
    b.floats = grow;
  }
  return b.ptr;
}

// Fixed partials storage for GpuAttentionFromCacheNoAlloc: a file-scope device
// array, so that entry point never allocates. Each device holds its own copy at
// its own address; host code must use the address hipGetSymbolAddress returns
// for the current device (AttnScratchForDevice), never the array's name, which
// on the host is only a registration handle.
constexpr size_t kNoAllocScratchFloats = size_t(1) << 19;  // 2 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

constexpr int kMaxScratchDevices = 64;

struct ScratchTable {
  std::mutex mu;
  float* ptr[kMaxScratchDevices] = {};
};
ScratchTable& Scratch() {
  static ScratchTable* t = new ScratchTable();
  return *t;
}

// Device address of `scratch` on the current device, looked up once per device.
float* ScratchForCurrentDevice() {
  int dev = -1;
  RPG_HIP_CHECK(hipGetDevice(&dev));
  RPG_CHECK(dev >= 0 && dev < kMaxScratchDevices, "device %d is beyond the %d devices the scratch table tracks", dev,
            kMaxScratchDevices);
  ScratchTable& t = Scratch();
  std::lock_guard<std::mutex> lock(t.mu);
  if (t.ptr[dev] == nullptr) {
    void* p = nullptr;
    RPG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    RPG_CHECK(p != nullptr, "hipGetSymbolAddress returned no address for the attention scratch on device %d", dev);
    t.ptr[dev] = static_cast<float*>(p);
  }
  return t.ptr[dev];
}

// Arrival counters of the one-launch split decode (AttnDecodeGroupKernel<G, kPrep,
// true>), one per (token, kv head) pair: zero at load, counted up by the pair's
// workgroups and put back to zero by the last of them, so they are zero between
// launches and a captured graph replays them as they are. The first half serves
// the allocating entry points, the second the no-allocation one. A split needs
// fewer than 2048 pairs (PlanGroupChunks gives one chunk from 2048 on).
constexpr int64_t kFusedCounterPairs = 2048;
static __device__ __align__(256) uint32_t pair_counters[2 * kFusedCounterPairs * kCounterStride];

struct CounterTable {
  std::mutex mu;
  uint32_t* ptr[kMaxScratchDevices] = {};
};
CounterTable& CounterTableInstance() {
  static CounterTable* t = new CounterTable();
  return *t;
}

// Device address of `pair_counters` on the current device, looked up once per device.
uint32_t* CountersForCurrentDevice() {
  int dev = -1;
  RPG_HIP_CHECK(hipGetDevice(&dev));
  RPG_CHECK(dev >= 0 && dev < kMaxScratchDevices, "device %d is beyond the %d devices the counter table tracks", dev,
            kMaxScratchDevices);
  CounterTable& t = CounterTableInstance();
  std::lock_guard<std::mutex> lock(t.mu);
  if (t.ptr[dev] == nullptr) {
    void* p = nullptr;
    RPG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(pair_counters)));
    RPG_CHECK(p != nullptr, "hipGetSymbolAddress returned no address for the attention counters on device %d", dev);
    t.ptr[dev] = static_cast<uint32_t*>(p);
  }
  return t.ptr[dev];
}

// Arrival counters of the prefill's fused chunk merge, one per (token tile,
// head), used the same way (zero between launches); first half for the allocating
// entry points, second for the no-allocation one. A launch with more (tile, head)
// pairs than a half holds merges in a separate launch.
static __device__ __align__(256) uint32_t fa_counters[2 * kFaCounterSlots * kFaCounterStride];

CounterTable& FaCounterTableInstance() {
  static CounterTable* t = new CounterTable();
  return *t;
}

// Device address of `fa_counters` on the current device, looked up once per device.
uint32_t* FaCountersForCurrentDevice() {
  int dev = -1;
  RPG_HIP_CHECK(hipGetDevice(&dev));
  RPG_CHECK(dev >= 0 && dev < kMaxScratchDevices, "device %d is beyond the %d devices the counter table tracks", dev,
            kMaxScratchDevices);
  CounterTable& t = FaCounterTableInstance();
  std::lock_guard<std::mutex> lock(t.mu);
  if (t.ptr[dev] == nullptr) {
    void* p = nullptr;
    RPG_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(fa_counters)));
    RPG_CHECK(p != nullptr, "hipGetSymbolAddress returned no address for the prefill counters on device %d", dev);
    t.ptr[dev] = static_cast<uint32_t*>(p);
  }
  return t.ptr[dev];
}

// Where a split-key launch keeps its chunk partials: the library's grow-only
// buffer (fixed == nullptr) or a fixed region that must already be big enough.
// The one-launch decode also takes its arrival counters from here.
struct PartialsSink {
  float* fixed = nullptr;
  size_t fixed_floats = 0;

  uint32_t* Counters() const {
    return CountersForCurrentDevice() + (fixed == nullptr ? 0 : kFusedCounterPairs * kCounterStride);
  }
  uint32_t* PrefillCounters() const {
    return FaCountersForCurrentDevice() + (fixed == nullptr ? 0 : kFaCounterSlots * kFaCounterStride);
  }

  float* Get(size_t floats) const {
    if (fixed == nullptr) return EnsurePartials(floats);
    RPG_CHECK(floats <= fixed_floats,
              "this attention call splits its keys into %zu floats of partials, more than the %zu floats (%zu MiB) "
              "of the no-allocation entry point's fixed scratch; use the allocating entry point for it",
              floats, fixed_floats, fixed_floats * sizeof(float) >> 20);
    return fixed;
  }

  // Floats a call may take (the library's buffer grows; a fixed region does not).
  size_t Capacity() const { return fixed == nullptr ? SIZE_MAX : fixed_floats; }
};

// Up to this many positions one chunk per (token, head) beats a split plus the
// merge launch (decode at Qwen3-1.7B: 8.2 vs 9.2 us at 128 keys, 14.1 vs 9.3 us
// at 256).
constexpr int64_t kSingleChunkPositions = 128;

// Chunking for `pairs` (t, h) pairs over a budget of `positions` keys: no split
// when the pairs alone fill the chip or the keys are few; otherwise enough
// chunks (of at least 64 keys, a multiple of 64) for ~2048 waves.
void PlanChunks(int64_t pairs, int64_t positions, int32_t* n_chunks, int64_t* chunk_len) {
  if (pairs >= kMaxSplitPairs || positions <= kSingleChunkPositions) {
    *n_chunks = 1;
    *chunk_len = positions;
    return;
  }
  int64_t want = (2048 + pairs - 1) / pairs;
  if (want > kMaxChunks) want = kMaxChunks;
  int64_t len = (positions + want - 1) / want;
  len = (len + 63) / 64 * 64;
  *chunk_len = len;
  *n_chunks = static_cast<int32_t>((positions + len - 1) / len);
}

// The same for the grouped decode kernel: `units` (token, kv head) pairs, chunks
// of a multiple of 32 keys, enough for ~2048 waves. Under graph capture the plan
// covers the position budget and the kernels use only the chunks live at the
// replayed position.
void PlanGroupChunks(int64_t units, int64_t positions, int32_t* n_chunks, int64_t* chunk_len) {
  if (units >= 2048 || positions <= kSingleChunkPositions) {
    *n_chunks = 1;
    *chunk_len = positions;
    return;
  }
  int64_t want = (2048 + units - 1) / units;
  if (want > kMaxGroupChunks) want = kMaxGroupChunks;
  int64_t len = (positions + want - 1) / want;
  len = (len + 31) / 32 * 32;
  *chunk_len = len;
  *n_chunks = static_cast<int32_t>((positions + len - 1) / len);
}

// Partials needed by any decode-sized call (seq 1, up to 64 heads, at most
// kMaxGroupChunks chunks): what a captured decode graph may replay.
size_t WarmupFloats(int64_t /*positions*/) { return static_cast<size_t>(64) * kMaxGroupChunks * kPartFloats; }

// A split grouped decode is one launch (AttnDecodeGroupKernel<G, kPrep, true>,
// merged by the last workgroup of each pair), whatever the position budget: a
// captured decode graph plans for the whole cache and replays at every position.
template <int G>
void LaunchDecodeGroup(const ModelMeta& c, const Pos0Arg& p0, const float* q_dev, int64_t seq,
                       const uint16_t* k_layer, const uint16_t* v_layer, int64_t max_seq, float scale,
                       int64_t positions, float* out_dev, const DecodePrep* prep = nullptr,
                       const PartialsSink& sink = PartialsSink{}) {
  int32_t n_chunks;
  int64_t chunk_len;
  // the kernel forms (token, kv head) indices and chunk offsets in 32 bits
  RPG_CHECK(seq * c.n_kv_heads < (int64_t{1} << 32) && max_seq <= INT32_MAX / (2 * kD),
            "decode attention over %lld (token, kv head) pairs and %lld cache rows exceeds the kernel's 32-bit "
            "indexing", static_cast<long long>(seq * c.n_kv_heads), static_cast<long long>(max_seq));
  PlanGroupChunks(seq * c.n_kv_heads, positions, &n_chunks, &chunk_len);
  const int64_t pairs = seq * c.n_heads;
  if (n_chunks > 1) {
    // one launch: workgroups of kFusedWaves chunks, merged by the pair's last workgroup
    const int64_t kv_pairs = seq * c.n_kv_heads;
    RPG_CHECK(kv_pairs <= kFusedCounterPairs, "a split decode over %lld (token, kv head) pairs exceeds the %lld "
              "arrival counters", static_cast<long long>(kv_pairs), static_cast<long long>(kFusedCounterPairs));
    const int32_t n_groups = (n_chunks + kFusedWaves - 1) / kFusedWaves;
    // one workgroup per pair holds every chunk: it merges in LDS and needs no partials
    float* part = n_groups > 1 ? sink.Get(static_cast<size_t>(pairs) * n_groups * kPartFloats) : nullptr;
    uint32_t* cnt = sink.Counters();
    const dim3 grid(static_cast<unsigned>(kv_pairs * n_groups));
    if (prep != nullptr) {
      Launch("AttnDecodePrepFusedKernel", AttnDecodeGroupKernel<G, true, true>, grid, dim3(64 * kFusedWaves), q_dev,
             k_layer, v_layer, max_seq, c.n_heads, c.n_kv_heads, scale, p0.value, p0.dev, seq, n_chunks, chunk_len,
             out_dev, part, *prep, cnt);
    } else {
      Launch("AttnDecodeFusedKernel", AttnDecodeGroupKernel<G, false, true>, grid, dim3(64 * kFusedWaves), q_dev,
             k_layer, v_layer, max_seq, c.n_heads, c.n_kv_heads, scale, p0.value, p0.dev, seq, n_chunks, chunk_len,
             out_dev, part, DecodePrep{}, cnt);
    }
    return;
  }
  // one chunk per (token, kv head): each wave writes its heads' outputs, no partials
  const int64_t units = seq * c.n_kv_heads;
  float* const part = nullptr;
  if (prep != nullptr) {
    Launch("AttnDecodePrepKernel", AttnDecodeGroupKernel<G, true>, dim3(GridFor(units, kWaves)),
           dim3(kBlockThreads), q_dev, k_layer, v_layer, max_seq, c.n_heads, c.n_kv_heads, scale, p0.value, p0.dev,
           seq, n_chunks, chunk_len, out_dev, part, *prep, static_cast<uint32_t*>(nullptr));
  } else {
    Launch("AttnDecodeGroupKernel", AttnDecodeGroupKernel<G>, dim3(GridFor(units, kWaves)), dim3(kBlockThreads),
           q_dev, k_layer, v_layer, max_seq, c.n_heads, c.n_kv_heads, scale, p0.value, p0.dev, seq, n_chunks,
           chunk_len, out_dev, part, DecodePrep{}, static_cast<uint32_t*>(nullptr));
  }
}

// GpuAttentionFromCache with the chunk partials taken from `sink`.
void AttentionFromCache(const ModelMeta& c, int64_t pos0, const float* q_dev, int64_t seq, const uint16_t* k_layer,
                        const uint16_t* v_layer, int64_t max_seq, float* out_dev, int64_t sh_positions,
                        const PartialsSink& sink) {
  RPG_CHECK(seq > 0, "attention: the query batch is empty (seq <= 0)");
  RPG_CHECK(pos0 >= 0, "attention: a negative start position");
  RPG_CHECK(c.n_heads > 0 && c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0,
            "n_heads (%d) must be a positive multiple of n_kv_heads (%d)", c.n_heads, c.n_kv_heads);
  RPG_CHECK(c.head_dim == kD, "attention supports head_dim %d (got %d)", kD, c.head_dim);
  RPG_CHECK(pos0 + seq <= max_seq, "positions [%lld, %lld) exceed the cache capacity %lld",
            static_cast<long long>(pos0), static_cast<long long>(pos0 + seq), static_cast<long long>(max_seq));
  const int64_t positions = sh_positions > 0 ? sh_positions : pos0 + seq;
  RPG_CHECK(positions >= pos0 + seq, "position budget (%lld) is smaller than the positions this call needs (%lld)",
            static_cast<long long>(positions), static_cast<long long>(pos0 + seq));
  RPG_CHECK(q_dev && k_layer && v_layer && out_dev, "attention got a null pointer");
  RPG_CHECK((reinterpret_cast<uintptr_t>(k_layer) & 15u) == 0 && (reinterpret_cast<uintptr_t>(v_layer) & 3u) == 0,
            "KV cache layers must be 16-byte (K) / 4-byte (V) aligned");
  const float scale = 1.0f / sqrtf(static_cast<float>(c.head_dim));
  const int64_t pairs = seq * c.n_heads;
  int32_t n_chunks;
  int64_t chunk_len;
  PlanChunks(pairs, positions, &n_chunks, &chunk_len);
  const Pos0Arg p0 = Pos0ForLaunch(pos0);
  if (seq >= kFaMinTokens) {
    // Key chunks of at most max(8, total / 512) key blocks per workgroup (two
    // workgroups per CU), counted over the position budget; the partials stay
    // within kFaMaxPartialFloats and within the sink (a fixed region that is
    // too small keeps one chunk, with no partials at all).
    const int64_t tiles = (seq + kFaTokens - 1) / kFaTokens;
    const int64_t first = positions - seq;  // position of token 0 in the budget
    int64_t total_blocks = 0;
    for (int64_t tt = 0; tt < tiles; ++tt) {
      const int64_t last = first + (tt + 1) * kFaTokens < positions ? first + (tt + 1) * kFaTokens : positions;
      total_blocks += (last + kFaKeys - 1) / kFaKeys;
    }
    total_blocks *= c.n_heads;
    const int64_t max_blocks = (positions + kFaKeys - 1) / kFaKeys;
    int64_t per = (total_blocks + 511) / 512;
    if (per < 8) per = 8;
    int64_t fa_chunks = (max_blocks + per - 1) / per;
    const int64_t room = static_cast<int64_t>(
        sink.Capacity() < static_cast<size_t>(kFaMaxPartialFloats) ? sink.Capacity() : kFaMaxPartialFloats);
    const int64_t per_chunk = std::max(seq * c.n_heads * kPartFloats, tiles * c.n_heads * kFaPartBlock);
    const int64_t cap = room / per_chunk;
    if (fa_chunks > cap) fa_chunks = cap;
    if (fa_chunks > kMaxChunks) fa_chunks = kMaxChunks;
    if (fa_chunks < 1) fa_chunks = 1;
    const int64_t fa_len = (max_blocks + fa_chunks - 1) / fa_chunks * kFaKeys;
    fa_chunks = (positions + fa_len - 1) / fa_len;
    // the fused merge's blocks cover whole tiles: tiles * 128 * 130 floats per (head, chunk), against
    // seq * 132 for the separate merge's rows
    const int64_t fused_floats = tiles * c.n_heads * fa_chunks * kFaPartBlock;
    const int64_t rows_floats = pairs * fa_chunks * kPartFloats;
    float* part = fa_chunks > 1 ? sink.Get(static_cast<size_t>(std::max(fused_floats, rows_floats))) : nullptr;
    const int64_t n_pairs = tiles * fa_chunks;
    RPG_CHECK(n_pairs * c.n_heads < (int64_t{1} << 31), "prefill attention grid too large");
    // (tile, chunk) pairs sorted by their key blocks over the position budget,
    // most first (ties: later tile first)
    FaOrder order;
    order.n = 0;
    if (n_pairs <= kFaOrderMax && tiles <= 1024) {
      std::vector<std::pair<int64_t, int32_t>> by_size;
      by_size.reserve(static_cast<size_t>(n_pairs));
      const int64_t len_blocks = fa_len / kFaKeys;
      for (int64_t tt = 0; tt < tiles; ++tt) {
        const int64_t last = first + (tt + 1) * kFaTokens < positions ? first + (tt + 1) * kFaTokens : positions;
        const int64_t n_blocks = (last + kFaKeys - 1) / kFaKeys;
        for (int64_t ch = 0; ch < fa_chunks; ++ch) {
          const int64_t size = std::min(std::max<int64_t>(n_blocks - ch * len_blocks, 0), len_blocks);
          by_size.emplace_back(-(size * 1024 + tt), static_cast<int32_t>((tt << 6) | ch));
        }
      }
      std::sort(by_size.begin(), by_size.end());
      for (int64_t i = 0; i < n_pairs; ++i) order.e[i] = static_cast<uint16_t>(by_size[i].second);
      order.n = static_cast<int32_t>(n_pairs);
    }
    // the last workgroup of each (tile, head) merges the tile's partials, unless the
    // counters cannot cover every (tile, head)
    uint32_t* cnt = fa_chunks > 1 && fa_chunks <= kFaFusedMaxChunks && tiles * c.n_heads <= kFaCounterSlots
                        ? sink.PrefillCounters()
                        : nullptr;
    Launch("AttnPrefillMfmaKernel", AttnPrefillMfmaKernel, dim3(static_cast<unsigned>(n_pairs * c.n_heads)),
           dim3(kBlockThreads), q_dev, k_layer, v_layer, max_seq, c.n_heads, c.n_heads / c.n_kv_heads, scale,
           p0.value, p0.dev, seq, static_cast<int32_t>(fa_chunks), fa_len, static_cast<int32_t>(tiles), out_dev,
           part, order, cnt);
    if (fa_chunks > 1 && cnt == nullptr) {
      Launch("AttnMergeRowsKernel", AttnMergeRowsKernel, dim3(GridFor(pairs * (kD / 4), kBlockThreads)),
             dim3(kBlockThreads), static_cast<const float*>(part), pairs, static_cast<int32_t>(fa_chunks), c.n_heads,
             fa_len, p0.value, p0.dev, out_dev);
    }
    return;
  }
  const int group = c.n_heads / c.n_kv_heads;
  const bool aligned = (reinterpret_cast<uintptr_t>(q_dev) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(v_layer) & 15u) == 0;
  if (aligned && group == 1) {
    return LaunchDecodeGroup<1>(c, p0, q_dev, seq, k_layer, v_layer, max_seq, scale, positions, out_dev, nullptr,
                                sink);
  }
  if (aligned && group == 2) {
    return LaunchDecodeGroup<2>(c, p0, q_dev, seq, k_layer, v_layer, max_seq, scale, positions, out_dev, nullptr,
                                sink);
  }
  if (aligned && group == 4) {
    return LaunchDecodeGroup<4>(c, p0, q_dev, seq, k_layer, v_layer, max_seq, scale, positions, out_dev, nullptr,
                                sink);
  }
  // other group sizes / alignments: one wave per query head
  float* part = nullptr;
  if (n_chunks > 1) part = sink.Get(static_cast<size_t>(pairs) * n_chunks * kPartFloats);
  const int64_t units = pairs * n_chunks;
  Launch("AttnChunkKernel", AttnChunkKernel<uint16_t>, dim3(GridFor(units, kWaves)), dim3(kBlockThreads), q_dev,
         k_layer, v_layer, max_seq * kD, static_cast<int64_t>(kD), max_seq, c.n_heads, c.n_heads / c.n_kv_heads,
         scale, p0.value, p0.dev, seq, n_chunks, chunk_len, out_dev, part);
  if (n_chunks > 1) {
    Launch("AttnMergeKernel", AttnMergeKernel, dim3(static_cast<unsigned>(pairs)), dim3(kBlockThreads), part, pairs,
           n_chunks, c.n_heads, chunk_len, p0.value, p0.dev, out_dev);
  }
}

}  // namespace

void GpuAttentionFromCache(const ModelMeta& c, int64_t pos0, const float* q_dev, int64_t seq, const uint16_t* k_layer,
                           const uint16_t* v_layer, int64_t max_seq, float* out_dev, int64_t sh_positions) {
  AttentionFromCache(c, pos0, q_dev, seq, k_layer, v_layer, max_seq, out_dev, sh_positions, PartialsSink{});
}

void GpuAttentionFromCacheNoAlloc(const ModelMeta& c, int64_t pos0, const float* q_dev, int64_t seq,
                                  const uint16_t* k_layer, const uint16_t* v_layer, int64_t max_seq, float* out_dev,
                                  int64_t sh_positions) {
  const PartialsSink sink{ScratchForCurrentDevice(), kNoAllocScratchFloats};
  AttentionFromCache(c, pos0, q_dev, seq, k_layer, v_layer, max_seq, out_dev, sh_positions, sink);
}

void GpuAttentionNoAllocInit() {
  (void)ScratchForCurrentDevice();
  (void)CountersForCurrentDevice();
  (void)FaCountersForCurrentDevice();
}

size_t GpuAttentionNoAllocScratchBytes() { return kNoAllocScratchFloats * sizeof(float); }

bool GpuQkNormRopeKvAttention(const ModelMeta& c, int64_t pos0, const float* q_dev, const float* k_dev,
                              const float* v_dev, const float* q_norm, const float* k_norm, const float* rope_tab,
                              int64_t rope_rows, uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq,
                              float* out_dev, int64_t sh_positions) {
  RPG_CHECK(pos0 >= 0, "attention: a negative start position");
  RPG_CHECK(c.n_heads > 0 && c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0,
            "n_heads (%d) must be a positive multiple of n_kv_heads (%d)", c.n_heads, c.n_kv_heads);
  RPG_CHECK(pos0 + 1 <= max_seq, "attention: position %lld has no slot in a cache of %lld positions", static_cast<long long>(pos0),
            static_cast<long long>(max_seq));
  RPG_CHECK(pos0 + 1 <= rope_rows, "position %lld exceeds the RoPE table (%lld rows)", static_cast<long long>(pos0),
            static_cast<long long>(rope_rows));
  const int64_t positions = sh_positions > 0 ? sh_positions : pos0 + 1;
  RPG_CHECK(positions >= pos0 + 1, "position budget (%lld) is smaller than the positions this call needs (%lld)",
            static_cast<long long>(positions), static_cast<long long>(pos0 + 1));
  RPG_CHECK(q_dev && k_dev && v_dev && q_norm && k_norm && rope_tab && k_layer && v_layer && out_dev,
            "QkNormRopeKvAttention got a null pointer");
  const int group = c.n_heads / c.n_kv_heads;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (c.head_dim != kD || !(group == 1 || group == 2 || group == 4) || !a16(q_dev) || !a16(k_dev) || !a16(v_dev) ||
      !a16(q_norm) || !a16(k_norm) || !a16(rope_tab) || !a16(k_layer) || !a16(v_layer) || !a16(out_dev)) {
    return false;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(c.head_dim));
  const Pos0Arg p0 = Pos0ForLaunch(pos0);
  const DecodePrep prep{k_dev, v_dev, q_norm, k_norm, rope_tab, rope_rows, c.rms_eps, k_layer, v_layer};
  if (group == 1) LaunchDecodeGroup<1>(c, p0, q_dev, 1, k_layer, v_layer, max_seq, scale, positions, out_dev, &prep);
  if (group == 2) LaunchDecodeGroup<2>(c, p0, q_dev, 1, k_layer, v_layer, max_seq, scale, positions, out_dev, &prep);
  if (group == 4) LaunchDecodeGroup<4>(c, p0, q_dev, 1, k_layer, v_layer, max_seq, scale, positions, out_dev, &prep);
  return true;
}

void GpuCausalAttention(const ModelMeta& c, const float* q_dev, const float* k_dev, const float* v_dev, int64_t seq,
                        float* out_dev) {
  RPG_CHECK(seq > 0, "attention: the query batch is empty (seq <= 0)");
  RPG_CHECK(c.n_heads > 0 && c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0,
            "n_heads (%d) must be a positive multiple of n_kv_heads (%d)", c.n_heads, c.n_kv_heads);
  RPG_CHECK(c.head_dim == kD, "attention supports head_dim %d (got %d)", kD, c.head_dim);
  RPG_CHECK(q_dev && k_dev && v_dev && out_dev, "attention got a null pointer");
  RPG_CHECK((reinterpret_cast<uintptr_t>(k_dev) & 15u) == 0 && (reinterpret_cast<uintptr_t>(v_dev) & 7u) == 0,
            "k / v rows must be 16-byte / 8-byte aligned");
  const float scale = 1.0f / sqrtf(static_cast<float>(c.head_dim));
  const int64_t pairs = seq * c.n_heads;
  int32_t n_chunks;
  int64_t chunk_len;
  PlanChunks(pairs, seq, &n_chunks, &chunk_len);
  float* part = nullptr;
  if (n_chunks > 1) part = EnsurePartials(static_cast<size_t>(pairs) * n_chunks * kPartFloats);
  const int64_t units = pairs * n_chunks;
  const int64_t row = static_cast<int64_t>(c.n_kv_heads) * kD;  // one token's k (or v) row
  Launch("AttnChunkKernel<f32>", AttnChunkKernel<float>, dim3(GridFor(units, kWaves)), dim3(kBlockThreads), q_dev,
         k_dev, v_dev, static_cast<int64_t>(kD), row, seq, c.n_heads, c.n_heads / c.n_kv_heads, scale,
         static_cast<int64_t>(0), static_cast<const int64_t*>(nullptr), seq, n_chunks, chunk_len, out_dev, part);
  if (n_chunks > 1) {
    Launch("AttnMergeKernel", AttnMergeKernel, dim3(static_cast<unsigned>(pairs)), dim3(kBlockThreads), part, pairs,
           n_chunks, c.n_heads, chunk_len, static_cast<int64_t>(0), static_cast<const int64_t*>(nullptr), out_dev);
  }
}

void GpuAttentionWarmupShmem(int64_t sh_positions) {
  RPG_CHECK(sh_positions > 0, "attention warmup: the position budget has to be at least 1 (got %lld)", static_cast<long long>(sh_positions));
  EnsurePartials(WarmupFloats(sh_positions));
  (void)CountersForCurrentDevice();
  (void)FaCountersForCurrentDevice();
}

}  // namespace rpg
