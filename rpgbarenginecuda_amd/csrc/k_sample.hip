// Device argmax (reference GpuArgMax, src/kernels_gpu.h:131-143, kernel
// src/kernels_gpu.cu:827-859) and the sampler (src/sampler_gpu.h; kernels
// src/sampler_gpu.cu:161-467). The semantics are listed in sampler_gpu.h.
//
// MI355X mapping. The reference filters in ONE 1024-thread block with 32-step
// binary searches (each step a pass over the vocabulary) and runs the inverse
// transform on ONE thread. A single CU needs several microseconds per pass over
// 151936 floats and ~20 us for a pass that evaluates expf, so here every pass
// is a grid of 1024-element slices (149 workgroups for Qwen3's vocabulary):
//   * top_k's threshold and top_p's cut are radix selects over the 32-bit order
//     keys with 12/12/8-bit digits. Level 1 is a histogram pass (each workgroup
//     histograms its slice in LDS and adds the non-zero bins to a global
//     histogram). In the next pass every workgroup picks level 1's digit from it
//     (same data, same order, same answer) and appends its keys with that digit
//     to a candidate list; the workgroup that arrives last selects the other 20
//     bits among the candidates in LDS. Two passes instead of 32;
//   * top_p's S(t) is summed as integers, p * 2^62 truncated, so the histogram
//     sums do not depend on the order of the atomics (they differ from the real
//     sums by less than n * 2^-62); the kept mass for the second normalisation
//     comes from the same integers;
//   * values that couple slices (max, sums, argmax) travel as per-slice
//     partials that every workgroup of the next kernel reduces in one fixed
//     order, so every result is the same from run to run;
//   * "the last workgroup to arrive" is one vector atomic per workgroup on a
//     counter that the last one puts back to zero; what it reads from the other
//     workgroups was stored device-scope write-through and is loaded
//     device-coherent. No workgroup ever waits for another (a grid barrier was
//     measured at ~3 us per barrier over 149 workgroups, no cheaper than a launch);
//   * the inverse transform keeps the serial double semantics exactly: a
//     fixed-point prefix (p * 2^52 truncated) over slices and then within one
//     slice finds the first index whose prefix exceeds u. The serial double sum
//     differs from the exact prefix by at most n * 2^-53 * max(prefix), so when
//     u is further than that (plus the truncation) from both neighbouring
//     prefixes the serial loop picks the same index. Otherwise (u within
//     ~1e-10 of a boundary) one thread runs the serial loop. The last workgroup
//     of the normalising pass runs it.
// Kernels, for T > 0 with top_p (the engine's default, top_k off):
//   Prep -> Sum -> TopP -> TopPCand -> Norm (+ inverse transform): 5 launches;
// top_k adds TopKCand after Prep (its level-1 histogram is built in Prep);
// without top_p the TopP kernels drop out. GpuArgMax is one launch.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "hip_common.h"
#include "kernels_gpu.h"
#include "launch.h"
#include "sampler_gpu.h"

namespace rpg {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSlice = 1024;  // elements per workgroup
constexpr int kPerThread = kSlice / kThreads;
constexpr int kMaxSlices = static_cast<int>(kSamplerMaxVocab / kSlice);
constexpr int kPartsPerThread = kMaxSlices / kThreads;  // partials one thread reduces
constexpr int kBins = 4096;                              // widest radix digit (12 bits)
enum ArriveCounter { kArriveArgMax, kArriveTopK, kArriveTopP, kArriveFinal, kArriveCounters };

// Radix levels: digit = (key >> shift) & (2^bits - 1); level L keeps only keys
// whose bits above its digit equal the prefix chosen by the levels before it.
__host__ __device__ constexpr int LevelShift(int level) { return level == 1 ? 20 : (level == 2 ? 8 : 0); }
__host__ __device__ constexpr int LevelBits(int level) { return level == 3 ? 8 : 12; }

struct SampleScratch {
  float max_part[kMaxSlices];
  double sum_part[kMaxSlices];
  float best_val[kMaxSlices];
  int32_t best_idx[kMaxSlices];
  uint64_t fix_part[kMaxSlices];
  double tot_part[kMaxSlices];
  uint32_t khist[kBins];  // top_k level-1 counts; zero between calls
  uint64_t phist[kBins];  // top_p level-1 weights; zero between calls
  uint32_t kth_key;       // top_k threshold key
  uint32_t cut_key;       // top_p: keys <= cut_key are cut (0xFFFFFFFF: no cut)
  uint64_t kept_w;        // top_p: Fix62 weight of the keys above the cut
  // Counters of the passes whose last workgroup finishes the step (zero between
  // calls: the last workgroup puts its counter back), one per 256 bytes.
  uint32_t arrive[kArriveCounters][64];
  uint32_t cand_count[kMaxSlices];  // candidates of each slice (at key[slice * kSlice ...])
};

// Candidate lists of the radix selects: the keys (and top_p weights) whose
// level-1 digit equals the selected one, each slice's in its own region (slice
// g at [g * kSlice, g * kSlice + cand_count[g])), resolved by the last
// workgroup. Sized for the whole vocabulary (ties can make every value a
// candidate).
struct SampleCandidates {
  uint32_t key[kSamplerMaxVocab];
  uint64_t w[kSamplerMaxVocab];
};

// ---------------------------------------------------------------- random source

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;  // SplitMix64's increment (2^64 / golden ratio)

// SplitMix64 (Steele, Lea & Flood, OOPSLA 2014): the state advanced by the
// golden-ratio increment, then the published 64-bit finaliser.
__host__ __device__ inline uint64_t SplitMix64Of(uint64_t x) {
  uint64_t z = x + kGamma;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t CounterRngOf(uint64_t seed, uint64_t counter) {
  return SplitMix64Of(seed + kGamma * counter);
}
__host__ __device__ inline float CounterUniformOf(uint64_t seed, uint64_t counter) {
  return static_cast<float>(static_cast<uint32_t>(CounterRngOf(seed, counter) >> 40)) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------- keys and fixed point

// Order-preserving map of float bit patterns onto uint32 (negative values are
// bit-inverted, non-negative ones get the sign bit set), and its inverse.
__device__ __forceinline__ uint32_t OrderKey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float FromOrderKey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// top_p weight: p * 2^62 truncated (p <= 2 keeps it below 2^63; anything else,
// NaN included, weighs 0).
__device__ __forceinline__ uint64_t Fix62(float p) {
  return (p >= 0.0f && p <= 2.0f) ? static_cast<uint64_t>(p * 0x1p62f) : 0ull;
}
// Inverse-transform weight: p * 2^52 truncated, exact floor for 0 <= p < 2.
__device__ __forceinline__ bool Fix52Valid(float p) { return p >= 0.0f && p < 2.0f; }
__device__ __forceinline__ uint64_t Fix52(float p) {
  return Fix52Valid(p) ? static_cast<uint64_t>(p * 0x1p52f) : 0ull;
}

// ---------------------------------------------------------------- block helpers (256 threads)

struct Best {
  float v;
  int32_t i;
};
// The larger value wins, ties go to the smaller index: a total order, so any
// reduction tree gives the same answer.
__device__ __forceinline__ Best Better(Best a, Best b) { return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a; }

__device__ __forceinline__ Best WaveBest(Best x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    Best o;
    o.v = __shfl_xor(x.v, off, 64);
    o.i = __shfl_xor(x.i, off, 64);
    x = Better(x, o);
  }
  return x;
}
__device__ __forceinline__ Best BlockBest(Best x, Best* sh) {
  x = WaveBest(x);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = x;
  __syncthreads();
  Best r = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = Better(r, sh[w]);
  __syncthreads();
  return r;
}

// Wave-level steps through DPP moves (VALU, a few cycles) instead of LDS
// permutes (a round trip through the LDS unit each, in dependent chains):
// a 64-bit value moved as two 32-bit halves; lanes the pattern gives no source
// (or rows outside row_mask) keep `old`.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ uint64_t DppU64(uint64_t v, uint64_t old) {
  const int lo = __builtin_amdgcn_update_dpp(static_cast<int>(static_cast<uint32_t>(old)),
                                             static_cast<int>(static_cast<uint32_t>(v)), kCtrl, kRowMask, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(static_cast<int>(static_cast<uint32_t>(old >> 32)),
                                             static_cast<int>(static_cast<uint32_t>(v >> 32)), kCtrl, kRowMask, 0xF,
                                             false);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ float DppF(float v, float old) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), kCtrl, kRowMask, 0xF, false));
}
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ double DppDbl(double v, double old) {
  return __builtin_bit_cast(double, DppU64<kCtrl, kRowMask>(__builtin_bit_cast(uint64_t, v),
                                                             __builtin_bit_cast(uint64_t, old)));
}
// Row steps (quad_perm [1,0,3,2], [2,3,0,1], half-row mirror, row mirror) leave
// every lane of a 16-lane row with the row's op-total; rows 1 and 3 then take
// rows 0 and 2 (row_bcast:15) and rows 2 and 3 take row 1 (row_bcast:31), so
// lane 63 ends with the wave's total. Every lane must be active.
__device__ __forceinline__ float WaveMaxTo63(float v) {
  v = fmaxf(v, DppF<0xB1>(v, v));
  v = fmaxf(v, DppF<0x4E>(v, v));
  v = fmaxf(v, DppF<0x141>(v, v));
  v = fmaxf(v, DppF<0x140>(v, v));
  v = fmaxf(v, DppF<0x142, 0xA>(v, -INFINITY));
  return fmaxf(v, DppF<0x143, 0xC>(v, -INFINITY));
}
__device__ __forceinline__ double WaveSumTo63(double v) {
  v += DppDbl<0xB1>(v, 0.0);
  v += DppDbl<0x4E>(v, 0.0);
  v += DppDbl<0x141>(v, 0.0);
  v += DppDbl<0x140>(v, 0.0);
  v += DppDbl<0x142, 0xA>(v, 0.0);
  return v + DppDbl<0x143, 0xC>(v, 0.0);
}
// Inclusive prefix sum over the wave: row_shr 1, 2, 4, 8 inside each row, then
// the rows' totals as above.
__device__ __forceinline__ uint64_t WaveInclScanU64(uint64_t v) {
  v += DppU64<0x111>(v, 0);
  v += DppU64<0x112>(v, 0);
  v += DppU64<0x114>(v, 0);
  v += DppU64<0x118>(v, 0);
  v += DppU64<0x142, 0xA>(v, 0);
  return v + DppU64<0x143, 0xC>(v, 0);
}

// Maximum of non-NaN values (callers never pass NaN: they only keep v > m).
__device__ __forceinline__ float BlockMax(float v, float* sh) {
  v = WaveMaxTo63(v);
  if ((threadIdx.x & 63) == 63) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, sh[w]);
  __syncthreads();
  return r;
}

// Sum in a fixed tree (the same in every workgroup and run): the wave's DPP
// tree, then the wave totals left to right.
__device__ __forceinline__ double BlockSumD(double v, double* sh) {
  v = WaveSumTo63(v);
  if ((threadIdx.x & 63) == 63) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r += sh[w];
  __syncthreads();
  return r;
}

// Exclusive prefix sum over the block in thread order; *total gets the sum.
__device__ __forceinline__ uint64_t BlockExclScan(uint64_t v, uint64_t* sh, uint64_t* total) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const uint64_t incl = WaveInclScanU64(v);
  if (lane == 63) sh[w] = incl;
  __syncthreads();
  uint64_t before = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    if (k < w) before += sh[k];
    tot += sh[k];
  }
  __syncthreads();
  *total = tot;
  return before + incl - v;
}

// ---------------------------------------------------------------- hand-off to the last workgroup

// Data that the last workgroup of the same launch reads crosses the XCDs'
// separate L2s: it is stored device-scope write-through (a relaxed agent-scope
// atomic store: a vector store with the sc1 policy), and the last workgroup
// takes an agent-scope acquire fence (invalidating its stale L1 / L2 lines)
// before its plain loads. kDev = false is the plain store, for data that a later
// launch reads (a kernel boundary orders it).
template <bool kDev, typename T>
__device__ __forceinline__ void St(T* p, T v) {
  if constexpr (kDev) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *p = v;
  }
}

// Called by every thread after its hand-off stores; returns true (uniformly) in
// the workgroup whose count arrives last, which puts the counter back to zero.
// Each wave waits for its stores to be acknowledged (device scope, so visible to
// every XCD) before the barrier ahead of the count, with no release fence (its
// L2 write-back costs more than the whole hand-off); the last workgroup takes an
// acquire fence after the barrier behind it. No workgroup waits for another.
// Measured against device-coherent (sc1) loads in the last workgroup instead of
// the fence: 1-1.6 us faster per hand-off.
__device__ bool ArriveLast(uint32_t* counter, int* flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before == gridDim.x - 1;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (*flag == 0) return false;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return true;
}

// Partials of all slices, reduced in one fixed order (identical in every workgroup).
__device__ float MaxOfParts(const float* parts, int n_slices, float* sh) {
  float m = -INFINITY;
  for (int g = threadIdx.x; g < n_slices; g += kThreads) m = fmaxf(m, parts[g]);
  return BlockMax(m, sh);
}
__device__ Best BestOfParts(const float* vals, const int32_t* idx, int n_slices, Best* sh) {
  Best b{-INFINITY, 0x7FFFFFFF};
  for (int g = threadIdx.x; g < n_slices; g += kThreads) b = Better(b, Best{vals[g], idx[g]});
  return BlockBest(b, sh);
}

// ---------------------------------------------------------------- radix digit selection

struct Pick {
  uint32_t digit;
  uint64_t carry;  // top_k: rank still to find within the digit; top_p: S below the digit
  int found;
};

// top_k: the largest digit d with count(digit >= d) >= rem; carry = rem - count(digit > d).
// Thread t owns bins [16t, 16t + 16).
template <int kNumBins>
__device__ Pick PickDescending(const uint32_t* hist, uint32_t rem, uint64_t* sh, Pick* pick) {
  constexpr int kPer = kNumBins / kThreads;
  uint32_t h[kPer];
  uint64_t s = 0;
#pragma unroll
  for (int b = 0; b < kPer; ++b) {
    h[b] = hist[threadIdx.x * kPer + b];
    s += h[b];
  }
  uint64_t total;
  const uint64_t below = BlockExclScan(s, sh, &total);
  const uint64_t above = total - below - s;  // bins of the threads after this one
  if (threadIdx.x == 0) *pick = Pick{0, 0, 0};
  __syncthreads();
  if (above < rem && rem <= above + s) {
    uint64_t acc = above;
    for (int b = kPer - 1; b >= 0; --b) {
      if (acc + h[b] >= rem) {
        *pick = Pick{static_cast<uint32_t>(threadIdx.x * kPer + b), rem - acc, 1};
        break;
      }
      acc += h[b];
    }
  }
  __syncthreads();
  const Pick r = *pick;
  __syncthreads();
  return r;
}

// top_p: the smallest digit d with base + sum(digit <= d) > thr; carry = base + sum(digit < d).
// *total_out (optional) gets the histogram's total.
template <int kNumBins>
__device__ Pick PickAscendingOf(const uint64_t (&h)[kNumBins / kThreads], uint64_t base, uint64_t thr, uint64_t* sh,
                                Pick* pick, uint64_t* total_out = nullptr) {
  constexpr int kPer = kNumBins / kThreads;
  uint64_t s = 0;
#pragma unroll
  for (int b = 0; b < kPer; ++b) s += h[b];
  uint64_t total;
  const uint64_t below = BlockExclScan(s, sh, &total);
  if (total_out != nullptr) *total_out = total;
  if (threadIdx.x == 0) *pick = Pick{0, 0, 0};
  __syncthreads();
  if (base + below <= thr && base + below + s > thr) {
    uint64_t acc = base + below;
    for (int b = 0; b < kPer; ++b) {
      if (acc + h[b] > thr) {
        *pick = Pick{static_cast<uint32_t>(threadIdx.x * kPer + b), acc, 1};
        break;
      }
      acc += h[b];
    }
  }
  __syncthreads();
  const Pick r = *pick;
  __syncthreads();
  return r;
}
template <int kNumBins>
__device__ Pick PickAscending(const uint64_t* hist, uint64_t base, uint64_t thr, uint64_t* sh, Pick* pick,
                              uint64_t* total_out = nullptr) {
  uint64_t h[kNumBins / kThreads];
#pragma unroll
  for (int b = 0; b < kNumBins / kThreads; ++b) h[b] = hist[threadIdx.x * (kNumBins / kThreads) + b];
  return PickAscendingOf<kNumBins>(h, base, thr, sh, pick, total_out);
}



// ---------------------------------------------------------------- value pipeline

struct Logits {
  const float* x;
  int64_t n;
  float inv_t;  // 1 / temperature
  int scale;    // temperature != 1
};

__device__ __forceinline__ float ScaleV(const Logits& lg, float raw) { return lg.scale ? raw * lg.inv_t : raw; }
__device__ __forceinline__ float LoadV(const Logits& lg, int64_t i) { return ScaleV(lg, lg.x[i]); }

struct ProbCtx {
  float mx;
  float inv;
  float kth;
  int topk;
};

__device__ __forceinline__ float MaskV(const ProbCtx& c, float v) { return (c.topk && v < c.kth) ? -INFINITY : v; }
__device__ __forceinline__ float MaskedV(const Logits& lg, const ProbCtx& c, int64_t i) {
  return MaskV(c, LoadV(lg, i));
}
// p of a raw logit (the one formula every pass uses)
__device__ __forceinline__ float ProbOfRaw(const Logits& lg, const ProbCtx& c, float raw) {
  return expf(MaskV(c, ScaleV(lg, raw)) - c.mx) * c.inv;
}
__device__ __forceinline__ float ProbAt(const Logits& lg, const ProbCtx& c, int64_t i) {
  return ProbOfRaw(lg, c, lg.x[i]);
}

__device__ __forceinline__ int NumSlices(int64_t n) { return static_cast<int>((n + kSlice - 1) / kSlice); }
__device__ __forceinline__ int64_t ElemIndex(int j) {
  return static_cast<int64_t>(blockIdx.x) * kSlice + threadIdx.x + j * kThreads;
}


// ---------------------------------------------------------------- kernels

// Per-slice max and first argmax of the (scaled) logits; with top_k also the
// level-1 count histogram of their keys (bits 31..20), added to khist; without
// top_k also the slice's sum of expf(v - m) against its own maximum m (the
// softmax normaliser then combines the slices, LoadProbCtx, and needs no launch
// of its own).
__global__ __launch_bounds__(kThreads) void SamplePrepKernel(Logits lg, int32_t topk, SampleScratch* __restrict__ s) {
  __shared__ uint32_t hist[kBins];
  __shared__ Best shb[kWaves];
  __shared__ double shd[kWaves];
  if (topk) {
    for (int b = threadIdx.x; b < kBins; b += kThreads) hist[b] = 0;
    __syncthreads();
  }
  Best b{-INFINITY, 0x7FFFFFFF};
  float v[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    v[j] = -INFINITY;
    if (i < lg.n) {
      v[j] = LoadV(lg, i);
      if (v[j] > b.v || (v[j] == b.v && b.i == 0x7FFFFFFF)) b = Best{v[j], static_cast<int32_t>(i)};
      if (topk) atomicAdd(&hist[OrderKey(v[j]) >> LevelShift(1)], 1u);
    }
  }
  b = BlockBest(b, shb);
  if (!topk) {
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      if (v[j] != -INFINITY) acc += static_cast<double>(expf(v[j] - b.v));
    }
    acc = BlockSumD(acc, shd);
    if (threadIdx.x == 0) s->sum_part[blockIdx.x] = acc;
  }
  if (threadIdx.x == 0) {
    s->max_part[blockIdx.x] = b.v;
    s->best_val[blockIdx.x] = b.v;
    s->best_idx[blockIdx.x] = b.i;
  }
  if (topk) {
    __syncthreads();
    for (int k = threadIdx.x; k < kBins; k += kThreads) {
      if (hist[k] != 0) atomicAdd(&s->khist[k], hist[k]);
    }
  }
}

// Stores this workgroup's elements that pass `match` in its slice's region of
// the candidate list, and their number in cand_count (both device-coherent, for
// the last workgroup).
template <typename F>
__device__ void StoreCandidates(const uint32_t (&key)[kPerThread], const uint64_t (&w)[kPerThread], F match,
                                bool with_w, SampleScratch* s, SampleCandidates* cand, uint64_t* sh) {
  uint64_t cnt = 0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) cnt += match(j) ? 1 : 0;
  uint64_t total;
  uint32_t at = static_cast<uint32_t>(blockIdx.x) * kSlice + static_cast<uint32_t>(BlockExclScan(cnt, sh, &total));
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    if (match(j)) {
      St<true>(&cand->key[at], key[j]);
      if (with_w) St<true>(&cand->w[at], w[j]);
      ++at;
    }
  }
  if (threadIdx.x == 0) St<true>(&s->cand_count[blockIdx.x], static_cast<uint32_t>(total));
}

// In the last workgroup: where each slice's candidates start in the compacted
// (slice-order) list, into lstart; returns the number of candidates. When they
// fit in LDS (kCap) they are copied there, keys to lkey and (kWithW) weights to
// lw; otherwise every level reads them from their slices' regions.
constexpr int kTopKCandLds = 8192;  // keys: 32 KB of LDS
constexpr int kTopPCandLds = 4096;  // keys and weights: 48 KB
__device__ __forceinline__ int SliceOf(const uint32_t* lstart, int n_slices, uint32_t i) {
  int lo = 0, hi = n_slices - 1;  // the largest g with lstart[g] <= i
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (lstart[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return lo;
}
template <bool kWithW, int kCap>
__device__ uint32_t GatherCandidates(const SampleScratch* s, const SampleCandidates* cand, int n_slices,
                                     uint32_t* lkey, uint64_t* lw, uint32_t* lstart, uint64_t* sh) {
  // thread t owns slices [t * kPartsPerThread, ...)
  uint32_t cnt[kPartsPerThread];
  uint64_t mine = 0;
#pragma unroll
  for (int k = 0; k < kPartsPerThread; ++k) {
    const int g = threadIdx.x * kPartsPerThread + k;
    cnt[k] = g < n_slices ? s->cand_count[g] : 0u;
    mine += cnt[k];
  }
  uint64_t total;
  uint64_t at = BlockExclScan(mine, sh, &total);
#pragma unroll
  for (int k = 0; k < kPartsPerThread; ++k) {
    const int g = threadIdx.x * kPartsPerThread + k;
    if (g < n_slices) lstart[g] = static_cast<uint32_t>(at);
    at += cnt[k];
  }
  __syncthreads();
  const uint32_t n_c = static_cast<uint32_t>(total);
  if (n_c <= kCap) {
    // every address first, then every load in flight at once, then the LDS copies
    constexpr int kItems = kCap / kThreads;
    uint32_t at_g[kItems];
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
      const uint32_t i = threadIdx.x + static_cast<uint32_t>(r) * kThreads;
      if (i < n_c) {
        const int g = SliceOf(lstart, n_slices, i);
        at_g[r] = static_cast<uint32_t>(g) * kSlice + (i - lstart[g]);
      }
    }
    uint32_t kv[kItems];
    uint64_t wv[kWithW ? kItems : 1];
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
      if (threadIdx.x + static_cast<uint32_t>(r) * kThreads < n_c) {
        kv[r] = cand->key[at_g[r]];
        if constexpr (kWithW) wv[r] = cand->w[at_g[r]];
      }
    }
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
      const uint32_t i = threadIdx.x + static_cast<uint32_t>(r) * kThreads;
      if (i < n_c) {
        lkey[i] = kv[r];
        if constexpr (kWithW) lw[i] = wv[r];
      }
    }
    __syncthreads();
  }
  return n_c;
}
// Candidate i of the compacted list: from LDS when it was copied there, else
// from its slice's region.
template <bool kWithW, int kCap>
__device__ __forceinline__ void CandidateAt(uint32_t i, uint32_t n_c, const uint32_t* lkey, const uint64_t* lw,
                                            const uint32_t* lstart, int n_slices, const SampleCandidates* cand,
                                            uint32_t* key, uint64_t* w) {
  if (n_c <= kCap) {
    *key = lkey[i];
    if (kWithW) *w = lw[i];
  } else {
    const int g = SliceOf(lstart, n_slices, i);
    const uint32_t at_g = static_cast<uint32_t>(g) * kSlice + (i - lstart[g]);
    *key = cand->key[at_g];
    if (kWithW) *w = cand->w[at_g];
  }
}

// top_k, levels 2 and 3: every workgroup picks level 1's digit from khist (the
// same data in every workgroup, so the same digit) and stores its keys with that
// digit; the last workgroup selects bits 19..8 and 7..0 among them in LDS,
// stores the threshold key and clears khist for the next call.
__global__ __launch_bounds__(kThreads) void SampleTopKCandKernel(Logits lg, int32_t top_k,
                                                                 SampleScratch* __restrict__ s,
                                                                 SampleCandidates* __restrict__ cand) {
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t lstart[kMaxSlices];
  __shared__ uint32_t lkey[kTopKCandLds];
  __shared__ uint64_t sh[kWaves];
  __shared__ Pick pick;
  __shared__ int last;
  uint32_t key[kPerThread];
  uint64_t none[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {  // requested before the pick's histogram reads
    const int64_t i = ElemIndex(j);
    key[j] = i < lg.n ? OrderKey(LoadV(lg, i)) : 0u;
    none[j] = 0;
  }
  const Pick p1 = PickDescending<kBins>(s->khist, static_cast<uint32_t>(top_k), sh, &pick);
  auto match = [&](int j) { return ElemIndex(j) < lg.n && (key[j] >> LevelShift(1)) == p1.digit; };
  StoreCandidates(key, none, match, false, s, cand, sh);
  if (!ArriveLast(&s->arrive[kArriveTopK][0], &last)) return;

  const int ns = static_cast<int>(gridDim.x);
  const uint32_t n_c = GatherCandidates<false, kTopKCandLds>(s, cand, ns, lkey, nullptr, lstart, sh);
  uint32_t prefix = p1.digit;
  uint32_t rem = static_cast<uint32_t>(p1.carry);
#pragma unroll
  for (int level = 2; level <= 3; ++level) {
    const int shift = LevelShift(level);
    const uint32_t mask = (1u << LevelBits(level)) - 1u;
    const int above = shift + LevelBits(level);
    for (int b = threadIdx.x; b < kBins; b += kThreads) hist[b] = 0;
    __syncthreads();
    if (n_c <= kTopKCandLds) {  // uniform: the LDS copy, read through an LDS address
      for (uint32_t c = threadIdx.x; c < n_c; c += kThreads) {
        const uint32_t k = lkey[c];
        if ((k >> above) == prefix) atomicAdd(&hist[(k >> shift) & mask], 1u);
      }
    } else {
      for (uint32_t c = threadIdx.x; c < n_c; c += kThreads) {
        uint32_t k;
        CandidateAt<false, kTopKCandLds>(c, n_c, lkey, nullptr, lstart, ns, cand, &k, nullptr);
        if ((k >> above) == prefix) atomicAdd(&hist[(k >> shift) & mask], 1u);
      }
    }
    __syncthreads();
    const Pick p = level == 3 ? PickDescending<256>(hist, rem, sh, &pick) : PickDescending<kBins>(hist, rem, sh, &pick);
    prefix = (prefix << LevelBits(level)) | p.digit;
    rem = static_cast<uint32_t>(p.carry);
  }
  if (threadIdx.x == 0) s->kth_key = prefix;
  for (int b = threadIdx.x; b < kBins; b += kThreads) s->khist[b] = 0;
}

// mx, inv and kth as every kernel after Sum sees them.
__device__ ProbCtx LoadProbCtx(const Logits& lg, int topk, const SampleScratch* s, float* shf, double* shd) {
  const int ns = NumSlices(lg.n);
  // both partials of a thread's slices requested at once (one memory round trip),
  // then the maximum and the normaliser: with top_k the slices' sums, otherwise
  // sum_g sum_part[g] exp(m_g - mx) over the slices' own maxima m_g (a slice of
  // -inf maxima adds its own sum, 0 or NaN); each term then differs from a direct
  // sum of expf(v - mx) by float rounding of the exponentials only (~1e-7)
  float mp[kPartsPerThread];
  double sp[kPartsPerThread];
#pragma unroll
  for (int k = 0; k < kPartsPerThread; ++k) {
    const int g = threadIdx.x + k * kThreads;
    mp[k] = g < ns ? s->max_part[g] : -INFINITY;
    sp[k] = g < ns ? s->sum_part[g] : 0.0;
  }
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPartsPerThread; ++k) m = fmaxf(m, mp[k]);
  ProbCtx c;
  c.mx = BlockMax(m, shf);
  // without top_k the slices' sums were taken against their own maxima (SamplePrepKernel)
  double t = 0.0;
#pragma unroll
  for (int k = 0; k < kPartsPerThread; ++k) {
    if (threadIdx.x + k * kThreads < ns) {
      t += (topk || mp[k] == -INFINITY) ? sp[k]
                                         : sp[k] * exp(static_cast<double>(mp[k]) - static_cast<double>(c.mx));
    }
  }
  c.inv = static_cast<float>(1.0 / BlockSumD(t, shd));
  c.topk = topk;
  c.kth = topk ? FromOrderKey(s->kth_key) : 0.0f;
  return c;
}

// Per-slice sum of e = expf(v - mx) (top_k's threshold applied).
__global__ __launch_bounds__(kThreads) void SampleSumKernel(Logits lg, int32_t topk, SampleScratch* __restrict__ s) {
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  ProbCtx c;
  c.mx = MaxOfParts(s->max_part, NumSlices(lg.n), shf);
  c.inv = 1.0f;
  c.topk = topk;
  c.kth = topk ? FromOrderKey(s->kth_key) : 0.0f;
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) acc += static_cast<double>(expf(MaskedV(lg, c, i) - c.mx));
  }
  acc = BlockSumD(acc, shd);
  if (threadIdx.x == 0) s->sum_part[blockIdx.x] = acc;
}

// top_p level 1: sum of Fix62(p) per key digit (bits 31..20), added to phist.
__global__ __launch_bounds__(kThreads) void SampleTopPKernel(Logits lg, int32_t topk, SampleScratch* __restrict__ s) {
  __shared__ uint64_t hist[kBins];
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  float raw[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {  // requested before the partials
    const int64_t i = ElemIndex(j);
    raw[j] = i < lg.n ? lg.x[i] : 0.0f;
  }
  for (int b = threadIdx.x; b < kBins; b += kThreads) hist[b] = 0;
  const ProbCtx c = LoadProbCtx(lg, topk, s, shf, shd);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) {
      const float p = ProbOfRaw(lg, c, raw[j]);
      const uint64_t w = Fix62(p);
      if (w != 0) atomicAdd(reinterpret_cast<unsigned long long*>(&hist[OrderKey(p) >> LevelShift(1)]),
                            static_cast<unsigned long long>(w));
    }
  }
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += kThreads) {
    if (hist[b] != 0)
      atomicAdd(reinterpret_cast<unsigned long long*>(&s->phist[b]), static_cast<unsigned long long>(hist[b]));
  }
}

// top_p, levels 2 and 3 and the cut: every workgroup picks level 1's digit (the
// smallest with S > thr) from phist and stores its (key, weight) pairs with
// that digit; the last workgroup selects bits 19..8 and 7..0 among them in LDS,
// which completes K* (the smallest key with S(K*) > thr), stores cut_key =
// K* - 1 and the weight of the keys above the cut (the total less S below K*),
// and clears phist for the next call. S never exceeding thr (no level-1 digit)
// means no cut.
__global__ __launch_bounds__(kThreads) void SampleTopPCandKernel(Logits lg, int32_t topk, uint64_t thr,
                                                                 SampleScratch* __restrict__ s,
                                                                 SampleCandidates* __restrict__ cand) {
  __shared__ uint64_t hist[kBins];
  __shared__ uint32_t lstart[kMaxSlices];
  __shared__ uint32_t lkey[kTopPCandLds];
  __shared__ uint64_t lw[kTopPCandLds];
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Pick pick;
  __shared__ int last;
  float v[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {  // requested before the partials and the histogram
    const int64_t i = ElemIndex(j);
    v[j] = i < lg.n ? lg.x[i] : 0.0f;
  }
  // the thread's level-1 bins, requested with the logits (before the barriers of
  // the partials' reductions, which would otherwise hold these loads back)
  uint64_t h1[kBins / kThreads];
#pragma unroll
  for (int b = 0; b < kBins / kThreads; ++b) h1[b] = s->phist[threadIdx.x * (kBins / kThreads) + b];
  const ProbCtx c = LoadProbCtx(lg, topk, s, shf, shd);
  uint64_t total = 0;
  const Pick p1 = PickAscendingOf<kBins>(h1, 0ull, thr, sh, &pick, &total);
  uint32_t key[kPerThread];
  uint64_t w[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const float p = ElemIndex(j) < lg.n ? ProbOfRaw(lg, c, v[j]) : 0.0f;
    key[j] = OrderKey(p);
    w[j] = Fix62(p);
  }
  auto match = [&](int j) {
    return p1.found && ElemIndex(j) < lg.n && w[j] != 0 && (key[j] >> LevelShift(1)) == p1.digit;
  };
  StoreCandidates(key, w, match, true, s, cand, sh);
  if (!ArriveLast(&s->arrive[kArriveTopP][0], &last)) return;

  uint32_t cut_key = 0xFFFFFFFFu;  // no cut
  uint64_t kept = total;
  if (p1.found) {
    const int ns = static_cast<int>(gridDim.x);
    const uint32_t n_c = GatherCandidates<true, kTopPCandLds>(s, cand, ns, lkey, lw, lstart, sh);
    uint32_t prefix = p1.digit;
    uint64_t base = p1.carry;
    bool found = true;
#pragma unroll
    for (int level = 2; level <= 3; ++level) {
      const int shift = LevelShift(level);
      const uint32_t mask = (1u << LevelBits(level)) - 1u;
      const int above = shift + LevelBits(level);
      for (int b = threadIdx.x; b < kBins; b += kThreads) hist[b] = 0;
      __syncthreads();
      if (n_c <= kTopPCandLds) {  // uniform: the LDS copy, read through LDS addresses
        for (uint32_t k = threadIdx.x; k < n_c; k += kThreads) {
          const uint32_t ck = lkey[k];
          if ((ck >> above) == prefix)
            atomicAdd(reinterpret_cast<unsigned long long*>(&hist[(ck >> shift) & mask]),
                      static_cast<unsigned long long>(lw[k]));
        }
      } else {
        for (uint32_t k = threadIdx.x; k < n_c; k += kThreads) {
          uint32_t ck;
          uint64_t cw;
          CandidateAt<true, kTopPCandLds>(k, n_c, lkey, lw, lstart, ns, cand, &ck, &cw);
          if ((ck >> above) == prefix)
            atomicAdd(reinterpret_cast<unsigned long long*>(&hist[(ck >> shift) & mask]),
                      static_cast<unsigned long long>(cw));
        }
      }
      __syncthreads();
      const Pick p = level == 3 ? PickAscending<256>(hist, base, thr, sh, &pick)
                                : PickAscending<kBins>(hist, base, thr, sh, &pick);
      found = found && p.found;
      prefix = (prefix << LevelBits(level)) | p.digit;
      base = p.carry;
    }
    if (found) {  // always, given level 1's digit: its candidates carry S past thr
      cut_key = prefix - 1u;
      kept = total - base;
    }
  }
  if (threadIdx.x == 0) {
    s->cut_key = cut_key;
    s->kept_w = kept;
  }
  for (int b = threadIdx.x; b < kBins; b += kThreads) s->phist[b] = 0;
}

// Per-slice inverse-transform partials of probs: Fix52 sum and the double sum
// (NaN when a value is outside [0, 2), which sends the transform to the serial loop).
template <bool kDev>
__device__ void WriteFixPartials(const float (&p)[kPerThread], const bool (&in)[kPerThread], SampleScratch* s,
                                 double* shd, uint64_t* sh) {
  uint64_t f = 0;
  double t = 0.0;
  bool ok = true;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    if (in[j]) {
      ok = ok && Fix52Valid(p[j]);
      f += Fix52(p[j]);
      t += static_cast<double>(p[j]);
    }
  }
  uint64_t ftot;
  (void)BlockExclScan(f, sh, &ftot);
  t = BlockSumD(ok ? t : NAN, shd);
  if (threadIdx.x == 0) {
    St<kDev>(&s->fix_part[blockIdx.x], ftot);
    St<kDev>(&s->tot_part[blockIdx.x], t);
  }
}

// Where the inverse transform takes u: the device counter when counter_dev is
// set, else u_val.
struct Draw {
  float u_val;
  uint64_t seed;
  const uint64_t* counter_dev;
  int32_t* out_idx;
};

// The draw with u resolved at kernel entry: the device counter is constant for
// the launch, so every workgroup reads it with its first loads and the last
// workgroup's inverse transform does not wait one more memory round trip for it.
__device__ __forceinline__ Draw ResolvedDraw(Draw d) {
  if (d.counter_dev != nullptr) {
    d.u_val = CounterUniformOf(d.seed, *d.counter_dev);
    d.counter_dev = nullptr;
    asm volatile("" ::"v"(d.u_val));  // formed here, not next to its use in the last workgroup
  }
  return d;
}

// The inverse transform over probs[0, n) by one workgroup, from the slices'
// Fix52 / double partials (in the last workgroup of the launch that wrote them,
// after ArriveLast's acquire fence, or in a later launch).
__device__ void InverseTransform(const float* __restrict__ probs, int64_t n, const Draw& d,
                                 const SampleScratch* __restrict__ s) {
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Best shb[kWaves];
  __shared__ float tile[kSlice];
  __shared__ int64_t hit;  // crossing index / slice, -1 none
  __shared__ uint64_t hit_lo, hit_hi;
  const float u = d.counter_dev != nullptr ? CounterUniformOf(d.seed, *d.counter_dev) : d.u_val;
  const int ns = static_cast<int>((n + kSlice - 1) / kSlice);

  // 1. slice totals: thread t owns slices [t * kPartsPerThread, ...)
  uint64_t f = 0;
  double t = 0.0;
  for (int k = 0; k < kPartsPerThread; ++k) {
    const int g = threadIdx.x * kPartsPerThread + k;
    if (g < ns) {
      f += s->fix_part[g];
      t += s->tot_part[g];
    }
  }
  const double tot = BlockSumD(t, shd);
  bool serial = !(tot < 4000.0);  // NaN / out-of-range values, or a fixed-point total that could overflow
  int64_t result = -1;
  if (!serial) {
    const uint64_t U = static_cast<uint64_t>(static_cast<double>(u) * 0x1p52);  // floor(u * 2^52)
    // serial-sum rounding (n * 2^-53 * max prefix) plus truncation (n * 2^-52), in 2^-52 units, with room
    const uint64_t margin = static_cast<uint64_t>(n) * (static_cast<uint64_t>(ceil(tot)) + 2ull) + 2ull;
    uint64_t ftot;
    uint64_t acc = BlockExclScan(f, sh, &ftot);
    if (threadIdx.x == 0) hit = -1;
    __syncthreads();
    for (int k = 0; k < kPartsPerThread; ++k) {
      const int g = threadIdx.x * kPartsPerThread + k;
      if (g < ns) {
        const uint64_t part = s->fix_part[g];
        if (acc <= U && U < acc + part) {
          hit = g;
          hit_lo = acc;
        }
        acc += part;
      }
    }
    __syncthreads();
    const int64_t g = hit;
    const uint64_t slice_lo = hit_lo;
    __syncthreads();
    if (g < 0) {
      // no prefix exceeds u: the serial loop also ends without a crossing when
      // the whole sum stays below u by the margin
      if (ftot + margin <= U) {
        result = -2;  // argmax fallback
      } else {
        serial = true;
      }
    } else {
      // 2. the crossing inside slice g: thread t owns elements 4t .. 4t + 3
      float p[kPerThread];
      uint64_t fs = 0;
#pragma unroll
      for (int j = 0; j < kPerThread; ++j) {
        const int64_t i = g * kSlice + threadIdx.x * kPerThread + j;
        p[j] = i < n ? probs[i] : 0.0f;
        fs += Fix52(p[j]);
      }
      uint64_t stot;
      uint64_t a = slice_lo + BlockExclScan(fs, sh, &stot);
      if (threadIdx.x == 0) hit = -1;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kPerThread; ++j) {
        const int64_t i = g * kSlice + threadIdx.x * kPerThread + j;
        const uint64_t fj = Fix52(p[j]);
        if (i < n && a <= U && U < a + fj) {
          hit = i;
          hit_lo = a;
          hit_hi = a + fj;
        }
        a += fj;
      }
      __syncthreads();
      const int64_t i = hit;
      const bool safe_hi = hit_hi > U + margin;               // serial sum at i exceeds u
      const bool safe_lo = i == 0 || hit_lo + margin <= U;   // serial sum before i does not
      __syncthreads();
      if (i >= 0 && safe_hi && safe_lo) {
        result = i;
      } else {
        serial = true;
      }
    }
  }

  if (serial) {
    // The reference loop itself: cum += (double)p in index order, first cum > u.
    // Tiles go through LDS so the one summing thread never waits on memory.
    if (threadIdx.x == 0) hit = -1;
    double cum = 0.0;
    const double ud = static_cast<double>(u);
    for (int64_t base = 0; base < n; base += kSlice) {
      __syncthreads();
      for (int j = threadIdx.x; j < kSlice; j += kThreads) tile[j] = base + j < n ? probs[base + j] : 0.0f;
      __syncthreads();
      if (threadIdx.x == 0) {
        const int m = n - base < kSlice ? static_cast<int>(n - base) : kSlice;
        for (int j = 0; j < m; ++j) {
          cum += static_cast<double>(tile[j]);
          if (cum > ud) {
            hit = base + j;
            break;
          }
        }
      }
      __syncthreads();
      if (hit >= 0) break;
    }
    result = hit >= 0 ? hit : -2;
  }

  if (result == -2) {
    // no crossing: the first maximum of probs, starting from probs[0]
    Best b{probs[0], 0};
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
      const float v = probs[i];
      if (v > b.v) b = Best{v, static_cast<int32_t>(i)};
    }
    b = BlockBest(b, shb);
    result = b.i;
  }
  if (threadIdx.x == 0) *d.out_idx = static_cast<int32_t>(result);
}

// Final probabilities: p = e * inv; with top_p the cut, the keep-one rule and
// the second normalisation (by the kept weight on the 2^-62 grid). Also the
// inverse-transform partials; with kSample the last workgroup then draws the
// token (probs and partials handed over device-coherent).
template <bool kSample>
__global__ __launch_bounds__(kThreads) void SampleNormKernel(Logits lg, int32_t topk, int32_t topp,
                                                             float* __restrict__ probs, SampleScratch* __restrict__ s,
                                                             Draw draw0) {
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Best shb[kWaves];
  __shared__ int last;
  const Draw draw = kSample ? ResolvedDraw(draw0) : draw0;
  __shared__ float best_raw;
  float raw[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {  // requested before the partials
    const int64_t i = ElemIndex(j);
    raw[j] = i < lg.n ? lg.x[i] : 0.0f;
  }
  // top_p's inputs requested with the logits, ahead of the partials' reductions
  // (whose barriers would otherwise hold each load back to a round trip of its
  // own): the cut, the kept weight, the slices' first maxima and the logit at
  // each thread's slice maximum (the block's argmax is one of them)
  const int ns = NumSlices(lg.n);
  uint32_t cut_key = 0;
  uint64_t kept_w = 0;
  Best bt{-INFINITY, 0x7FFFFFFF};
  float bt_raw = 0.0f;
  if (topp) {
    cut_key = s->cut_key;
    kept_w = s->kept_w;
    for (int g = threadIdx.x; g < ns; g += kThreads) bt = Better(bt, Best{s->best_val[g], s->best_idx[g]});
    if (bt.i >= 0 && bt.i < lg.n) bt_raw = lg.x[bt.i];
  }
  const ProbCtx c = LoadProbCtx(lg, topk, s, shf, shd);
  float cut = 0.0f, inv2 = 1.0f;
  bool forced = false, rescale = false;
  int32_t best = 0;
  if (topp) {
    cut = FromOrderKey(cut_key);  // NaN when there is no cut: nothing compares <= it
    const Best b = BlockBest(bt, shb);  // the first maximum of the scaled logits
    best = b.i;
    if (bt.i == b.i && b.i >= 0 && b.i < lg.n) best_raw = bt_raw;  // threads holding that index agree
    __syncthreads();
    // p is non-decreasing in the logit, so nothing survives the cut exactly when
    // the largest p does not: then the argmax is kept with 1 (no argmax: every
    // logit NaN)
    forced = best >= 0 && best < lg.n && ProbOfRaw(lg, c, best_raw) <= cut;
    const double sum2 = forced ? 1.0 : static_cast<double>(kept_w) * 0x1p-62;
    rescale = sum2 > 0.0;
    if (rescale) inv2 = static_cast<float>(1.0 / sum2);
  }
  float p[kPerThread];
  bool in[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    in[j] = i < lg.n;
    p[j] = 0.0f;
    if (in[j]) {
      float v = ProbOfRaw(lg, c, raw[j]);
      if (topp) {
        if (v <= cut) v = 0.0f;
        if (forced && i == best) v = 1.0f;
        if (rescale) v *= inv2;
      }
      p[j] = v;
      St<kSample>(probs + i, v);
    }
  }
  WriteFixPartials<kSample>(p, in, s, shd, sh);
  if constexpr (kSample) {
    if (ArriveLast(&s->arrive[kArriveFinal][0], &last)) InverseTransform(probs, lg.n, draw, s);
  }
}

// The inverse transform as a launch of its own (one workgroup), after a Norm
// launch without the draw.
__global__ __launch_bounds__(kThreads) void SampleInverseKernel(const float* __restrict__ probs, int64_t n,
                                                                const SampleScratch* __restrict__ s, Draw draw) {
  InverseTransform(probs, n, draw, s);
}

// Inverse-transform partials of caller-provided probabilities; the last
// workgroup then draws the token.
__global__ __launch_bounds__(kThreads) void SampleFixKernel(const float* __restrict__ probs, int64_t n,
                                                            SampleScratch* __restrict__ s, Draw draw0) {
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ int last;
  const Draw draw = ResolvedDraw(draw0);
  float p[kPerThread];
  bool in[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    in[j] = i < n;
    p[j] = in[j] ? probs[i] : 0.0f;
  }
  WriteFixPartials<true>(p, in, s, shd, sh);
  // probs came from the caller (ordered by the launch); only the partials cross workgroups
  if (ArriveLast(&s->arrive[kArriveFinal][0], &last)) InverseTransform(probs, n, draw, s);
}

// Per-slice argmax: values above `init` only, ties to the smaller index. With
// out_idx the last workgroup reduces the partials into it (GpuArgMax);
// otherwise a later launch reads them.
__global__ __launch_bounds__(kThreads) void ArgMaxPartKernel(const float* __restrict__ x, int64_t n, float init,
                                                             SampleScratch* __restrict__ s,
                                                             int32_t* __restrict__ out_idx) {
  __shared__ Best shb[kWaves];
  __shared__ int last;
  Best b{init, 0};
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < n) {
      const float v = x[i];
      if (v > b.v) b = Best{v, static_cast<int32_t>(i)};
    }
  }
  b = BlockBest(b, shb);
  if (out_idx == nullptr) {
    if (threadIdx.x == 0) {
      s->best_val[blockIdx.x] = b.v;
      s->best_idx[blockIdx.x] = b.i;
    }
    return;
  }
  if (threadIdx.x == 0) {
    St<true>(&s->best_val[blockIdx.x], b.v);
    St<true>(&s->best_idx[blockIdx.x], b.i);
  }
  if (!ArriveLast(&s->arrive[kArriveArgMax][0], &last)) return;
  const Best r = BestOfParts(s->best_val, s->best_idx, static_cast<int>(gridDim.x), shb);
  if (threadIdx.x == 0) *out_idx = r.i;
}

// Greedy FilterToProbs: one-hot at the argmax.
__global__ __launch_bounds__(kThreads) void OneHotKernel(int64_t n, float* __restrict__ probs,
                                                         const SampleScratch* __restrict__ s) {
  __shared__ Best shb[kWaves];
  const Best b = BestOfParts(s->best_val, s->best_idx, NumSlices(n), shb);
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < n) probs[i] = i == b.i ? 1.0f : 0.0f;
  }
}

// ---------------------------------------------------------------- scratch

// Library-owned, allocated once, never freed (a destructor running after the
// HIP runtime has shut down can hang). Grid-sized state lives here, so sampling
// allocates nothing after the first call or GpuSamplerWarmup.
struct SamplerBuffers {
  SampleScratch* s = nullptr;
  SampleCandidates* cand = nullptr;
};
std::mutex g_scratch_mu;
SamplerBuffers g_buffers;

SamplerBuffers Buffers() {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_buffers.s == nullptr) {
    RPG_CHECK(!StreamIsCapturing(),
              "the sampler's scratch block is allocated on first use, which cannot happen during graph capture; "
              "call GpuSamplerWarmup() before capturing");
    void* p = nullptr;
    void* c = nullptr;
    RPG_HIP_CHECK(hipMalloc(&p, sizeof(SampleScratch)));
    RPG_HIP_CHECK(hipMemset(p, 0, sizeof(SampleScratch)));  // outside capture (checked above): counters, histograms
    RPG_HIP_CHECK(hipMalloc(&c, sizeof(SampleCandidates)));
    RPG_HIP_CHECK(hipDeviceSynchronize());
    g_buffers.s = static_cast<SampleScratch*>(p);
    g_buffers.cand = static_cast<SampleCandidates*>(c);
  }
  return g_buffers;
}

void CheckVocab(int64_t n) {
  RPG_CHECK(n > 0, "sampler: empty vocabulary (n = %lld)", static_cast<long long>(n));
  RPG_CHECK(n <= kSamplerMaxVocab, "vocab size %lld exceeds the device sampler's limit %lld",
            static_cast<long long>(n), static_cast<long long>(kSamplerMaxVocab));
}

unsigned Slices(int64_t n) { return static_cast<unsigned>((n + kSlice - 1) / kSlice); }

// The token drawn by the last workgroup of the normalising launch rather than
// by a launch of its own.
constexpr bool kDrawInNorm = true;

// FilterToProbs launches for T > 0, then (draw.out_idx set) the token: Prep
// [-> TopKCand] -> Sum [-> TopP -> TopPCand] -> Norm, the last workgroup of Norm
// drawing the token.
void LaunchSample(const float* logits, int64_t n, const SampleOptions& opt, float* probs, const SamplerBuffers& b,
                  const Draw& draw) {
  const dim3 grid(Slices(n)), block(kThreads);
  Logits lg{logits, n, 1.0f / opt.temperature, opt.temperature != 1.0f ? 1 : 0};
  const int32_t topk = (opt.top_k > 1 && opt.top_k < n) ? 1 : 0;
  const int32_t topp = (opt.top_p > 0.0f && opt.top_p < 1.0f) ? 1 : 0;
  // S(t) <= 1 - top_p, on the 2^-62 grid of the weights
  const uint64_t thr = topp ? static_cast<uint64_t>(floor((1.0 - static_cast<double>(opt.top_p)) * 0x1p62)) : 0ull;
  Launch("SamplePrepKernel", SamplePrepKernel, grid, block, lg, topk, b.s);
  if (topk) Launch("SampleTopKCandKernel", SampleTopKCandKernel, grid, block, lg, opt.top_k, b.s, b.cand);
  if (topk) Launch("SampleSumKernel", SampleSumKernel, grid, block, lg, topk, b.s);  // else formed by Prep
  if (topp) {
    Launch("SampleTopPKernel", SampleTopPKernel, grid, block, lg, topk, b.s);
    Launch("SampleTopPCandKernel", SampleTopPCandKernel, grid, block, lg, topk, thr, b.s, b.cand);
  }
  if (draw.out_idx != nullptr && kDrawInNorm) {
    Launch("SampleNormKernel", SampleNormKernel<true>, grid, block, lg, topk, topp, probs, b.s, draw);
  } else {
    Launch("SampleNormKernel", SampleNormKernel<false>, grid, block, lg, topk, topp, probs, b.s, draw);
    if (draw.out_idx != nullptr) {
      Launch("SampleInverseKernel", SampleInverseKernel, dim3(1), block, static_cast<const float*>(probs), n, b.s,
             draw);
    }
  }
}

void CheckBuffers(const void* a, const void* b) {
  RPG_CHECK(a != nullptr && b != nullptr, "sampler: a probability buffer is null");
}

}  // namespace

// ---------------------------------------------------------------- public API

uint64_t DevSplitMix64(uint64_t x) { return SplitMix64Of(x); }
uint64_t DevCounterRng(uint64_t seed, uint64_t counter) { return CounterRngOf(seed, counter); }
float DevCounterUniform(uint64_t seed, uint64_t counter) { return CounterUniformOf(seed, counter); }

void GpuSamplerWarmup() { (void)Buffers(); }

void GpuArgMax(const float* x_dev, int64_t n, int32_t* out_idx_dev) {
  CheckBuffers(x_dev, out_idx_dev);
  CheckVocab(n);
  const SamplerBuffers b = Buffers();
  Launch("ArgMaxPartKernel", ArgMaxPartKernel, dim3(Slices(n)), dim3(kThreads), x_dev, n, -FLT_MAX, b.s,
         out_idx_dev);
}

void GpuFilterToProbs(const float* logits_dev, int64_t n, const SampleOptions& opt, float* probs_dev) {
  CheckBuffers(logits_dev, probs_dev);
  CheckVocab(n);
  const SamplerBuffers b = Buffers();
  if (!(opt.temperature > 0.0f)) {
    const dim3 grid(Slices(n)), block(kThreads);
    Launch("ArgMaxPartKernel", ArgMaxPartKernel, grid, block, logits_dev, n, -INFINITY, b.s,
           static_cast<int32_t*>(nullptr));
    Launch("OneHotKernel", OneHotKernel, grid, block, n, probs_dev, b.s);
    return;
  }
  LaunchSample(logits_dev, n, opt, probs_dev, b, Draw{0.0f, 0, nullptr, nullptr});
}

void GpuInverseSample(const float* probs_dev, int64_t n, float u, int32_t* out_idx_dev) {
  CheckBuffers(probs_dev, out_idx_dev);
  CheckVocab(n);
  RPG_CHECK(u >= 0.0f && u < 1.0f, "inverse sampling needs a uniform draw in [0, 1), got %g", static_cast<double>(u));
  RPG_CHECK(!StreamIsCapturing(),
            "GpuInverseSample takes u from the host and is therefore not capturable; use GpuSampleTokenDev inside a "
            "graph");
  const SamplerBuffers b = Buffers();
  Launch("SampleFixKernel", SampleFixKernel, dim3(Slices(n)), dim3(kThreads), probs_dev, n, b.s,
         Draw{u, 0, nullptr, out_idx_dev});
}

void GpuSampleToken(const float* logits_dev, int64_t n, const SampleOptions& opt, uint64_t seed, uint64_t counter,
                    float* probs_dev, int32_t* out_idx_dev) {
  if (!(opt.temperature > 0.0f)) {  // greedy consumes no random number
    GpuArgMax(logits_dev, n, out_idx_dev);
    return;
  }
  CheckBuffers(logits_dev, out_idx_dev);
  RPG_CHECK(probs_dev != nullptr, "sampler: a probability buffer is null");
  CheckVocab(n);
  RPG_CHECK(!StreamIsCapturing(),
            "GpuSampleToken takes the counter from the host and is therefore not capturable; use GpuSampleTokenDev "
            "inside a graph");
  LaunchSample(logits_dev, n, opt, probs_dev, Buffers(), Draw{CounterUniformOf(seed, counter), 0, nullptr, out_idx_dev});
}

void GpuSampleTokenDev(const float* logits_dev, int64_t n, const SampleOptions& opt, uint64_t seed,
                       const uint64_t* counter_dev, float* probs_dev, int32_t* out_idx_dev) {
  if (!(opt.temperature > 0.0f)) {
    GpuArgMax(logits_dev, n, out_idx_dev);
    return;
  }
  RPG_CHECK(counter_dev != nullptr, "sampler: counter_dev is null");
  CheckBuffers(logits_dev, out_idx_dev);
  RPG_CHECK(probs_dev != nullptr, "sampler: a probability buffer is null");
  CheckVocab(n);
  LaunchSample(logits_dev, n, opt, probs_dev, Buffers(), Draw{0.0f, seed, counter_dev, out_idx_dev});
}

}  // namespace rpg
