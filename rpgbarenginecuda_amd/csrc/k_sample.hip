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
//     keys with 12/12/8-bit digits: 3 passes instead of 32. Each workgroup
//     histograms its slice in LDS and adds the non-zero bins to a global
//     histogram; every workgroup of the next kernel picks the digit from it
//     (same data, same order, same answer) and workgroup 0 records the state;
//   * top_p's S(t) is summed as integers, p * 2^62 truncated, so the histogram
//     sums do not depend on the order of the atomics (they differ from the real
//     sums by less than n * 2^-62);
//   * values that couple slices (max, sums, argmax) travel as per-slice
//     partials that every workgroup of the next kernel reduces in one fixed
//     order, so every result is the same from run to run;
//   * the inverse transform keeps the serial double semantics exactly: a
//     fixed-point prefix (p * 2^52 truncated) over slices and then within one
//     slice finds the first index whose prefix exceeds u. The serial double sum
//     differs from the exact prefix by at most n * 2^-53 * max(prefix), so when
//     u is further than that (plus the truncation) from both neighbouring
//     prefixes the serial loop picks the same index. Otherwise (u within
//     ~1e-10 of a boundary) one thread runs the serial loop.
// Kernels, for T > 0 with top_p (the engine's default, top_k off):
//   Prep -> Sum -> TopP x3 -> Cut -> Norm -> Inverse (8 launches);
// top_k adds TopK x3 after Prep; without top_p the TopP and Cut kernels drop out.
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

// Radix levels: digit = (key >> shift) & (2^bits - 1); level L keeps only keys
// whose bits above its digit equal the prefix chosen by the levels before it.
__host__ __device__ constexpr int LevelShift(int level) { return level == 1 ? 20 : (level == 2 ? 8 : 0); }
__host__ __device__ constexpr int LevelBits(int level) { return level == 3 ? 8 : 12; }

struct KState {  // top_k select after a level: key prefix, rank still to find
  uint32_t prefix;
  uint32_t rem;
};
struct PState {  // top_p select after a level: key prefix, S below the prefix range, no-cut flag
  uint64_t prefix;
  uint64_t base;
  uint64_t none;
};

struct SampleScratch {
  float max_part[kMaxSlices];
  double sum_part[kMaxSlices];
  double sum2_part[kMaxSlices];
  float best_val[kMaxSlices];
  int32_t best_idx[kMaxSlices];
  uint64_t fix_part[kMaxSlices];
  double tot_part[kMaxSlices];
  uint32_t khist[3][kBins];
  uint64_t phist[3][kBins];
  KState kstate[4];  // index = level
  PState pstate[4];
  uint32_t kth_key;
  uint32_t cut_key;
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

// Maximum of non-NaN values (callers never pass NaN: they only keep v > m).
__device__ __forceinline__ float BlockMax(float v, float* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, sh[w]);
  __syncthreads();
  return r;
}

// Sum in a fixed tree: the butterfly gives every lane the same value
// (each pair adds the same two operands), then the wave totals left to right.
__device__ __forceinline__ double BlockSumD(double v, double* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
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
  uint64_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint64_t o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
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

// Partials of all slices, reduced in one fixed order (identical in every workgroup).
__device__ float MaxOfParts(const float* parts, int n_slices, float* sh) {
  float m = -INFINITY;
  for (int g = threadIdx.x; g < n_slices; g += kThreads) m = fmaxf(m, parts[g]);
  return BlockMax(m, sh);
}
__device__ double SumOfParts(const double* parts, int n_slices, double* sh) {
  double s = 0.0;
  for (int g = threadIdx.x; g < n_slices; g += kThreads) s += parts[g];
  return BlockSumD(s, sh);
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
template <int kNumBins>
__device__ Pick PickAscending(const uint64_t* hist, uint64_t base, uint64_t thr, uint64_t* sh, Pick* pick) {
  constexpr int kPer = kNumBins / kThreads;
  uint64_t h[kPer];
  uint64_t s = 0;
#pragma unroll
  for (int b = 0; b < kPer; ++b) {
    h[b] = hist[threadIdx.x * kPer + b];
    s += h[b];
  }
  uint64_t total;
  const uint64_t below = BlockExclScan(s, sh, &total);
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

template <typename F>
__device__ __forceinline__ auto PickLevel(int level, F&& f) {
  return level == 3 ? f(std::integral_constant<int, 256>{}) : f(std::integral_constant<int, kBins>{});
}

// ---------------------------------------------------------------- value pipeline

struct Logits {
  const float* x;
  int64_t n;
  float inv_t;  // 1 / temperature
  int scale;    // temperature != 1
};

__device__ __forceinline__ float LoadV(const Logits& lg, int64_t i) {
  const float v = lg.x[i];
  return lg.scale ? v * lg.inv_t : v;
}

struct ProbCtx {
  float mx;
  float inv;
  float kth;
  int topk;
};

__device__ __forceinline__ float MaskedV(const Logits& lg, const ProbCtx& c, int64_t i) {
  const float v = LoadV(lg, i);
  return (c.topk && v < c.kth) ? -INFINITY : v;
}
__device__ __forceinline__ float ProbAt(const Logits& lg, const ProbCtx& c, int64_t i) {
  return expf(MaskedV(lg, c, i) - c.mx) * c.inv;
}

__device__ __forceinline__ int NumSlices(int64_t n) { return static_cast<int>((n + kSlice - 1) / kSlice); }
__device__ __forceinline__ int64_t ElemIndex(int j) {
  return static_cast<int64_t>(blockIdx.x) * kSlice + threadIdx.x + j * kThreads;
}

// mx, inv and kth as every kernel after Sum sees them.
__device__ ProbCtx LoadProbCtx(const Logits& lg, int topk, const SampleScratch* s, float* shf, double* shd) {
  const int ns = NumSlices(lg.n);
  ProbCtx c;
  c.mx = MaxOfParts(s->max_part, ns, shf);
  c.inv = static_cast<float>(1.0 / SumOfParts(s->sum_part, ns, shd));
  c.topk = topk;
  c.kth = topk ? FromOrderKey(s->kth_key) : 0.0f;
  return c;
}

// ---------------------------------------------------------------- kernels

// Per-slice max of the (scaled) logits; zeroes the radix histograms.
__global__ __launch_bounds__(kThreads) void SamplePrepKernel(Logits lg, SampleScratch* __restrict__ s) {
  __shared__ float shf[kWaves];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) {
      const float v = LoadV(lg, i);
      if (v > m) m = v;
    }
  }
  m = BlockMax(m, shf);
  if (threadIdx.x == 0) s->max_part[blockIdx.x] = m;
  uint32_t* kh = &s->khist[0][0];
  uint64_t* ph = &s->phist[0][0];
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k < 3 * kBins;
       k += static_cast<int64_t>(gridDim.x) * kThreads) {
    kh[k] = 0;
    ph[k] = 0;
  }
}

// Resolves top_k's level (level - 1) digit (from the histogram of the previous
// kernel) and returns the key prefix after it; workgroup 0 records the state.
__device__ KState ResolveTopK(int level, int32_t top_k, SampleScratch* s, uint64_t* sh, Pick* pick) {
  const KState prev = level - 1 == 1 ? KState{0u, static_cast<uint32_t>(top_k)} : s->kstate[level - 2];
  const int lv = level - 1;
  const Pick p = PickLevel(lv, [&](auto nb) { return PickDescending<decltype(nb)::value>(s->khist[lv - 1], prev.rem, sh, pick); });
  const KState st{(prev.prefix << LevelBits(lv)) | p.digit, static_cast<uint32_t>(p.carry)};
  if (blockIdx.x == 0 && threadIdx.x == 0) s->kstate[lv] = st;
  return st;
}

// top_k level histogram (count of keys per digit among keys matching the prefix).
__global__ __launch_bounds__(kThreads) void SampleTopKKernel(Logits lg, int32_t top_k, int32_t level,
                                                             SampleScratch* __restrict__ s) {
  __shared__ uint32_t hist[kBins];
  __shared__ uint64_t sh[kWaves];
  __shared__ Pick pick;
  uint32_t prefix = 0;
  if (level > 1) prefix = ResolveTopK(level, top_k, s, sh, &pick).prefix;
  for (int b = threadIdx.x; b < kBins; b += kThreads) hist[b] = 0;
  __syncthreads();
  const int shift = LevelShift(level);
  const uint32_t mask = (1u << LevelBits(level)) - 1u;
  const int above = shift + LevelBits(level);
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) {
      const uint32_t key = OrderKey(LoadV(lg, i));
      if (level == 1 || (key >> above) == prefix) atomicAdd(&hist[(key >> shift) & mask], 1u);
    }
  }
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += kThreads) {
    if (hist[b] != 0) atomicAdd(&s->khist[level - 1][b], hist[b]);
  }
}

// Per-slice sum of e = expf(v - mx) (resolving top_k's threshold first).
__global__ __launch_bounds__(kThreads) void SampleSumKernel(Logits lg, int32_t topk, int32_t top_k,
                                                            SampleScratch* __restrict__ s) {
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Pick pick;
  ProbCtx c;
  c.mx = MaxOfParts(s->max_part, NumSlices(lg.n), shf);
  c.inv = 1.0f;
  c.topk = topk;
  c.kth = 0.0f;
  if (topk) {
    const KState st = ResolveTopK(4, top_k, s, sh, &pick);  // level 3's digit completes the key
    c.kth = FromOrderKey(st.prefix);
    if (blockIdx.x == 0 && threadIdx.x == 0) s->kth_key = st.prefix;
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) acc += static_cast<double>(expf(MaskedV(lg, c, i) - c.mx));
  }
  acc = BlockSumD(acc, shd);
  if (threadIdx.x == 0) s->sum_part[blockIdx.x] = acc;
}

// Resolves top_p's level (level - 1) digit; workgroup 0 records the state.
__device__ PState ResolveTopP(int level, uint64_t thr, SampleScratch* s, uint64_t* sh, Pick* pick) {
  const PState prev = level - 1 == 1 ? PState{0ull, 0ull, 0ull} : s->pstate[level - 2];
  const int lv = level - 1;
  PState st = prev;
  if (!prev.none) {
    const Pick p =
        PickLevel(lv, [&](auto nb) { return PickAscending<decltype(nb)::value>(s->phist[lv - 1], prev.base, thr, sh, pick); });
    if (p.found) {
      st = PState{(prev.prefix << LevelBits(lv)) | p.digit, p.carry, 0ull};
    } else {
      st = PState{0ull, 0ull, 1ull};  // S never exceeds the threshold: no cut
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) s->pstate[lv] = st;
  return st;
}

// top_p level histogram: sum of Fix62(p) per digit among keys matching the prefix.
__global__ __launch_bounds__(kThreads) void SampleTopPKernel(Logits lg, int32_t topk, uint64_t thr, int32_t level,
                                                             SampleScratch* __restrict__ s) {
  __shared__ uint64_t hist[kBins];
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Pick pick;
  const ProbCtx c = LoadProbCtx(lg, topk, s, shf, shd);
  uint64_t prefix = 0;
  if (level > 1) {
    const PState st = ResolveTopP(level, thr, s, sh, &pick);
    if (st.none) return;  // uniform across the grid: every workgroup resolved the same state
    prefix = st.prefix;
  }
  for (int b = threadIdx.x; b < kBins; b += kThreads) hist[b] = 0;
  __syncthreads();
  const int shift = LevelShift(level);
  const uint32_t mask = (1u << LevelBits(level)) - 1u;
  const int above = shift + LevelBits(level);
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) {
      const float p = ProbAt(lg, c, i);
      const uint32_t key = OrderKey(p);
      if (level == 1 || (key >> above) == prefix) {
        const uint64_t w = Fix62(p);
        if (w != 0) atomicAdd(reinterpret_cast<unsigned long long*>(&hist[(key >> shift) & mask]),
                              static_cast<unsigned long long>(w));
      }
    }
  }
  __syncthreads();
  for (int b = threadIdx.x; b < kBins; b += kThreads) {
    if (hist[b] != 0)
      atomicAdd(reinterpret_cast<unsigned long long*>(&s->phist[level - 1][b]), static_cast<unsigned long long>(hist[b]));
  }
}

// Applies top_p's cut: per-slice argmax (from -inf) and double sum of what is left.
__global__ __launch_bounds__(kThreads) void SampleCutKernel(Logits lg, int32_t topk, uint64_t thr,
                                                            SampleScratch* __restrict__ s) {
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Best shb[kWaves];
  __shared__ Pick pick;
  const ProbCtx c = LoadProbCtx(lg, topk, s, shf, shd);
  const PState st = ResolveTopP(4, thr, s, sh, &pick);  // level 3's digit completes the key K*
  // cut = the largest key with S <= thr, i.e. K* - 1; no K* means no cut (NaN compares false)
  const uint32_t cut_key = st.none ? 0xFFFFFFFFu : static_cast<uint32_t>(st.prefix) - 1u;
  if (blockIdx.x == 0 && threadIdx.x == 0) s->cut_key = cut_key;
  const float cut = FromOrderKey(cut_key);
  Best b{-INFINITY, 0};
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    if (i < lg.n) {
      float p = ProbAt(lg, c, i);
      if (p <= cut) p = 0.0f;
      if (p > b.v) b = Best{p, static_cast<int32_t>(i)};
      acc += static_cast<double>(p);
    }
  }
  b = BlockBest(b, shb);
  acc = BlockSumD(acc, shd);
  if (threadIdx.x == 0) {
    s->best_val[blockIdx.x] = b.v;
    s->best_idx[blockIdx.x] = b.i;
    s->sum2_part[blockIdx.x] = acc;
  }
}

// Per-slice inverse-transform partials of probs: Fix52 sum and the double sum
// (NaN when a value is outside [0, 2), which sends the transform to the serial loop).
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
    s->fix_part[blockIdx.x] = ftot;
    s->tot_part[blockIdx.x] = t;
  }
}

// Final probabilities: p = e * inv; with top_p the cut, the keep-one rule and
// the second normalisation. Also the inverse-transform partials.
__global__ __launch_bounds__(kThreads) void SampleNormKernel(Logits lg, int32_t topk, int32_t topp,
                                                             float* __restrict__ probs, SampleScratch* __restrict__ s) {
  __shared__ float shf[kWaves];
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Best shb[kWaves];
  const ProbCtx c = LoadProbCtx(lg, topk, s, shf, shd);
  float cut = 0.0f, inv2 = 1.0f;
  bool forced = false, rescale = false;
  int32_t best = 0;
  if (topp) {
    const int ns = NumSlices(lg.n);
    cut = FromOrderKey(s->cut_key);
    const Best b = BestOfParts(s->best_val, s->best_idx, ns, shb);
    best = b.i;
    forced = b.v == 0.0f;  // nothing survived the cut: the argmax is kept with 1
    const double sum2 = SumOfParts(s->sum2_part, ns, shd) + (forced ? 1.0 : 0.0);
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
      float v = ProbAt(lg, c, i);
      if (topp) {
        if (v <= cut) v = 0.0f;
        if (forced && i == best) v = 1.0f;
        if (rescale) v *= inv2;
      }
      p[j] = v;
      probs[i] = v;
    }
  }
  WriteFixPartials(p, in, s, shd, sh);
}

// Inverse-transform partials of caller-provided probabilities.
__global__ __launch_bounds__(kThreads) void SampleFixKernel(const float* __restrict__ probs, int64_t n,
                                                            SampleScratch* __restrict__ s) {
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  float p[kPerThread];
  bool in[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t i = ElemIndex(j);
    in[j] = i < n;
    p[j] = in[j] ? probs[i] : 0.0f;
  }
  WriteFixPartials(p, in, s, shd, sh);
}

// The inverse transform (one workgroup). u comes from the device counter when
// counter_dev is set, else from u_val.
__global__ __launch_bounds__(kThreads) void SampleInverseKernel(const float* __restrict__ probs, int64_t n, float u_val,
                                                                uint64_t seed, const uint64_t* __restrict__ counter_dev,
                                                                int32_t* __restrict__ out_idx,
                                                                const SampleScratch* __restrict__ s) {
  __shared__ double shd[kWaves];
  __shared__ uint64_t sh[kWaves];
  __shared__ Best shb[kWaves];
  __shared__ float tile[kSlice];
  __shared__ int64_t hit;  // crossing index / slice, -1 none
  __shared__ uint64_t hit_lo, hit_hi;
  const float u = counter_dev != nullptr ? CounterUniformOf(seed, *counter_dev) : u_val;
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
  if (threadIdx.x == 0) *out_idx = static_cast<int32_t>(result);
}

// Per-slice argmax: values above `init` only, ties to the smaller index.
__global__ __launch_bounds__(kThreads) void ArgMaxPartKernel(const float* __restrict__ x, int64_t n, float init,
                                                             SampleScratch* __restrict__ s) {
  __shared__ Best shb[kWaves];
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
  if (threadIdx.x == 0) {
    s->best_val[blockIdx.x] = b.v;
    s->best_idx[blockIdx.x] = b.i;
  }
}

// GpuArgMax's result from the slice partials (one workgroup).
__global__ __launch_bounds__(kThreads) void ArgMaxFinalKernel(int64_t n, int32_t* __restrict__ out_idx,
                                                              const SampleScratch* __restrict__ s) {
  __shared__ Best shb[kWaves];
  const Best b = BestOfParts(s->best_val, s->best_idx, static_cast<int>((n + kSlice - 1) / kSlice), shb);
  if (threadIdx.x == 0) *out_idx = b.i;
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
std::mutex g_scratch_mu;
SampleScratch* g_scratch = nullptr;

SampleScratch* Scratch() {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch == nullptr) {
    RPG_CHECK(!StreamIsCapturing(),
              "the sampler's scratch block is allocated on first use, which cannot happen during graph capture; "
              "call GpuSamplerWarmup() before capturing");
    void* p = nullptr;
    RPG_HIP_CHECK(hipMalloc(&p, sizeof(SampleScratch)));
    RPG_HIP_CHECK(hipMemset(p, 0, sizeof(SampleScratch)));  // outside capture (checked above)
    g_scratch = static_cast<SampleScratch*>(p);
  }
  return g_scratch;
}

void CheckVocab(int64_t n) {
  RPG_CHECK(n > 0, "sampler: empty vocabulary (n = %lld)", static_cast<long long>(n));
  RPG_CHECK(n <= kSamplerMaxVocab, "vocab size %lld exceeds the device sampler's limit %lld",
            static_cast<long long>(n), static_cast<long long>(kSamplerMaxVocab));
}

unsigned Slices(int64_t n) { return static_cast<unsigned>((n + kSlice - 1) / kSlice); }

// FilterToProbs launches (T > 0 or greedy); returns nothing, writes probs.
void LaunchFilter(const float* logits, int64_t n, const SampleOptions& opt, float* probs, SampleScratch* s) {
  const dim3 grid(Slices(n)), block(kThreads);
  if (!(opt.temperature > 0.0f)) {
    Launch("ArgMaxPartKernel", ArgMaxPartKernel, grid, block, logits, n, -INFINITY, s);
    Launch("OneHotKernel", OneHotKernel, grid, block, n, probs, s);
    return;
  }
  Logits lg{logits, n, 1.0f / opt.temperature, opt.temperature != 1.0f ? 1 : 0};
  const int32_t topk = (opt.top_k > 1 && opt.top_k < n) ? 1 : 0;
  const int32_t topp = (opt.top_p > 0.0f && opt.top_p < 1.0f) ? 1 : 0;
  // S(t) <= 1 - top_p, on the 2^-62 grid of the weights
  const uint64_t thr = topp ? static_cast<uint64_t>(floor((1.0 - static_cast<double>(opt.top_p)) * 0x1p62)) : 0ull;
  Launch("SamplePrepKernel", SamplePrepKernel, grid, block, lg, s);
  if (topk) {
    for (int32_t level = 1; level <= 3; ++level)
      Launch("SampleTopKKernel", SampleTopKKernel, grid, block, lg, opt.top_k, level, s);
  }
  Launch("SampleSumKernel", SampleSumKernel, grid, block, lg, topk, opt.top_k, s);
  if (topp) {
    for (int32_t level = 1; level <= 3; ++level)
      Launch("SampleTopPKernel", SampleTopPKernel, grid, block, lg, topk, thr, level, s);
    Launch("SampleCutKernel", SampleCutKernel, grid, block, lg, topk, thr, s);
  }
  Launch("SampleNormKernel", SampleNormKernel, grid, block, lg, topk, topp, probs, s);
}

void CheckBuffers(const void* a, const void* b) {
  RPG_CHECK(a != nullptr && b != nullptr, "sampler: a probability buffer is null");
}

}  // namespace

// ---------------------------------------------------------------- public API

uint64_t DevSplitMix64(uint64_t x) { return SplitMix64Of(x); }
uint64_t DevCounterRng(uint64_t seed, uint64_t counter) { return CounterRngOf(seed, counter); }
float DevCounterUniform(uint64_t seed, uint64_t counter) { return CounterUniformOf(seed, counter); }

void GpuSamplerWarmup() { (void)Scratch(); }

void GpuArgMax(const float* x_dev, int64_t n, int32_t* out_idx_dev) {
  CheckBuffers(x_dev, out_idx_dev);
  CheckVocab(n);
  SampleScratch* s = Scratch();
  Launch("ArgMaxPartKernel", ArgMaxPartKernel, dim3(Slices(n)), dim3(kThreads), x_dev, n, -FLT_MAX, s);
  Launch("ArgMaxFinalKernel", ArgMaxFinalKernel, dim3(1), dim3(kThreads), n, out_idx_dev, s);
}

void GpuFilterToProbs(const float* logits_dev, int64_t n, const SampleOptions& opt, float* probs_dev) {
  CheckBuffers(logits_dev, probs_dev);
  CheckVocab(n);
  LaunchFilter(logits_dev, n, opt, probs_dev, Scratch());
}

void GpuInverseSample(const float* probs_dev, int64_t n, float u, int32_t* out_idx_dev) {
  CheckBuffers(probs_dev, out_idx_dev);
  CheckVocab(n);
  RPG_CHECK(u >= 0.0f && u < 1.0f, "inverse sampling needs a uniform draw in [0, 1), got %g", static_cast<double>(u));
  RPG_CHECK(!StreamIsCapturing(),
            "GpuInverseSample takes u from the host and is therefore not capturable; use GpuSampleTokenDev inside a "
            "graph");
  SampleScratch* s = Scratch();
  Launch("SampleFixKernel", SampleFixKernel, dim3(Slices(n)), dim3(kThreads), probs_dev, n, s);
  Launch("SampleInverseKernel", SampleInverseKernel, dim3(1), dim3(kThreads), probs_dev, n, u, uint64_t{0},
         static_cast<const uint64_t*>(nullptr), out_idx_dev, s);
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
  SampleScratch* s = Scratch();
  LaunchFilter(logits_dev, n, opt, probs_dev, s);
  Launch("SampleInverseKernel", SampleInverseKernel, dim3(1), dim3(kThreads), static_cast<const float*>(probs_dev), n,
         CounterUniformOf(seed, counter), uint64_t{0}, static_cast<const uint64_t*>(nullptr), out_idx_dev, s);
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
  SampleScratch* s = Scratch();
  LaunchFilter(logits_dev, n, opt, probs_dev, s);
  Launch("SampleInverseKernel", SampleInverseKernel, dim3(1), dim3(kThreads), static_cast<const float*>(probs_dev), n,
         0.0f, seed, counter_dev, out_idx_dev, s);
}

}  // namespace rpg
