// Device argmax and token sampling: the step after lm_head.
//
// Same C++ signatures as the reference sampler (src/sampler_gpu.h:62-128,
// src/sampler.h:35-46) so the generate loop (src/qwen3_gpu.cu:416, :553) links
// unchanged; GpuArgMax itself is declared with the layer operators in
// kernels_gpu.h (reference src/kernels_gpu.h:131-143).
//
// Semantics (what the parity tests hold the kernels to):
//   * temperature <= 0 (or NaN) is greedy: FilterToProbs gives a one-hot at the
//     argmax, SampleToken is GpuArgMax and consumes no random number;
//   * logits are scaled by float(1/T) when T != 1;
//   * top_k (1 < k < n): the threshold is the k-th largest value in the total
//     order of float bit patterns; values below it (float compare) are dropped,
//     ties with it kept;
//   * softmax: e = expf(v - max), summed in double, p = e * float(1/sum);
//   * top_p (0 < p < 1): with S(t) = sum of p_i over bit-pattern keys <= t, the
//     cut is the largest key with S <= 1 - top_p; every p_i <= cut becomes 0;
//     if nothing is left the argmax gets 1; then p *= float(1/sum) again, the
//     sum of the kept p taken on the same 2^-62 grid (within n * 2^-62 of the
//     double sum);
//   * inverse transform: the first index whose running double sum of p exceeds
//     u; if none does, the first maximum of p;
//   * u = CounterUniform(seed, counter) = (SplitMix64 of seed + gamma*counter)
//     >> 40, times 2^-24.
#ifndef RPG_AMD_SAMPLER_GPU_H_
#define RPG_AMD_SAMPLER_GPU_H_

#include <cstdint>

namespace rpg {

// Sampling parameters (reference src/sampler.h:35-46): temperature <= 0 is
// greedy; top_k 0 disables the top-k filter; top_p 1 disables the nucleus cut.
struct SampleOptions {
  float temperature = 1.0f;
  int32_t top_k = 0;
  float top_p = 1.0f;
};

// Largest vocabulary the device sampler accepts (the per-slice partials live
// in a fixed-size scratch block).
constexpr int64_t kSamplerMaxVocab = int64_t(1) << 22;

// Counter-based random source, host side (reference src/sampler_gpu.h:71-73).
uint64_t DevSplitMix64(uint64_t x);
uint64_t DevCounterRng(uint64_t seed, uint64_t counter);
float DevCounterUniform(uint64_t seed, uint64_t counter);

// logits -> filtered, normalised probabilities (reference src/sampler_gpu.h:86-87).
// probs_dev holds >= n floats; logits_dev is not modified.
void GpuFilterToProbs(const float* logits_dev, int64_t n, const SampleOptions& opt, float* probs_dev);

// Inverse transform with a host u in [0, 1) (reference src/sampler_gpu.h:95-96).
// Not capturable (u would be frozen into the graph): throws while the engine
// stream is capturing.
void GpuInverseSample(const float* probs_dev, int64_t n, float u, int32_t* out_idx_dev);

// One token: greedy -> GpuArgMax; otherwise FilterToProbs then the inverse
// transform with u = CounterUniform(seed, counter) (reference src/sampler_gpu.h:108-110).
void GpuSampleToken(const float* logits_dev, int64_t n, const SampleOptions& opt, uint64_t seed, uint64_t counter,
                    float* probs_dev, int32_t* out_idx_dev);

// The same with the counter read on the device (the pos0 staging scalar), so a
// captured graph draws a fresh u on every replay (reference src/sampler_gpu.h:124-126).
void GpuSampleTokenDev(const float* logits_dev, int64_t n, const SampleOptions& opt, uint64_t seed,
                       const uint64_t* counter_dev, float* probs_dev, int32_t* out_idx_dev);

// Allocates the sampler's scratch block; call once before capturing a graph
// that samples or takes an argmax (reference src/sampler_gpu.h:130).
void GpuSamplerWarmup();

}  // namespace rpg

#endif  // RPG_AMD_SAMPLER_GPU_H_
