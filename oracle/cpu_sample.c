/* cpu_sample.c -- CPU oracle for device argmax and sampling.
 *
 * TEST INFRASTRUCTURE ONLY (see cpu_ref.h). A plain-C restatement of the
 * reference's sampling semantics: GpuArgMax (src/kernels_gpu.cu:827-859),
 * FilterProbsKernel (src/sampler_gpu.cu:161-298), InverseSampleKernel
 * (src/sampler_gpu.cu:321-343), SampleToken / the counter-based random source
 * (src/sampler_gpu.cu:41-55, 430-446). The reference's CPU sampler
 * (sampler.cc) is not part of /root/reference; its contract is the header
 * src/sampler.h:35-62, which these functions follow.
 *
 * Where the reference uses a binary search over the key space (top_k's k-th
 * largest value, top_p's cut) this restatement sorts, which is what the search
 * computes; top_p's cumulative mass is summed exactly (fixed point with 2^-125
 * resolution) so the oracle states the real-number decision the reference's
 * double sums approximate.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "cpu_ref.h"

#define ORA_GAMMA 0x9E3779B97F4A7C15ull

/* SplitMix64 (Steele, Lea & Flood 2014); src/sampler_gpu.cu:41-46. */
uint64_t ora_split_mix64(uint64_t x) {
  uint64_t z = x + ORA_GAMMA;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* src/sampler_gpu.cu:48-55. */
uint64_t ora_counter_rng(uint64_t seed, uint64_t counter) { return ora_split_mix64(seed + ORA_GAMMA * counter); }

float ora_counter_uniform(uint64_t seed, uint64_t counter) {
  const uint32_t bits = (uint32_t)(ora_counter_rng(seed, counter) >> 40);
  return (float)bits * (1.0f / 16777216.0f);
}

/* First index of the largest value strictly above `init` (none: 0);
 * src/kernels_gpu.cu:827-859 with init = -FLT_MAX, src/sampler_gpu.cu:129-156
 * with init = -inf. */
int32_t ora_argmax(const float* x, int64_t n, float init) {
  float bv = init;
  int32_t bi = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (x[i] > bv) {
      bv = x[i];
      bi = (int32_t)i;
    }
  }
  return bi;
}

static uint32_t order_key(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static float from_order_key(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static int cmp_u32_desc(const void* a, const void* b) {
  const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

typedef struct {
  uint32_t key;
  float p;
} KeyProb;

static int cmp_keyprob_asc(const void* a, const void* b) {
  const uint32_t x = ((const KeyProb*)a)->key, y = ((const KeyProb*)b)->key;
  return x < y ? -1 : (x > y ? 1 : 0);
}

/* p * 2^125 truncated (exact for p >= 2^-125; p <= 8 fits). */
static unsigned __int128 fix125(double p) {
  if (!(p > 0.0)) return 0;
  const long double s = (long double)p * 0x1p125L;
  return (unsigned __int128)s;
}

static double unfix125(unsigned __int128 v) { return (double)((long double)v * 0x1p-125L); }

/* p * 2^62 truncated: the weight the device's top_p histograms sum (exact
 * integers, so the sum does not depend on the order of the atomics). */
static unsigned __int128 fix62(float p) {
  if (!(p > 0.0f)) return 0;
  return (unsigned __int128)(uint64_t)ldexp((double)p, 62);
}

/* The top_p cut (src/sampler_gpu.cu:243-270): with S(t) the mass of the
 * probabilities whose order key is <= t, the cut is the largest t with
 * S(t) <= 1 - top_p, and every p <= cut is dropped. Returns the cut's order
 * key (0 on allocation failure: no real cut is 0). `rule` decides how S(t) is
 * compared:
 *   ORA_TOPP_EXACT   the real number (fixed point at 2^-125: exact for fp32
 *                    probabilities); the oracle's semantics;
 *   ORA_TOPP_GRID62  the device kernel's: every p truncated to the 2^-62 grid,
 *                    summed as integers, against floor((1 - top_p) * 2^62);
 *   ORA_TOPP_DOUBLE  the reference's: S(t) as a double sum (here in index
 *                    order; the reference sums strided per thread, then over the
 *                    block) against the double 1 - top_p.
 * The three agree unless S(t) lies within rounding of 1 - top_p: about
 * n * 2^-53 S for the double sums, n * 2^-62 for the grid.
 * *margin (may be NULL; EXACT only) receives the distance between 1 - top_p
 * and the nearest cumulative mass that decides the cut. */
uint32_t ora_top_p_cut_key(const float* probs, int64_t n, float top_p, int rule, double* margin) {
  const double threshold = 1.0 - (double)top_p;
  const unsigned __int128 thr = rule == ORA_TOPP_GRID62 ? (unsigned __int128)(uint64_t)floor(ldexp(threshold, 62))
                                                        : fix125(threshold);
  KeyProb* kp = (KeyProb*)malloc((size_t)n * sizeof(KeyProb));
  if (!kp) return 0u;
  for (int64_t i = 0; i < n; ++i) {
    kp[i].key = order_key(probs[i]);
    kp[i].p = probs[i];
  }
  uint32_t cut_key = 0xFFFFFFFFu;
  if (rule == ORA_TOPP_DOUBLE) {
    /* the reference's binary search, literally: the largest key t whose double
     * S(t) <= threshold (S is monotone in t) */
    uint32_t lo = 0u, hi = 0xFFFFFFFFu;
    while (lo < hi) {
      const uint32_t mid = (uint32_t)(lo + (((uint64_t)hi - lo + 1) >> 1));
      double sm = 0.0;
      for (int64_t i = 0; i < n; ++i)
        if (kp[i].key <= mid) sm += (double)kp[i].p;
      if (sm <= threshold) {
        lo = mid;
      } else {
        hi = mid - 1;
      }
    }
    free(kp);
    return lo;
  }
  qsort(kp, (size_t)n, sizeof(KeyProb), cmp_keyprob_asc);
  /* one below the smallest key whose cumulative mass exceeds the threshold */
  unsigned __int128 sum = 0;
  double m = INFINITY;
  int64_t i = 0;
  while (i < n) {
    const uint32_t key = kp[i].key;
    unsigned __int128 s_next = sum;
    for (; i < n && kp[i].key == key; ++i) s_next += rule == ORA_TOPP_GRID62 ? fix62(kp[i].p) : fix125(kp[i].p);
    if (s_next > thr) {
      cut_key = key - 1u;
      m = fmin(unfix125(s_next - thr), unfix125(thr - sum));
      break;
    }
    sum = s_next;
  }
  if (cut_key == 0xFFFFFFFFu) m = unfix125(thr - sum);
  free(kp);
  if (margin && rule == ORA_TOPP_EXACT) *margin = m;
  return cut_key;
}

/* FilterProbsKernel semantics (src/sampler_gpu.cu:161-298). *margin (may be
 * NULL) receives, when top_p is active, the distance between 1 - top_p and the
 * nearest cumulative mass that decides the cut: agreement with any other
 * accurate implementation is expected when it is well above their rounding. */
int ora_filter_to_probs(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p, float* probs,
                        double* margin) {
  if (n <= 0) return -1;
  if (margin) *margin = INFINITY;
  if (!(temperature > 0.0f)) { /* greedy: one-hot at the argmax (from -inf) */
    const int32_t best = ora_argmax(logits, n, -INFINITY);
    for (int64_t i = 0; i < n; ++i) probs[i] = 0.0f;
    probs[best] = 1.0f;
    return 0;
  }
  for (int64_t i = 0; i < n; ++i) probs[i] = logits[i];
  if (temperature != 1.0f) {
    const float inv = 1.0f / temperature;
    for (int64_t i = 0; i < n; ++i) probs[i] *= inv;
  }
  if (top_k > 1 && top_k < n) { /* threshold = k-th largest key */
    uint32_t* keys = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
    if (!keys) return -1;
    for (int64_t i = 0; i < n; ++i) keys[i] = order_key(probs[i]);
    qsort(keys, (size_t)n, sizeof(uint32_t), cmp_u32_desc);
    const float kth = from_order_key(keys[top_k - 1]);
    free(keys);
    for (int64_t i = 0; i < n; ++i)
      if (probs[i] < kth) probs[i] = -INFINITY;
  }
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    if (probs[i] > mx) mx = probs[i];
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const float e = expf(probs[i] - mx);
    probs[i] = e;
    sum += (double)e;
  }
  const float inv = (float)(1.0 / sum);
  for (int64_t i = 0; i < n; ++i) probs[i] *= inv;

  if (top_p > 0.0f && top_p < 1.0f) {
    const uint32_t cut_key = ora_top_p_cut_key(probs, n, top_p, ORA_TOPP_EXACT, margin);
    if (cut_key == 0u) return -1;
    const float cut = from_order_key(cut_key);
    for (int64_t j = 0; j < n; ++j)
      if (probs[j] <= cut) probs[j] = 0.0f;
    const int32_t best = ora_argmax(probs, n, -INFINITY);
    if (probs[best] == 0.0f) probs[best] = 1.0f;
    double sum2 = 0.0;
    for (int64_t j = 0; j < n; ++j) sum2 += (double)probs[j];
    if (sum2 > 0.0) {
      const float inv2 = (float)(1.0 / sum2);
      for (int64_t j = 0; j < n; ++j) probs[j] *= inv2;
    }
  }
  return 0;
}

/* InverseSampleKernel (src/sampler_gpu.cu:321-343): the first i whose running
 * double sum exceeds u; none -> the first maximum starting from probs[0]. */
int32_t ora_inverse_sample(const float* probs, int64_t n, float u) {
  const double ud = (double)u;
  double cum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    cum += (double)probs[i];
    if (cum > ud) return (int32_t)i;
  }
  float bv = probs[0];
  int32_t bi = 0;
  for (int64_t i = 1; i < n; ++i) {
    if (probs[i] > bv) {
      bv = probs[i];
      bi = (int32_t)i;
    }
  }
  return bi;
}

/* GpuSampleToken (src/sampler_gpu.cu:430-446): greedy is GpuArgMax and draws
 * no random number; otherwise filter, then the inverse transform at
 * u = CounterUniform(seed, counter). probs: n floats of scratch. */
int32_t ora_sample_token(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p, uint64_t seed,
                         uint64_t counter, float* probs) {
  if (!(temperature > 0.0f)) return ora_argmax(logits, n, -FLT_MAX);
  if (ora_filter_to_probs(logits, n, temperature, top_k, top_p, probs, NULL) != 0) return -1;
  return ora_inverse_sample(probs, n, ora_counter_uniform(seed, counter));
}
