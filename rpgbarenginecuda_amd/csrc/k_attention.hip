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
//   * prefill (many (t, h) pairs) uses a single chunk per pair and writes the
//     normalised output directly; decode (few pairs) splits the keys into up to
//     kMaxChunks chunks so the whole chip streams the cache, each chunk storing
//     (m, l, o) to a partials buffer that a second kernel merges;
//   * the partials buffer is library-owned and grows on demand;
//     GpuAttentionWarmupShmem(max positions) sizes it before a graph capture,
//     where allocating is not allowed.
// Under graph capture pos0 comes from the staging scalar, so chunk ranges are
// laid out for the position budget (sh_positions) and checked against the
// actual position inside the kernel.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>

#include "dev_util.h"
#include "kernels_gpu.h"
#include "launch.h"

namespace rpg {
namespace {

constexpr int kD = 128;          // head_dim of the fast path
constexpr int kBlockThreads = 256;
constexpr int kWaves = kBlockThreads / 64;
constexpr int kMaxChunks = 64;
constexpr int kPartFloats = kD + 2;  // o[128], m, l

__device__ __forceinline__ int64_t ReadPos0(int64_t value, const int64_t* dev) { return dev != nullptr ? *dev : value; }

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
__device__ __forceinline__ float WaveMax(float v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) v = fmaxf(v, DppMov(v, k));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float WaveSumF(float v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) v += DppMov(v, k);
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

__device__ __forceinline__ float HalfToF(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// Merges the chunks of one (t, h): M = max m_c, L = sum l_c e^(m_c - M),
// out = sum o_c e^(m_c - M) / L. Lane c holds chunk c's (m, l) and weight; the
// partial outputs are read 16 chunks at a time (lane l owns dims 2l, 2l + 1).
// n_chunks <= 64.
__device__ __forceinline__ void MergeChunks(const float* pp, int32_t n_chunks, int lane, float* ot) {
  const bool has = lane < n_chunks;
  const float mc = has ? pp[lane * kPartFloats + kD] : -INFINITY;
  const float lc = has ? pp[lane * kPartFloats + kD + 1] : 0.0f;
  const float mx = WaveMax(mc);
  const float f = mc == -INFINITY ? 0.0f : expf(mc - mx);
  const float L = WaveSumF(lc * f);
  float o0 = 0.0f, o1 = 0.0f;
  for (int c0 = 0; c0 < n_chunks; c0 += 16) {
    float2 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = c0 + i < n_chunks ? c0 + i : n_chunks - 1;  // clamped: its weight is used only if c0 + i < n
      v[i] = *reinterpret_cast<const float2*>(pp + c * kPartFloats + 2 * lane);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float fc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), c0 + i));
      if (c0 + i < n_chunks) {
        o0 = __builtin_fmaf(v[i].x, fc, o0);
        o1 = __builtin_fmaf(v[i].y, fc, o1);
      }
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  ot[2 * lane] = o0 * inv;
  ot[2 * lane + 1] = o1 * inv;
}

// One wave per (t, h, chunk). part == nullptr: a single chunk, the output is
// written normalised; otherwise (m, l, o) of the chunk go to part.
__global__ __launch_bounds__(kBlockThreads) void AttnChunkKernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t max_seq,
    int32_t n_heads, int32_t group, float scale, int64_t pos0_val, const int64_t* __restrict__ pos0_dev, int64_t seq,
    int32_t n_chunks, int64_t chunk_len, float* __restrict__ out, float* __restrict__ part) {
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

  const int64_t lo = static_cast<int64_t>(c) * chunk_len;
  int64_t hi = lo + chunk_len;
  if (hi > pos + 1) hi = pos + 1;
  if (hi > max_seq) hi = max_seq;  // only reachable through a replayed graph with a bad staged pos0

  const uint16_t* kb = kc + static_cast<int64_t>(kh) * max_seq * kD;
  const uint16_t* vb = vc + static_cast<int64_t>(kh) * max_seq * kD;
  float m = -INFINITY;
  float l = 0.0f;
  float o0 = 0.0f, o1 = 0.0f;

  for (int64_t base = lo; base < hi; base += 64) {
    const int64_t s = base + lane;
    const bool valid = s < hi;
    // score of key s: its 256-byte row against q
    float sc = -INFINITY;
    if (valid) {
      const uint4* kr = reinterpret_cast<const uint4*>(kb + s * kD);
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four interleaved partial sums: a 32-deep chain
#pragma unroll
      for (int i = 0; i < kD / 8; ++i) {
        const uint4 w = kr[i];
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[k] = __builtin_fmaf(qs[wv][8 * i + 2 * k], HalfToF(wd[k] & 0xFFFFu), acc[k]);
          acc[k] = __builtin_fmaf(qs[wv][8 * i + 2 * k + 1], HalfToF(wd[k] >> 16), acc[k]);
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
    // row (one 256-byte row per wave load); 16 rows are requested before any is
    // used so their latencies overlap.
    const int64_t nk = hi - base < 64 ? hi - base : 64;
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(vb + base * kD) + lane;
    for (int j0 = 0; j0 < 64; j0 += 16) {
      if (j0 >= nk) break;
      uint32_t vv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = j0 + i < nk ? j0 + i : static_cast<int>(nk) - 1;  // clamped: stays in the block
        vv[i] = vr[static_cast<int64_t>(j) * (kD / 2)];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // p of a key past the block's end is 0 (invalid lanes), so the clamped
        // duplicate rows add nothing
        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), j0 + i));
        o0 = __builtin_fmaf(pj, HalfToF(vv[i] & 0xFFFFu), o0);
        o1 = __builtin_fmaf(pj, HalfToF(vv[i] >> 16), o1);
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

// One wave per (t, h): merges its n_chunks partials into out. (A merge by the
// last chunk to arrive would save this launch, but its device-scope release
// fence writes the whole L2 back once per chunk, which costs more.)
__global__ __launch_bounds__(kBlockThreads) void AttnMergeKernel(const float* __restrict__ part, int64_t pairs,
                                                                  int32_t n_chunks, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t th = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (th >= pairs) return;
  MergeChunks(part + th * n_chunks * kPartFloats, n_chunks, lane, out + th * kD);
}

// ---------------------------------------------------------------- partials buffer

// Grow-only device buffer for the chunk partials. Deliberately never freed at
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
    if (b.ptr != nullptr) {
      RPG_HIP_CHECK(hipDeviceSynchronize());
      RPG_HIP_CHECK(hipFree(b.ptr));
      b.ptr = nullptr;
      b.floats = 0;
    }
    RPG_HIP_CHECK(hipMalloc(&b.ptr, floats * sizeof(float)));
    b.floats = floats;
  }
  return b.ptr;
}

// Chunking for `pairs` (t, h) pairs over a budget of `positions` keys: no split
// when the pairs alone fill the chip; otherwise enough chunks (of at least 64
// keys, a multiple of 64) for ~2048 waves.
void PlanChunks(int64_t pairs, int64_t positions, int32_t* n_chunks, int64_t* chunk_len) {
  if (pairs >= kMaxSplitPairs || positions <= 64) {
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

// Partials needed for decode-sized calls with up to `positions` keys (seq 1,
// up to 64 heads), the worst case a decode graph replays.
size_t WarmupFloats(int64_t positions) {
  int32_t n_chunks;
  int64_t len;
  PlanChunks(64, positions, &n_chunks, &len);
  return static_cast<size_t>(64) * n_chunks * kPartFloats;
}

}  // namespace

void GpuAttentionFromCache(const ModelMeta& c, int64_t pos0, const float* q_dev, int64_t seq, const uint16_t* k_layer,
                           const uint16_t* v_layer, int64_t max_seq, float* out_dev, int64_t sh_positions) {
  RPG_CHECK(seq > 0, "attention seq must be positive");
  RPG_CHECK(pos0 >= 0, "pos0 must not be negative");
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
  float* part = nullptr;
  if (n_chunks > 1) part = EnsurePartials(static_cast<size_t>(pairs) * n_chunks * kPartFloats);
  const Pos0Arg p0 = Pos0ForLaunch(pos0);
  const int64_t units = pairs * n_chunks;
  Launch("AttnChunkKernel", AttnChunkKernel, dim3(GridFor(units, kWaves)), dim3(kBlockThreads), q_dev, k_layer,
         v_layer, max_seq, c.n_heads, c.n_heads / c.n_kv_heads, scale, p0.value, p0.dev, seq, n_chunks, chunk_len,
         out_dev, part);
  if (n_chunks > 1) {
    Launch("AttnMergeKernel", AttnMergeKernel, dim3(GridFor(pairs, kWaves)), dim3(kBlockThreads), part, pairs,
           n_chunks, out_dev);
  }
}

void GpuAttentionWarmupShmem(int64_t sh_positions) {
  RPG_CHECK(sh_positions > 0, "sh_positions must be positive (got %lld)", static_cast<long long>(sh_positions));
  EnsurePartials(WarmupFloats(sh_positions));
}

}  // namespace rpg
