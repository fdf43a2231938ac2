// NeoX RoPE, the fp32 -> fp16 KV-cache write, and their fusion with the
// per-head q/k RMSNorm.
//
// Reference semantics:
//   RoPE (src/kernels_gpu.cu:598-621): x is [rows][heads][head_dim]; the pair is
//     (i, i + head_dim/2); with c = tab[(pos0+row)*head_dim + i] and
//     s = tab[(pos0+row)*head_dim + head_dim/2 + i]:
//       x_i <- a*c - b*s,   x_{i+half} <- b*c + a*s.
//   KV write (src/kernels_gpu.cu:708-727): source [t][h][d] fp32, destination
//     [h][pos0+t][d] fp16 with IEEE round-to-nearest-even; host checks
//     pos0 >= 0 and pos0 + seq <= max_seq (src/kernels_gpu.cu:1024-1028).
//   Layer order (src/qwen3_gpu.cu:77-91): q/k RMSNorm, then RoPE on q and k,
//     then the K/V cache write; V is never normalised or rotated.
//
// MI355X mapping for head_dim = 128: 8 lanes own one head row (head_row.h), so
// both members of every RoPE pair sit in the same lane and the norm reduction is
// a 3-step butterfly inside the 8-lane group. The fused kernel reads q, k, v once
// (streaming loads), writes q back (fp32) and k, v as fp16 straight into the
// cache (each head row of the cache is 256 contiguous bytes).
//
// pos0 arrives by value on eager launches; a launch being captured into a graph
// receives the staging address instead (Pos0ForLaunch) and reads it on device.
#include <hip/hip_runtime.h>

#include "dev_util.h"
#include "head_row.h"
#include "kernels_gpu.h"
#include "launch.h"

namespace rpg {
namespace {

using dev::HeadRow;
using dev::kHeadLanes;
using dev::LoadStream4;
using dev::PackHalf4;
using dev::StoreStreamHalf4;

constexpr int kBlock = 256;
constexpr int kHeadDim = 128;

bool Aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

__device__ __forceinline__ int64_t ReadPos0(int64_t value, const int64_t* dev) {
  return dev != nullptr ? *dev : value;
}

// ---------------------------------------------------------------- RoPE

__global__ __launch_bounds__(kBlock) void RopeHead128Kernel(float* x, int32_t n_heads, const float* __restrict__ tab,
                                                            int64_t pos0_val, const int64_t* __restrict__ pos0_dev,
                                                            int64_t n_units) {
  const int l = threadIdx.x % kHeadLanes;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * (kBlock / kHeadLanes) + threadIdx.x / kHeadLanes;
  if (unit >= n_units) return;
  const int64_t row = unit / n_heads;
  float* p = x + unit * kHeadDim;
  HeadRow r = dev::LoadHeadRowStream(p, l);
  const HeadRow trig = dev::LoadHeadVec(tab + (ReadPos0(pos0_val, pos0_dev) + row) * kHeadDim, l);
  dev::RotateHeadRow(r, trig, true);
  dev::StoreHeadRowStream(p, l, r);
}

// Any even head_dim: one thread per rotation pair.
__global__ __launch_bounds__(kBlock) void RopePairKernel(float* x, int32_t n_heads, int32_t head_dim,
                                                         const float* __restrict__ tab, int64_t pos0_val,
                                                         const int64_t* __restrict__ pos0_dev, int64_t total) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= total) return;
  const int32_t half = head_dim / 2;
  const int64_t per_row = static_cast<int64_t>(n_heads) * half;
  const int64_t row = idx / per_row;
  const int64_t rem = idx - row * per_row;
  const int32_t h = static_cast<int32_t>(rem / half);
  const int32_t i = static_cast<int32_t>(rem - static_cast<int64_t>(h) * half);
  const float* c_t = tab + (ReadPos0(pos0_val, pos0_dev) + row) * head_dim;
  float* xh = x + (row * n_heads + h) * head_dim;
  const float a = xh[i];
  const float b = xh[i + half];
  const float c = c_t[i];
  const float s = c_t[half + i];
  xh[i] = a * c - b * s;
  xh[i + half] = b * c + a * s;
}

// ---------------------------------------------------------------- KV write

// Four consecutive elements per thread (head_dim % 4 == 0): one float4 load per
// tensor, one 8-byte store of four halves per tensor.
__global__ __launch_bounds__(kBlock) void KvWriteVec4Kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                            int32_t n_kv_heads, int32_t head_dim, int64_t pos0_val,
                                                            const int64_t* __restrict__ pos0_dev, int64_t max_seq,
                                                            int64_t total4, uint16_t* __restrict__ kc,
                                                            uint16_t* __restrict__ vc) {
  const int64_t i4 = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i4 >= total4) return;
  const int64_t i = 4 * i4;
  const int64_t dd = i % head_dim;
  const int64_t r = i / head_dim;  // t * n_kv_heads + h
  const int64_t h = r % n_kv_heads;
  const int64_t t = r / n_kv_heads;
  const int64_t pos = ReadPos0(pos0_val, pos0_dev) + t;
  if (pos < 0 || pos >= max_seq) return;  // only reachable through a replayed graph with a bad staged pos0
  const int64_t dst = (h * max_seq + pos) * head_dim + dd;
  StoreStreamHalf4(kc + dst, PackHalf4(LoadStream4(k + i)));
  StoreStreamHalf4(vc + dst, PackHalf4(LoadStream4(v + i)));
}

__global__ __launch_bounds__(kBlock) void KvWriteScalarKernel(const float* __restrict__ k, const float* __restrict__ v,
                                                              int32_t n_kv_heads, int32_t head_dim, int64_t pos0_val,
                                                              const int64_t* __restrict__ pos0_dev, int64_t max_seq,
                                                              int64_t total, uint16_t* __restrict__ kc,
                                                              uint16_t* __restrict__ vc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= total) return;
  const int64_t dd = i % head_dim;
  const int64_t r = i / head_dim;
  const int64_t h = r % n_kv_heads;
  const int64_t t = r / n_kv_heads;
  const int64_t pos = ReadPos0(pos0_val, pos0_dev) + t;
  if (pos < 0 || pos >= max_seq) return;
  const int64_t dst = (h * max_seq + pos) * head_dim + dd;
  kc[dst] = static_cast<uint16_t>(dev::FloatToHalfBits(k[i]));
  vc[dst] = static_cast<uint16_t>(dev::FloatToHalfBits(v[i]));
}

// ---------------------------------------------------------------- fused q/k norm + RoPE + KV

// Work units per token: n_heads q rows, then n_kv k rows, then n_kv v rows;
// 8 lanes per unit, 32 units per 256-thread block. With n_heads and n_kv
// multiples of 8 every wave handles units of a single kind.
//
// Store policies (kBuf, when q and one cache layer each span less than 2 GiB, so
// 32-bit buffer offsets reach every row): q rows go out as device-scope
// write-through stores with the streaming hint (sc1 | nt), the fp16 cache rows as
// plain stores. Measured on MI355X at n = 2811 in the layer's kernel order over 28
// rotated layers, against every pair of {plain, nt, sc1, sc1|nt, sc0|sc1,
// sc0|sc1|nt}: q stores without the streaming hint, or cache stores with it, were
// 3-12% slower. With the buffers carved from one allocation this pair took 13.95 us
// against 14.33 us for nontemporal q / plain cache global stores; with separately
// allocated tensors (as torch allocates them) every good pair lands within 1% of
// 14.7 us.
template <bool kWriteK, bool kBuf>
__global__ __launch_bounds__(kBlock) void QkNormRopeKvKernel(
    float* q, float* k, const float* __restrict__ v, const float* __restrict__ qw, const float* __restrict__ kw,
    int32_t n_heads, int32_t n_kv, const float* __restrict__ tab, int64_t rope_rows, int64_t pos0_val,
    const int64_t* __restrict__ pos0_dev, uint32_t n_units, float eps, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int64_t max_seq, uint32_t q_bytes, uint32_t cache_bytes) {
  // All kernel arguments in one batch of scalar loads at entry: the empty asm takes
  // them as scalar inputs (it emits nothing). Left to itself the compiler loads each
  // argument next to its first use, behind the unit-range and unit-kind branches,
  // and the first waves on each CU then wait for four scalar round trips (two of
  // them cache-line misses) before their first activation load.
  asm volatile("" ::"s"(q), "s"(k), "s"(v), "s"(qw), "s"(kw), "s"(n_heads), "s"(n_kv), "s"(tab), "s"(rope_rows),
               "s"(pos0_val), "s"(pos0_dev), "s"(n_units), "s"(eps), "s"(kc), "s"(vc), "s"(max_seq), "s"(q_bytes),
               "s"(cache_bytes));
  const int l = threadIdx.x % kHeadLanes;
  const uint32_t unit = blockIdx.x * (kBlock / kHeadLanes) + threadIdx.x / kHeadLanes;
  if (unit >= n_units) return;
  const uint32_t per_tok = static_cast<uint32_t>(n_heads + 2 * n_kv);
  const uint32_t t = unit / per_tok;
  const int32_t j = static_cast<int32_t>(unit - t * per_tok);
  const int64_t pos = ReadPos0(pos0_val, pos0_dev) + t;
  const bool kv_slot_ok = pos >= 0 && pos < max_seq;

  if (j < n_heads + n_kv) {
    const bool is_q = j < n_heads;
    const int32_t h = is_q ? j : j - n_heads;
    float* p = is_q ? q + (static_cast<int64_t>(t) * n_heads + h) * kHeadDim
                    : k + (static_cast<int64_t>(t) * n_kv + h) * kHeadDim;
    // The RoPE row index is clamped so the load is always in bounds; a position
    // outside the table (reachable only through a replayed graph with a bad
    // staged pos0) leaves the row unrotated.
    const bool rope_ok = pos >= 0 && pos < rope_rows;
    const HeadRow trig = dev::LoadHeadVec(tab + (rope_ok ? pos : 0) * kHeadDim, l);
    HeadRow r = dev::LoadHeadRowStream(p, l);
    // Keep the table and activation loads ahead of the reduction: each RoPE row is
    // read by a single block per launch, so it usually comes from HBM, not L2.
    __builtin_amdgcn_sched_barrier(0);
    const HeadRow w = dev::LoadHeadVec(is_q ? qw : kw, l);
    dev::NormHeadRow(r, w, eps);
    dev::RotateHeadRow(r, trig, rope_ok);
    if constexpr (kBuf) {
      if (is_q) {
        const uint32_t off = (t * static_cast<uint32_t>(n_heads) + static_cast<uint32_t>(h)) * (4u * kHeadDim);
        dev::StoreHeadRowBuf<dev::kStoreDeviceThroughPolicy>(dev::OutResource(q, q_bytes), off, l, r);
      } else {
        if (kWriteK) dev::StoreHeadRowStream(p, l, r);
        if (kv_slot_ok) {
          const uint32_t off = static_cast<uint32_t>(static_cast<int64_t>(h) * max_seq + pos) * (2u * kHeadDim);
          dev::StoreHeadRowHalfBuf<dev::kStorePlainPolicy>(dev::OutResource(kc, cache_bytes), off, l, r);
        }
      }
    } else {
      if (is_q || kWriteK) dev::StoreHeadRowStream(p, l, r);
      if (!is_q && kv_slot_ok) dev::StoreHeadRowHalf(kc + (static_cast<int64_t>(h) * max_seq + pos) * kHeadDim, l, r);
    }
  } else {
    const int32_t h = j - n_heads - n_kv;
    const HeadRow r = dev::LoadHeadRowStream(v + (static_cast<int64_t>(t) * n_kv + h) * kHeadDim, l);
    if (kv_slot_ok) {
      if constexpr (kBuf) {
        const uint32_t off = static_cast<uint32_t>(static_cast<int64_t>(h) * max_seq + pos) * (2u * kHeadDim);
        dev::StoreHeadRowHalfBuf<dev::kStorePlainPolicy>(dev::OutResource(vc, cache_bytes), off, l, r);
      } else {
        dev::StoreHeadRowHalf(vc + (static_cast<int64_t>(h) * max_seq + pos) * kHeadDim, l, r);
      }
    }
  }
}

}  // namespace

void GpuRope(float* x, int32_t n_heads, int32_t head_dim, const float* rope_tab, int64_t pos0, int64_t n_rows) {
  RPG_CHECK(head_dim > 0 && head_dim % 2 == 0, "RoPE rotates pairs (i, i + head_dim/2), so head_dim has to be even and positive (got %d)", head_dim);
  RPG_CHECK(n_heads > 0 && n_rows >= 0, "invalid Rope arguments");
  RPG_CHECK(pos0 >= 0, "RoPE position %lld must not be negative", static_cast<long long>(pos0));
  if (n_rows == 0) return;
  RPG_CHECK(x != nullptr && rope_tab != nullptr, "Rope got a null pointer");
  const Pos0Arg p0 = Pos0ForLaunch(pos0);
  if (head_dim == kHeadDim && Aligned(x, 16) && Aligned(rope_tab, 16)) {
    const int64_t units = n_rows * n_heads;
    Launch("RopeHead128Kernel", RopeHead128Kernel, dim3(GridFor(units, kBlock / kHeadLanes)), dim3(kBlock), x, n_heads,
           rope_tab, p0.value, p0.dev, units);
    return;
  }
  const int64_t total = n_rows * n_heads * (head_dim / 2);
  Launch("RopePairKernel", RopePairKernel, dim3(GridFor(total, kBlock)), dim3(kBlock), x, n_heads, head_dim, rope_tab,
         p0.value, p0.dev, total);
}

void GpuKvWrite(const float* k_dev, const float* v_dev, int32_t n_kv_heads, int32_t head_dim, int64_t pos0,
                int64_t seq, uint16_t* k_cache_layer, uint16_t* v_cache_layer, int64_t max_seq) {
  RPG_CHECK(seq > 0 && n_kv_heads > 0 && head_dim > 0, "KV write: seq, n_kv_heads and head_dim have to be positive");
  RPG_CHECK(pos0 >= 0, "KV write: start position %lld is negative", static_cast<long long>(pos0));
  RPG_CHECK(pos0 + seq <= max_seq, "KV write: positions [%lld, %lld) run past the %lld cache slots",
            static_cast<long long>(pos0), static_cast<long long>(pos0 + seq), static_cast<long long>(max_seq));
  RPG_CHECK(k_dev != nullptr && v_dev != nullptr && k_cache_layer != nullptr && v_cache_layer != nullptr,
            "KvWrite got a null pointer");
  const int64_t total = seq * n_kv_heads * head_dim;
  const Pos0Arg p0 = Pos0ForLaunch(pos0);
  if (head_dim % 4 == 0 && Aligned(k_dev, 16) && Aligned(v_dev, 16) && Aligned(k_cache_layer, 8) &&
      Aligned(v_cache_layer, 8)) {
    const int64_t total4 = total / 4;
    Launch("KvWriteVec4Kernel", KvWriteVec4Kernel, dim3(GridFor(total4, kBlock)), dim3(kBlock), k_dev, v_dev,
           n_kv_heads, head_dim, p0.value, p0.dev, max_seq, total4, k_cache_layer, v_cache_layer);
    return;
  }
  Launch("KvWriteScalarKernel", KvWriteScalarKernel, dim3(GridFor(total, kBlock)), dim3(kBlock), k_dev, v_dev,
         n_kv_heads, head_dim, p0.value, p0.dev, max_seq, total, k_cache_layer, v_cache_layer);
}

void GpuQkNormRopeKv(float* q, float* k, const float* v, const float* q_norm, const float* k_norm, int32_t n_heads,
                     int32_t n_kv_heads, int32_t head_dim, const float* rope_tab, int64_t rope_rows, int64_t pos0,
                     int64_t seq, float eps, uint16_t* k_cache_layer, uint16_t* v_cache_layer, int64_t max_seq,
                     bool write_k_f32) {
  RPG_CHECK(seq > 0 && n_heads > 0 && n_kv_heads > 0 && head_dim > 0, "invalid QkNormRopeKv arguments");
  RPG_CHECK(head_dim % 2 == 0, "head_dim %d must be even", head_dim);
  RPG_CHECK(pos0 >= 0, "KV write: start position %lld is negative", static_cast<long long>(pos0));
  RPG_CHECK(pos0 + seq <= max_seq, "KV write: positions [%lld, %lld) run past the %lld cache slots",
            static_cast<long long>(pos0), static_cast<long long>(pos0 + seq), static_cast<long long>(max_seq));
  RPG_CHECK(pos0 + seq <= rope_rows, "positions [%lld, %lld) exceed the RoPE table (%lld rows)",
            static_cast<long long>(pos0), static_cast<long long>(pos0 + seq), static_cast<long long>(rope_rows));
  RPG_CHECK(q && k && v && q_norm && k_norm && rope_tab && k_cache_layer && v_cache_layer,
            "QkNormRopeKv got a null pointer");
  const int64_t units = seq * (n_heads + 2 * static_cast<int64_t>(n_kv_heads));
  const bool fast = head_dim == kHeadDim && units <= 0x7FFFFFFF && Aligned(q, 16) && Aligned(k, 16) &&
                    Aligned(v, 16) && Aligned(q_norm, 16) && Aligned(k_norm, 16) && Aligned(rope_tab, 16) &&
                    Aligned(k_cache_layer, 16) && Aligned(v_cache_layer, 16);
  if (!fast) {
    // Other head sizes / layouts: the unfused reference sequence (k then holds
    // the rotated values, as it does in the reference layer).
    GpuRmsNorm(q, q_norm, seq * n_heads, head_dim, head_dim, eps, q);
    GpuRmsNorm(k, k_norm, seq * n_kv_heads, head_dim, head_dim, eps, k);
    GpuRope(q, n_heads, head_dim, rope_tab, pos0, seq);
    GpuRope(k, n_kv_heads, head_dim, rope_tab, pos0, seq);
    GpuKvWrite(k, v, n_kv_heads, head_dim, pos0, seq, k_cache_layer, v_cache_layer, max_seq);
    return;
  }
  const Pos0Arg p0 = Pos0ForLaunch(pos0);
  const unsigned grid = GridFor(units, kBlock / kHeadLanes);
  // Buffer stores need every q row and every slot of a cache layer within 2 GiB of
  // the tensor's start (32-bit offsets); larger tensors take global stores. Short
  // launches (decode) take them too: there the write-through acknowledgement of the
  // q rows only lengthens a latency-bound kernel (n = 1: 2.66 against 2.35 us).
  const int64_t q_bytes = seq * n_heads * kHeadDim * 4;
  const int64_t cache_bytes = static_cast<int64_t>(n_kv_heads) * max_seq * kHeadDim * 2;
  const bool buf = seq >= 64 && q_bytes < (int64_t{1} << 31) && cache_bytes < (int64_t{1} << 31);
  auto* kern = write_k_f32 ? (buf ? QkNormRopeKvKernel<true, true> : QkNormRopeKvKernel<true, false>)
                           : (buf ? QkNormRopeKvKernel<false, true> : QkNormRopeKvKernel<false, false>);
  Launch(write_k_f32 ? "QkNormRopeKvKernel<write_k>" : "QkNormRopeKvKernel", kern, dim3(grid), dim3(kBlock), q, k, v,
         q_norm, k_norm, n_heads, n_kv_heads, rope_tab, rope_rows, p0.value, p0.dev, static_cast<uint32_t>(units), eps,
         k_cache_layer, v_cache_layer, max_seq, static_cast<uint32_t>(buf ? q_bytes : 0),
         static_cast<uint32_t>(buf ? cache_bytes : 0));
}

}  // namespace rpg
