// GpuKvCache storage and the host-built RoPE table.
#include <cmath>
#include <cstdio>
#include <limits>
#include <vector>

#include "kernels_gpu.h"

namespace rpg {

GpuKvCache::GpuKvCache(const ModelMeta& c, int64_t max_seq)
    : n_layers_(c.n_layers), n_kv_heads_(c.n_kv_heads), head_dim_(c.head_dim), max_seq_(max_seq) {
  if (n_layers_ <= 0 || n_kv_heads_ <= 0 || head_dim_ <= 0) {
    Throw("GpuKvCache needs a model shape with layers, kv heads and a head size; got %d / %d / %d", n_layers_,
          n_kv_heads_, head_dim_);
  }
  if (max_seq_ <= 0) Throw("GpuKvCache: a cache of %lld positions holds nothing", static_cast<long long>(max_seq_));
  // Element count of one plane and of the whole block, refusing anything whose
  // byte size would not fit a size_t (a corrupt model shape, not a real cache).
  const double total = 2.0 * n_layers_ * static_cast<double>(n_kv_heads_) * static_cast<double>(max_seq_) *
                       head_dim_ * sizeof(uint16_t);
  if (total > static_cast<double>(std::numeric_limits<int64_t>::max() / 2)) {
    Throw("GpuKvCache: %d layers x %d kv heads x %lld positions x %d is too large to address", n_layers_,
          n_kv_heads_, static_cast<long long>(max_seq_), head_dim_);
  }
  plane_elems_ = static_cast<int64_t>(n_kv_heads_) * max_seq_ * head_dim_;
  // The whole capacity is reserved now, so running out of device memory is an
  // error of session creation rather than of a later generation step. No
  // clearing: rows at positions >= len() are never read, and every position
  // below it has been written by the fused q/k kernel or GpuKvWrite.
  store_.Alloc(static_cast<size_t>(2 * n_layers_ * plane_elems_) * sizeof(uint16_t));
}

uint16_t* GpuKvCache::Plane(int32_t layer, int plane) const {
  if (layer < 0 || layer >= n_layers_) {
    Throw("GpuKvCache has layers 0..%d; layer %d was requested", n_layers_ - 1, layer);
  }
  uint16_t* base = static_cast<uint16_t*>(const_cast<void*>(store_.data()));
  return base + (static_cast<int64_t>(plane) * n_layers_ + layer) * plane_elems_;
}

void GpuKvCache::SetLen(int64_t n) {
  if (n < 0 || n > max_seq_) {
    Throw("GpuKvCache: cannot mark %lld positions as filled in a cache of %lld", static_cast<long long>(n),
          static_cast<long long>(max_seq_));
  }
  len_ = n;
}

std::string GpuKvCache::Describe() const {
  char text[224];
  std::snprintf(text, sizeof(text),
                "fp16 KV cache: %d layers, %d kv heads, head_dim %d, %lld positions (%lld filled), %.1f MiB in one "
                "block",
                n_layers_, n_kv_heads_, head_dim_, static_cast<long long>(max_seq_), static_cast<long long>(len_),
                static_cast<double>(bytes()) / (1024.0 * 1024.0));
  return text;
}

// tab[p][i] = cos(p * w_i), tab[p][head_dim/2 + i] = sin(p * w_i) with
// w_i = 1 / theta^(2i / head_dim), every angle in double and rounded to fp32 once
// (the table src/gpu_model.cu:90-120 uploads). The inverse frequency is formed as a
// reciprocal of the power, as the reference forms it: pow(theta, -2i/d) differs from
// it in the last double bit for about a third of the i, which moves some fp32 table
// entries at positions past ~6500.
std::vector<float> BuildRopeTable(int32_t head_dim, double theta, int64_t n_pos) {
  RPG_CHECK(head_dim > 0 && head_dim % 2 == 0, "RoPE needs an even head size, got %d", head_dim);
  RPG_CHECK(theta > 0.0, "RoPE base theta must be positive, got %g", theta);
  const int64_t rows = n_pos > 0 ? n_pos : 1;
  const int32_t pairs = head_dim / 2;
  std::vector<double> freq(static_cast<size_t>(pairs));
  for (int32_t i = 0; i < pairs; ++i) {
    freq[static_cast<size_t>(i)] = 1.0 / std::pow(theta, static_cast<double>(2 * i) / static_cast<double>(head_dim));
  }
  std::vector<float> tab(static_cast<size_t>(rows * head_dim));
  float* out = tab.data();
  for (int64_t p = 0; p < rows; ++p, out += head_dim) {
    for (int32_t i = 0; i < pairs; ++i) {
      const double angle = static_cast<double>(p) * freq[static_cast<size_t>(i)];
      out[i] = static_cast<float>(std::cos(angle));
      out[pairs + i] = static_cast<float>(std::sin(angle));
    }
  }
  return tab;
}

}  // namespace rpg
