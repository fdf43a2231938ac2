// GpuKvCache (layout and per-layer base pointers) and the host-built RoPE table.
#include <cmath>
#include <cstdio>
#include <vector>

#include "kernels_gpu.h"

namespace rpg {

GpuKvCache::GpuKvCache(const ModelMeta& c, int64_t max_seq)
    : n_layers_(c.n_layers), n_kv_heads_(c.n_kv_heads), head_dim_(c.head_dim), max_seq_(max_seq) {
  RPG_CHECK(n_layers_ > 0 && n_kv_heads_ > 0 && head_dim_ > 0,
            "incomplete model config, cannot build a KV cache (%d layers / %d KV heads / head_dim %d)", n_layers_,
            n_kv_heads_, head_dim_);
  RPG_CHECK(max_seq_ > 0, "max_seq must be positive, got %lld", static_cast<long long>(max_seq_));
  const size_t per = static_cast<size_t>(n_layers_) * static_cast<size_t>(LayerElems()) * sizeof(uint16_t);
  // Full capacity up front: an allocation failure shows at session creation,
  // not in the middle of a generation. Contents are left uninitialised; what
  // is visible is decided by len().
  k_.Alloc(per);
  v_.Alloc(per);
}

uint16_t* GpuKvCache::k_layer(int32_t layer) {
  RPG_CHECK(layer >= 0 && layer < n_layers_, "layer index %d out of range (%d layers)", layer, n_layers_);
  return static_cast<uint16_t*>(k_.data()) + static_cast<int64_t>(layer) * LayerElems();
}

uint16_t* GpuKvCache::v_layer(int32_t layer) {
  RPG_CHECK(layer >= 0 && layer < n_layers_, "layer index %d out of range (%d layers)", layer, n_layers_);
  return static_cast<uint16_t*>(v_.data()) + static_cast<int64_t>(layer) * LayerElems();
}

const uint16_t* GpuKvCache::k_layer(int32_t layer) const { return const_cast<GpuKvCache*>(this)->k_layer(layer); }

void GpuKvCache::SetLen(int64_t n) {
  RPG_CHECK(n >= 0 && n <= max_seq_, "length %lld out of range (capacity %lld)", static_cast<long long>(n),
            static_cast<long long>(max_seq_));
  len_ = n;
}

std::string GpuKvCache::Describe() const {
  char buf[192];
  std::snprintf(buf, sizeof(buf), "KV cache (fp16) %d layers x %d KV heads x %lld x %d = %.1f MiB (len %lld)",
                n_layers_, n_kv_heads_, static_cast<long long>(max_seq_), head_dim_,
                static_cast<double>(bytes()) / 1048576.0, static_cast<long long>(len_));
  return std::string(buf);
}

std::vector<float> BuildRopeTable(int32_t head_dim, double theta, int64_t n_pos) {
  RPG_CHECK(head_dim > 0 && head_dim % 2 == 0, "head_dim %d must be even", head_dim);
  RPG_CHECK(theta > 0.0, "rope theta must be positive");
  if (n_pos <= 0) n_pos = 1;
  const int32_t half = head_dim / 2;
  std::vector<double> inv(static_cast<size_t>(half));
  for (int32_t i = 0; i < half; ++i) {
    inv[static_cast<size_t>(i)] = 1.0 / std::pow(theta, static_cast<double>(2 * i) / static_cast<double>(head_dim));
  }
  std::vector<float> tab(static_cast<size_t>(n_pos) * static_cast<size_t>(head_dim));
  for (int64_t p = 0; p < n_pos; ++p) {
    float* row = tab.data() + p * head_dim;
    for (int32_t i = 0; i < half; ++i) {
      const double ang = static_cast<double>(p) * inv[static_cast<size_t>(i)];
      row[i] = static_cast<float>(std::cos(ang));
      row[half + i] = static_cast<float>(std::sin(ang));
    }
  }
  return tab;
}

}  // namespace rpg
