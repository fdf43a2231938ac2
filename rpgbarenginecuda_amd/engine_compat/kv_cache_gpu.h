// GpuKvCache with the reference interface (src/kv_cache_gpu.h:50-100), backed
// by a librpg_ops cache (rpg_kv_create_shape): fp16 K and V, each
// [n_layers][n_kv_heads][max_seq][head_dim], allocated in full at creation.
// The filled length lives in the library (its forward advances it), so len()
// asks it every time.
#ifndef RPG_AMD_COMPAT_KV_CACHE_GPU_H_
#define RPG_AMD_COMPAT_KV_CACHE_GPU_H_

#include <cstdint>
#include <string>

#include "cuda_common.h"
#include "model_meta.h"

struct rpg_kv;

namespace rpg {

class GpuKvCache {
 public:
  GpuKvCache() = default;
  GpuKvCache(const ModelMeta& c, int64_t max_seq);
  GpuKvCache(GpuKvCache&& o) noexcept;
  GpuKvCache& operator=(GpuKvCache&& o) noexcept;
  GpuKvCache(const GpuKvCache&) = delete;
  GpuKvCache& operator=(const GpuKvCache&) = delete;
  ~GpuKvCache();

  int64_t len() const;
  int64_t max_seq() const { return max_seq_; }
  int32_t n_layers() const { return n_layers_; }
  int32_t n_kv_heads() const { return n_kv_heads_; }
  int32_t head_dim() const { return head_dim_; }
  bool valid() const { return handle_ != nullptr; }

  uint16_t* k_layer(int32_t layer);
  uint16_t* v_layer(int32_t layer);

  void Reset() { SetLen(0); }
  void SetLen(int64_t n);
  void AddLen(int64_t n) { SetLen(len() + n); }
  int64_t bytes() const;
  std::string Describe() const;

  rpg_kv* handle() const { return handle_; }

 private:
  rpg_kv* handle_ = nullptr;
  int32_t n_layers_ = 0;
  int32_t n_kv_heads_ = 0;
  int32_t head_dim_ = 0;
  int64_t max_seq_ = 0;
};

}  // namespace rpg

#endif  // RPG_AMD_COMPAT_KV_CACHE_GPU_H_
