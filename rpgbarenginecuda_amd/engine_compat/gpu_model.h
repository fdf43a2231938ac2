// GpuModel with the interface the reference engine uses (src/gpu_model.h:81-103:
// Load, config, gguf, tokenizer, path, rope_positions, device_bytes, Describe).
// The weights live in librpg_ops (rpg_model_load: one device arena, staged
// upload); the metadata, shapes and tokenizer come from the engine's own host
// layer (GgufFile, ReadModelMeta, Tokenizer::FromGguf) on the same file, and
// the two readings of the file are cross-checked at load.
#ifndef RPG_AMD_COMPAT_GPU_MODEL_H_
#define RPG_AMD_COMPAT_GPU_MODEL_H_

#include <cstdint>
#include <string>

#include "cuda_common.h"
#include "gguf.h"
#include "model_meta.h"
#include "tokenizer.h"

struct rpg_model;

namespace rpg {

class GpuModel {
 public:
  static GpuModel Load(const std::string& path, int32_t max_pos = 4096);

  GpuModel(GpuModel&& o) noexcept;
  GpuModel& operator=(GpuModel&& o) noexcept;
  GpuModel(const GpuModel&) = delete;
  GpuModel& operator=(const GpuModel&) = delete;
  ~GpuModel();

  const ModelMeta& config() const { return cfg_; }
  const GgufFile& gguf() const { return gguf_; }
  const Tokenizer& tokenizer() const { return tokenizer_; }
  const std::string& path() const { return gguf_.path(); }
  int64_t rope_positions() const { return rope_positions_; }
  int64_t device_bytes() const;
  std::string Describe() const;

  // The librpg_ops handle the forward and generation calls take.
  rpg_model* handle() const { return handle_; }

 private:
  GpuModel() = default;

  GgufFile gguf_;
  ModelMeta cfg_;
  Tokenizer tokenizer_;
  rpg_model* handle_ = nullptr;
  int64_t rope_positions_ = 0;
};

}  // namespace rpg

#endif  // RPG_AMD_COMPAT_GPU_MODEL_H_
