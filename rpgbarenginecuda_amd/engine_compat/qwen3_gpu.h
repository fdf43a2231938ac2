// Forward and generation with the interface the reference engine uses
// (src/qwen3_gpu.h:47-211: GpuScratch, GpuForwardOptions, GpuForwardFull,
// GpuForwardStep, GpuForwardStepDev, GpuGenerateOptions, GpuGenerate,
// GpuGenerateGreedy), each a call into librpg_ops (rpg_forward_*, rpg_generate).
// SampleOptions is the engine's own (sampler.h).
#ifndef RPG_AMD_COMPAT_QWEN3_GPU_H_
#define RPG_AMD_COMPAT_QWEN3_GPU_H_

#include <cstdint>
#include <vector>

#include "cuda_common.h"
#include "gpu_model.h"
#include "kv_cache_gpu.h"
#include "model_meta.h"
#include "sampler.h"

struct rpg_scratch;

namespace rpg {

// Grow-only device activations of a forward plus the captured decode graph,
// owned by librpg_ops. Creating one touches no device (the engine constructs
// a session's scratch before it knows whether a GPU exists).
class GpuScratch {
 public:
  // The logits of the last forward, [seq, vocab] fp32 in device memory.
  class LogitsView {
   public:
    explicit LogitsView(const GpuScratch* owner) : owner_(owner) {}
    const void* data() const;

   private:
    const GpuScratch* owner_;
  };

  GpuScratch() : logits(this) {}
  ~GpuScratch();
  GpuScratch(const GpuScratch&) = delete;
  GpuScratch& operator=(const GpuScratch&) = delete;
  GpuScratch(GpuScratch&&) = delete;
  GpuScratch& operator=(GpuScratch&&) = delete;

  LogitsView logits;

  rpg_scratch* handle();

 private:
  rpg_scratch* handle_ = nullptr;
};

struct GpuForwardOptions {
  int32_t layer_limit = 0;                        // 0 = every layer
  std::vector<float>* capture_hidden = nullptr;   // [layers run + 1, seq, hidden]
};

void GpuForwardFull(const GpuModel& m, const int32_t* tokens, int64_t seq, GpuScratch* s, std::vector<float>* logits,
                    const GpuForwardOptions& opt = GpuForwardOptions(), GpuKvCache* kv = nullptr);
void GpuForwardStep(const GpuModel& m, int32_t token, int64_t pos, GpuKvCache* kv, GpuScratch* s,
                    std::vector<float>* logits);
void GpuForwardStepDev(const GpuModel& m, const int32_t* token_dev, int64_t pos, GpuKvCache* kv, GpuScratch* s);

struct GpuGenerateOptions {
  int32_t max_tokens = 64;
  std::vector<int32_t> stop_ids;
  SampleOptions sample;
  uint64_t seed = 0;
  std::vector<float>* step_logits = nullptr;  // [tokens returned, vocab] when set
  bool use_graph = false;
};

void GpuGenerate(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                 const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids);
void GpuGenerateGreedy(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                       const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids);

}  // namespace rpg

#endif  // RPG_AMD_COMPAT_QWEN3_GPU_H_
