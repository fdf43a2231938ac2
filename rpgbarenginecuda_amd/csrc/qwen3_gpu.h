// Qwen3 forward and generation on the device, composed from this library's
// operators: the caller of the hot path, with the reference's interface
// (src/qwen3_gpu.h:47-211, src/qwen3_gpu.cu:47-658).
//
//   GpuScratch          src/qwen3_gpu.h:47-113     grow-only activations + the decode graph
//   GpuForwardOptions   src/qwen3_gpu.h:115-122    layer_limit, capture_hidden
//   GpuForwardFull      src/qwen3_gpu.h:136-139    whole segment, with or without the KV cache
//   GpuForwardStep      src/qwen3_gpu.h:145-146    one token at pos == cache length
//   GpuForwardStepDev   src/qwen3_gpu.h:151-152    the same with the token already on the device
//   GpuGenerateOptions  src/qwen3_gpu.h:156-181
//   GpuGenerate         src/qwen3_gpu.h:197-199    sample -> forward loop, optionally as a HIP graph
//   GpuGenerateGreedy   src/qwen3_gpu.h:207-210
//
// What differs from the reference layer (src/qwen3_gpu.cu:47-109), same maths:
//   * the residual add of each sub-layer is folded into the RMSNorm that reads
//     the sum next (GpuAddRmsNorm: the next layer's attn_norm, the ffn_norm, or
//     the output norm), so x is read and written once per sub-layer; at one
//     token the add and the norm run inside the matmul that reads the norm
//     (GpuNormMatMulQuantGroup / GpuNormMatMulQuantSwiGLU), and the residual
//     alternates between x and x_alt;
//   * q / k RMSNorm, RoPE and the fp16 K/V store run as one pass
//     (GpuQkNormRopeKv) on the cache path, and at one token inside the
//     attention launch (GpuQkNormRopeKvAttention);
//   * q / k / v go through GpuMatMulQuantGroup (at one token one launch per
//     same-type run, bit-identical to separate calls), and gate / up with the
//     SwiGLU through GpuMatMulQuantSwiGLU (at one token one launch that writes
//     silu(gate) * up from each row pair's totals);
//   * the decode graph reads the sampled token straight from the sampler's
//     output slot instead of copying it into the token buffer first.
// The no-cache path keeps the reference's separate norm / RoPE steps and runs
// attention on the fp32 k / v rows (GpuCausalAttention).
#ifndef RPG_AMD_QWEN3_GPU_H_
#define RPG_AMD_QWEN3_GPU_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

#include "gpu_model.h"
#include "kernels_gpu.h"
#include "sampler_gpu.h"

namespace rpg {

// Device activations of one forward (src/qwen3_gpu.h:47-113). Buffers only
// grow: indices inside a forward are segment-local, and a buffer sized for the
// longest segment seen serves every shorter one.
class GpuScratch {
 public:
  GpuScratch() = default;
  ~GpuScratch();
  GpuScratch(const GpuScratch&) = delete;
  GpuScratch& operator=(const GpuScratch&) = delete;
  GpuScratch(GpuScratch&&) = delete;
  GpuScratch& operator=(GpuScratch&&) = delete;

  void Ensure(const ModelMeta& c, int64_t seq);
  int64_t bytes() const;

  DeviceBuffer x;       // [seq, hidden] residual stream
  DeviceBuffer x_alt;   // [hidden] the residual stream's second buffer at one token
  DeviceBuffer h;       // [seq, hidden] normalised input of a sub-layer
  DeviceBuffer q;       // [seq, q_dim]
  DeviceBuffer k;       // [seq, kv_dim]
  DeviceBuffer v;       // [seq, kv_dim]
  DeviceBuffer attn;    // [seq, q_dim]
  DeviceBuffer proj;    // [seq, hidden] sub-layer output, added to x by the next norm
  DeviceBuffer gate;    // [seq, intermediate]
  DeviceBuffer up;      // [seq, intermediate]
  DeviceBuffer toks;    // [seq] int32
  DeviceBuffer logits;  // [seq, vocab]
  DeviceBuffer probs;   // [vocab] sampling distribution
  DeviceBuffer argmax_idx;  // [1] int32: the sampled / argmax token

  // The captured decode step (sample -> forward) and everything it baked in:
  // the device addresses it reads and writes (model, cache layers, every
  // scratch buffer), the shapes and the sampling options. The graph is
  // replayed only while a fresh signature compares equal, element by element.
  hipGraphExec_t graph_exec = nullptr;
  std::vector<uint64_t> graph_signature;

  // Every device buffer above, in declaration order.
  std::vector<const DeviceBuffer*> buffers() const;
};

struct GpuForwardOptions {
  // Run only the first layer_limit layers (0 = all); the output norm and
  // lm_head are then skipped and logits come back empty.
  int32_t layer_limit = 0;
  // When set: the residual stream after the embedding and after every layer,
  // [n_use + 1, seq, hidden].
  std::vector<float>* capture_hidden = nullptr;
};

// Whole segment (src/qwen3_gpu.h:136-139). tokens are host ids. With kv the
// segment is appended at position kv->len() and attends to the whole cache;
// kv->len() grows by seq. logits == nullptr keeps the result on the device
// (s->logits, [seq, vocab]).
void GpuForwardFull(const GpuModel& m, const int32_t* tokens, int64_t seq, GpuScratch* s,
                    std::vector<float>* logits, const GpuForwardOptions& opt = GpuForwardOptions(),
                    GpuKvCache* kv = nullptr);

// One token at pos == kv->len() (src/qwen3_gpu.h:145-146).
void GpuForwardStep(const GpuModel& m, int32_t token, int64_t pos, GpuKvCache* kv, GpuScratch* s,
                    std::vector<float>* logits);

// The same with the token id in device memory (src/qwen3_gpu.h:151-152). An id
// outside [0, vocab) embeds as a zero row (the gather never reads out of range).
void GpuForwardStepDev(const GpuModel& m, const int32_t* token_dev, int64_t pos, GpuKvCache* kv, GpuScratch* s);

struct GpuGenerateOptions {
  int32_t max_tokens = 64;
  std::vector<int32_t> stop_ids;  // the stop token itself is returned
  SampleOptions sample{0.0f, 0, 1.0f};  // temperature 0: greedy
  uint64_t seed = 0;
  std::vector<float>* step_logits = nullptr;  // [returned tokens, vocab] when set
  bool use_graph = false;                     // ignored (with a warning) when step_logits is set
};

// Generation from the distribution at first_logits_dev ([vocab] on the device,
// usually the last row of s->logits after a prefill), appending the returned
// ids to out_ids (src/qwen3_gpu.h:197-199). Every returned token, the stop token
// included, is written to the cache, so kv->len() == prompt + returned tokens.
// The sampling counter of a token is its absolute position (kv->len() before
// it is written). A full context is an error, not a silent stop.
void GpuGenerate(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                 const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids);

// GpuGenerate with temperature 0 (src/qwen3_gpu.h:207-210).
void GpuGenerateGreedy(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                       const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids);

}  // namespace rpg

#endif  // RPG_AMD_QWEN3_GPU_H_
