// A Qwen3 GGUF model resident in device memory: quantized weights as their raw
// GGUF bytes, norms as fp32, and the RoPE table.
//
// Interface of the reference's GpuModel and ReadModelMeta (src/gpu_model.h:
// 57-133, src/model_meta.h:67, src/model_meta.cc:11-78); the upload is this
// project's own design for MI355X:
//   * every weight lands in ONE device arena (one hipMalloc, 256-byte aligned
//     slices), so a model is a single allocation that cannot fragment across
//     288 GB of HBM, and GpuTensor::buf is a non-owning view into it;
//   * the file's bytes travel through a ring of pinned staging buffers: host
//     threads pread chunk c+1 out of the page cache while the DMA engine moves
//     chunk c over PCIe on a dedicated copy stream, instead of one synchronous
//     pageable copy per tensor out of the memory map;
//   * norms stored quantized (Q4_K / Q6_K) are dequantized on the device by the
//     same kernel as GpuDequantRow (bit-exact with the reference's host dequant).
// Only F32, Q4_K and Q6_K tensors are accepted, as in the reference
// (src/gpu_model.cu:26-38); anything else is rejected at load time.
#ifndef RPG_AMD_GPU_MODEL_H_
#define RPG_AMD_GPU_MODEL_H_

#include <cstdint>
#include <string>
#include <vector>

#include "gguf.h"
#include "kernels_gpu.h"

namespace rpg {

// Shapes and hyper-parameters from the GGUF metadata (src/model_meta.cc:11-78):
// architecture must be qwen3; head_dim from attention.key_length (else
// hidden / n_heads); vocab = rows of token_embd; tied when neither
// output.weight nor lm_head.weight exists.
ModelMeta ReadModelMeta(const GgufFile& g);

struct GpuLayer {
  GpuTensor attn_norm;  // [hidden] f32
  GpuTensor ffn_norm;   // [hidden] f32
  GpuTensor q_norm;     // [head_dim] f32
  GpuTensor k_norm;     // [head_dim] f32

  GpuTensor attn_q;  // [n_heads*head_dim, hidden]
  GpuTensor attn_k;  // [n_kv_heads*head_dim, hidden]
  GpuTensor attn_v;  // [n_kv_heads*head_dim, hidden]
  GpuTensor attn_o;  // [hidden, n_heads*head_dim]

  GpuTensor ffn_gate;  // [intermediate, hidden]
  GpuTensor ffn_up;    // [intermediate, hidden]
  GpuTensor ffn_down;  // [hidden, intermediate]
};

struct UploadStats {
  int64_t bytes = 0;         // file bytes moved to the device
  double parse_seconds = 0;  // GGUF header, metadata and tensor table
  double upload_seconds = 0; // arena allocation to the last byte on the device
  int32_t chunks = 0;        // staging chunks
  int32_t host_threads = 0;  // threads filling the staging buffers
};

class GpuModel {
 public:
  // max_pos: positions of the RoPE table (capped at context_length, at least 1).
  static GpuModel Load(const std::string& path, int32_t max_pos = 4096);

  const ModelMeta& config() const { return cfg_; }
  const GgufFile& gguf() const { return gguf_; }
  const std::string& path() const { return gguf_.path(); }

  const GpuTensor& token_embd() const { return token_embd_; }
  const GpuTensor& lm_head() const { return cfg_.tied_embeddings ? token_embd_ : lm_head_; }
  const GpuTensor& output_norm() const { return output_norm_; }
  const std::vector<GpuLayer>& layers() const { return layers_; }

  // [rope_positions(), head_dim] fp32, cos | sin per row.
  const float* rope_dev() const { return static_cast<const float*>(rope_.data()); }
  int64_t rope_positions() const { return n_rope_pos_; }

  // The device tensor loaded from the GGUF tensor `name` (output.weight resolves
  // to token_embd when tied); nullptr if there is none.
  const GpuTensor* FindTensor(const std::string& name) const;

  int64_t device_bytes() const;
  const UploadStats& upload_stats() const { return stats_; }
  std::string Describe() const;

 private:
  GgufFile gguf_;
  ModelMeta cfg_;
  DeviceBuffer arena_;
  GpuTensor token_embd_;
  GpuTensor lm_head_;
  GpuTensor output_norm_;
  std::vector<GpuLayer> layers_;
  DeviceBuffer rope_;
  int64_t n_rope_pos_ = 0;
  UploadStats stats_;
};

}  // namespace rpg

#endif  // RPG_AMD_GPU_MODEL_H_
