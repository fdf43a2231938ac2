// extern "C" boundary (include/rpg_ops.h): each entry forwards to the C++
// operator layer and converts exceptions into the negative-status /
// thread-local-message convention.
#include "../../include/rpg_ops.h"

#include <algorithm>
#include <cstring>
#include <exception>
#include <new>
#include <utility>
#include <vector>

#include "common.h"
#include "hip_common.h"
#include "kernels_gpu.h"
#include "gpu_model.h"
#include "qwen3_gpu.h"
#include "sampler_gpu.h"

namespace {

template <typename F>
int32_t Guard(F&& f) {
  try {
    f();
    return RPG_OPS_OK;
  } catch (const rpg::Error&) {
    return -1;  // Throw already recorded the message
  } catch (const std::bad_alloc&) {
    rpg::SetLastError("out of host memory");
    return -2;
  } catch (const std::exception& e) {
    rpg::SetLastError(e.what());
    return -3;
  } catch (...) {
    rpg::SetLastError("unknown error");
    return -4;
  }
}

int32_t CopyText(const std::string& text, char* buf, int32_t cap) {
  if (buf != nullptr && cap > 0) {
    const size_t n = std::min(text.size(), static_cast<size_t>(cap - 1));
    std::memcpy(buf, text.data(), n);
    buf[n] = '\0';
  }
  return static_cast<int32_t>(std::min<size_t>(text.size(), 0x7FFFFFFF));
}

void FillMeta(const rpg::ModelMeta& c, rpg_model_meta_t* out) {
  RPG_CHECK(out != nullptr, "null output pointer");
  std::memset(out, 0, sizeof(*out));
  CopyText(c.arch, out->arch, sizeof(out->arch));
  CopyText(c.name, out->name, sizeof(out->name));
  out->n_layers = c.n_layers;
  out->hidden = c.hidden;
  out->n_heads = c.n_heads;
  out->n_kv_heads = c.n_kv_heads;
  out->head_dim = c.head_dim;
  out->value_dim = c.value_dim;
  out->intermediate = c.intermediate;
  out->vocab = c.vocab;
  out->context_length = c.context_length;
  out->rope_theta = c.rope_theta;
  out->rms_eps = c.rms_eps;
  out->tied_embeddings = c.tied_embeddings ? 1 : 0;
  out->bos_id = c.bos_id;
  out->eos_id = c.eos_id;
  out->pad_id = c.pad_id;
  out->add_bos = c.add_bos ? 1 : 0;
  out->weight_bytes = c.weight_bytes;
}

rpg::SampleOptions Options(float temperature, int32_t top_k, float top_p) {
  rpg::SampleOptions o;
  o.temperature = temperature;
  o.top_k = top_k;
  o.top_p = top_p;
  return o;
}

}  // namespace

struct rpg_gguf {
  rpg::GgufFile file;
};

struct rpg_model {
  rpg::GpuModel model;
};

struct rpg_kv {
  rpg::GpuKvCache kv;
};

struct rpg_scratch {
  rpg::GpuScratch s;
};

extern "C" {

const char* rpg_ops_version(void) { return "0.1.0"; }

const char* rpg_ops_last_error(void) { return rpg::LastError(); }

int32_t rpg_ops_init(void) {
  return Guard([] {
    (void)rpg::PosStagingPtr();
    rpg::GpuAttentionNoAllocInit();
  });
}

int32_t rpg_ops_set_stream(void* stream) {
  return Guard([&] { rpg::SetEngineStream(static_cast<hipStream_t>(stream)); });
}

void* rpg_ops_get_stream(void) { return static_cast<void*>(rpg::EngineStream()); }

int64_t* rpg_ops_pos_staging_ptr(void) {
  int64_t* p = nullptr;
  if (Guard([&] { p = rpg::PosStagingPtr(); }) != RPG_OPS_OK) return nullptr;
  return p;
}

int32_t rpg_ops_stage_pos0(int64_t pos) {
  return Guard([&] { rpg::StagePos0(pos); });
}

int32_t rpg_ops_device_info(char* buf, int32_t cap) {
  int32_t avail = 0;
  const int32_t rc = Guard([&] {
    RPG_CHECK(buf != nullptr && cap > 0, "device_info needs a buffer");
    const rpg::DeviceInfo d = rpg::QueryDevice(0);
    const std::string s = rpg::DescribeDevice(d);
    std::strncpy(buf, s.c_str(), static_cast<size_t>(cap) - 1);
    buf[cap - 1] = '\0';
    avail = d.available ? 1 : 0;
  });
  return rc < 0 ? rc : avail;
}

int64_t rpg_ops_type_row_bytes(uint32_t type, int64_t n_elems) {
  int64_t out = -1;
  const int32_t rc = Guard([&] { out = rpg::TypeRowBytes(type, n_elems); });
  return rc < 0 ? rc : out;
}

int32_t rpg_ops_build_rope_table(int32_t head_dim, double theta, int64_t n_pos, float* out_host) {
  return Guard([&] {
    RPG_CHECK(out_host != nullptr && n_pos > 0, "build_rope_table needs n_pos > 0 and an output buffer");
    const std::vector<float> t = rpg::BuildRopeTable(head_dim, theta, n_pos);
    std::memcpy(out_host, t.data(), t.size() * sizeof(float));
  });
}

int32_t rpg_op_dequant_row(uint32_t type, const uint8_t* src_dev, int64_t n_elems, float* dst_dev) {
  return Guard([&] { rpg::GpuDequantRow(type, src_dev, n_elems, dst_dev); });
}

int32_t rpg_op_rms_norm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, float eps,
                        float* out) {
  return Guard([&] { rpg::GpuRmsNorm(x, w, n_rows, n, stride, eps, out); });
}

int32_t rpg_op_rope(float* x, int32_t n_heads, int32_t head_dim, const float* rope_tab, int64_t pos0,
                    int64_t n_rows) {
  return Guard([&] { rpg::GpuRope(x, n_heads, head_dim, rope_tab, pos0, n_rows); });
}

int32_t rpg_op_kv_write(const float* k, const float* v, int32_t n_kv_heads, int32_t head_dim, int64_t pos0,
                        int64_t seq, uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq) {
  return Guard([&] { rpg::GpuKvWrite(k, v, n_kv_heads, head_dim, pos0, seq, k_layer, v_layer, max_seq); });
}

int32_t rpg_op_silu_mul_inplace(float* gate, const float* up, int64_t n) {
  return Guard([&] { rpg::GpuSiluMulInPlace(gate, up, n); });
}

int32_t rpg_op_vec_add_inplace(float* a, const float* b, int64_t n) {
  return Guard([&] { rpg::GpuVecAddInPlace(a, b, n); });
}

int32_t rpg_op_embedding_lookup(uint32_t type, const uint8_t* emb, int64_t rows, int64_t cols, const int32_t* toks,
                                int64_t seq, float* x) {
  return Guard([&] { rpg::GpuEmbeddingLookupRaw(type, emb, rows, cols, toks, seq, x); });
}

int32_t rpg_op_attention_from_cache(const float* q, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                    int64_t pos0, int64_t seq, const uint16_t* k_layer, const uint16_t* v_layer,
                                    int64_t max_seq, float* out, int64_t sh_positions) {
  return Guard([&] {
    rpg::ModelMeta c;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.head_dim = head_dim;
    rpg::GpuAttentionFromCache(c, pos0, q, seq, k_layer, v_layer, max_seq, out, sh_positions);
  });
}

int32_t rpg_op_qk_norm_rope_kv_attention(const float* q, const float* k, const float* v, const float* q_norm,
                                         const float* k_norm, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                         const float* rope_tab, int64_t rope_rows, int64_t pos0, float eps,
                                         uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq, float* out,
                                         int64_t sh_positions, int32_t* fused) {
  return Guard([&] {
    RPG_CHECK(fused != nullptr, "qk_norm_rope_kv_attention: null flag");
    *fused = 0;
    rpg::ModelMeta c;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.head_dim = head_dim;
    c.rms_eps = eps;
    *fused = rpg::GpuQkNormRopeKvAttention(c, pos0, q, k, v, q_norm, k_norm, rope_tab, rope_rows, k_layer, v_layer,
                                           max_seq, out, sh_positions)
                 ? 1
                 : 0;
  });
}

int32_t rpg_op_attention_from_cache_noalloc(const float* q, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                            int64_t pos0, int64_t seq, const uint16_t* k_layer,
                                            const uint16_t* v_layer, int64_t max_seq, float* out,
                                            int64_t sh_positions) {
  return Guard([&] {
    rpg::ModelMeta c;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.head_dim = head_dim;
    rpg::GpuAttentionFromCacheNoAlloc(c, pos0, q, seq, k_layer, v_layer, max_seq, out, sh_positions);
  });
}

int32_t rpg_op_attention_warmup(int64_t sh_positions) {
  return Guard([&] { rpg::GpuAttentionWarmupShmem(sh_positions); });
}

int32_t rpg_gguf_open(const char* path, rpg_gguf** out) {
  return Guard([&] {
    RPG_CHECK(path != nullptr && out != nullptr, "null argument");
    *out = nullptr;
    auto* g = new rpg_gguf{rpg::GgufFile::Open(path)};
    *out = g;
  });
}

int32_t rpg_gguf_close(rpg_gguf* g) {
  delete g;
  return RPG_OPS_OK;
}

int64_t rpg_gguf_tensor_count(const rpg_gguf* g) {
  if (g == nullptr) {
    rpg::SetLastError("null GGUF handle");
    return -1;
  }
  return static_cast<int64_t>(g->file.tensors().size());
}

int32_t rpg_gguf_tensor_info(const rpg_gguf* g, int64_t index, char* name, int32_t cap, rpg_tensor_info_t* out) {
  return Guard([&] {
    RPG_CHECK(g != nullptr && out != nullptr, "null argument");
    const auto& ts = g->file.tensors();
    RPG_CHECK(index >= 0 && index < static_cast<int64_t>(ts.size()), "tensor index %lld out of range (%zu)",
              static_cast<long long>(index), ts.size());
    const rpg::GgufTensor& t = ts[static_cast<size_t>(index)];
    CopyText(t.name, name, cap);
    std::memset(out, 0, sizeof(*out));
    out->data = g->file.TensorBytes(t);
    out->type = t.type;
    out->n_dims = static_cast<int32_t>(t.dims.size());
    for (size_t d = 0; d < t.dims.size(); ++d) out->dims[d] = t.dims[d];
    out->n_elements = t.n_elements;
    out->n_bytes = t.n_bytes;
    out->file_offset = g->file.TensorFileOffset(t);
  });
}

int32_t rpg_gguf_meta(const rpg_gguf* g, const char* key, int64_t item, int32_t* kind, double* num, char* str,
                      int32_t cap, int64_t* n_items) {
  int32_t len = 0;
  const int32_t rc = Guard([&] {
    RPG_CHECK(g != nullptr && key != nullptr && kind != nullptr, "null argument");
    const rpg::GgufValue* v = &g->file.Meta(key);
    if (item >= 0) {
      RPG_CHECK(v->IsArray(), "metadata %s is not an array", key);
      RPG_CHECK(item < static_cast<int64_t>(v->items.size()), "item %lld out of range for %s (%zu items)",
                static_cast<long long>(item), key, v->items.size());
      v = &v->items[static_cast<size_t>(item)];
    }
    if (num) *num = 0.0;
    if (n_items) *n_items = 0;
    switch (v->kind) {
      case rpg::GgufValue::Kind::kNone: *kind = 0; break;
      case rpg::GgufValue::Kind::kNumber:
        *kind = 1;
        if (num) *num = v->num;
        break;
      case rpg::GgufValue::Kind::kBool:
        *kind = 2;
        if (num) *num = v->flag ? 1.0 : 0.0;
        break;
      case rpg::GgufValue::Kind::kString:
        *kind = 3;
        len = CopyText(v->str, str, cap);
        break;
      case rpg::GgufValue::Kind::kArray:
        *kind = 4;
        if (n_items) *n_items = static_cast<int64_t>(v->items.size());
        break;
    }
  });
  return rc < 0 ? rc : len;
}

int32_t rpg_gguf_model_meta(const rpg_gguf* g, rpg_model_meta_t* out) {
  return Guard([&] {
    RPG_CHECK(g != nullptr, "null GGUF handle");
    FillMeta(rpg::ReadModelMeta(g->file), out);
  });
}

int32_t rpg_gguf_describe(const rpg_gguf* g, char* buf, int32_t cap) {
  int32_t len = 0;
  const int32_t rc = Guard([&] {
    RPG_CHECK(g != nullptr, "null GGUF handle");
    len = CopyText(g->file.Describe(), buf, cap);
  });
  return rc < 0 ? rc : len;
}

int32_t rpg_model_load(const char* path, int32_t max_pos, rpg_model** out) {
  return Guard([&] {
    RPG_CHECK(path != nullptr && out != nullptr, "null argument");
    *out = nullptr;
    auto* m = new rpg_model{rpg::GpuModel::Load(path, max_pos)};
    *out = m;
  });
}

int32_t rpg_model_free(rpg_model* m) {
  delete m;
  return RPG_OPS_OK;
}

int32_t rpg_model_meta(const rpg_model* m, rpg_model_meta_t* out) {
  return Guard([&] {
    RPG_CHECK(m != nullptr, "null model handle");
    FillMeta(m->model.config(), out);
  });
}

int32_t rpg_model_tensor(const rpg_model* m, const char* name, rpg_tensor_info_t* out) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && name != nullptr && out != nullptr, "null argument");
    const rpg::GpuTensor* t = m->model.FindTensor(name);
    RPG_CHECK(t != nullptr && t->valid(), "the model has no tensor %s", name);
    std::memset(out, 0, sizeof(*out));
    out->data = t->buf.data();
    out->type = t->type;
    out->n_dims = t->matrix ? 2 : 1;
    out->dims[0] = t->matrix ? t->cols : t->n_elements;
    out->dims[1] = t->matrix ? t->rows : 1;
    out->n_elements = t->n_elements;
    out->n_bytes = t->bytes();
    const rpg::GgufTensor* src = m->model.gguf().Find(
        std::string(name) == "output.weight" && m->model.config().tied_embeddings ? "token_embd.weight" : name);
    out->file_offset = src != nullptr ? m->model.gguf().TensorFileOffset(*src) : -1;
  });
}

int32_t rpg_model_rope(const rpg_model* m, const float** tab, int64_t* n_pos) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && tab != nullptr && n_pos != nullptr, "null argument");
    *tab = m->model.rope_dev();
    *n_pos = m->model.rope_positions();
  });
}

int32_t rpg_model_describe(const rpg_model* m, char* buf, int32_t cap) {
  int32_t len = 0;
  const int32_t rc = Guard([&] {
    RPG_CHECK(m != nullptr, "null model handle");
    len = CopyText(m->model.Describe(), buf, cap);
  });
  return rc < 0 ? rc : len;
}

int32_t rpg_model_device_bytes(const rpg_model* m, int64_t* out) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && out != nullptr, "null argument");
    *out = m->model.device_bytes();
  });
}

int32_t rpg_model_upload_stats(const rpg_model* m, int64_t* bytes, double* parse_seconds, double* upload_seconds) {
  return Guard([&] {
    RPG_CHECK(m != nullptr, "null model handle");
    const rpg::UploadStats& s = m->model.upload_stats();
    if (bytes) *bytes = s.bytes;
    if (parse_seconds) *parse_seconds = s.parse_seconds;
    if (upload_seconds) *upload_seconds = s.upload_seconds;
  });
}

int32_t rpg_kv_create(const rpg_model* m, int64_t max_seq, rpg_kv** out) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && out != nullptr, "null argument");
    *out = nullptr;
    *out = new rpg_kv{rpg::GpuKvCache(m->model.config(), max_seq)};
  });
}

int32_t rpg_kv_create_shape(int32_t n_layers, int32_t n_kv_heads, int32_t head_dim, int64_t max_seq, rpg_kv** out) {
  return Guard([&] {
    RPG_CHECK(out != nullptr, "null argument");
    *out = nullptr;
    rpg::ModelMeta c;
    c.n_layers = n_layers;
    c.n_kv_heads = n_kv_heads;
    c.head_dim = head_dim;
    *out = new rpg_kv{rpg::GpuKvCache(c, max_seq)};
  });
}

int32_t rpg_kv_free(rpg_kv* kv) {
  delete kv;
  return RPG_OPS_OK;
}

int32_t rpg_kv_info(const rpg_kv* kv, int64_t* len, int64_t* max_seq, int64_t* bytes) {
  return Guard([&] {
    RPG_CHECK(kv != nullptr, "null cache handle");
    if (len) *len = kv->kv.len();
    if (max_seq) *max_seq = kv->kv.max_seq();
    if (bytes) *bytes = kv->kv.bytes();
  });
}

int32_t rpg_kv_set_len(rpg_kv* kv, int64_t len) {
  return Guard([&] {
    RPG_CHECK(kv != nullptr, "null cache handle");
    kv->kv.SetLen(len);
  });
}

int32_t rpg_kv_layer(rpg_kv* kv, int32_t layer, uint16_t** k, uint16_t** v) {
  return Guard([&] {
    RPG_CHECK(kv != nullptr && k != nullptr && v != nullptr, "null argument");
    *k = kv->kv.k_layer(layer);
    *v = kv->kv.v_layer(layer);
  });
}

int32_t rpg_scratch_create(rpg_scratch** out) {
  return Guard([&] {
    RPG_CHECK(out != nullptr, "null argument");
    *out = new rpg_scratch();
  });
}

int32_t rpg_scratch_free(rpg_scratch* s) {
  delete s;
  return RPG_OPS_OK;
}

int32_t rpg_scratch_logits(rpg_scratch* s, const float** logits_dev, const int32_t** token_dev) {
  return Guard([&] {
    RPG_CHECK(s != nullptr, "null scratch handle");
    RPG_CHECK(!s->s.logits.empty(), "the scratch holds no logits yet (run a forward first)");
    if (logits_dev) *logits_dev = static_cast<const float*>(s->s.logits.data());
    if (token_dev) *token_dev = static_cast<const int32_t*>(s->s.argmax_idx.data());
  });
}

int32_t rpg_forward_full(const rpg_model* m, const int32_t* tokens, int64_t seq, rpg_scratch* s, float* logits,
                         int32_t layer_limit, float* hidden, rpg_kv* kv) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && s != nullptr, "null model or scratch handle");
    RPG_CHECK(layer_limit >= 0, "layer_limit must not be negative");
    const rpg::ModelMeta& c = m->model.config();
    RPG_CHECK(logits == nullptr || layer_limit == 0 || layer_limit >= c.n_layers,
              "logits were requested from a truncated forward (layer_limit %d of %d layers)", layer_limit,
              c.n_layers);
    std::vector<float> hid;
    std::vector<float> lg;
    rpg::GpuForwardOptions opt;
    opt.layer_limit = layer_limit;
    if (hidden != nullptr) opt.capture_hidden = &hid;
    rpg::GpuForwardFull(m->model, tokens, seq, &s->s, logits != nullptr ? &lg : nullptr, opt,
                        kv != nullptr ? &kv->kv : nullptr);
    if (hidden != nullptr) std::memcpy(hidden, hid.data(), hid.size() * sizeof(float));
    if (logits != nullptr) std::memcpy(logits, lg.data(), lg.size() * sizeof(float));
  });
}

int32_t rpg_forward_step(const rpg_model* m, int32_t token, int64_t pos, rpg_kv* kv, rpg_scratch* s, float* logits) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && s != nullptr && kv != nullptr, "null handle");
    std::vector<float> lg;
    rpg::GpuForwardStep(m->model, token, pos, &kv->kv, &s->s, logits != nullptr ? &lg : nullptr);
    if (logits != nullptr) std::memcpy(logits, lg.data(), lg.size() * sizeof(float));
  });
}

int32_t rpg_forward_step_dev(const rpg_model* m, const int32_t* token_dev, int64_t pos, rpg_kv* kv, rpg_scratch* s) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && s != nullptr && kv != nullptr, "null handle");
    rpg::GpuForwardStepDev(m->model, token_dev, pos, &kv->kv, &s->s);
  });
}

int32_t rpg_generate(const rpg_model* m, rpg_kv* kv, rpg_scratch* s, const float* first_logits_dev,
                     const rpg_generate_opts_t* opts, int32_t* out_ids, int32_t out_cap, int32_t* n_out) {
  return Guard([&] {
    RPG_CHECK(m != nullptr && s != nullptr && kv != nullptr && opts != nullptr, "null handle");
    RPG_CHECK(out_ids != nullptr && n_out != nullptr, "null output");
    *n_out = 0;
    RPG_CHECK(opts->max_tokens > 0 && opts->max_tokens <= out_cap, "max_tokens (%d) must be in [1, out_cap = %d]",
              opts->max_tokens, out_cap);
    RPG_CHECK(opts->n_stop >= 0 && (opts->n_stop == 0 || opts->stop_ids != nullptr), "bad stop id list");
    const int64_t vocab = m->model.config().vocab;
    rpg::GpuGenerateOptions g;
    g.max_tokens = opts->max_tokens;
    g.stop_ids.assign(opts->stop_ids, opts->stop_ids + opts->n_stop);
    g.sample.temperature = opts->temperature;
    g.sample.top_k = opts->top_k;
    g.sample.top_p = opts->top_p;
    g.seed = opts->seed;
    g.use_graph = opts->use_graph != 0;
    std::vector<float> steps;
    if (opts->step_logits != nullptr) {
      RPG_CHECK(opts->step_logits_cap >= static_cast<int64_t>(opts->max_tokens) * vocab,
                "step_logits holds %lld floats, max_tokens x vocab = %lld are needed",
                static_cast<long long>(opts->step_logits_cap),
                static_cast<long long>(static_cast<int64_t>(opts->max_tokens) * vocab));
      g.step_logits = &steps;
    }
    std::vector<int32_t> ids;
    rpg::GpuGenerate(m->model, &kv->kv, &s->s, first_logits_dev, g, &ids);
    std::memcpy(out_ids, ids.data(), ids.size() * sizeof(int32_t));
    if (opts->step_logits != nullptr) std::memcpy(opts->step_logits, steps.data(), steps.size() * sizeof(float));
    *n_out = static_cast<int32_t>(ids.size());
  });
}

int32_t rpg_op_argmax(const float* x, int64_t n, int32_t* out_idx) {
  return Guard([&] { rpg::GpuArgMax(x, n, out_idx); });
}

uint64_t rpg_sample_split_mix64(uint64_t x) { return rpg::DevSplitMix64(x); }

uint64_t rpg_sample_counter_rng(uint64_t seed, uint64_t counter) { return rpg::DevCounterRng(seed, counter); }

float rpg_sample_counter_uniform(uint64_t seed, uint64_t counter) { return rpg::DevCounterUniform(seed, counter); }

int32_t rpg_op_filter_to_probs(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p,
                               float* probs) {
  return Guard([&] { rpg::GpuFilterToProbs(logits, n, Options(temperature, top_k, top_p), probs); });
}

int32_t rpg_op_inverse_sample(const float* probs, int64_t n, float u, int32_t* out_idx) {
  return Guard([&] { rpg::GpuInverseSample(probs, n, u, out_idx); });
}

int32_t rpg_op_sample_token(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p,
                            uint64_t seed, uint64_t counter, float* probs, int32_t* out_idx) {
  return Guard(
      [&] { rpg::GpuSampleToken(logits, n, Options(temperature, top_k, top_p), seed, counter, probs, out_idx); });
}

int32_t rpg_op_sample_token_dev(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p,
                                uint64_t seed, const uint64_t* counter_dev, float* probs, int32_t* out_idx) {
  return Guard([&] {
    rpg::GpuSampleTokenDev(logits, n, Options(temperature, top_k, top_p), seed, counter_dev, probs, out_idx);
  });
}

int32_t rpg_op_sampler_warmup(void) {
  return Guard([] { rpg::GpuSamplerWarmup(); });
}

int32_t rpg_op_matmul_quant(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const float* x,
                            int64_t n_tokens, float* out) {
  return Guard([&] { rpg::GpuMatMulQuantRaw(type, w, rows, cols, x, n_tokens, out); });
}

int32_t rpg_op_set_force_generic_matmul(int32_t force) {
  return Guard([&] { rpg::GpuSetForceGenericMatMul(force != 0); });
}

int32_t rpg_op_force_generic_matmul(void) { return rpg::GpuForceGenericMatMul() ? 1 : 0; }

int32_t rpg_op_matmul_quant_swiglu(uint32_t type, const uint8_t* w_gate, const uint8_t* w_up, int64_t rows,
                                   int64_t cols, const float* x, int64_t n_tokens, float* gate, float* up) {
  return Guard([&] {
    RPG_CHECK(w_gate != nullptr && w_up != nullptr, "null weight pointer");
    RPG_CHECK(rows > 0 && cols > 0, "invalid matrix shape [%lld, %lld]", static_cast<long long>(rows),
              static_cast<long long>(cols));
    const int64_t rb = rpg::TypeRowBytes(type, cols);
    RPG_CHECK(rb > 0, "unsupported matrix type %u or width %lld", type, static_cast<long long>(cols));
    rpg::GpuTensor g, u;
    for (auto [t, p] : {std::pair<rpg::GpuTensor*, const uint8_t*>{&g, w_gate}, {&u, w_up}}) {
      t->buf = rpg::DeviceBuffer::View(const_cast<uint8_t*>(p), static_cast<size_t>(rows * rb));
      t->type = type;
      t->matrix = true;
      t->rows = rows;
      t->cols = cols;
      t->n_elements = rows * cols;
    }
    rpg::GpuMatMulQuantSwiGLU(g, u, x, n_tokens, gate, up);
  });
}

namespace {

// Non-owning GpuTensor views of n matrices of one width (the group entry points).
void GroupViews(int32_t n, const uint32_t* types, const uint8_t* const* ws, const int64_t* rows, int64_t cols,
                std::vector<rpg::GpuTensor>* t, std::vector<const rpg::GpuTensor*>* p) {
  RPG_CHECK(n > 0 && n <= 64 && types && ws && rows, "matmul group: bad arguments (n = %d)", n);
  t->resize(static_cast<size_t>(n));
  p->resize(static_cast<size_t>(n));
  for (int32_t i = 0; i < n; ++i) {
    RPG_CHECK(ws[i] != nullptr && rows[i] > 0 && cols > 0, "matmul group: matrix %d is empty", i);
    const int64_t rb = rpg::TypeRowBytes(types[i], cols);
    RPG_CHECK(rb > 0, "matmul group: unsupported type %u or width %lld", types[i], static_cast<long long>(cols));
    rpg::GpuTensor& g = (*t)[static_cast<size_t>(i)];
    g.type = types[i];
    g.matrix = true;
    g.rows = rows[i];
    g.cols = cols;
    g.n_elements = rows[i] * cols;
    g.buf = rpg::DeviceBuffer::View(const_cast<uint8_t*>(ws[i]), static_cast<size_t>(rows[i] * rb));
    (*p)[static_cast<size_t>(i)] = &g;
  }
}

}  // namespace

int32_t rpg_op_matmul_quant_group(int32_t n, const uint32_t* types, const uint8_t* const* ws, const int64_t* rows,
                                  int64_t cols, const float* x, int64_t n_tokens, float* const* outs) {
  return Guard([&] {
    RPG_CHECK(outs != nullptr, "matmul group: null output array");
    std::vector<rpg::GpuTensor> t;
    std::vector<const rpg::GpuTensor*> p;
    GroupViews(n, types, ws, rows, cols, &t, &p);
    rpg::GpuMatMulQuantGroup(p.data(), n, x, n_tokens, outs);
  });
}

int32_t rpg_op_norm_matmul_quant_group(int32_t n, const uint32_t* types, const uint8_t* const* ws,
                                       const int64_t* rows, int64_t cols, const float* x, const float* d,
                                       const float* norm_w, float eps, float* x_out, float* const* outs,
                                       int32_t* fused) {
  return Guard([&] {
    RPG_CHECK(outs != nullptr && fused != nullptr, "norm matmul group: null output array or flag");
    *fused = 0;
    std::vector<rpg::GpuTensor> t;
    std::vector<const rpg::GpuTensor*> p;
    GroupViews(n, types, ws, rows, cols, &t, &p);
    *fused = rpg::GpuNormMatMulQuantGroup(rpg::GpuNormIn{x, d, norm_w, eps, x_out}, p.data(), n, outs) ? 1 : 0;
  });
}

int32_t rpg_op_norm_matmul_quant_swiglu(uint32_t type, const uint8_t* w_gate, const uint8_t* w_up, int64_t rows,
                                        int64_t cols, const float* x, const float* d, const float* norm_w, float eps,
                                        float* x_out, float* gate, float* up, int32_t* fused) {
  return Guard([&] {
    RPG_CHECK(fused != nullptr, "norm matmul swiglu: null flag");
    *fused = 0;
    const uint32_t types[2] = {type, type};
    const uint8_t* ws[2] = {w_gate, w_up};
    const int64_t rs[2] = {rows, rows};
    std::vector<rpg::GpuTensor> t;
    std::vector<const rpg::GpuTensor*> p;
    GroupViews(2, types, ws, rs, cols, &t, &p);
    *fused = rpg::GpuNormMatMulQuantSwiGLU(rpg::GpuNormIn{x, d, norm_w, eps, x_out}, t[0], t[1], gate, up) ? 1 : 0;
  });
}

int32_t rpg_op_add_rms_norm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n, float eps,
                            float* out) {
  return Guard([&] { rpg::GpuAddRmsNorm(x, d, w, n_rows, n, eps, out); });
}

int32_t rpg_op_qk_norm_rope_kv(float* q, float* k, const float* v, const float* q_norm, const float* k_norm,
                               int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const float* rope_tab,
                               int64_t rope_rows, int64_t pos0, int64_t seq, float eps, uint16_t* k_layer,
                               uint16_t* v_layer, int64_t max_seq, int32_t write_k_f32) {
  return Guard([&] {
    rpg::GpuQkNormRopeKv(q, k, v, q_norm, k_norm, n_heads, n_kv_heads, head_dim, rope_tab, rope_rows, pos0, seq,
                         eps, k_layer, v_layer, max_seq, write_k_f32 != 0);
  });
}

int32_t rpg_op_stream_copy(const void* src, void* dst, int64_t bytes) {
  return Guard([&] { rpg::GpuStreamCopy(src, dst, bytes); });
}

int32_t rpg_op_stream_read(const void* src, int64_t bytes, uint32_t key, uint32_t* sink) {
  return Guard([&] { rpg::GpuStreamRead(src, bytes, key, sink); });
}

int32_t rpg_op_stream_fill(void* dst, int64_t bytes, uint32_t pattern) {
  return Guard([&] { rpg::GpuStreamFill(dst, bytes, pattern); });
}

int32_t rpg_op_f16_sweep(float* out_dev) {
  return Guard([&] { rpg::GpuF16Sweep(out_dev); });
}

int32_t rpg_ops_profile_start(int32_t max_launches) {
  return Guard([&] { rpg::ProfileStart(max_launches); });
}

int32_t rpg_ops_profile_stop(void) {
  return Guard([] { rpg::ProfileStop(); });
}

int32_t rpg_ops_profile_report(char* buf, int32_t cap) {
  int32_t len = 0;
  const int32_t rc = Guard([&] {
    RPG_CHECK(buf != nullptr && cap > 0, "profile_report needs a buffer");
    const std::string s = rpg::ProfileReport();
    std::strncpy(buf, s.c_str(), static_cast<size_t>(cap) - 1);
    buf[cap - 1] = '\0';
    len = static_cast<int32_t>(s.size());
  });
  return rc < 0 ? rc : len;
}

}  // extern "C"
