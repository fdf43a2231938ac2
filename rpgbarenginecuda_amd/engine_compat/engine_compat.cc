// The reference GPU layer's C++ interface (cuda_common.h, gpu_model.h,
// kv_cache_gpu.h, qwen3_gpu.h in this directory) implemented over
// librpg_ops.so's C ABI. Every failure of the library becomes rpg::Throw with
// the library's message, so the engine's ABI boundary reports it exactly as
// it reports its own errors (src/engine.cc:231-239).
#include <algorithm>
#include <cstdio>
#include <utility>
#include <vector>

#include "cuda_common.h"
#include "gpu_model.h"
#include "kv_cache_gpu.h"
#include "qwen3_gpu.h"
#include "rpg_ops.h"

namespace rpg {
namespace {

void Check(int32_t rc, const char* what) {
  if (rc >= 0) return;
  const char* why = rpg_ops_last_error();
  Throw("%s: %s", what, (why != nullptr && *why != '\0') ? why : "librpg_ops reported an error");
}

}  // namespace

// ---------------------------------------------------------------- device

DeviceInfo QueryDevice(int index) {
  DeviceInfo d;
  if (index != 0) {
    d.reason = "librpg_ops drives device 0 of the process (HIP_VISIBLE_DEVICES selects which GPU that is)";
    return d;
  }
  char text[512] = {0};
  const int32_t rc = rpg_ops_device_info(text, static_cast<int32_t>(sizeof(text)));
  d.available = rc == 1;
  if (d.available) {
    d.name = text;
  } else {
    d.reason = rc < 0 ? std::string(rpg_ops_last_error()) : std::string(text);
    if (d.reason.empty()) d.reason = "no usable HIP device";
  }
  return d;
}

std::string DescribeDevice(const DeviceInfo& d) { return d.available ? d.name : "no usable GPU: " + d.reason; }

// ---------------------------------------------------------------- model

GpuModel GpuModel::Load(const std::string& path, int32_t max_pos) {
  GpuModel m;
  m.gguf_ = GgufFile::Open(path);
  m.cfg_ = ReadModelMeta(m.gguf_);
  m.tokenizer_ = Tokenizer::FromGguf(m.gguf_);
  Check(rpg_model_load(path.c_str(), max_pos, &m.handle_), "rpg_model_load");
  // The library read the same file with its own GGUF reader: the shapes it
  // uploaded must be the ones the engine derived.
  rpg_model_meta_t lib{};
  Check(rpg_model_meta(m.handle_, &lib), "rpg_model_meta");
  const ModelMeta& c = m.cfg_;
  const bool same = lib.n_layers == c.n_layers && lib.hidden == c.hidden && lib.n_heads == c.n_heads &&
                    lib.n_kv_heads == c.n_kv_heads && lib.head_dim == c.head_dim &&
                    lib.intermediate == c.intermediate && lib.vocab == c.vocab &&
                    (lib.tied_embeddings != 0) == c.tied_embeddings;
  if (!same) {
    Throw("%s: librpg_ops read %d layers / hidden %d / %d x %d heads of %d / ffn %d / vocab %d, the engine's "
          "metadata says %d / %d / %d x %d of %d / %d / %d",
          path.c_str(), lib.n_layers, lib.hidden, lib.n_heads, lib.n_kv_heads, lib.head_dim, lib.intermediate,
          lib.vocab, c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.intermediate, c.vocab);
  }
  const float* tab = nullptr;
  Check(rpg_model_rope(m.handle_, &tab, &m.rope_positions_), "rpg_model_rope");
  return m;
}

GpuModel::GpuModel(GpuModel&& o) noexcept
    : gguf_(std::move(o.gguf_)),
      cfg_(std::move(o.cfg_)),
      tokenizer_(std::move(o.tokenizer_)),
      handle_(std::exchange(o.handle_, nullptr)),
      rope_positions_(o.rope_positions_) {}

GpuModel& GpuModel::operator=(GpuModel&& o) noexcept {
  if (this != &o) {
    if (handle_ != nullptr) rpg_model_free(handle_);
    gguf_ = std::move(o.gguf_);
    cfg_ = std::move(o.cfg_);
    tokenizer_ = std::move(o.tokenizer_);
    handle_ = std::exchange(o.handle_, nullptr);
    rope_positions_ = o.rope_positions_;
  }
  return *this;
}

GpuModel::~GpuModel() {
  if (handle_ != nullptr) rpg_model_free(handle_);
}

int64_t GpuModel::device_bytes() const {
  int64_t b = 0;
  Check(rpg_model_device_bytes(handle_, &b), "rpg_model_device_bytes");
  return b;
}

std::string GpuModel::Describe() const {
  char text[1024] = {0};
  Check(rpg_model_describe(handle_, text, static_cast<int32_t>(sizeof(text))), "rpg_model_describe");
  return text;
}

// ---------------------------------------------------------------- KV cache

GpuKvCache::GpuKvCache(const ModelMeta& c, int64_t max_seq)
    : n_layers_(c.n_layers), n_kv_heads_(c.n_kv_heads), head_dim_(c.head_dim), max_seq_(max_seq) {
  Check(rpg_kv_create_shape(c.n_layers, c.n_kv_heads, c.head_dim, max_seq, &handle_), "rpg_kv_create_shape");
}

GpuKvCache::GpuKvCache(GpuKvCache&& o) noexcept
    : handle_(std::exchange(o.handle_, nullptr)),
      n_layers_(o.n_layers_),
      n_kv_heads_(o.n_kv_heads_),
      head_dim_(o.head_dim_),
      max_seq_(o.max_seq_) {}

GpuKvCache& GpuKvCache::operator=(GpuKvCache&& o) noexcept {
  if (this != &o) {
    if (handle_ != nullptr) rpg_kv_free(handle_);
    handle_ = std::exchange(o.handle_, nullptr);
    n_layers_ = o.n_layers_;
    n_kv_heads_ = o.n_kv_heads_;
    head_dim_ = o.head_dim_;
    max_seq_ = o.max_seq_;
  }
  return *this;
}

GpuKvCache::~GpuKvCache() {
  if (handle_ != nullptr) rpg_kv_free(handle_);
}

int64_t GpuKvCache::len() const {
  int64_t n = 0;
  Check(rpg_kv_info(handle_, &n, nullptr, nullptr), "rpg_kv_info");
  return n;
}

void GpuKvCache::SetLen(int64_t n) { Check(rpg_kv_set_len(handle_, n), "rpg_kv_set_len"); }

uint16_t* GpuKvCache::k_layer(int32_t layer) {
  uint16_t *k = nullptr, *v = nullptr;
  Check(rpg_kv_layer(handle_, layer, &k, &v), "rpg_kv_layer");
  return k;
}

uint16_t* GpuKvCache::v_layer(int32_t layer) {
  uint16_t *k = nullptr, *v = nullptr;
  Check(rpg_kv_layer(handle_, layer, &k, &v), "rpg_kv_layer");
  return v;
}

int64_t GpuKvCache::bytes() const {
  int64_t b = 0;
  Check(rpg_kv_info(handle_, nullptr, nullptr, &b), "rpg_kv_info");
  return b;
}

std::string GpuKvCache::Describe() const {
  char text[192];
  std::snprintf(text, sizeof(text), "librpg_ops fp16 KV cache: %d layers x %d kv heads x %lld x %d, %lld filled",
                n_layers_, n_kv_heads_, static_cast<long long>(max_seq_), head_dim_,
                static_cast<long long>(valid() ? len() : 0));
  return text;
}

// ---------------------------------------------------------------- scratch

rpg_scratch* GpuScratch::handle() {
  if (handle_ == nullptr) Check(rpg_scratch_create(&handle_), "rpg_scratch_create");
  return handle_;
}

GpuScratch::~GpuScratch() {
  if (handle_ != nullptr) rpg_scratch_free(handle_);
}

const void* GpuScratch::LogitsView::data() const {
  GpuScratch* s = const_cast<GpuScratch*>(owner_);
  if (s->handle_ == nullptr) return nullptr;
  const float* lg = nullptr;
  Check(rpg_scratch_logits(s->handle_, &lg, nullptr), "rpg_scratch_logits");
  return lg;
}

// ---------------------------------------------------------------- forward

void GpuForwardFull(const GpuModel& m, const int32_t* tokens, int64_t seq, GpuScratch* s, std::vector<float>* logits,
                    const GpuForwardOptions& opt, GpuKvCache* kv) {
  RPG_CHECK(s != nullptr, "GpuForwardFull needs a scratch");
  const ModelMeta& c = m.config();
  const bool truncated = opt.layer_limit > 0 && opt.layer_limit < c.n_layers;
  const int32_t layers_run = truncated ? opt.layer_limit : c.n_layers;
  float* lg = nullptr;
  if (logits != nullptr) {
    logits->clear();  // a truncated run has no logits
    if (!truncated && seq > 0) {
      logits->assign(static_cast<size_t>(seq) * static_cast<size_t>(c.vocab), 0.0f);
      lg = logits->data();
    }
  }
  float* hid = nullptr;
  if (opt.capture_hidden != nullptr && seq > 0) {
    opt.capture_hidden->assign(static_cast<size_t>(layers_run + 1) * static_cast<size_t>(seq) * c.hidden, 0.0f);
    hid = opt.capture_hidden->data();
  }
  Check(rpg_forward_full(m.handle(), tokens, seq, s->handle(), lg, opt.layer_limit, hid,
                         kv != nullptr ? kv->handle() : nullptr),
        "rpg_forward_full");
}

void GpuForwardStep(const GpuModel& m, int32_t token, int64_t pos, GpuKvCache* kv, GpuScratch* s,
                    std::vector<float>* logits) {
  RPG_CHECK(kv != nullptr && s != nullptr, "GpuForwardStep needs a KV cache and a scratch");
  float* lg = nullptr;
  if (logits != nullptr) {
    logits->assign(static_cast<size_t>(m.config().vocab), 0.0f);
    lg = logits->data();
  }
  Check(rpg_forward_step(m.handle(), token, pos, kv->handle(), s->handle(), lg), "rpg_forward_step");
}

void GpuForwardStepDev(const GpuModel& m, const int32_t* token_dev, int64_t pos, GpuKvCache* kv, GpuScratch* s) {
  RPG_CHECK(kv != nullptr && s != nullptr, "GpuForwardStepDev needs a KV cache and a scratch");
  Check(rpg_forward_step_dev(m.handle(), token_dev, pos, kv->handle(), s->handle()), "rpg_forward_step_dev");
}

// ---------------------------------------------------------------- generation

void GpuGenerate(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                 const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids) {
  RPG_CHECK(kv != nullptr && s != nullptr && out_ids != nullptr, "GpuGenerate needs a KV cache, a scratch and an "
                                                                 "output vector");
  RPG_CHECK(opt.max_tokens > 0, "GpuGenerate: max_tokens has to be at least 1 (got %d)", opt.max_tokens);
  out_ids->clear();
  const int64_t vocab = m.config().vocab;
  rpg_generate_opts_t o{};
  o.max_tokens = opt.max_tokens;
  o.stop_ids = opt.stop_ids.data();
  o.n_stop = static_cast<int32_t>(opt.stop_ids.size());
  o.temperature = opt.sample.temperature;
  o.top_k = opt.sample.top_k;
  o.top_p = opt.sample.top_p;
  o.seed = opt.seed;
  // Per-step logits are downloaded after every step, which a replayed graph
  // cannot do: such a call runs the per-step loop, and says so.
  if (opt.use_graph && opt.step_logits != nullptr) {
    RPG_LOG_WARN("GpuGenerate: step_logits are requested, so the decode loop runs without a HIP graph");
  }
  o.use_graph = (opt.use_graph && opt.step_logits == nullptr) ? 1 : 0;
  // One row of `vocab` floats per generated token, appended after whatever the
  // caller's vector already holds.
  std::vector<float> rows;
  if (opt.step_logits != nullptr) {
    rows.assign(static_cast<size_t>(opt.max_tokens) * static_cast<size_t>(vocab), 0.0f);
    o.step_logits = rows.data();
    o.step_logits_cap = static_cast<int64_t>(rows.size());
  }
  std::vector<int32_t> ids(static_cast<size_t>(opt.max_tokens));
  int32_t n = 0;
  Check(rpg_generate(m.handle(), kv->handle(), s->handle(), first_logits_dev, &o, ids.data(), opt.max_tokens, &n),
        "rpg_generate");
  out_ids->assign(ids.begin(), ids.begin() + n);
  if (opt.step_logits != nullptr) {
    opt.step_logits->insert(opt.step_logits->end(), rows.begin(),
                            rows.begin() + static_cast<std::ptrdiff_t>(n) * static_cast<std::ptrdiff_t>(vocab));
  }
}

void GpuGenerateGreedy(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                       const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids) {
  GpuGenerateOptions greedy = opt;
  greedy.sample.temperature = 0.0f;
  GpuGenerate(m, kv, s, first_logits_dev, greedy, out_ids);
}

}  // namespace rpg
