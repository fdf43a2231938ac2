// Qwen3 forward / generation over the device operators (reference
// src/qwen3_gpu.cu:47-658; interface and the differences from the reference's
// layer are described in qwen3_gpu.h).
#include "qwen3_gpu.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <utility>

namespace rpg {
namespace {

float* F(DeviceBuffer& b) { return static_cast<float*>(b.data()); }

// Sub-layer input normalisation with the pending residual folded in: when the
// previous sub-layer left its output in proj, x += proj happens inside the norm
// (GpuAddRmsNorm); the bits of x are those of the reference's separate
// GpuVecAddInPlace (one IEEE add per element).
class Residual {
 public:
  Residual(float* x, float* x_alt, float* proj, float* h, int64_t seq, int64_t hidden, float eps)
      : x_(x), alt_(x_alt), proj_(proj), h_(h), seq_(seq), hidden_(hidden), eps_(eps) {}

  // The residual stream (x or x_alt: a fused norm writes x + proj to the other).
  float* x() const { return x_; }

  // At one token the norm runs inside the matmul that reads it (GpuNormIn):
  // the sum x + proj, when pending, goes to the other buffer (keep) or nowhere
  // (the output norm, after which x is not read). Returns the fused call's
  // result; false leaves everything as it was, for NormInto.
  template <typename Call>
  bool Fused(const float* w, bool keep, Call&& call) {
    if (seq_ != 1) return false;
    const bool write = pending_ && keep;
    const GpuNormIn in{x_, pending_ ? proj_ : nullptr, w, eps_, write ? alt_ : nullptr};
    if (!call(in)) return false;
    if (write) std::swap(x_, alt_);
    pending_ = false;
    return true;
  }

  void NormInto(const float* w) {
    if (pending_) {
      GpuAddRmsNorm(x_, proj_, w, seq_, hidden_, eps_, h_);
    } else {
      GpuRmsNorm(x_, w, seq_, hidden_, hidden_, eps_, h_);
    }
    pending_ = false;
  }
  // proj now holds a sub-layer output that belongs to x.
  void Defer() { pending_ = true; }
  // Makes x the residual stream itself (before it is read back).
  void Settle() {
    if (pending_) GpuVecAddInPlace(x_, proj_, seq_ * hidden_);
    pending_ = false;
  }

 private:
  float* x_;
  float* alt_;
  float* proj_;
  float* h_;
  int64_t seq_;
  int64_t hidden_;
  float eps_;
  bool pending_ = false;
};

// One decoder layer (reference GpuForwardLayer, src/qwen3_gpu.cu:47-109):
//   h = RMSNorm(x) * attn_norm; q, k, v = h W_q^T, h W_k^T, h W_v^T
//   q, k <- RoPE(RMSNorm_head(.) * q_norm / k_norm)   (v is not rotated)
//   cache path: k, v -> fp16 cache at pos0 + t, attention over the cache
//   x += attn W_o^T; h = RMSNorm(x) * ffn_norm
//   x += (silu(h W_gate^T) * h W_up^T) W_down^T
void ForwardLayer(const GpuModel& m, int32_t layer, int64_t pos0, GpuScratch* s, int64_t seq, GpuKvCache* kv,
                  int64_t attn_sh_positions, Residual* res) {
  const ModelMeta& c = m.config();
  const GpuLayer& w = m.layers()[static_cast<size_t>(layer)];
  const int32_t hd = c.head_dim;
  float* q = F(s->q);
  float* k = F(s->k);
  float* v = F(s->v);
  float* attn = F(s->attn);
  float* h = F(s->h);

  {
    const float* nw = static_cast<const float*>(w.attn_norm.buf.data());
    const GpuTensor* mats[3] = {&w.attn_q, &w.attn_k, &w.attn_v};
    float* outs[3] = {q, k, v};
    if (!res->Fused(nw, true, [&](const GpuNormIn& in) { return GpuNormMatMulQuantGroup(in, mats, 3, outs); })) {
      res->NormInto(nw);
      GpuMatMulQuantGroup(mats, 3, h, seq, outs);
    }
  }
  const float* qn = static_cast<const float*>(w.q_norm.buf.data());
  const float* kn = static_cast<const float*>(w.k_norm.buf.data());
  if (kv != nullptr) {
    // One token: norm, RoPE, the K/V store and attention in one decode launch.
    const bool fused = seq == 1 && GpuQkNormRopeKvAttention(c, pos0, q, k, v, qn, kn, m.rope_dev(),
                                                            m.rope_positions(), kv->k_layer(layer),
                                                            kv->v_layer(layer), kv->max_seq(), attn,
                                                            attn_sh_positions);
    if (!fused) {
      // the segment's K/V must be in the cache before attention reads it: token t
      // attends to positions <= pos0 + t, including those written just now
      GpuQkNormRopeKv(q, k, v, qn, kn, c.n_heads, c.n_kv_heads, hd, m.rope_dev(), m.rope_positions(), pos0, seq,
                      c.rms_eps, kv->k_layer(layer), kv->v_layer(layer), kv->max_seq(), false);
      GpuAttentionFromCache(c, pos0, q, seq, kv->k_layer(layer), kv->v_layer(layer), kv->max_seq(), attn,
                            attn_sh_positions);
    }
  } else {
    GpuRmsNorm(q, qn, seq * c.n_heads, hd, hd, c.rms_eps, q);
    GpuRmsNorm(k, kn, seq * c.n_kv_heads, hd, hd, c.rms_eps, k);
    GpuRope(q, c.n_heads, hd, m.rope_dev(), pos0, seq);
    GpuRope(k, c.n_kv_heads, hd, m.rope_dev(), pos0, seq);
    GpuCausalAttention(c, q, k, v, seq, attn);
  }
  GpuMatMulQuant(w.attn_o, attn, seq, F(s->proj));
  res->Defer();

  // gate <- silu(gate) * up
  const float* fw = static_cast<const float*>(w.ffn_norm.buf.data());
  if (!res->Fused(fw, true, [&](const GpuNormIn& in) {
        return GpuNormMatMulQuantSwiGLU(in, w.ffn_gate, w.ffn_up, F(s->gate), F(s->up));
      })) {
    res->NormInto(fw);
    GpuMatMulQuantSwiGLU(w.ffn_gate, w.ffn_up, h, seq, F(s->gate), F(s->up));
  }
  GpuMatMulQuant(w.ffn_down, F(s->gate), seq, F(s->proj));
  res->Defer();
}

// Forward of a segment whose token ids are already on the device
// (reference ForwardCore, src/qwen3_gpu.cu:120-180): embedding, the layers,
// output norm and lm_head into s->logits. No host checks and no cache length
// update: the callers do those, which keeps this part capturable.
void ForwardCore(const GpuModel& m, int64_t seq, GpuScratch* s, const int32_t* toks_dev,
                 std::vector<float>* logits, const GpuForwardOptions& opt, GpuKvCache* kv,
                 int64_t attn_sh_positions) {
  const ModelMeta& c = m.config();
  const int64_t hidden = c.hidden;
  const int64_t pos0 = kv != nullptr ? kv->len() : 0;
  const int32_t n_use = opt.layer_limit > 0 && opt.layer_limit < c.n_layers ? opt.layer_limit : c.n_layers;
  const size_t row_floats = static_cast<size_t>(seq) * static_cast<size_t>(hidden);
  if (opt.capture_hidden != nullptr) opt.capture_hidden->assign(static_cast<size_t>(n_use + 1) * row_floats, 0.0f);

  s->Ensure(c, seq);
  // Qwen3 does not scale the embedding by sqrt(hidden)
  GpuEmbeddingLookup(m.token_embd(), toks_dev, seq, F(s->x));
  if (opt.capture_hidden != nullptr) s->x.Download(opt.capture_hidden->data(), row_floats * sizeof(float));

  Residual res(F(s->x), F(s->x_alt), F(s->proj), F(s->h), seq, hidden, c.rms_eps);
  for (int32_t l = 0; l < n_use; ++l) {
    ForwardLayer(m, l, pos0, s, seq, kv, attn_sh_positions, &res);
    if (opt.capture_hidden != nullptr) {
      res.Settle();
      (res.x() == F(s->x) ? s->x : s->x_alt).Download(opt.capture_hidden->data() + static_cast<size_t>(l + 1) * row_floats, row_floats * sizeof(float));
    }
  }
  if (n_use < c.n_layers) {
    // truncated run: the output norm and lm_head depend on the deeper layers
    res.Settle();
    if (logits != nullptr) logits->clear();
    return;
  }
  // Always computed, also when logits == nullptr: decoding reads s->logits.
  const float* ow = static_cast<const float*>(m.output_norm().buf.data());
  const GpuTensor* head[1] = {&m.lm_head()};
  float* head_out[1] = {F(s->logits)};
  if (!res.Fused(ow, false, [&](const GpuNormIn& in) { return GpuNormMatMulQuantGroup(in, head, 1, head_out); })) {
    res.NormInto(ow);
    GpuMatMulQuant(m.lm_head(), F(s->h), seq, F(s->logits));
  }
  if (logits == nullptr) return;
  logits->assign(static_cast<size_t>(seq) * static_cast<size_t>(c.vocab), 0.0f);
  s->logits.Download(logits->data(), logits->size() * sizeof(float));
}

// Host-side admission of a segment of `seq` tokens starting at position pos0:
// it must fit the RoPE table and, on the cache path, the cache.
void CheckPositions(const GpuModel& m, const GpuKvCache* kv, int64_t pos0, int64_t seq) {
  const long long end = static_cast<long long>(pos0 + seq);
  if (pos0 + seq > m.rope_positions()) {
    Throw("positions up to %lld requested, but the RoPE table was built for %lld (load the model with a larger "
          "max_pos, or reset the cache)",
          end, static_cast<long long>(m.rope_positions()));
  }
  if (kv != nullptr && pos0 + seq > kv->max_seq()) {
    Throw("positions up to %lld do not fit the KV cache capacity of %lld", end, static_cast<long long>(kv->max_seq()));
  }
}

void CheckCache(const GpuModel& m, const GpuKvCache* kv) {
  const ModelMeta& c = m.config();
  const bool same = kv->valid() && kv->n_layers() == c.n_layers && kv->n_kv_heads() == c.n_kv_heads &&
                    kv->head_dim() == c.head_dim;
  if (!same) {
    Throw("the KV cache was built for %d layers / %d kv heads / head_dim %d, the model has %d / %d / %d",
          kv->n_layers(), kv->n_kv_heads(), kv->head_dim(), c.n_layers, c.n_kv_heads, c.head_dim);
  }
}

// Decode steps append: the step's position must be the cache's current length.
void CheckAppend(const GpuKvCache* kv, int64_t pos) {
  if (pos != kv->len()) {
    Throw("a decode step writes at the end of the cache (length %lld); position %lld was given",
          static_cast<long long>(kv->len()), static_cast<long long>(pos));
  }
}

}  // namespace

// ---------------------------------------------------------------- GpuScratch

std::vector<const DeviceBuffer*> GpuScratch::buffers() const {
  return {&x, &x_alt, &h, &q, &k, &v, &attn, &proj, &gate, &up, &toks, &logits, &probs, &argmax_idx};
}

void GpuScratch::Ensure(const ModelMeta& c, int64_t seq) {
  if (seq <= 0) Throw("GpuScratch::Ensure: a segment of %lld tokens needs no buffers", static_cast<long long>(seq));
  const int64_t fp = sizeof(float);
  // Bytes each buffer must hold for a segment of `seq` tokens: per-token
  // activations scale with seq; x_alt (the one-token residual twin), the
  // sampling distribution and the sampled id do not.
  const std::pair<DeviceBuffer*, int64_t> sizes[] = {
      {&x, seq * c.hidden * fp},          {&x_alt, c.hidden * fp},
      {&h, seq * c.hidden * fp},          {&q, seq * c.q_dim() * fp},
      {&k, seq * c.kv_dim() * fp},        {&v, seq * c.kv_dim() * fp},
      {&attn, seq * c.q_dim() * fp},      {&proj, seq * c.hidden * fp},
      {&gate, seq * c.intermediate * fp}, {&up, seq * c.intermediate * fp},
      {&toks, seq * 4},                   {&logits, seq * c.vocab * fp},
      {&probs, c.vocab * fp},             {&argmax_idx, 4},
  };
  for (const auto& [buf, want] : sizes) {
    if (static_cast<int64_t>(buf->size()) < want) buf->Alloc(static_cast<size_t>(want));
  }
}

int64_t GpuScratch::bytes() const {
  int64_t total = 0;
  for (const DeviceBuffer* b : buffers()) total += static_cast<int64_t>(b->size());
  return total;
}

GpuScratch::~GpuScratch() {
  if (graph_exec == nullptr) return;
  // A destructor cannot report failure; the only realistic one is a runtime
  // already torn down at process exit, where the graph is gone anyway.
  const hipError_t e = hipGraphExecDestroy(graph_exec);
  if (e != hipSuccess) RPG_LOG_WARN("decode graph not released (%s)", hipGetErrorString(e));
  graph_exec = nullptr;
}

// ---------------------------------------------------------------- forward

void GpuForwardFull(const GpuModel& m, const int32_t* tokens, int64_t seq, GpuScratch* s, std::vector<float>* logits,
                    const GpuForwardOptions& opt, GpuKvCache* kv) {
  const ModelMeta& c = m.config();
  if (s == nullptr || tokens == nullptr) Throw("GpuForwardFull: %s is null", s == nullptr ? "scratch" : "tokens");
  if (seq <= 0) Throw("GpuForwardFull: the token segment is empty");
  if (kv != nullptr) CheckCache(m, kv);
  const int64_t pos0 = kv != nullptr ? kv->len() : 0;
  CheckPositions(m, kv, pos0, seq);
  // Ids are checked here, on the host: the device gather turns a bad id into a
  // zero row instead of failing, which would hide the caller's mistake.
  const int32_t* bad = std::find_if(tokens, tokens + seq, [&c](int32_t id) { return id < 0 || id >= c.vocab; });
  if (bad != tokens + seq) {
    Throw("token %lld of the segment is %d, out of range for a vocabulary of %d",
          static_cast<long long>(bad - tokens), *bad, c.vocab);
  }
  s->Ensure(c, seq);
  RPG_HIP_CHECK(hipMemcpyAsync(s->toks.data(), tokens, static_cast<size_t>(seq) * sizeof(int32_t),
                               hipMemcpyHostToDevice, EngineStream()));
  ForwardCore(m, seq, s, static_cast<const int32_t*>(s->toks.data()), logits, opt, kv, -1);
  // The cache grows only once every layer has been written.
  if (kv != nullptr) kv->SetLen(pos0 + seq);
}

void GpuForwardStep(const GpuModel& m, int32_t token, int64_t pos, GpuKvCache* kv, GpuScratch* s,
                    std::vector<float>* logits) {
  if (kv == nullptr) Throw("GpuForwardStep: a decode step needs the KV cache");
  CheckAppend(kv, pos);
  GpuForwardFull(m, &token, 1, s, logits, GpuForwardOptions(), kv);
}

void GpuForwardStepDev(const GpuModel& m, const int32_t* token_dev, int64_t pos, GpuKvCache* kv, GpuScratch* s) {
  if (kv == nullptr || s == nullptr || token_dev == nullptr) {
    Throw("GpuForwardStepDev: the %s is null", kv == nullptr ? "KV cache" : s == nullptr ? "scratch" : "token pointer");
  }
  CheckCache(m, kv);
  CheckAppend(kv, pos);
  CheckPositions(m, kv, pos, 1);
  ForwardCore(m, 1, s, token_dev, nullptr, GpuForwardOptions(), kv, kv->max_seq());
  kv->SetLen(pos + 1);
}

// ---------------------------------------------------------------- generation

namespace {

// Everything a captured decode step depends on, as plain words. Two
// signatures compare equal only if a replay would touch exactly the same
// memory with the same shapes and sampling parameters; no hashing, so no
// collision can ever replay a stale graph.
std::vector<uint64_t> DecodeStepSignature(const GpuModel& m, const GpuKvCache* kv, const GpuScratch* s,
                                          const GpuGenerateOptions& opt) {
  const ModelMeta& c = m.config();
  auto bits = [](float f) {
    uint32_t u;
    std::memcpy(&u, &f, sizeof(u));
    return static_cast<uint64_t>(u);
  };
  std::vector<uint64_t> sig = {
      reinterpret_cast<uintptr_t>(&m),
      reinterpret_cast<uintptr_t>(m.token_embd().buf.data()),
      reinterpret_cast<uintptr_t>(m.lm_head().buf.data()),
      reinterpret_cast<uintptr_t>(m.rope_dev()),
      reinterpret_cast<uintptr_t>(kv),
      reinterpret_cast<uintptr_t>(kv->k_layer(0)),
      reinterpret_cast<uintptr_t>(kv->v_layer(0)),
      static_cast<uint64_t>(kv->max_seq()),
      static_cast<uint64_t>(c.n_layers),
      static_cast<uint64_t>(c.hidden),
      static_cast<uint64_t>(c.intermediate),
      static_cast<uint64_t>(c.vocab),
      static_cast<uint64_t>(c.n_heads) << 32 | static_cast<uint32_t>(c.n_kv_heads),
      static_cast<uint64_t>(c.head_dim),
      bits(opt.sample.temperature) << 32 | bits(opt.sample.top_p),
      static_cast<uint64_t>(static_cast<uint32_t>(opt.sample.top_k)),
      opt.seed,
  };
  for (const DeviceBuffer* b : s->buffers()) sig.push_back(reinterpret_cast<uintptr_t>(b->data()));
  return sig;
}

// Captures one decode step on the capture stream: sample the next token from
// s->logits (counter = the staged position), then the forward of that token,
// which overwrites s->logits. Everything the step allocates is allocated first.
hipGraphExec_t CaptureDecodeStep(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const GpuGenerateOptions& opt) {
  const hipStream_t cap = CaptureStream();
  if (cap == nullptr) return nullptr;
  const ModelMeta& c = m.config();
  GpuSamplerWarmup();
  int64_t* pos_dev = PosStagingPtr();
  s->Ensure(c, 1);
  GpuAttentionWarmupShmem(kv->max_seq());
  float* probs = F(s->probs);
  int32_t* idx = static_cast<int32_t*>(s->argmax_idx.data());

  hipGraph_t graph = nullptr;
  {
    ScopedEngineStream guard(cap);
    const hipError_t be = hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal);
    if (be != hipSuccess) {
      (void)hipGetLastError();
      RPG_LOG_WARN("hipStreamBeginCapture failed (%s); generating with per-step launches", hipGetErrorString(be));
      return nullptr;
    }
    try {
      GpuSampleTokenDev(F(s->logits), c.vocab, opt.sample, opt.seed, reinterpret_cast<const uint64_t*>(pos_dev),
                        probs, idx);
      ForwardCore(m, 1, s, idx, nullptr, GpuForwardOptions(), kv, kv->max_seq());
      RPG_HIP_CHECK(hipStreamEndCapture(cap, &graph));
    } catch (...) {
      (void)hipStreamEndCapture(cap, &graph);
      if (graph != nullptr) (void)hipGraphDestroy(graph);
      throw;
    }
  }
  if (graph == nullptr) return nullptr;
  hipGraphExec_t exec = nullptr;
  const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (ie != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return exec;
}

bool IsStop(const GpuGenerateOptions& opt, int32_t id) {
  for (const int32_t sid : opt.stop_ids) {
    if (sid == id) return true;
  }
  return false;
}

void CheckRoom(const GpuModel& m, const GpuKvCache* kv, int32_t generated) {
  RPG_CHECK(kv->len() < kv->max_seq(),
            "KV cache has no free slot: all %lld positions are taken after %d generated tokens (reset it, or size it for more positions)",
            static_cast<long long>(kv->max_seq()), generated);
  RPG_CHECK(kv->len() + 1 <= m.rope_positions(), "position %lld is beyond the %lld positions the RoPE table covers",
            static_cast<long long>(kv->len() + 1), static_cast<long long>(m.rope_positions()));
}

bool GenerateGraph(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const GpuGenerateOptions& opt,
                   const float* first_logits_dev, std::vector<int32_t>* out_ids) {
  const ModelMeta& c = m.config();
  const hipStream_t cap = CaptureStream();
  if (cap == nullptr) return false;
  ScopedEngineStream guard(cap);
  if (first_logits_dev != F(s->logits)) {
    RPG_HIP_CHECK(hipMemcpyAsync(s->logits.data(), first_logits_dev, static_cast<size_t>(c.vocab) * sizeof(float),
                                 hipMemcpyDeviceToDevice, cap));
  }
  CheckRoom(m, kv, 1);  // the capture itself appends at kv->len()
  std::vector<uint64_t> sig = DecodeStepSignature(m, kv, s, opt);
  if (s->graph_exec != nullptr && s->graph_signature != sig) {
    (void)hipGraphExecDestroy(s->graph_exec);
    s->graph_exec = nullptr;
    s->graph_signature.clear();
  }
  if (s->graph_exec == nullptr) {
    s->graph_exec = CaptureDecodeStep(m, kv, s, opt);
    // Capturing may have grown nothing (everything is allocated first), but the
    // signature is taken again so it describes exactly what was captured.
    if (s->graph_exec != nullptr) s->graph_signature = DecodeStepSignature(m, kv, s, opt);
  }
  if (s->graph_exec == nullptr) {
    RPG_LOG_WARN("HIP graph capture is unavailable; generating with per-step launches");
    return false;
  }
  const int32_t* idx = static_cast<const int32_t*>(s->argmax_idx.data());
  for (int32_t i = 0; i < opt.max_tokens; ++i) {
    CheckRoom(m, kv, i + 1);
    const int64_t pos = kv->len();
    StagePos0(pos);  // the position the token is written at, and its sampling counter
    RPG_HIP_CHECK(hipGraphLaunch(s->graph_exec, cap));
    int32_t next = 0;
    RPG_HIP_CHECK(hipMemcpyAsync(&next, idx, sizeof(int32_t), hipMemcpyDeviceToHost, cap));
    RPG_HIP_CHECK(hipStreamSynchronize(cap));
    out_ids->push_back(next);
    kv->SetLen(pos + 1);
    if (IsStop(opt, next)) break;
  }
  return true;
}

void GenerateNoGraph(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const GpuGenerateOptions& opt,
                     const float* first_logits_dev, std::vector<int32_t>* out_ids) {
  const ModelMeta& c = m.config();
  float* probs = F(s->probs);
  int32_t* idx = static_cast<int32_t*>(s->argmax_idx.data());
  const float* cur = first_logits_dev;
  for (int32_t i = 0; i < opt.max_tokens; ++i) {
    GpuSampleToken(cur, c.vocab, opt.sample, opt.seed, static_cast<uint64_t>(kv->len()), probs, idx);
    int32_t next = 0;
    RPG_HIP_CHECK(hipMemcpyAsync(&next, idx, sizeof(int32_t), hipMemcpyDeviceToHost, EngineStream()));
    RPG_HIP_CHECK(hipStreamSynchronize(EngineStream()));
    out_ids->push_back(next);
    if (opt.step_logits != nullptr) {
      const size_t base = opt.step_logits->size();
      opt.step_logits->resize(base + static_cast<size_t>(c.vocab));
      RPG_HIP_CHECK(hipMemcpyAsync(opt.step_logits->data() + base, cur, static_cast<size_t>(c.vocab) * sizeof(float),
                                   hipMemcpyDeviceToHost, EngineStream()));
      RPG_HIP_CHECK(hipStreamSynchronize(EngineStream()));
    }
    const bool stop = IsStop(opt, next);
    CheckRoom(m, kv, i + 1);
    GpuForwardStep(m, next, kv->len(), kv, s, nullptr);
    cur = F(s->logits);
    if (stop) break;
  }
}

}  // namespace

void GpuGenerate(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                 const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids) {
  const ModelMeta& c = m.config();
  RPG_CHECK(kv != nullptr, "GpuGenerate: no KV cache was given");
  RPG_CHECK(s != nullptr && out_ids != nullptr, "GpuGenerate got a null scratch or output");
  RPG_CHECK(first_logits_dev != nullptr, "GpuGenerate: first_logits_dev is null; the first token is sampled from the last prefill row's logits");
  RPG_CHECK(opt.max_tokens > 0, "GpuGenerate: max_tokens has to be at least 1 (got %d)", opt.max_tokens);
  RPG_CHECK(!s->argmax_idx.empty() && s->probs.size() >= static_cast<size_t>(c.vocab) * sizeof(float),
            "the scratch has not been sized yet (run a prefill first)");
  CheckCache(m, kv);
  if (opt.use_graph && opt.step_logits != nullptr) {
    RPG_LOG_WARN("GpuGenerate: step_logits are requested, so the decode loop runs without a HIP graph");
  }
  const bool use_graph = opt.use_graph && opt.step_logits == nullptr;
  if (use_graph && GenerateGraph(m, kv, s, opt, first_logits_dev, out_ids)) return;
  GenerateNoGraph(m, kv, s, opt, first_logits_dev, out_ids);
}

void GpuGenerateGreedy(const GpuModel& m, GpuKvCache* kv, GpuScratch* s, const float* first_logits_dev,
                       const GpuGenerateOptions& opt, std::vector<int32_t>* out_ids) {
  GpuGenerateOptions g = opt;
  g.sample.temperature = 0.0f;
  GpuGenerate(m, kv, s, first_logits_dev, g, out_ids);
}

}  // namespace rpg
