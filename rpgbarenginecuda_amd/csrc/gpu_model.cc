// GGUF -> device upload (see gpu_model.h for the design).
#include "gpu_model.h"

#include <hip/hip_runtime_api.h>

#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>

#include "common.h"

namespace rpg {

// ---------------------------------------------------------------- metadata

ModelMeta ReadModelMeta(const GgufFile& g) {
  ModelMeta m;
  m.arch = g.architecture();
  RPG_CHECK(m.arch == "qwen3", "model architecture is %s; this engine implements qwen3 only", m.arch.c_str());
  m.name = g.MetaStr("general.name", g.MetaStr("general.basename", "(unnamed)"));

  m.n_layers = static_cast<int32_t>(g.ArchInt("block_count", 0));
  m.hidden = static_cast<int32_t>(g.ArchInt("embedding_length", 0));
  m.n_heads = static_cast<int32_t>(g.ArchInt("attention.head_count", 0));
  m.n_kv_heads = static_cast<int32_t>(g.ArchInt("attention.head_count_kv", m.n_heads));
  m.intermediate = static_cast<int32_t>(g.ArchInt("feed_forward_length", 0));
  m.context_length = static_cast<int32_t>(g.ArchInt("context_length", 4096));

  // head_dim comes from key_length; hidden / n_heads only when the key is absent
  const int64_t key_len = g.ArchInt("attention.key_length", 0);
  if (key_len > 0) {
    m.head_dim = static_cast<int32_t>(key_len);
  } else {
    RPG_CHECK(m.n_heads > 0 && m.hidden % m.n_heads == 0,
              "GGUF has no attention.key_length and hidden %d is not a multiple of %d heads", m.hidden, m.n_heads);
    RPG_LOG_WARN("GGUF has no attention.key_length; head_dim = hidden / heads = %d", m.hidden / m.n_heads);
    m.head_dim = m.hidden / m.n_heads;
  }
  m.value_dim = static_cast<int32_t>(g.ArchInt("attention.value_length", m.head_dim));
  m.rope_theta = g.ArchFloat("rope.freq_base", 10000.0f);
  m.rms_eps = g.ArchFloat("attention.layer_norm_rms_epsilon", 1e-6f);

  m.bos_id = static_cast<int32_t>(g.MetaInt("tokenizer.ggml.bos_token_id", -1));
  m.eos_id = static_cast<int32_t>(g.MetaInt("tokenizer.ggml.eos_token_id", -1));
  m.pad_id = static_cast<int32_t>(g.MetaInt("tokenizer.ggml.padding_token_id", -1));
  m.add_bos = g.MetaBool("tokenizer.ggml.add_bos_token", false);

  const GgufTensor* emb = g.Find("token_embd.weight");
  RPG_CHECK(emb != nullptr, "GGUF has no token_embd.weight");
  m.vocab = static_cast<int32_t>(emb->rows());

  RPG_CHECK(m.n_layers > 0 && m.hidden > 0 && m.n_heads > 0 && m.n_kv_heads > 0 && m.head_dim > 0 &&
                m.intermediate > 0 && m.vocab > 0,
            "incomplete GGUF metadata: layers=%d hidden=%d heads=%d kv=%d head_dim=%d ffn=%d vocab=%d", m.n_layers,
            m.hidden, m.n_heads, m.n_kv_heads, m.head_dim, m.intermediate, m.vocab);
  RPG_CHECK(m.n_heads % m.n_kv_heads == 0, "%d query heads are not a multiple of %d KV heads", m.n_heads,
            m.n_kv_heads);
  RPG_CHECK(m.value_dim == m.head_dim, "value_length %d differs from key_length %d", m.value_dim, m.head_dim);

  m.tied_embeddings = g.Find("output.weight") == nullptr && g.Find("lm_head.weight") == nullptr;
  for (const GgufTensor& t : g.tensors()) m.weight_bytes += t.n_bytes;
  return m;
}

namespace {

constexpr int64_t kArenaAlign = 256;
constexpr int kStagingBuffers = 4;
constexpr size_t kStagingBytes = size_t{32} << 20;
constexpr size_t kParallelCopyMin = size_t{4} << 20;

int64_t AlignArena(int64_t x) { return (x + kArenaAlign - 1) / kArenaAlign * kArenaAlign; }

bool DeviceType(uint32_t t) { return t == kGgmlF32 || t == kGgmlQ4_K || t == kGgmlQ6_K; }

void CheckGpuType(const GgufTensor& t) {
  RPG_CHECK(DeviceType(t.type),
            "tensor %s has type %s; the MI355X backend implements only F32 / Q4_K / Q6_K (the Q4_K + Q6_K pair of "
            "Q4_K_M / Q5_K_M files)",
            t.name.c_str(), GgufTypeName(t.type));
}

const GgufTensor& Require(const GgufFile& g, const std::string& name) {
  const GgufTensor* t = g.Find(name);
  if (t == nullptr) {
    Throw("tensor %s not found in the GGUF (arch %s, %zu tensors)", name.c_str(), g.architecture().c_str(),
          g.tensors().size());
  }
  return *t;
}

void CheckShape(const GgufTensor& t, int64_t rows, int64_t cols) {
  if (!t.is_matrix()) {
    Throw("tensor %s has the wrong shape: expected [%lld,%lld] (rows x cols), got %zu dims, not a matrix",
          t.name.c_str(), static_cast<long long>(rows), static_cast<long long>(cols), t.dims.size());
  }
  if (t.rows() != rows || t.cols() != cols) {
    Throw("tensor %s has the wrong shape: expected [%lld,%lld] (rows x cols), got [%lld,%lld]", t.name.c_str(),
          static_cast<long long>(rows), static_cast<long long>(cols), static_cast<long long>(t.rows()),
          static_cast<long long>(t.cols()));
  }
  CheckGpuType(t);
}

// Copies file byte ranges to device addresses through a ring of pinned staging
// buffers: the host fills buffer i (several threads pread from the file) while
// the copy stream drains the buffers filled before it.
// The pinned staging buffers, their events and the copy stream: created on the
// first load and kept for the process (pinning 4 x 32 MiB costs more than a
// small model's whole transfer), one load at a time.
struct StagingRing {
  std::mutex mu;
  bool ready = false;
  hipStream_t stream = nullptr;
  uint8_t* bufs[kStagingBuffers] = {};
  hipEvent_t ev[kStagingBuffers] = {};

  void Init() {
    if (ready) return;
    RPG_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    for (int i = 0; i < kStagingBuffers; ++i) {
      void* p = nullptr;
      RPG_HIP_CHECK(hipHostMalloc(&p, kStagingBytes, hipHostMallocDefault));
      bufs[i] = static_cast<uint8_t*>(p);
      RPG_HIP_CHECK(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
    }
    ready = true;
  }
};

StagingRing& Ring() {
  static StagingRing* r = new StagingRing();  // never destroyed: the HIP runtime may be gone at exit
  return *r;
}

class StagedUploader {
 public:
  StagedUploader(const MappedFile& f, int64_t total) : file_(f), lock_(Ring().mu) {
    StagingRing& r = Ring();
    r.Init();
    stream_ = r.stream;
    for (int i = 0; i < kStagingBuffers; ++i) {
      bufs_[i] = r.bufs[i];
      ev_[i] = r.ev[i];
    }
    cap_ = static_cast<size_t>(std::min<int64_t>(static_cast<int64_t>(kStagingBytes), std::max<int64_t>(total, 1)));
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    threads_ = static_cast<int>(std::min(8u, hw));
  }
  ~StagedUploader() {
    if (stream_ != nullptr) (void)hipStreamSynchronize(stream_);  // the buffers are reused by the next load
  }
  StagedUploader(const StagedUploader&) = delete;
  StagedUploader& operator=(const StagedUploader&) = delete;

  void Copy(int64_t file_off, int64_t n, void* dst) {
    RPG_CHECK(file_off >= 0 && n >= 0 && static_cast<uint64_t>(file_off + n) <= file_.size(),
              "upload range outside the file");
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n > 0) {
      const size_t take = std::min(static_cast<size_t>(n), cap_ - fill_);
      Fill(bufs_[cur_] + fill_, file_off, take);
      pending_.push_back(Piece{fill_, take, d});
      fill_ += take;
      file_off += static_cast<int64_t>(take);
      d += take;
      n -= static_cast<int64_t>(take);
      if (fill_ == cap_) Flush();
    }
  }

  void Finish() {
    if (fill_ > 0) Flush();
    RPG_HIP_CHECK(hipStreamSynchronize(stream_));
  }

  int chunks() const { return chunks_; }
  int threads() const { return threads_; }

 private:
  struct Piece {
    size_t off;
    size_t n;
    uint8_t* dst;
  };

  // File bytes [off, off + n) -> dst with pread: the kernel copies straight out of
  // the page cache, so the mapping's pages are never faulted in (one fault per
  // 4 KiB page was the cost of copying out of the mapping). Large pieces are
  // split over several threads.
  void ReadRange(uint8_t* dst, int64_t off, size_t n) const {
    while (n > 0) {
      const ssize_t got = pread(file_.fd(), dst, n, static_cast<off_t>(off));
      if (got < 0 && errno == EINTR) continue;
      RPG_CHECK(got > 0, "reading %s at %lld failed: %s", file_.path().c_str(), static_cast<long long>(off),
                got < 0 ? std::strerror(errno) : "unexpected end of file");
      dst += got;
      off += got;
      n -= static_cast<size_t>(got);
    }
  }

  void Fill(uint8_t* dst, int64_t off, size_t n) {
    if (n < kParallelCopyMin || threads_ <= 1) {
      ReadRange(dst, off, n);
      return;
    }
    std::vector<std::thread> pool;
    std::vector<std::string> errors(static_cast<size_t>(threads_));
    const size_t per = (n + threads_ - 1) / threads_;
    for (int t = 0; t < threads_; ++t) {
      const size_t lo = per * t;
      if (lo >= n) break;
      const size_t len = std::min(per, n - lo);
      pool.emplace_back([=, &errors] {
        try {
          ReadRange(dst + lo, off + static_cast<int64_t>(lo), len);
        } catch (const std::exception& e) {
          errors[static_cast<size_t>(t)] = e.what();
        }
      });
    }
    for (std::thread& th : pool) th.join();
    for (const std::string& e : errors) RPG_CHECK(e.empty(), "%s", e.c_str());
  }

  void Flush() {
    for (const Piece& p : pending_)
      RPG_HIP_CHECK(hipMemcpyAsync(p.dst, bufs_[cur_] + p.off, p.n, hipMemcpyHostToDevice, stream_));
    RPG_HIP_CHECK(hipEventRecord(ev_[cur_], stream_));
    inflight_[cur_] = true;
    pending_.clear();
    fill_ = 0;
    ++chunks_;
    cur_ = (cur_ + 1) % kStagingBuffers;
    if (inflight_[cur_]) {  // the next buffer is reused only after its copies have landed
      RPG_HIP_CHECK(hipEventSynchronize(ev_[cur_]));
      inflight_[cur_] = false;
    }
  }

  const MappedFile& file_;
  std::lock_guard<std::mutex> lock_;
  size_t cap_ = 0;
  int threads_ = 1;
  hipStream_t stream_ = nullptr;
  uint8_t* bufs_[kStagingBuffers] = {};
  hipEvent_t ev_[kStagingBuffers] = {};
  bool inflight_[kStagingBuffers] = {};
  int cur_ = 0;
  size_t fill_ = 0;
  int chunks_ = 0;
  std::vector<Piece> pending_;
};

// One planned tensor: where its bytes go.
struct Slot {
  const GgufTensor* src;
  GpuTensor* dst;
  bool norm;
  int64_t arena_off;  // the tensor as used (raw bytes, or fp32 for a norm)
  int64_t raw_off;    // quantized norm: raw bytes in the staging region of the arena, else -1
};

}  // namespace

GpuModel GpuModel::Load(const std::string& path, int32_t max_pos) {
  const DeviceInfo dev = QueryDevice(0);
  if (!dev.available) Throw("no usable HIP device, cannot upload the weights: %s", dev.reason.c_str());

  GpuModel m;
  const auto t0 = std::chrono::steady_clock::now();
  m.gguf_ = GgufFile::Open(path);
  m.cfg_ = ReadModelMeta(m.gguf_);
  const ModelMeta& c = m.cfg_;
  const auto t1 = std::chrono::steady_clock::now();

  // ---- plan: shape/type checks first, nothing is allocated until all pass
  std::vector<Slot> slots;
  auto matrix = [&](const std::string& name, int64_t rows, int64_t cols, GpuTensor* dst) {
    const GgufTensor& t = Require(m.gguf_, name);
    CheckShape(t, rows, cols);
    slots.push_back(Slot{&t, dst, false, 0, -1});
  };
  auto norm = [&](const std::string& name, int64_t n, GpuTensor* dst) {
    const GgufTensor& t = Require(m.gguf_, name);
    CheckGpuType(t);
    RPG_CHECK(t.dims.size() == 1, "tensor %s should be a 1-D norm weight, got %zu dims", t.name.c_str(),
              t.dims.size());
    RPG_CHECK(n < 0 || t.n_elements == n, "norm %s has %lld elements, expected %lld", t.name.c_str(),
              static_cast<long long>(t.n_elements), static_cast<long long>(n));
    slots.push_back(Slot{&t, dst, true, 0, -1});
  };

  matrix("token_embd.weight", c.vocab, c.hidden, &m.token_embd_);
  if (!c.tied_embeddings) matrix("output.weight", c.vocab, c.hidden, &m.lm_head_);
  norm("output_norm.weight", c.hidden, &m.output_norm_);
  m.layers_.resize(static_cast<size_t>(c.n_layers));
  for (int32_t l = 0; l < c.n_layers; ++l) {
    GpuLayer& w = m.layers_[static_cast<size_t>(l)];
    const std::string p = "blk." + std::to_string(l) + ".";
    norm(p + "attn_norm.weight", -1, &w.attn_norm);
    norm(p + "ffn_norm.weight", -1, &w.ffn_norm);
    norm(p + "attn_q_norm.weight", -1, &w.q_norm);
    norm(p + "attn_k_norm.weight", -1, &w.k_norm);
    matrix(p + "attn_q.weight", c.q_dim(), c.hidden, &w.attn_q);
    matrix(p + "attn_k.weight", c.kv_dim(), c.hidden, &w.attn_k);
    matrix(p + "attn_v.weight", c.kv_dim(), c.hidden, &w.attn_v);
    matrix(p + "attn_output.weight", c.hidden, c.q_dim(), &w.attn_o);
    matrix(p + "ffn_gate.weight", c.intermediate, c.hidden, &w.ffn_gate);
    matrix(p + "ffn_up.weight", c.intermediate, c.hidden, &w.ffn_up);
    matrix(p + "ffn_down.weight", c.hidden, c.intermediate, &w.ffn_down);
  }

  // ---- arena layout: used tensors, then the raw bytes of quantized norms
  int64_t off = 0;
  for (Slot& s : slots) {
    s.arena_off = off;
    off = AlignArena(off + (s.norm ? 4 * s.src->n_elements : s.src->n_bytes));
  }
  for (Slot& s : slots) {
    if (s.norm && s.src->type != kGgmlF32) {
      s.raw_off = off;
      off = AlignArena(off + s.src->n_bytes);
    }
  }
  m.arena_.Alloc(static_cast<size_t>(std::max<int64_t>(off, kArenaAlign)));
  uint8_t* base = static_cast<uint8_t*>(m.arena_.data());

  // ---- copies in file order (sequential reads of the mapping)
  std::vector<const Slot*> order;
  int64_t total = 0;
  for (const Slot& s : slots) {
    order.push_back(&s);
    total += s.src->n_bytes;
  }
  std::sort(order.begin(), order.end(), [](const Slot* a, const Slot* b) { return a->src->offset < b->src->offset; });
  {
    StagedUploader up(m.gguf_.file(), total);
    for (const Slot* s : order) {
      const int64_t dst = s->raw_off >= 0 ? s->raw_off : s->arena_off;
      up.Copy(m.gguf_.TensorFileOffset(*s->src), s->src->n_bytes, base + dst);
    }
    up.Finish();
    m.stats_.chunks = up.chunks();
    m.stats_.host_threads = up.threads();
  }
  m.stats_.bytes = total;

  // ---- device views; quantized norms dequantized in place on the device
  bool dequant = false;
  for (const Slot& s : slots) {
    GpuTensor& g = *s.dst;
    const GgufTensor& t = *s.src;
    g.n_elements = t.n_elements;
    if (s.norm) {
      g.type = kGgmlF32;
      g.matrix = false;
      g.rows = t.n_elements;
      g.cols = 1;
      g.buf = DeviceBuffer::View(base + s.arena_off, static_cast<size_t>(4 * t.n_elements));
      if (s.raw_off >= 0) {
        GpuDequantRow(t.type, base + s.raw_off, t.n_elements, static_cast<float*>(g.buf.data()));
        dequant = true;
      }
    } else {
      g.type = t.type;
      g.matrix = true;
      g.rows = t.rows();
      g.cols = t.cols();
      g.buf = DeviceBuffer::View(base + s.arena_off, static_cast<size_t>(t.n_bytes));
    }
  }
  if (dequant) RPG_HIP_CHECK(hipStreamSynchronize(EngineStream()));

  // ---- RoPE table
  m.n_rope_pos_ = max_pos > c.context_length ? c.context_length : max_pos;
  if (m.n_rope_pos_ <= 0) m.n_rope_pos_ = 1;
  const std::vector<float> tab = BuildRopeTable(c.head_dim, static_cast<double>(c.rope_theta), m.n_rope_pos_);
  m.rope_.Alloc(tab.size() * sizeof(float));
  m.rope_.Upload(tab.data(), tab.size() * sizeof(float));

  const auto t2 = std::chrono::steady_clock::now();
  m.stats_.parse_seconds = std::chrono::duration<double>(t1 - t0).count();
  m.stats_.upload_seconds = std::chrono::duration<double>(t2 - t1).count();
  return m;
}

const GpuTensor* GpuModel::FindTensor(const std::string& name) const {
  if (name == "token_embd.weight") return &token_embd_;
  if (name == "output.weight") return &lm_head();
  if (name == "output_norm.weight") return &output_norm_;
  int layer = -1, used = 0;
  char suffix[64] = {0};
  if (std::sscanf(name.c_str(), "blk.%d.%63s%n", &layer, suffix, &used) != 2 || layer < 0 ||
      layer >= static_cast<int>(layers_.size()) || used != static_cast<int>(name.size())) {
    return nullptr;
  }
  const GpuLayer& w = layers_[static_cast<size_t>(layer)];
  const std::string s = suffix;
  if (s == "attn_norm.weight") return &w.attn_norm;
  if (s == "ffn_norm.weight") return &w.ffn_norm;
  if (s == "attn_q_norm.weight") return &w.q_norm;
  if (s == "attn_k_norm.weight") return &w.k_norm;
  if (s == "attn_q.weight") return &w.attn_q;
  if (s == "attn_k.weight") return &w.attn_k;
  if (s == "attn_v.weight") return &w.attn_v;
  if (s == "attn_output.weight") return &w.attn_o;
  if (s == "ffn_gate.weight") return &w.ffn_gate;
  if (s == "ffn_up.weight") return &w.ffn_up;
  if (s == "ffn_down.weight") return &w.ffn_down;
  return nullptr;
}

int64_t GpuModel::device_bytes() const { return static_cast<int64_t>(arena_.size() + rope_.size()); }

std::string GpuModel::Describe() const {
  const UploadStats& s = stats_;
  const double gbps = s.upload_seconds > 0 ? static_cast<double>(s.bytes) / s.upload_seconds / 1e9 : 0.0;
  char buf[768];
  std::snprintf(buf, sizeof(buf),
                "%s (%s): %d layers, hidden %d, ffn %d, %d q heads / %d kv heads x %d, vocab %d, rope theta %.6g "
                "(%lld positions), eps %.3g, %s; %lld weight bytes in one %.2f GiB device arena; upload %.3f s "
                "(%.2f GB/s, %d chunks, %d host threads), parse %.3f s",
                cfg_.name.c_str(), cfg_.arch.c_str(), cfg_.n_layers, cfg_.hidden, cfg_.intermediate, cfg_.n_heads,
                cfg_.n_kv_heads, cfg_.head_dim, cfg_.vocab, static_cast<double>(cfg_.rope_theta),
                static_cast<long long>(n_rope_pos_), static_cast<double>(cfg_.rms_eps),
                cfg_.tied_embeddings ? "tied lm_head" : "separate output.weight", static_cast<long long>(s.bytes),
                static_cast<double>(arena_.size()) / (1024.0 * 1024.0 * 1024.0), s.upload_seconds, gbps, s.chunks,
                s.host_threads, s.parse_seconds);
  return buf;
}

}  // namespace rpg
