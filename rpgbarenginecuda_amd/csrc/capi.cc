// extern "C" boundary (include/rpg_ops.h): each entry forwards to the C++
// operator layer and converts exceptions into the negative-status /
// thread-local-message convention.
#include "../../include/rpg_ops.h"

#include <cstring>
#include <exception>
#include <new>
#include <vector>

#include "common.h"
#include "hip_common.h"
#include "kernels_gpu.h"
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

rpg::SampleOptions Options(float temperature, int32_t top_k, float top_p) {
  rpg::SampleOptions o;
  o.temperature = temperature;
  o.top_k = top_k;
  o.top_p = top_p;
  return o;
}

}  // namespace

extern "C" {

const char* rpg_ops_version(void) { return "0.1.0"; }

const char* rpg_ops_last_error(void) { return rpg::LastError(); }

int32_t rpg_ops_init(void) {
  return Guard([] { (void)rpg::PosStagingPtr(); });
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

int32_t rpg_op_attention_warmup(int64_t sh_positions) {
  return Guard([&] { rpg::GpuAttentionWarmupShmem(sh_positions); });
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
