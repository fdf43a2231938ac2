// Hot-path operators of the Qwen3 layer, MI355X (gfx950) implementation.
//
// The seven reference operators keep their exact C++ signatures
// (reference src/kernels_gpu.h), so the engine code that sequences them
// (src/qwen3_gpu.cu:47-109, 139-140, 168) links against this library unchanged:
//   GpuDequantRow        src/kernels_gpu.h:39-40
//   GpuRmsNorm           src/kernels_gpu.h:65-66
//   GpuRope              src/kernels_gpu.h:71-72
//   GpuKvWrite           src/kernels_gpu.h:97-99
//   GpuSiluMulInPlace    src/kernels_gpu.h:147
//   GpuVecAddInPlace     src/kernels_gpu.h:150
//   GpuEmbeddingLookup   src/kernels_gpu.h:153-154
// and three fused operators replace the unfused sequences of GpuForwardLayer:
//   GpuAddRmsNorm        GpuVecAddInPlace(x += d) ; GpuRmsNorm(x -> out)
//                        (src/qwen3_gpu.cu:100 -> 103, and :108 -> next layer's :69)
//   GpuQkNormRopeKv      GpuRmsNorm(q), GpuRmsNorm(k), GpuRope(q), GpuRope(k),
//                        GpuKvWrite(k, v)   (src/qwen3_gpu.cu:77-91)
//   GpuSiluMulInPlace    already one kernel in the reference (src/qwen3_gpu.cu:106)
//
// Conventions (same as the reference operator layer):
//   * every pointer is a device pointer; the caller owns all buffers;
//   * launches are asynchronous on EngineStream(); nothing synchronises;
//   * argument errors throw rpg::Error before anything is launched;
//   * out may alias x for RMSNorm / RoPE / SiLU-mul / add.
//
// Numerics (what the parity tests hold each operator to):
//   * dequant / gather: bit-exact with the reference CPU dequant (quant.cc):
//     Q4_K y = (d*sc)*q - (dmin*m), Q6_K y = (d*sc)*q, each op rounded
//     separately (the library is built with -ffp-contract=off);
//   * residual add: one IEEE fp32 add, bit-exact;
//   * fp16 KV store: IEEE round-to-nearest-even, bit-exact;
//   * RMSNorm: sum of squares accumulated in double, scale = float(1/sqrt(ss/n + eps)),
//     out = (x*scale)*w in fp32;  RoPE: a*c - b*s, b*c + a*s;  SiLU-mul: v/(1+exp(-v))*up.
#ifndef RPG_AMD_KERNELS_GPU_H_
#define RPG_AMD_KERNELS_GPU_H_

#include <cstdint>
#include <string>
#include <vector>

#include "hip_common.h"
#include "quant_types.h"

namespace rpg {

// ---------------------------------------------------------------- shapes

// Shapes and hyper-parameters of a model, with the reference's field names and
// types (src/model_meta.h:27-65); filled from a GGUF by ReadModelMeta
// (gpu_model.h) or by hand for single-operator use.
struct ModelMeta {
  std::string arch;  // "qwen3"
  std::string name;

  int32_t n_layers = 0;
  int32_t hidden = 0;
  int32_t n_heads = 0;
  int32_t n_kv_heads = 0;
  int32_t head_dim = 0;   // qwen3.attention.key_length
  int32_t value_dim = 0;  // qwen3.attention.value_length (== head_dim)
  int32_t intermediate = 0;
  int32_t vocab = 0;  // rows of token_embd
  int32_t context_length = 0;

  float rope_theta = 10000.0f;
  float rms_eps = 1e-6f;

  bool tied_embeddings = false;  // no output.weight / lm_head.weight: lm_head is token_embd

  int32_t bos_id = -1;
  int32_t eos_id = -1;
  int32_t pad_id = -1;
  bool add_bos = false;

  int64_t weight_bytes = 0;  // sum of every tensor's bytes in the file

  int32_t q_dim() const { return n_heads * head_dim; }
  int32_t kv_dim() const { return n_kv_heads * head_dim; }
  int32_t heads_per_kv() const { return n_kv_heads > 0 ? n_heads / n_kv_heads : 0; }
};

// A weight tensor resident in device memory as its raw GGUF bytes
// (reference src/gpu_model.h:42-55).
struct GpuTensor {
  DeviceBuffer buf;
  uint32_t type = kGgmlF32;
  bool matrix = false;
  int64_t rows = 0;  // dims[1]
  int64_t cols = 0;  // dims[0]
  int64_t n_elements = 0;

  bool valid() const { return !buf.empty(); }
  const char* type_name() const { return TypeName(type); }
  int64_t bytes() const { return static_cast<int64_t>(buf.size()); }
  int64_t row_bytes() const { return TypeRowBytes(type, cols); }
};

// Device-resident fp16 KV cache with the reference's layout: K, and V, each
// [n_layers][n_kv_heads][max_seq][head_dim] (src/kv_cache_gpu.h:1-30, :50-100),
// reached through the per-layer bases. The interface is the reference's; the
// storage is one device block per cache (all K layers, then all V layers), so
// a session costs a single allocation.
class GpuKvCache {
 public:
  GpuKvCache() = default;
  GpuKvCache(const ModelMeta& c, int64_t max_seq);

  int64_t len() const { return len_; }
  int64_t max_seq() const { return max_seq_; }
  int32_t n_layers() const { return n_layers_; }
  int32_t n_kv_heads() const { return n_kv_heads_; }
  int32_t head_dim() const { return head_dim_; }
  bool valid() const { return max_seq_ > 0; }

  // Base of layer `layer`: [n_kv_heads][max_seq][head_dim] fp16 bits.
  uint16_t* k_layer(int32_t layer) { return Plane(layer, 0); }
  uint16_t* v_layer(int32_t layer) { return Plane(layer, 1); }
  const uint16_t* k_layer(int32_t layer) const { return Plane(layer, 0); }
  const uint16_t* v_layer(int32_t layer) const { return Plane(layer, 1); }

  // Positions [0, len()) hold valid K / V rows; nothing else is ever read.
  void Reset() { len_ = 0; }
  void SetLen(int64_t n);
  void AddLen(int64_t n) { SetLen(len_ + n); }
  int64_t bytes() const { return static_cast<int64_t>(store_.size()); }
  std::string Describe() const;

 private:
  // Base of `layer` in plane 0 (K) or 1 (V).
  uint16_t* Plane(int32_t layer, int plane) const;

  int32_t n_layers_ = 0;
  int32_t n_kv_heads_ = 0;
  int32_t head_dim_ = 0;
  int64_t max_seq_ = 0;
  int64_t len_ = 0;
  int64_t plane_elems_ = 0;  // n_kv_heads * max_seq * head_dim
  DeviceBuffer store_;
};

// Host-built RoPE table, [n_pos][head_dim] fp32, cos in the first half of a row and
// sin in the second; angles computed in double (reference src/gpu_model.cu:90-120).
// n_pos = min(max_pos, context_length), at least 1.
std::vector<float> BuildRopeTable(int32_t head_dim, double theta, int64_t n_pos);

// ---------------------------------------------------------------- reference operators

void GpuDequantRow(uint32_t type, const uint8_t* src_dev, int64_t n_elems, float* dst_dev);

void GpuRmsNorm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, float eps,
                float* out);

void GpuRope(float* x, int32_t n_heads, int32_t head_dim, const float* rope_tab, int64_t pos0,
             int64_t n_rows);

void GpuKvWrite(const float* k_dev, const float* v_dev, int32_t n_kv_heads, int32_t head_dim, int64_t pos0,
                int64_t seq, uint16_t* k_cache_layer, uint16_t* v_cache_layer, int64_t max_seq);

void GpuSiluMulInPlace(float* gate_dev, const float* up_dev, int64_t n);

void GpuVecAddInPlace(float* a_dev, const float* b_dev, int64_t n);

void GpuEmbeddingLookup(const GpuTensor& emb, const int32_t* toks_dev, int64_t seq, float* x_dev);

// ---------------------------------------------------------------- fused operators

// x[r] += d[r] (one IEEE add, written back to x), then out[r] = RMSNorm(x[r]) * w.
// Rows are contiguous with stride n. out must not alias x or d.
void GpuAddRmsNorm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n, float eps, float* out);

// Per token t (position pos0 + t):
//   q[t,h,:]  <- RoPE(RMSNorm(q[t,h,:]) * q_norm)          in place, h < n_heads
//   k'        <- RoPE(RMSNorm(k[t,h,:]) * k_norm)          h < n_kv_heads
//   k_layer[h][pos0+t][:] <- fp16_rne(k');  v_layer[h][pos0+t][:] <- fp16_rne(v[t,h,:])
//   if write_k_f32: k[t,h,:] <- k' (needed only by the no-cache attention path)
// rope_rows is the number of rows in rope_tab (bounds check on pos0 + seq).
void GpuQkNormRopeKv(float* q, float* k, const float* v, const float* q_norm, const float* k_norm,
                     int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const float* rope_tab,
                     int64_t rope_rows, int64_t pos0, int64_t seq, float eps, uint16_t* k_cache_layer,
                     uint16_t* v_cache_layer, int64_t max_seq, bool write_k_f32);

// Embedding gather from a raw (non-owning) device table; GpuEmbeddingLookup
// forwards here. Token ids outside [0, rows) produce a zero row instead of an
// out-of-bounds read.
void GpuEmbeddingLookupRaw(uint32_t type, const uint8_t* emb_dev, int64_t rows, int64_t cols,
                           const int32_t* toks_dev, int64_t seq, float* x_dev);

// ---------------------------------------------------------------- attention

// Causal attention over the fp16 KV cache (src/kernels_gpu.h:113-116): for token
// t (absolute position pos0 + t) and query head h, softmax((q . k_j) / sqrt(d))
// over the cached positions j <= pos0 + t of kv head h / (n_heads / n_kv_heads),
// then the weighted sum of the v rows. q and out are [seq][n_heads][head_dim]
// fp32; k_layer / v_layer are one layer of the cache, [n_kv_heads][max_seq][d]
// fp16 bits. sh_positions > 0 fixes the position budget (needed under graph
// capture, where pos0 is read from the staging scalar at replay); otherwise
// pos0 + seq. head_dim must be 128.
void GpuAttentionFromCache(const ModelMeta& c, int64_t pos0, const float* q_dev, int64_t seq, const uint16_t* k_layer,
                           const uint16_t* v_layer, int64_t max_seq, float* out_dev, int64_t sh_positions = -1);

// One token at position pos0: GpuQkNormRopeKv (q / k per-head RMSNorm with
// q_norm / k_norm and eps = c.rms_eps, RoPE at pos0, k and v rounded to fp16
// into k_layer / v_layer at pos0) and GpuAttentionFromCache in one decode launch
// (plus the chunk merge when the keys are split), bit-identical to the two
// calls; q, k, v are the projections' raw [heads][128] rows and are not
// modified. Returns false, having launched nothing, when the shape has no fused
// kernel (head_dim != 128, a GQA group other than 1, 2, 4, pointers not 16-byte
// aligned); the caller then makes the two calls. No counterpart in the
// reference (src/qwen3_gpu.cu:77-96 runs norm, RoPE, KV write and attention as
// separate launches).
bool GpuQkNormRopeKvAttention(const ModelMeta& c, int64_t pos0, const float* q_dev, const float* k_dev,
                              const float* v_dev, const float* q_norm, const float* k_norm, const float* rope_tab,
                              int64_t rope_rows, uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq,
                              float* out_dev, int64_t sh_positions = -1);

// Causal attention without a cache (src/kernels_gpu.h:82-84): the same maths
// over the segment's own fp32 rows, k / v [seq][n_kv_heads][head_dim], token t
// attending to tokens 0..t. The no-cache forward uses it; the difference from
// GpuAttentionFromCache on the same tokens is the fp16 rounding of k and v only.
void GpuCausalAttention(const ModelMeta& c, const float* q_dev, const float* k_dev, const float* v_dev, int64_t seq,
                        float* out_dev);

// GpuAttentionFromCache for callers that cannot allocate (code under HIP graph
// capture, serving loops that forbid hipMalloc): the same kernels and results,
// with the chunk partials in a fixed 8 MiB device array of the library instead
// of the grow-only buffer, so nothing is ever allocated. A call whose key split
// needs more partials than that (seq * n_heads * chunks * 132 floats > 2^21;
// the split aims at ~2048 waves, so this is reached only with GQA groups of 4
// and more than ~2000 (token, kv head) pairs) is rejected before anything
// launches. Every call on a device shares that
// device's array: calls that overlap on one device (two streams) race. No
// counterpart in the reference.
void GpuAttentionFromCacheNoAlloc(const ModelMeta& c, int64_t pos0, const float* q_dev, int64_t seq,
                                  const uint16_t* k_layer, const uint16_t* v_layer, int64_t max_seq, float* out_dev,
                                  int64_t sh_positions = -1);
// Looks up the fixed array's address on the current device (once per device;
// the entry point does it on first use if this was not called).
void GpuAttentionNoAllocInit();
size_t GpuAttentionNoAllocScratchBytes();

// Sizes the attention's partials buffer for up to sh_positions cached positions
// (decode calls), so that a graph capture of the decode step allocates nothing
// (src/kernels_gpu.h:128; there it raises the shared-memory limit instead).
void GpuAttentionWarmupShmem(int64_t sh_positions);

// ---------------------------------------------------------------- quantised matmul

// OUT[t, r] = dot(row r of W, row t of X), i.e. OUT = X . W^T (src/kernels_gpu.h:42-49):
//   W   [rows, cols] quantised (raw GGUF bytes on the device, Q4_K / Q6_K / F32)
//   X   [n_tokens, cols] fp32, row-major
//   OUT [n_tokens, rows] fp32, row-major
// Weights are dequantised bit-exactly and accumulated in fp32 (fused multiply-add).
void GpuMatMulQuant(const GpuTensor& w, const float* X_dev, int64_t n_tokens, float* OUT_dev);

// Path-equivalence switch (src/kernels_gpu.h:51-58): while set, GpuMatMulQuant
// and the grouped / fused matmul entry points run the generic kernel
// (MatMulGenericKernel: per-element decode, one wave per output) instead of the
// decode, tiled and matrix-core kernels; the norm-fused entry points then
// return false. For verification only: the specialised kernels are checked bit
// for bit against it on inputs where every summation order is exact. Off by
// default; the flag is process-wide.
void GpuSetForceGenericMatMul(bool force);
bool GpuForceGenericMatMul();

// GpuMatMulQuant over several matrices that read the same X (a layer's q / k / v,
// or gate / up): OUT_i = X . W_i^T. At n_tokens = 1, up to 4 Q4_K / Q6_K
// matrices (either type or both) are decoded in one launch, else each run of
// consecutive same-type matrices is; on the matrix-core path
// X is split once for all the matrices; otherwise one call per matrix. Every
// output is bit-identical to its own GpuMatMulQuant call. No counterpart in the
// reference (which launches once per matrix).
void GpuMatMulQuantGroup(const GpuTensor* const* ws, int32_t n_mats, const float* X_dev, int64_t n_tokens,
                         float* const* OUTs);

// The layer's gate / up projections and SwiGLU (src/qwen3_gpu.cu:104-106):
// gate <- silu(X . W_gate^T) * (X . W_up^T); up is scratch (it holds X . W_up^T
// after a multi-token call, and is left untouched at one token). At one token on
// same-type matrices of <= 2048 columns it is one launch: each wave computes
// row p of both matrices and writes the SwiGLU of the two totals. Bit-identical
// to GpuMatMulQuantGroup({gate, up}) + GpuSiluMulInPlace. No counterpart in the
// reference.
void GpuMatMulQuantSwiGLU(const GpuTensor& w_gate, const GpuTensor& w_up, const float* X_dev, int64_t n_tokens,
                          float* gate_dev, float* up_dev);

// The sub-layer norm in front of a one-token matmul (the reference runs
// GpuVecAddInPlace, GpuRmsNorm and the matmul as separate launches,
// src/qwen3_gpu.cu:69-76,100-104,168): v = x + d (d == nullptr: v = x),
// h = RMSNorm(v) * w as GpuAddRmsNorm computes it, and the matmul of h. Each
// launch forms h itself, so no h buffer is written; x_out (optional) receives v,
// bit-exact, and must not alias x or d. The scale's double sum of squares is
// taken in another order than GpuAddRmsNorm's, so h can differ from it in the
// last fp32 bit. All of x, d, w, x_out 16-byte aligned.
struct GpuNormIn {
  const float* x;
  const float* d;
  const float* w;
  float eps;
  float* x_out;
};

// GpuMatMulQuantGroup at one token on RMSNorm(x + d) * w. Returns false, having
// launched nothing, when the group has no fused form (a matrix that is not
// Q4_K / Q6_K, more than 2048 columns, misaligned pointers); the caller then
// runs GpuAddRmsNorm and GpuMatMulQuantGroup. No counterpart in the reference.
bool GpuNormMatMulQuantGroup(const GpuNormIn& in, const GpuTensor* const* ws, int32_t n_mats, float* const* OUTs);

// GpuMatMulQuantSwiGLU at one token on RMSNorm(x + d) * w; false as above. No
// counterpart in the reference.
bool GpuNormMatMulQuantSwiGLU(const GpuNormIn& in, const GpuTensor& w_gate, const GpuTensor& w_up, float* gate_dev,
                              float* up_dev);

// The same on a raw (non-owning) weight pointer; GpuMatMulQuant forwards here.
void GpuMatMulQuantRaw(uint32_t type, const uint8_t* w_dev, int64_t rows, int64_t cols, const float* x_dev,
                       int64_t n_tokens, float* out_dev);

// ---------------------------------------------------------------- argmax

// Index of the largest of x[0..n) (src/kernels_gpu.h:131-143): only values above
// -FLT_MAX count (none -> 0), ties go to the smallest index, NaN never wins.
// n <= kSamplerMaxVocab (sampler_gpu.h, which declares the sampler around it).
void GpuArgMax(const float* x_dev, int64_t n, int32_t* out_idx_dev);

// ---------------------------------------------------------------- measurement / verification

// Streaming copy of `bytes` (multiple of 16) used to calibrate bandwidth and
// HBM counters (the reference's streaming-bandwidth probe, tools/matmul_bench.cu:230-289).
void GpuStreamCopy(const void* src, void* dst, int64_t bytes);

// Write-only probe: every 32-bit word of dst <- pattern (`bytes` a multiple of 16).
void GpuStreamFill(void* dst, int64_t bytes, uint32_t pattern);

// Read-only probe: reads `bytes` (a multiple of 16) of src and writes nothing
// unless the XOR fold of some thread's words equals `key` (then that fold goes to
// *sink). The reference's read probe (BwReadKernel, tools/matmul_bench.cu:239-250).
void GpuStreamRead(const void* src, int64_t bytes, uint32_t key, uint32_t* sink);

// out[i] = binary16 bits i converted to fp32, i in [0, 65536): exhaustive check
// of the device f16 -> f32 conversion (tools/dequant_check.cu:44-48).
void GpuF16Sweep(float* out_dev);

}  // namespace rpg

#endif  // RPG_AMD_KERNELS_GPU_H_
