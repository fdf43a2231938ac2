/* rpg_ops.h -- C ABI of the MI355X hot-path operators of the Qwen3 layer.
 *
 * librpg_ops.so exports exactly the functions declared here. Every argument is a
 * plain pointer or integer; every pointer named *_dev / x / q / k / v / w / out is
 * a device pointer owned by the caller. Launches are asynchronous on the engine
 * stream (rpg_ops_set_stream; NULL = the null stream) and nothing synchronises.
 *
 * Status convention (the reference ABI's, include/rpg_engine.h:46-55): 0 on
 * success, a negative value on failure with the reason available from
 * rpg_ops_last_error() (thread-local). Argument errors are detected on the host
 * before anything is launched, and no C++ exception crosses this boundary.
 *
 * Each operator cites the reference interface it replaces. The C++ operator
 * layer with the reference's own signatures (namespace rpg, src/kernels_gpu.h)
 * lives in rpgbarenginecuda_amd/csrc/kernels_gpu.h; these entry points forward
 * to it one to one.
 */
#ifndef RPG_OPS_H
#define RPG_OPS_H

#include <stdint.h>

#if defined(__GNUC__)
#define RPG_OPS_API __attribute__((visibility("default")))
#else
#define RPG_OPS_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define RPG_OPS_OK 0

/* ggml type ids accepted by the device path (src/quant.h:22-38). */
#define RPG_GGML_F32 0u
#define RPG_GGML_Q4_K 12u
#define RPG_GGML_Q6_K 14u

/* ---------------------------------------------------------------- library */

/* Version string of this library, e.g. "0.1.0". */
RPG_OPS_API const char* rpg_ops_version(void);

/* Text of the last failure on the calling thread (do not free).
 * Replaces: rpg_engine_last_error, include/rpg_engine.h:55. */
RPG_OPS_API const char* rpg_ops_last_error(void);

/* Allocates the fixed-address pos0 scalar on the current device and looks up
 * the current device's address of the no-allocation attention scratch. Must be
 * called once before any operator is captured into a HIP graph (allocation is
 * illegal during capture). Replaces: PosStagingPtr, src/cuda_common.h:153. */
RPG_OPS_API int32_t rpg_ops_init(void);

/* Routes every following launch to `stream` (a hipStream_t; NULL = null stream).
 * Replaces: ScopedEngineStream / EngineStream, src/cuda_common.h:116-137. */
RPG_OPS_API int32_t rpg_ops_set_stream(void* stream);
RPG_OPS_API void* rpg_ops_get_stream(void);

/* Device address of the pos0 staging scalar (allocating it on first use, so
 * call it before any capture). The graph path's sampler reads its counter
 * there. Replaces: PosStagingPtr, src/cuda_common.h:153. */
RPG_OPS_API int64_t* rpg_ops_pos_staging_ptr(void);

/* Writes pos into the pos0 scalar read by captured (graph) launches; a graph
 * replay loop calls it before each replay. Replaces: StagePos0,
 * src/cuda_common.h:154. */
RPG_OPS_API int32_t rpg_ops_stage_pos0(int64_t pos);

/* One-line description of device 0 written into buf (NUL-terminated).
 * Returns 1 if a device is available, 0 if not (buf says why), <0 on error.
 * Replaces: QueryDevice / DescribeDevice, src/cuda_common.h:52-56. */
RPG_OPS_API int32_t rpg_ops_device_info(char* buf, int32_t cap);

/* Bytes of n_elems elements of a device type (n_elems a block multiple);
 * negative on error. Replaces: TypeRowBytes, src/quant.h:57. */
RPG_OPS_API int64_t rpg_ops_type_row_bytes(uint32_t type, int64_t n_elems);

/* Host RoPE table [n_pos][head_dim] fp32 (cos half | sin half), angles in
 * double, into caller-provided host memory of n_pos*head_dim floats.
 * Replaces: GpuModel::BuildRopeTable, src/gpu_model.cu:90-120. */
RPG_OPS_API int32_t rpg_ops_build_rope_table(int32_t head_dim, double theta, int64_t n_pos, float* out_host);

/* ---------------------------------------------------------------- reference operators */

/* One row of n_elems elements of `type` -> fp32, bit-exact with the CPU dequant.
 * Replaces: GpuDequantRow, src/kernels_gpu.h:39-40. */
RPG_OPS_API int32_t rpg_op_dequant_row(uint32_t type, const uint8_t* src_dev, int64_t n_elems, float* dst_dev);

/* out[r] = x[r] * float(1/sqrt(sum(x[r]^2)/n + eps)) * w over n_rows rows of n
 * elements spaced `stride` apart; out may equal x.
 * Replaces: GpuRmsNorm, src/kernels_gpu.h:65-66. */
RPG_OPS_API int32_t rpg_op_rms_norm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride,
                                    float eps, float* out);

/* NeoX RoPE in place on x[n_rows][n_heads][head_dim] at positions pos0 + row;
 * rope_tab is [positions][head_dim] (cos | sin).
 * Replaces: GpuRope, src/kernels_gpu.h:71-72. */
RPG_OPS_API int32_t rpg_op_rope(float* x, int32_t n_heads, int32_t head_dim, const float* rope_tab, int64_t pos0,
                                int64_t n_rows);

/* k, v [seq][n_kv_heads][head_dim] fp32 -> k_layer, v_layer [n_kv_heads][max_seq][head_dim]
 * fp16 bits (IEEE round-to-nearest-even) at positions pos0..pos0+seq-1.
 * Replaces: GpuKvWrite, src/kernels_gpu.h:97-99. */
RPG_OPS_API int32_t rpg_op_kv_write(const float* k, const float* v, int32_t n_kv_heads, int32_t head_dim,
                                    int64_t pos0, int64_t seq, uint16_t* k_layer, uint16_t* v_layer,
                                    int64_t max_seq);

/* gate[i] = silu(gate[i]) * up[i]; n <= 0 is a no-op.
 * Replaces: GpuSiluMulInPlace, src/kernels_gpu.h:147. */
RPG_OPS_API int32_t rpg_op_silu_mul_inplace(float* gate, const float* up, int64_t n);

/* a[i] += b[i]; n <= 0 is a no-op. Replaces: GpuVecAddInPlace, src/kernels_gpu.h:150. */
RPG_OPS_API int32_t rpg_op_vec_add_inplace(float* a, const float* b, int64_t n);

/* x[t] = dequantised row toks[t] of the [rows][cols] table of `type` (raw GGUF
 * bytes); ids outside [0, rows) give a zero row.
 * Replaces: GpuEmbeddingLookup, src/kernels_gpu.h:153-154 (its GpuTensor
 * argument flattened to type / data / rows / cols). */
RPG_OPS_API int32_t rpg_op_embedding_lookup(uint32_t type, const uint8_t* emb, int64_t rows, int64_t cols,
                                            const int32_t* toks, int64_t seq, float* x);

/* Causal attention over one layer of the fp16 KV cache: q / out are
 * [seq][n_heads][head_dim] fp32 (head_dim 128), k_layer / v_layer
 * [n_kv_heads][max_seq][head_dim] fp16 bits; token t attends to positions
 * [0, pos0 + t]. sh_positions > 0: position budget for graph capture.
 * Replaces: GpuAttentionFromCache, src/kernels_gpu.h:113-116 (its ModelMeta
 * argument flattened to the three head counts). */
RPG_OPS_API int32_t rpg_op_attention_from_cache(const float* q, int32_t n_heads, int32_t n_kv_heads,
                                                int32_t head_dim, int64_t pos0, int64_t seq,
                                                const uint16_t* k_layer, const uint16_t* v_layer, int64_t max_seq,
                                                float* out, int64_t sh_positions);

/* One token at pos0: rpg_op_qk_norm_rope_kv (q / k per-head RMSNorm with q_norm /
 * k_norm and eps, RoPE from rope_tab at pos0, k and v stored as fp16 at pos0)
 * followed by rpg_op_attention_from_cache, in one decode launch, bit-identical
 * to the two calls. q, k, v are the raw projections ([n_heads] / [n_kv_heads]
 * rows of 128 floats) and are not modified. *fused = 0 when the shape has no
 * fused kernel (head_dim != 128, n_heads / n_kv_heads not 1, 2 or 4, pointers
 * not 16-byte aligned): nothing ran. No counterpart in the reference
 * (src/qwen3_gpu.cu:77-96 runs these as separate launches). */
RPG_OPS_API int32_t rpg_op_qk_norm_rope_kv_attention(const float* q, const float* k, const float* v,
                                                     const float* q_norm, const float* k_norm, int32_t n_heads,
                                                     int32_t n_kv_heads, int32_t head_dim, const float* rope_tab,
                                                     int64_t rope_rows, int64_t pos0, float eps, uint16_t* k_layer,
                                                     uint16_t* v_layer, int64_t max_seq, float* out,
                                                     int64_t sh_positions, int32_t* fused);

/* rpg_op_attention_from_cache for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc): same arguments, same kernels, bit-identical results, but the
 * partials of a split-key decode live in a fixed 2 MiB device array of the
 * library (one per GPU, held until the process ends), and the arrival counters
 * of the split decode and of the prefill's in-launch chunk merge in fixed arrays
 * beside it, so no call ever allocates.
 * Limit: a call whose split needs more than 2^19 floats of partials fails with
 * an error and launches nothing. A split decode keeps 132 floats per (token,
 * query head, workgroup of 4 key chunks), none when one workgroup takes every
 * chunk; the split aims at ~2048 waves, so the only calls over the limit have a
 * GQA group of 4, 497 to 511 (token, kv head) pairs and a split of 5 to 8 chunks
 * (1056 floats per pair; 496 pairs fit). Prefill-sized calls keep fewer key
 * chunks when the array is too small for their partials.
 * Calls that overlap on one GPU (different streams) share the arrays and race.
 * No counterpart in the reference: it exists for callers that cannot allocate. */
RPG_OPS_API int32_t rpg_op_attention_from_cache_noalloc(const float* q, int32_t n_heads, int32_t n_kv_heads,
                                                        int32_t head_dim, int64_t pos0, int64_t seq,
                                                        const uint16_t* k_layer, const uint16_t* v_layer,
                                                        int64_t max_seq, float* out, int64_t sh_positions);

/* Pre-sizes the attention's partials buffer for graph capture.
 * Replaces: GpuAttentionWarmupShmem, src/kernels_gpu.h:128. */
RPG_OPS_API int32_t rpg_op_attention_warmup(int64_t sh_positions);

/* out[t * rows + r] = dot(row r of the [rows][cols] matrix w of `type`, row t of
 * x), i.e. OUT[n_tokens, rows] = X[n_tokens, cols] . W^T. Weights are dequantised
 * bit-exactly and summed in fp32.
 * Replaces: GpuMatMulQuant, src/kernels_gpu.h:42-49 (its GpuTensor argument
 * flattened to type / data / rows / cols). */
RPG_OPS_API int32_t rpg_op_matmul_quant(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols,
                                        const float* x, int64_t n_tokens, float* out);

/* Path-equivalence switch: force != 0 makes every matmul entry point run the
 * generic per-element kernel instead of the decode / tiled / matrix-core
 * kernels (the norm-fused ones then report *fused = 0). For verification only;
 * process-wide, off by default. rpg_op_force_generic_matmul returns 1 or 0.
 * Replaces: GpuSetForceGenericMatMul / GpuForceGenericMatMul, src/kernels_gpu.h:57-58. */
RPG_OPS_API int32_t rpg_op_set_force_generic_matmul(int32_t force);
RPG_OPS_API int32_t rpg_op_force_generic_matmul(void);

/* rpg_op_matmul_quant over n matrices sharing x (a layer's q / k / v, or gate /
 * up): out[i] = x . w[i]^T, each w[i] [rows[i]][cols] of types[i]; all arrays
 * are host arrays of n entries (ws / outs hold device pointers). At n_tokens = 1
 * up to 4 Q4_K / Q6_K matrices (either type or both) are one launch, every
 * output bit-identical to its own rpg_op_matmul_quant. No counterpart in the
 * reference (one launch per matrix, src/qwen3_gpu.cu:72-74, :104-105). */
RPG_OPS_API int32_t rpg_op_matmul_quant_group(int32_t n, const uint32_t* types, const uint8_t* const* ws,
                                              const int64_t* rows, int64_t cols, const float* x, int64_t n_tokens,
                                              float* const* outs);

/* A layer's gate / up projections and SwiGLU: gate <- silu(x . w_gate^T) *
 * (x . w_up^T), both matrices [rows][cols] of `type`; up is scratch. At n_tokens
 * = 1 (<= 2048 columns) one launch forms the SwiGLU from each row pair's totals.
 * Bit-identical to rpg_op_matmul_quant_group + rpg_op_silu_mul_inplace. No
 * counterpart in the reference (src/qwen3_gpu.cu:104-106 makes three calls). */
RPG_OPS_API int32_t rpg_op_matmul_quant_swiglu(uint32_t type, const uint8_t* w_gate, const uint8_t* w_up,
                                               int64_t rows, int64_t cols, const float* x, int64_t n_tokens,
                                               float* gate, float* up);

/* One token: v = x + d (d may be NULL: v = x), h = RMSNorm(v) * norm_w (the
 * rpg_op_add_rms_norm maths) formed inside the matmul launches that read it,
 * then out[i] = h . w[i]^T as rpg_op_matmul_quant_group. x_out (may be NULL)
 * receives v, bit-exact; it must not alias x or d. x, d, norm_w, x_out hold
 * cols floats, 16-byte aligned. *fused = 1 when launched; 0 when the group has
 * no fused form (a matrix not Q4_K / Q6_K, cols > 2048), in which case nothing
 * ran and the caller runs rpg_op_add_rms_norm + rpg_op_matmul_quant_group. h can
 * differ from rpg_op_add_rms_norm's in the last fp32 bit (the double sum of
 * squares is taken in another order). No counterpart in the reference
 * (GpuVecAddInPlace, GpuRmsNorm and the matmuls are separate launches,
 * src/qwen3_gpu.cu:69-76,100-104,168). */
RPG_OPS_API int32_t rpg_op_norm_matmul_quant_group(int32_t n, const uint32_t* types, const uint8_t* const* ws,
                                                   const int64_t* rows, int64_t cols, const float* x, const float* d,
                                                   const float* norm_w, float eps, float* x_out, float* const* outs,
                                                   int32_t* fused);

/* The same in front of rpg_op_matmul_quant_swiglu (gate <- silu(h . w_gate^T) *
 * (h . w_up^T); up is left untouched). No counterpart in the reference. */
RPG_OPS_API int32_t rpg_op_norm_matmul_quant_swiglu(uint32_t type, const uint8_t* w_gate, const uint8_t* w_up,
                                                    int64_t rows, int64_t cols, const float* x, const float* d,
                                                    const float* norm_w, float eps, float* x_out, float* gate,
                                                    float* up, int32_t* fused);

/* ---------------------------------------------------------------- GGUF files and the device model
 * rpg_gguf: a parsed GGUF file (host only, no GPU needed). rpg_model: a qwen3
 * GGUF uploaded to the device (F32 / Q4_K / Q6_K tensors only): quantized
 * matrices as raw GGUF bytes, norms as fp32, in one device arena, plus the RoPE
 * table. Replaces: GgufFile (src/gguf.h:43-97), ReadModelMeta
 * (src/model_meta.cc:11-78) and GpuModel::Load (src/gpu_model.cu:148-246). */
typedef struct rpg_gguf rpg_gguf;
typedef struct rpg_model rpg_model;

/* ModelMeta (src/model_meta.h:27-65) as plain fields; booleans as 0 / 1. */
typedef struct {
  char arch[32];
  char name[128];
  int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, value_dim, intermediate, vocab, context_length;
  float rope_theta, rms_eps;
  int32_t tied_embeddings, bos_id, eos_id, pad_id, add_bos;
  int64_t weight_bytes;
} rpg_model_meta_t;

/* A tensor: data is a host pointer into the file mapping (rpg_gguf) or a device
 * pointer (rpg_model); dims[0] varies fastest; norms of a model are fp32. */
typedef struct {
  const void* data;
  uint32_t type;
  int32_t n_dims;
  int64_t dims[4];
  int64_t n_elements, n_bytes, file_offset;
} rpg_tensor_info_t;

RPG_OPS_API int32_t rpg_gguf_open(const char* path, rpg_gguf** out);
RPG_OPS_API int32_t rpg_gguf_close(rpg_gguf* g);
RPG_OPS_API int64_t rpg_gguf_tensor_count(const rpg_gguf* g);
/* Tensor `index` in file order; its name is copied into name[cap]. */
RPG_OPS_API int32_t rpg_gguf_tensor_info(const rpg_gguf* g, int64_t index, char* name, int32_t cap,
                                         rpg_tensor_info_t* out);
/* Metadata value of `key` (item < 0) or item `item` of an array value: *kind = 0
 * absent, 1 number (*num), 2 bool (*num = 0 / 1), 3 string (copied into str[cap];
 * the return value is its full length), 4 array (*n_items). */
RPG_OPS_API int32_t rpg_gguf_meta(const rpg_gguf* g, const char* key, int64_t item, int32_t* kind, double* num,
                                  char* str, int32_t cap, int64_t* n_items);
/* ReadModelMeta of the file (qwen3 only). */
RPG_OPS_API int32_t rpg_gguf_model_meta(const rpg_gguf* g, rpg_model_meta_t* out);
/* One-line summary; returns its full length. */
RPG_OPS_API int32_t rpg_gguf_describe(const rpg_gguf* g, char* buf, int32_t cap);

/* Parses and uploads a qwen3 GGUF; max_pos = positions of the RoPE table. */
RPG_OPS_API int32_t rpg_model_load(const char* path, int32_t max_pos, rpg_model** out);
RPG_OPS_API int32_t rpg_model_free(rpg_model* m);
RPG_OPS_API int32_t rpg_model_meta(const rpg_model* m, rpg_model_meta_t* out);
/* The device tensor loaded from GGUF tensor `name` (output.weight is token_embd
 * when the embeddings are tied). */
RPG_OPS_API int32_t rpg_model_tensor(const rpg_model* m, const char* name, rpg_tensor_info_t* out);
/* Device RoPE table [*n_pos][head_dim] fp32 (cos | sin per row). */
RPG_OPS_API int32_t rpg_model_rope(const rpg_model* m, const float** tab, int64_t* n_pos);
RPG_OPS_API int32_t rpg_model_describe(const rpg_model* m, char* buf, int32_t cap);
/* File bytes moved to the device, and the parse / upload wall times. */
RPG_OPS_API int32_t rpg_model_upload_stats(const rpg_model* m, int64_t* bytes, double* parse_seconds,
                                           double* upload_seconds);
/* Device bytes the model holds (weight arena and RoPE table).
 * Replaces: GpuModel::device_bytes, src/gpu_model.h:101. */
RPG_OPS_API int32_t rpg_model_device_bytes(const rpg_model* m, int64_t* out);

/* ---------------------------------------------------------------- forward and generation
 * The Qwen3 layer chain over the operators above, for a loaded rpg_model.
 * rpg_kv: the fp16 KV cache [n_layers][n_kv_heads][max_seq][head_dim], allocated
 * in full at creation (Replaces: GpuKvCache, src/kv_cache_gpu.h:50-100).
 * rpg_scratch: the grow-only device activations of a forward plus the captured
 * decode graph (Replaces: GpuScratch, src/qwen3_gpu.h:47-113). A model, its caches
 * and scratches are used from one host thread at a time. */
typedef struct rpg_kv rpg_kv;
typedef struct rpg_scratch rpg_scratch;

RPG_OPS_API int32_t rpg_kv_create(const rpg_model* m, int64_t max_seq, rpg_kv** out);
/* The same cache from the three shape numbers it depends on, with no loaded model
 * at hand (the engine sizes its session caches from ModelMeta alone).
 * Replaces: GpuKvCache::GpuKvCache(const ModelMeta&, int64_t), src/kv_cache_gpu.h:56. */
RPG_OPS_API int32_t rpg_kv_create_shape(int32_t n_layers, int32_t n_kv_heads, int32_t head_dim, int64_t max_seq,
                                        rpg_kv** out);
RPG_OPS_API int32_t rpg_kv_free(rpg_kv* kv);
/* Current length (positions filled), capacity and K + V bytes. */
RPG_OPS_API int32_t rpg_kv_info(const rpg_kv* kv, int64_t* len, int64_t* max_seq, int64_t* bytes);
/* Sets the length (0 <= len <= max_seq); 0 is GpuKvCache::Reset, src/kv_cache_gpu.h:75. */
RPG_OPS_API int32_t rpg_kv_set_len(rpg_kv* kv, int64_t len);
/* Device bases of one layer's K and V (fp16 bits). */
RPG_OPS_API int32_t rpg_kv_layer(rpg_kv* kv, int32_t layer, uint16_t** k, uint16_t** v);

RPG_OPS_API int32_t rpg_scratch_create(rpg_scratch** out);
RPG_OPS_API int32_t rpg_scratch_free(rpg_scratch* s);
/* Device address of the scratch's logits [seq, vocab] (valid after a forward),
 * and of its sampled-token slot (int32). */
RPG_OPS_API int32_t rpg_scratch_logits(rpg_scratch* s, const float** logits_dev, const int32_t** token_dev);

/* Forward of `seq` host token ids. kv == NULL: the no-cache path (attention over
 * the segment's fp32 k / v); otherwise the segment is appended at the cache's
 * length and attends to the whole cache, whose length then grows by seq.
 * layer_limit > 0 runs only that many layers (no logits then). logits (host,
 * [seq, vocab]) and hidden (host, [n_use + 1, seq, hidden]: the residual stream
 * after the embedding and after each layer) are optional (NULL).
 * Replaces: GpuForwardFull, src/qwen3_gpu.h:136-139. */
RPG_OPS_API int32_t rpg_forward_full(const rpg_model* m, const int32_t* tokens, int64_t seq, rpg_scratch* s,
                                     float* logits, int32_t layer_limit, float* hidden, rpg_kv* kv);
/* One token at pos == the cache length; logits (host [vocab]) optional.
 * Replaces: GpuForwardStep, src/qwen3_gpu.h:145-146. */
RPG_OPS_API int32_t rpg_forward_step(const rpg_model* m, int32_t token, int64_t pos, rpg_kv* kv, rpg_scratch* s,
                                     float* logits);
/* The same with the token id on the device; logits stay in the scratch.
 * Replaces: GpuForwardStepDev, src/qwen3_gpu.h:151-152. */
RPG_OPS_API int32_t rpg_forward_step_dev(const rpg_model* m, const int32_t* token_dev, int64_t pos, rpg_kv* kv,
                                         rpg_scratch* s);

/* Generation options (GpuGenerateOptions, src/qwen3_gpu.h:156-181). temperature
 * <= 0 is greedy; step_logits (host, step_logits_cap floats, or NULL) receives
 * the distribution each token was drawn from; use_graph replays the decode step
 * as a HIP graph (ignored when step_logits is set). */
typedef struct {
  int32_t max_tokens;
  const int32_t* stop_ids;
  int32_t n_stop;
  float temperature;
  int32_t top_k;
  float top_p;
  uint64_t seed;
  int32_t use_graph;
  float* step_logits;
  int64_t step_logits_cap;
} rpg_generate_opts_t;

/* Generates from the distribution at first_logits_dev ([vocab], device; e.g.
 * the last row of rpg_scratch_logits after a prefill), writing up to out_cap
 * ids and *n_out. Every returned token (the stop token included) is in the cache
 * afterwards. Replaces: GpuGenerate, src/qwen3_gpu.h:197-199. */
RPG_OPS_API int32_t rpg_generate(const rpg_model* m, rpg_kv* kv, rpg_scratch* s, const float* first_logits_dev,
                                 const rpg_generate_opts_t* opts, int32_t* out_ids, int32_t out_cap, int32_t* n_out);

/* ---------------------------------------------------------------- argmax and sampling
 * n (the vocabulary) is at most 2^22 for all of these. Semantics: greedy
 * (temperature <= 0) is argmax, ties to the smallest index; otherwise logits *
 * (1/T), top_k threshold (k-th largest, ties kept), softmax with a double sum,
 * top_p cut (largest key whose cumulative mass <= 1 - top_p, at least one
 * token kept, renormalised), and the inverse transform (first running double
 * sum > u). */

/* *out_idx = index of the largest x[i] above -FLT_MAX (none: 0).
 * Replaces: GpuArgMax, src/kernels_gpu.h:131-143. */
RPG_OPS_API int32_t rpg_op_argmax(const float* x, int64_t n, int32_t* out_idx);

/* Host-side counter-based random source: SplitMix64, H(seed, counter) and
 * u = (H >> 40) * 2^-24 in [0, 1).
 * Replaces: DevSplitMix64 / DevCounterRng / DevCounterUniform, src/sampler_gpu.h:71-73. */
RPG_OPS_API uint64_t rpg_sample_split_mix64(uint64_t x);
RPG_OPS_API uint64_t rpg_sample_counter_rng(uint64_t seed, uint64_t counter);
RPG_OPS_API float rpg_sample_counter_uniform(uint64_t seed, uint64_t counter);

/* probs[0..n) <- filtered, normalised distribution of logits.
 * Replaces: GpuFilterToProbs, src/sampler_gpu.h:86-87 (SampleOptions flattened). */
RPG_OPS_API int32_t rpg_op_filter_to_probs(const float* logits, int64_t n, float temperature, int32_t top_k,
                                           float top_p, float* probs);

/* *out_idx = first i whose running double sum of probs exceeds u (u in [0, 1));
 * none: the first maximum. Not capturable.
 * Replaces: GpuInverseSample, src/sampler_gpu.h:95-96. */
RPG_OPS_API int32_t rpg_op_inverse_sample(const float* probs, int64_t n, float u, int32_t* out_idx);

/* One token with u = CounterUniform(seed, counter); greedy is rpg_op_argmax.
 * probs is scratch of n floats. Not capturable (use the _dev form).
 * Replaces: GpuSampleToken, src/sampler_gpu.h:108-110. */
RPG_OPS_API int32_t rpg_op_sample_token(const float* logits, int64_t n, float temperature, int32_t top_k,
                                        float top_p, uint64_t seed, uint64_t counter, float* probs,
                                        int32_t* out_idx);

/* The same with the counter read on the device from counter_dev (the pos0
 * staging scalar in the engine's graph path).
 * Replaces: GpuSampleTokenDev, src/sampler_gpu.h:124-126. */
RPG_OPS_API int32_t rpg_op_sample_token_dev(const float* logits, int64_t n, float temperature, int32_t top_k,
                                            float top_p, uint64_t seed, const uint64_t* counter_dev, float* probs,
                                            int32_t* out_idx);

/* Allocates the sampler's scratch block (call before a graph capture that
 * samples or takes an argmax). Replaces: GpuSamplerWarmup, src/sampler_gpu.h:130. */
RPG_OPS_API int32_t rpg_op_sampler_warmup(void);

/* ---------------------------------------------------------------- fused operators */

/* x[r] += d[r] (bit-exact fp32 add, written back), then out[r] = RMSNorm(x[r]) * w,
 * rows contiguous (stride n); out must not alias x or d.
 * Replaces: GpuVecAddInPlace + GpuRmsNorm, src/qwen3_gpu.cu:100->103 and :108->69. */
RPG_OPS_API int32_t rpg_op_add_rms_norm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n,
                                        float eps, float* out);

/* Per token t (position pos0 + t): q <- RoPE(RMSNorm(q) * q_norm) in place;
 * k' = RoPE(RMSNorm(k) * k_norm); k_layer/v_layer[h][pos0+t] <- fp16_rne(k'), fp16_rne(v);
 * k <- k' only if write_k_f32 != 0 (head_dim != 128 always writes it).
 * rope_rows = rows of rope_tab. q [seq][n_heads][head_dim], k/v [seq][n_kv_heads][head_dim].
 * Replaces: GpuRmsNorm(q), GpuRmsNorm(k), GpuRope(q), GpuRope(k), GpuKvWrite,
 * src/qwen3_gpu.cu:77-91. */
RPG_OPS_API int32_t rpg_op_qk_norm_rope_kv(float* q, float* k, const float* v, const float* q_norm,
                                           const float* k_norm, int32_t n_heads, int32_t n_kv_heads,
                                           int32_t head_dim, const float* rope_tab, int64_t rope_rows,
                                           int64_t pos0, int64_t seq, float eps, uint16_t* k_layer,
                                           uint16_t* v_layer, int64_t max_seq, int32_t write_k_f32);

/* ---------------------------------------------------------------- measurement / verification */

/* dst <- src, `bytes` a positive multiple of 16, both 16-byte aligned: the
 * streaming-bandwidth probe. Replaces: BwCopyKernel, tools/matmul_bench.cu:230-289. */
RPG_OPS_API int32_t rpg_op_stream_copy(const void* src, void* dst, int64_t bytes);

/* Every 32-bit word of dst <- pattern, `bytes` a positive multiple of 16, dst
 * 16-byte aligned: the write-only bandwidth probe (the ceiling of write-dominated
 * ops such as the embedding gather). No counterpart in the reference, which
 * probes copies only (tools/matmul_bench.cu:230-289). */
RPG_OPS_API int32_t rpg_op_stream_fill(void* dst, int64_t bytes, uint32_t pattern);

/* Reads `bytes` (a positive multiple of 16) of src (16-byte aligned) and writes
 * nothing, unless the XOR fold of one thread's 16 words equals `key`; then that
 * fold is stored to *sink (device memory, one word). The read-only bandwidth
 * probe (the ceiling of read-dominated kernels: decode matvecs, the output
 * projection, decode attention). Replaces: BwReadKernel,
 * tools/matmul_bench.cu:239-250,269-286. */
RPG_OPS_API int32_t rpg_op_stream_read(const void* src, int64_t bytes, uint32_t key, uint32_t* sink);

/* out_dev[i] = fp32 value of the binary16 bit pattern i, i in [0, 65536).
 * Replaces: F16SweepKernel, tools/dequant_check.cu:44-48. */
RPG_OPS_API int32_t rpg_op_f16_sweep(float* out_dev);

/* Kernel-execution timing: after rpg_ops_profile_start(n), each of the next n
 * launches (outside graph capture) carries a HIP start/stop event pair attached
 * to its dispatch. rpg_ops_profile_report synchronises on the last launch and
 * writes per-kernel JSON {"<kernel>": {"count", "avg_us", "min_us", "max_us",
 * "total_us"}} into buf; it returns the length of the JSON (which may exceed
 * cap-1, then the text is truncated) or a negative status. Takes the place of
 * the reference's host-clock timing in tools/matmul_bench.cu:45-49,114-133. */
RPG_OPS_API int32_t rpg_ops_profile_start(int32_t max_launches);
RPG_OPS_API int32_t rpg_ops_profile_stop(void);
RPG_OPS_API int32_t rpg_ops_profile_report(char* buf, int32_t cap);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RPG_OPS_H */
