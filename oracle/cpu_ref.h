/* cpu_ref.h -- CPU oracle for the hot-path operators.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * algorithms, used as the checker by tests/, by __graft_entry__.smoke() and by
 * the cpu_baseline leg of bench.py. The product (librpg_ops.so) never links,
 * loads or calls it.
 *
 * Built with gcc -O2 -ffp-contract=off (oracle/Makefile) so every fp32 op is
 * rounded separately, as in the reference CPU build (CMakeLists.txt:120-127).
 *
 * Pinning (how each function is checked independently of its own formula; the
 * tests named here live in tests/test_oracle.py):
 *   ora_f16_to_f32       exhaustive 65536 values vs numpy float16->float32, and
 *                        vs the reference's own F16ToF32 (oracle/_ref) when built
 *   ora_f32_to_f16_rne   numpy astype(float16) (an independent IEEE RNE routine)
 *                        on random values, every tie class, subnormals, overflow
 *   ora_dequantize_row   golden vectors written by the reference quant.cc
 *                        (tests/golden/), oracle/_ref directly when built, a
 *                        per-element pure-Python restatement on tiny inputs,
 *                        and closed-form special blocks
 *   ora_embedding_lookup row-by-row equality with ora_dequantize_row
 *   ora_rms_norm         float64 closed forms (constant rows), scale invariance,
 *                        unit-RMS output with w = 1, numpy float64 restatement
 *   ora_build_rope_table numpy float64 cos/sin cast to float32
 *   ora_rope             pos 0 is the identity, pair norms preserved, complex
 *                        multiplication form (x_i + j x_{i+64}) * e^{j*angle}
 *   ora_kv_write         the reference's integer-coded KAT
 *                        (tools/kv_map_check.cu:51-186) plus "untouched stays 0"
 *   ora_silu_mul         silu(0)=0, v->-inf gives -0, v>>0 gives v*up, numpy f64
 *   ora_vec_add          numpy float32 addition, bitwise
 *   ora_matmul_quant_f64 numpy float64 dot products (BLAS) of the dequantised
 *                        matrix, one-hot inputs select exact matrix columns,
 *                        linearity in X
 *   ora_attention_f64    numpy float64 softmax attention, equal keys give the
 *                        mean of v, a dominant score selects its v row,
 *                        rows past the causal limit do not matter
 *   ora_split_mix64 /    SplitMix64's published outputs for seed 0 (the first
 *   ora_counter_rng      five), which CounterRng(0, c) reproduces for c = 0..4
 *   ora_counter_uniform  24-bit grid, range [0, 1), mean over many counters
 *   ora_argmax           numpy argmax (first maximum), the -FLT_MAX / -inf floors
 *   ora_filter_to_probs  a numpy restatement by sorting (np.sort keys for top_k,
 *                        float64 cumsum for top_p), one-hot for T <= 0, tie
 *                        groups kept whole, the mass bounds that define the cut
 *   ora_inverse_sample   np.cumsum (sequential float64) + searchsorted, exact
 *                        boundaries, the no-crossing fallback
 */
#ifndef RPG_ORACLE_CPU_REF_H
#define RPG_ORACLE_CPU_REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORA_GGML_F32 0u
#define ORA_GGML_Q4_K 12u
#define ORA_GGML_Q6_K 14u

/* ---- fp16 ---------------------------------------------------------------- */
float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_f16_rne(float f);
void ora_f16_to_f32_array(const uint16_t* src, int64_t n, float* dst);
void ora_f32_to_f16_rne_array(const float* src, int64_t n, uint16_t* dst);

/* ---- dequant / gather ----------------------------------------------------- */
int64_t ora_type_row_bytes(uint32_t type, int64_t n_elems); /* <0 if unsupported */
int ora_dequantize_row(uint32_t type, const uint8_t* src, int64_t n_elems, float* dst);
int ora_embedding_lookup(uint32_t type, const uint8_t* emb, int64_t rows, int64_t cols, const int32_t* toks,
                         int64_t seq, float* x);

/* ---- attention over the fp16 KV cache --------------------------------------- */
/* src/kernels_gpu.cu:737-823 (AttentionFromCacheKernel) in double: for token t
 * (position pos0 + t) and head h, kv head h / (n_heads / n_kv_heads):
 * s_j = (q . k_j) * scale, scale = (double)(1.0f / sqrtf((float)d)), over j in
 * [0, pos0 + t]; p = softmax(s); out = sum_j p_j v_j. q / out [seq][n_heads][d];
 * caches [n_kv][max_seq][d] fp16 bits. Optional outputs per (t, h): smag =
 * max_j scale * sum_d |q_d k_jd| (the scale of the scores' rounding) and
 * vmax = max_j max_d |v_jd|. Returns 0, or -1 on bad arguments. */
int ora_attention_f64(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t max_seq, int32_t n_heads,
                      int32_t n_kv_heads, int32_t d, int64_t pos0, int64_t seq, double* out, double* smag,
                      double* vmax);

/* ---- quantized matmul ------------------------------------------------------ */
/* OUT[t][r] = sum_e W[r][e] * X[t][e] for the raw [rows][row_bytes] matrix W
 * (src/kernels_gpu.h:42-49 GpuMatMulQuant: OUT = X . W^T, OUT [n_tokens][rows]).
 * Each row is dequantised exactly (ora_dequantize_row) and the products are
 * summed in double, so `out` is the dot product to double accuracy; `absdot`
 * (may be NULL) receives sum_e |W[r][e] * X[t][e]|, the scale of any fp32
 * summation error. Returns 0, or -1 for an unsupported type / shape. */
int ora_matmul_quant_f64(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const float* x,
                         int64_t n_tokens, double* out, double* absdot);

/* ---- argmax and sampling (cpu_sample.c) ------------------------------------ */
uint64_t ora_split_mix64(uint64_t x);
uint64_t ora_counter_rng(uint64_t seed, uint64_t counter);
float ora_counter_uniform(uint64_t seed, uint64_t counter);
int32_t ora_argmax(const float* x, int64_t n, float init);
int ora_filter_to_probs(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p, float* probs,
                        double* margin);
int32_t ora_inverse_sample(const float* probs, int64_t n, float u);
/* The top_p cut's order key under three rules for comparing S(t) with 1 - top_p:
 * the exact mass (the oracle's), the device's 2^-62 grid, the reference's double
 * sums (see cpu_sample.c). */
#define ORA_TOPP_EXACT 0
#define ORA_TOPP_GRID62 1
#define ORA_TOPP_DOUBLE 2
uint32_t ora_top_p_cut_key(const float* probs, int64_t n, float top_p, int rule, double* margin);
int32_t ora_sample_token(const float* logits, int64_t n, float temperature, int32_t top_k, float top_p, uint64_t seed,
                         uint64_t counter, float* probs);

/* ---- layer ops, fp32 in the reference's op order -------------------------- */
void ora_rms_norm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, float eps, float* out);
void ora_build_rope_table(int32_t head_dim, double theta, int64_t n_pos, float* out);
void ora_rope(float* x, int32_t n_heads, int32_t head_dim, const float* tab, int64_t pos0, int64_t n_rows);
int ora_kv_write(const float* k, const float* v, int32_t n_kv_heads, int32_t head_dim, int64_t pos0, int64_t seq,
                 uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq);
void ora_silu_mul(float* gate, const float* up, int64_t n);
void ora_vec_add(float* a, const float* b, int64_t n);

/* Compositions the fused operators must equal (src/qwen3_gpu.cu:77-91, :100-103). */
void ora_add_rms_norm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n, float eps, float* out);
int ora_qk_norm_rope_kv(float* q, float* k, const float* v, const float* q_norm, const float* k_norm,
                        int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const float* tab, int64_t pos0,
                        int64_t seq, float eps, uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq);

/* ---- float64 restatements (the tolerance gate's reference values) ---------- */
void ora_rms_norm_f64(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, double eps,
                      double* out);
void ora_rope_f64(const float* x, int32_t n_heads, int32_t head_dim, const float* tab, int64_t pos0, int64_t n_rows,
                  double* out);
void ora_silu_mul_f64(const float* gate, const float* up, int64_t n, double* out);
void ora_norm_rope_f64(const float* x, const float* w, int32_t n_heads, int32_t head_dim, const float* tab,
                       int64_t pos0, int64_t n_rows, double eps, double* out);

/* ---- CPU baseline timing (bench.py cpu_baseline leg) ----------------------- */
/* Runs the one-layer chain (residual add + RMSNorm over [n,H], q/k norm + RoPE +
 * fp16 KV write over [n,Hq|Hkv,128], SwiGLU over [n,I]) `reps` times on
 * `threads` threads (rows partitioned), on synthetic inputs it allocates
 * itself. Returns the median seconds per chain, or a negative value on error. */
double ora_bench_layer_chain(int threads, int64_t n, int64_t hidden, int32_t n_heads, int32_t n_kv_heads,
                             int64_t inter, int reps);
/* One op of the chain alone: op 1 residual add + RMSNorm, 2 q/k norm + RoPE + KV, 3 SwiGLU (0 = all). */
double ora_bench_layer_op(int op, int threads, int64_t n, int64_t hidden, int32_t n_heads, int32_t n_kv_heads,
                          int64_t inter, int reps);
/* Same for the embedding gather of `seq` ids from a rows x cols table of `type`. */
double ora_bench_gather(int threads, uint32_t type, int64_t rows, int64_t cols, int64_t seq, int reps);
double ora_bench_matmul(uint32_t type, int64_t rows, int64_t cols, int reps);

#ifdef __cplusplus
}
#endif

#endif /* RPG_ORACLE_CPU_REF_H */
