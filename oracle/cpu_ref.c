/* cpu_ref.c -- CPU oracle for the hot-path operators (TEST INFRASTRUCTURE ONLY;
 * see cpu_ref.h for what it is, who may use it, and how each function is pinned).
 *
 * Each function cites the reference file:line whose behaviour it restates.
 */
#include "cpu_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

/* binary16 -> binary32, restating src/dtypes.h:21-47: zero keeps its sign,
 * subnormals are normalised by shifting the mantissa until the implicit bit
 * appears, Inf/NaN keep the payload shifted into the fp32 mantissa. */
float ora_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {
      int e = -14; /* value = man * 2^-24 = (man / 2^10) * 2^-14 */
      while ((man & 0x400u) == 0) {
        man <<= 1;
        --e;
      }
      out = sign | ((uint32_t)(e + 127) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 31) {
    out = sign | 0x7F800000u | (man << 13);
  } else {
    out = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

/* binary32 -> binary16 with IEEE 754 round-to-nearest, ties to even: the
 * conversion the reference's KV write performs on the device (__float2half_rn,
 * src/kernels_gpu.cu:725-726). Deliberately NOT src/dtypes.h:50-76, which rounds
 * ties away from zero. NaN -> quiet NaN with the top payload bits kept. */
uint16_t ora_f32_to_f16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) {
    if (a == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
  }
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to Inf */
  if (a < 0x38800000u) {                                    /* below 2^-14: subnormal or zero */
    if (a <= 0x33000000u) return (uint16_t)sign;             /* <= 2^-25 (the tie goes to even 0) */
    const uint32_t e = a >> 23;                              /* 102..112 */
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;                         /* 14..24 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((((a >> 23) - 112u)) << 10) | ((a & 0x7FFFFFu) >> 13);
  const uint32_t rem = a & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q; /* a carry walks into the exponent */
  return (uint16_t)(sign | q);
}

void ora_f16_to_f32_array(const uint16_t* src, int64_t n, float* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = ora_f16_to_f32(src[i]);
}

void ora_f32_to_f16_rne_array(const float* src, int64_t n, uint16_t* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = ora_f32_to_f16_rne(src[i]);
}

/* ------------------------------------------------------------------ dequant */

static float half_at(const uint8_t* p) { return ora_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Block table restated from src/quant.cc:29-45 (device types only). */
int64_t ora_type_row_bytes(uint32_t type, int64_t n_elems) {
  switch (type) {
    case ORA_GGML_F32:
      return n_elems * 4;
    case ORA_GGML_Q4_K:
      return (n_elems % 256) ? -1 : (n_elems / 256) * 144;
    case ORA_GGML_Q6_K:
      return (n_elems % 256) ? -1 : (n_elems / 256) * 210;
    default:
      return -1;
  }
}

/* 6-bit scale/min unpack of sub-block j, src/quant.cc:159-167. */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* src/quant.cc:252-279: per 64-element group, (d1, m1) for the low nibbles and
 * (d2, m2) for the high nibbles; y = d1*q - m1 with separately rounded ops. */
static void deq_q4_k(const uint8_t* src, int64_t n, float* dst) {
  const int64_t nb = n / 256;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* p = src + b * 144;
    const float d = half_at(p);
    const float dmin = half_at(p + 2);
    const uint8_t* scales = p + 4;
    const uint8_t* q = p + 16;
    float* y = dst + b * 256;
    for (int grp = 0; grp < 4; ++grp) {
      uint8_t sc, m;
      scale_min_k4(2 * grp, scales, &sc, &m);
      const float d1 = d * (float)sc;
      const float m1 = dmin * (float)m;
      scale_min_k4(2 * grp + 1, scales, &sc, &m);
      const float d2 = d * (float)sc;
      const float m2 = dmin * (float)m;
      for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0x0F) - m1;
      for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - m2;
      q += 32;
    }
  }
}

/* src/quant.cc:321-354: per 128-element half, four 32-element quarters whose
 * 6-bit values combine a nibble of ql with two bits of qh; y = d*sc*q left to right. */
static void deq_q6_k(const uint8_t* src, int64_t n, float* dst) {
  const int64_t nb = n / 256;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* p = src + b * 210;
    const uint8_t* ql = p;
    const uint8_t* qh = p + 128;
    const int8_t* sc = (const int8_t*)(p + 192);
    const float d = half_at(p + 208);
    float* y = dst + b * 256;
    for (int hf = 0; hf < 2; ++hf) {
      for (int l = 0; l < 32; ++l) {
        const int is = l / 16;
        const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
        const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        y[l] = d * (float)sc[is + 0] * (float)q1;
        y[l + 32] = d * (float)sc[is + 2] * (float)q2;
        y[l + 64] = d * (float)sc[is + 4] * (float)q3;
        y[l + 96] = d * (float)sc[is + 6] * (float)q4;
      }
      y += 128;
      ql += 64;
      qh += 32;
      sc += 8;
    }
  }
}

/* src/quant.cc:416-436, restricted to the device types. */
int ora_dequantize_row(uint32_t type, const uint8_t* src, int64_t n_elems, float* dst) {
  if (ora_type_row_bytes(type, n_elems) < 0) return -1;
  switch (type) {
    case ORA_GGML_F32:
      memcpy(dst, src, (size_t)n_elems * 4);
      return 0;
    case ORA_GGML_Q4_K:
      deq_q4_k(src, n_elems, dst);
      return 0;
    case ORA_GGML_Q6_K:
      deq_q6_k(src, n_elems, dst);
      return 0;
    default:
      return -1;
  }
}

/* src/kernels_gpu.cu:737-823: softmax over the cached positions in double (the
 * reference subtracts the max, exponentiates in fp32 and sums in double; here
 * every step is double, the exact answer to compare against). */
int ora_attention_f64(const float* q, const uint16_t* kc, const uint16_t* vc, int64_t max_seq, int32_t n_heads,
                      int32_t n_kv_heads, int32_t d, int64_t pos0, int64_t seq, double* out, double* smag,
                      double* vmax) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || d <= 0 || pos0 < 0 || seq < 0 ||
      pos0 + seq > max_seq)
    return -1;
  const int32_t group = n_heads / n_kv_heads;
  const double scale = (double)(1.0f / sqrtf((float)d));
  double* s = (double*)malloc((size_t)(pos0 + seq + 1) * sizeof(double));
  if (s == NULL) return -1;
  for (int64_t t = 0; t < seq; ++t) {
    const int64_t pos = pos0 + t;
    for (int32_t h = 0; h < n_heads; ++h) {
      const int32_t kh = h / group;
      const float* qt = q + (t * n_heads + h) * d;
      const uint16_t* kb = kc + (int64_t)kh * max_seq * d;
      const uint16_t* vb = vc + (int64_t)kh * max_seq * d;
      double mx = -INFINITY, mag = 0.0, vm = 0.0;
      for (int64_t j = 0; j <= pos; ++j) {
        double acc = 0.0, a = 0.0;
        for (int32_t e = 0; e < d; ++e) {
          const double p = (double)qt[e] * (double)ora_f16_to_f32(kb[j * d + e]);
          acc += p;
          a += fabs(p);
        }
        s[j] = acc * scale;
        if (s[j] > mx) mx = s[j];
        if (a * scale > mag) mag = a * scale;
        for (int32_t e = 0; e < d; ++e) {
          const double v = fabs((double)ora_f16_to_f32(vb[j * d + e]));
          if (v > vm) vm = v;
        }
      }
      double sum = 0.0;
      for (int64_t j = 0; j <= pos; ++j) {
        s[j] = exp(s[j] - mx);
        sum += s[j];
      }
      double* ot = out + (t * n_heads + h) * d;
      for (int32_t e = 0; e < d; ++e) {
        double acc = 0.0;
        for (int64_t j = 0; j <= pos; ++j) acc += s[j] * (double)ora_f16_to_f32(vb[j * d + e]);
        ot[e] = acc / sum;
      }
      if (smag != NULL) smag[t * n_heads + h] = mag;
      if (vmax != NULL) vmax[t * n_heads + h] = vm;
    }
  }
  free(s);
  return 0;
}

/* src/kernels_gpu.cu:166-560 (MatMulQuantKernel and its Q4_K / Q6_K forms):
 * OUT[t * rows + r] = dot(dequantised row r of W, row t of X). The reference sums
 * in fp32 in a thread-strided order plus a tree; here every product is exact in
 * double (fp32 x fp32 fits in 48 bits) and the sum is taken in double. */
int ora_matmul_quant_f64(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const float* x,
                         int64_t n_tokens, double* out, double* absdot) {
  const int64_t rb = ora_type_row_bytes(type, cols);
  if (rb < 0 || rows < 0 || n_tokens < 0) return -1;
  float* row = (float*)malloc((size_t)(cols > 0 ? cols : 1) * sizeof(float));
  if (row == NULL) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    ora_dequantize_row(type, w + r * rb, cols, row);
    for (int64_t t = 0; t < n_tokens; ++t) {
      const float* xt = x + t * cols;
      double s = 0.0, a = 0.0;
      for (int64_t e = 0; e < cols; ++e) {
        const double p = (double)row[e] * (double)xt[e];
        s += p;
        a += fabs(p);
      }
      out[t * rows + r] = s;
      if (absdot != NULL) absdot[t * rows + r] = a;
    }
  }
  free(row);
  return 0;
}

/* src/kernels_gpu.cu:877-889 (x[t] = dequantised row toks[t]); ids outside
 * [0, rows) give a zero row, the behaviour the device gather defines. */
int ora_embedding_lookup(uint32_t type, const uint8_t* emb, int64_t rows, int64_t cols, const int32_t* toks,
                         int64_t seq, float* x) {
  const int64_t rb = ora_type_row_bytes(type, cols);
  if (rb < 0) return -1;
  for (int64_t t = 0; t < seq; ++t) {
    float* out = x + t * cols;
    const int64_t tok = toks[t];
    if (tok < 0 || tok >= rows) {
      memset(out, 0, (size_t)cols * 4);
      continue;
    }
    ora_dequantize_row(type, emb + tok * rb, cols, out);
  }
  return 0;
}

/* ------------------------------------------------------------------ layer ops */

/* Sum of squares in double, in the reference kernel's order: 128 strided
 * partial sums followed by a halving tree (src/kernels_gpu.cu:572-581). */
static double sumsq_ref_order(const float* xr, int64_t n) {
  double red[128];
  for (int t = 0; t < 128; ++t) {
    double s = 0.0;
    for (int64_t i = t; i < n; i += 128) {
      const double v = (double)xr[i];
      s += v * v;
    }
    red[t] = s;
  }
  for (int st = 64; st > 0; st >>= 1)
    for (int t = 0; t < st; ++t) red[t] += red[t + st];
  return red[0];
}

/* src/kernels_gpu.cu:564-591: scale = (float)(1/sqrt(ss/n + eps)) in double,
 * out = x*scale*w in fp32, left to right; out may equal x. */
void ora_rms_norm(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, float eps, float* out) {
  for (int64_t r = 0; r < n_rows; ++r) {
    const float* xr = x + r * stride;
    float* orow = out + r * stride;
    const double mean = sumsq_ref_order(xr, n) / (double)n;
    const float scale = (float)(1.0 / sqrt(mean + (double)eps));
    for (int64_t i = 0; i < n; ++i) orow[i] = xr[i] * scale * w[i];
  }
}

/* src/gpu_model.cu:90-120. */
void ora_build_rope_table(int32_t head_dim, double theta, int64_t n_pos, float* out) {
  const int32_t half = head_dim / 2;
  for (int64_t p = 0; p < n_pos; ++p) {
    float* row = out + p * head_dim;
    for (int32_t i = 0; i < half; ++i) {
      const double inv = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
      const double ang = (double)p * inv;
      row[i] = (float)cos(ang);
      row[half + i] = (float)sin(ang);
    }
  }
}

/* src/kernels_gpu.cu:598-621: pairs (i, i+half), table row pos0 + row. */
void ora_rope(float* x, int32_t n_heads, int32_t head_dim, const float* tab, int64_t pos0, int64_t n_rows) {
  const int32_t half = head_dim / 2;
  for (int64_t r = 0; r < n_rows; ++r) {
    const float* cs = tab + (pos0 + r) * head_dim;
    for (int32_t h = 0; h < n_heads; ++h) {
      float* xh = x + (r * n_heads + h) * head_dim;
      for (int32_t i = 0; i < half; ++i) {
        const float a = xh[i];
        const float b = xh[i + half];
        const float c = cs[i];
        const float s = cs[half + i];
        xh[i] = a * c - b * s;
        xh[i + half] = b * c + a * s;
      }
    }
  }
}

/* src/kernels_gpu.cu:708-727 with the host checks of :1024-1028: source
 * [t][h][d] -> destination [h][pos0+t][d], fp16 round-to-nearest-even. */
int ora_kv_write(const float* k, const float* v, int32_t n_kv_heads, int32_t head_dim, int64_t pos0, int64_t seq,
                 uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq) {
  if (seq <= 0 || n_kv_heads <= 0 || head_dim <= 0 || pos0 < 0 || pos0 + seq > max_seq) return -1;
  for (int64_t t = 0; t < seq; ++t)
    for (int32_t h = 0; h < n_kv_heads; ++h)
      for (int32_t d = 0; d < head_dim; ++d) {
        const int64_t src = (t * n_kv_heads + h) * head_dim + d;
        const int64_t dst = ((int64_t)h * max_seq + pos0 + t) * head_dim + d;
        k_layer[dst] = ora_f32_to_f16_rne(k[src]);
        v_layer[dst] = ora_f32_to_f16_rne(v[src]);
      }
  return 0;
}

/* src/kernels_gpu.cu:863-869. */
void ora_silu_mul(float* gate, const float* up, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = gate[i];
    gate[i] = (v / (1.0f + expf(-v))) * up[i];
  }
}

/* src/kernels_gpu.cu:871-875. */
void ora_vec_add(float* a, const float* b, int64_t n) {
  for (int64_t i = 0; i < n; ++i) a[i] += b[i];
}

/* src/qwen3_gpu.cu:100 then :103 (GpuVecAddInPlace, then GpuRmsNorm x -> h). */
void ora_add_rms_norm(float* x, const float* d, const float* w, int64_t n_rows, int64_t n, float eps, float* out) {
  ora_vec_add(x, d, n_rows * n);
  ora_rms_norm(x, w, n_rows, n, n, eps, out);
}

/* src/qwen3_gpu.cu:77-91: q/k norm, RoPE on q and k, then the cache write. */
int ora_qk_norm_rope_kv(float* q, float* k, const float* v, const float* q_norm, const float* k_norm,
                        int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const float* tab, int64_t pos0,
                        int64_t seq, float eps, uint16_t* k_layer, uint16_t* v_layer, int64_t max_seq) {
  if (pos0 < 0 || pos0 + seq > max_seq) return -1;
  ora_rms_norm(q, q_norm, seq * n_heads, head_dim, head_dim, eps, q);
  ora_rms_norm(k, k_norm, seq * n_kv_heads, head_dim, head_dim, eps, k);
  ora_rope(q, n_heads, head_dim, tab, pos0, seq);
  ora_rope(k, n_kv_heads, head_dim, tab, pos0, seq);
  return ora_kv_write(k, v, n_kv_heads, head_dim, pos0, seq, k_layer, v_layer, max_seq);
}

/* ------------------------------------------------------------------ float64 restatements */

void ora_rms_norm_f64(const float* x, const float* w, int64_t n_rows, int64_t n, int64_t stride, double eps,
                      double* out) {
  for (int64_t r = 0; r < n_rows; ++r) {
    const float* xr = x + r * stride;
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += (double)xr[i] * (double)xr[i];
    const double scale = 1.0 / sqrt(ss / (double)n + eps);
    for (int64_t i = 0; i < n; ++i) out[r * n + i] = (double)xr[i] * scale * (double)w[i];
  }
}

void ora_rope_f64(const float* x, int32_t n_heads, int32_t head_dim, const float* tab, int64_t pos0, int64_t n_rows,
                  double* out) {
  const int32_t half = head_dim / 2;
  for (int64_t r = 0; r < n_rows; ++r) {
    const float* cs = tab + (pos0 + r) * head_dim;
    for (int32_t h = 0; h < n_heads; ++h) {
      const float* xh = x + (r * n_heads + h) * head_dim;
      double* oh = out + (r * n_heads + h) * head_dim;
      for (int32_t i = 0; i < half; ++i) {
        const double a = xh[i], b = xh[i + half], c = cs[i], s = cs[half + i];
        oh[i] = a * c - b * s;
        oh[i + half] = b * c + a * s;
      }
    }
  }
}

void ora_silu_mul_f64(const float* gate, const float* up, int64_t n, double* out) {
  for (int64_t i = 0; i < n; ++i) {
    const double v = gate[i];
    out[i] = v / (1.0 + exp(-v)) * (double)up[i];
  }
}

/* q/k path of the fused operator in double: RMSNorm then RoPE on the
 * normalised row, no fp32 rounding in between. */
void ora_norm_rope_f64(const float* x, const float* w, int32_t n_heads, int32_t head_dim, const float* tab,
                       int64_t pos0, int64_t n_rows, double eps, double* out) {
  const int32_t half = head_dim / 2;
  for (int64_t r = 0; r < n_rows; ++r) {
    const float* cs = tab + (pos0 + r) * head_dim;
    for (int32_t h = 0; h < n_heads; ++h) {
      const float* xh = x + (r * n_heads + h) * head_dim;
      double* oh = out + (r * n_heads + h) * head_dim;
      double ss = 0.0;
      for (int32_t i = 0; i < head_dim; ++i) ss += (double)xh[i] * (double)xh[i];
      const double scale = 1.0 / sqrt(ss / (double)head_dim + eps);
      for (int32_t i = 0; i < half; ++i) {
        const double a = (double)xh[i] * scale * (double)w[i];
        const double b = (double)xh[i + half] * scale * (double)w[i + half];
        const double c = cs[i], s = cs[half + i];
        oh[i] = a * c - b * s;
        oh[i + half] = b * c + a * s;
      }
    }
  }
}
