/* cpu_bench.c -- CPU baseline timing for bench.py (TEST INFRASTRUCTURE ONLY).
 *
 * Times the oracle's restatement of the layer-op chain and of the embedding
 * gather on the host cores, rows partitioned over pthreads. Inputs follow the
 * benchmark configuration's distributions (activations N(0,1), norm weights
 * N(1,0.1); Q4_K / Q6_K tables with fp16 d, dmin = |N(0,0.01)| and uniform
 * scale / quant bytes), drawn from SplitMix64 through Box-Muller, allocated
 * here and never read back.
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "cpu_ref.h"

static uint64_t splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Normal(mean, sd) floats: Box-Muller on two 53-bit uniforms in double. */
static void fill_normal(float* p, int64_t n, uint64_t seed, float mean, float sd) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740993.0);
    const double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    p[i] = (float)(mean + sd * r * cos(6.283185307179586 * u2));
    if (i + 1 < n) p[i + 1] = (float)(mean + sd * r * sin(6.283185307179586 * u2));
  }
}

static void fill_uniform(float* p, int64_t n, uint64_t seed, float lo, float hi) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; ++i) {
    const double u = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    p[i] = (float)(lo + (hi - lo) * u);
  }
}

/* A [rows, row_bytes] Q4_K / Q6_K table: uniform bytes, then every block's fp16
 * scale fields set to fp16(|N(0, 0.01)|) (Q4_K d and dmin, Q6_K d). */
static void fill_quant_table(uint8_t* emb, int64_t rows, int64_t rb, uint32_t type, uint64_t seed) {
  uint64_t s = seed;
  const int64_t total = rows * rb;
  for (int64_t i = 0; i < total; i += 8) {
    const uint64_t r = splitmix64(&s);
    const int64_t m = total - i < 8 ? total - i : 8;
    memcpy(emb + i, &r, (size_t)m);
  }
  const int64_t bb = type == ORA_GGML_Q4_K ? 144 : 210;
  const int n_scales = type == ORA_GGML_Q4_K ? 2 : 1;
  const int64_t first = type == ORA_GGML_Q4_K ? 0 : 208;
  float sc[2];
  for (int64_t b = 0; b < total / bb; ++b) {
    fill_normal(sc, n_scales, seed + 0x9E37u * (uint64_t)(b + 1), 0.0f, 0.01f);
    for (int j = 0; j < n_scales; ++j) {
      const uint16_t h = ora_f32_to_f16_rne(fabsf(sc[j]));
      memcpy(emb + b * bb + first + 2 * j, &h, 2);
    }
  }
}

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int cmp_double(const void* a, const void* b) {
  const double x = *(const double*)a, y = *(const double*)b;
  return (x > y) - (x < y);
}

/* ------------------------------------------------------------------ layer chain */

typedef struct {
  int op; /* 0: the whole chain, 1: residual add + RMSNorm, 2: q/k norm + RoPE + KV, 3: SwiGLU */
  int64_t n, hidden, inter;
  int32_t n_heads, n_kv;
  float *x, *d, *h, *wn, *q, *k, *v, *qn, *kn, *tab, *gate, *up;
  uint16_t *kc, *vc;
  int64_t max_seq;
  int64_t t0, t1; /* token range of this worker */
} ChainArgs;

static void* chain_worker(void* p) {
  const ChainArgs* a = (const ChainArgs*)p;
  const int64_t rows = a->t1 - a->t0;
  if (rows <= 0) return NULL;
  if (a->op == 0 || a->op == 1)
    ora_add_rms_norm(a->x + a->t0 * a->hidden, a->d + a->t0 * a->hidden, a->wn, rows, a->hidden, 1e-6f,
                     a->h + a->t0 * a->hidden);
  /* q/k norm + RoPE + KV write for this worker's tokens (positions t0..t1-1). */
  if (a->op == 0 || a->op == 2)
    ora_qk_norm_rope_kv(a->q + a->t0 * a->n_heads * 128, a->k + a->t0 * a->n_kv * 128,
                        a->v + a->t0 * a->n_kv * 128, a->qn, a->kn, a->n_heads, a->n_kv, 128, a->tab, a->t0, rows,
                        1e-6f, a->kc, a->vc, a->max_seq);
  if (a->op == 0 || a->op == 3) ora_silu_mul(a->gate + a->t0 * a->inter, a->up + a->t0 * a->inter, rows * a->inter);
  return NULL;
}

double ora_bench_layer_op(int op, int threads, int64_t n, int64_t hidden, int32_t n_heads, int32_t n_kv_heads,
                          int64_t inter, int reps) {
  if (op < 0 || op > 3 || threads < 1 || threads > 256 || n <= 0 || reps < 1 || reps > 64) return -1.0;
  ChainArgs base;
  memset(&base, 0, sizeof(base));
  base.op = op;
  base.n = n;
  base.hidden = hidden;
  base.inter = inter;
  base.n_heads = n_heads;
  base.n_kv = n_kv_heads;
  base.max_seq = n;
  base.x = malloc((size_t)(n * hidden) * 4);
  base.d = malloc((size_t)(n * hidden) * 4);
  base.h = malloc((size_t)(n * hidden) * 4);
  base.wn = malloc((size_t)hidden * 4);
  base.q = malloc((size_t)(n * n_heads * 128) * 4);
  base.k = malloc((size_t)(n * n_kv_heads * 128) * 4);
  base.v = malloc((size_t)(n * n_kv_heads * 128) * 4);
  base.qn = malloc(128 * 4);
  base.kn = malloc(128 * 4);
  base.tab = malloc((size_t)(n * 128) * 4);
  base.gate = malloc((size_t)(n * inter) * 4);
  base.up = malloc((size_t)(n * inter) * 4);
  base.kc = malloc((size_t)(n_kv_heads * n * 128) * 2);
  base.vc = malloc((size_t)(n_kv_heads * n * 128) * 2);
  double result = -2.0;
  if (!base.x || !base.d || !base.h || !base.wn || !base.q || !base.k || !base.v || !base.qn || !base.kn ||
      !base.tab || !base.gate || !base.up || !base.kc || !base.vc)
    goto done;
  fill_normal(base.x, n * hidden, 1, 0.f, 1.f);
  fill_normal(base.d, n * hidden, 2, 0.f, 1.f);
  fill_normal(base.wn, hidden, 3, 1.f, 0.1f);
  fill_normal(base.q, n * n_heads * 128, 4, 0.f, 1.f);
  fill_normal(base.k, n * n_kv_heads * 128, 5, 0.f, 1.f);
  fill_normal(base.v, n * n_kv_heads * 128, 6, 0.f, 1.f);
  fill_normal(base.qn, 128, 7, 1.f, 0.1f);
  fill_normal(base.kn, 128, 8, 1.f, 0.1f);
  ora_build_rope_table(128, 1e6, n, base.tab);
  fill_normal(base.gate, n * inter, 9, 0.f, 1.f);
  fill_normal(base.up, n * inter, 10, 0.f, 1.f);

  {
    pthread_t tid[256];
    ChainArgs args[256];
    double times[64];
    for (int r = 0; r < reps; ++r) {
      const double t_start = now_s();
      for (int i = 0; i < threads; ++i) {
        args[i] = base;
        args[i].t0 = n * i / threads;
        args[i].t1 = n * (i + 1) / threads;
        pthread_create(&tid[i], NULL, chain_worker, &args[i]);
      }
      for (int i = 0; i < threads; ++i) pthread_join(tid[i], NULL);
      times[r] = now_s() - t_start;
    }
    qsort(times, (size_t)reps, sizeof(double), cmp_double);
    result = times[reps / 2];
  }
done:
  free(base.x); free(base.d); free(base.h); free(base.wn); free(base.q); free(base.k); free(base.v);
  free(base.qn); free(base.kn); free(base.tab); free(base.gate); free(base.up); free(base.kc); free(base.vc);
  return result;
}

/* ------------------------------------------------------------------ gather */

typedef struct {
  uint32_t type;
  const uint8_t* emb;
  int64_t rows, cols;
  const int32_t* toks;
  float* x;
  int64_t t0, t1;
} GatherArgs;

static void* gather_worker(void* p) {
  const GatherArgs* a = (const GatherArgs*)p;
  if (a->t1 > a->t0)
    ora_embedding_lookup(a->type, a->emb, a->rows, a->cols, a->toks + a->t0, a->t1 - a->t0, a->x + a->t0 * a->cols);
  return NULL;
}

double ora_bench_gather(int threads, uint32_t type, int64_t rows, int64_t cols, int64_t seq, int reps) {
  const int64_t rb = ora_type_row_bytes(type, cols);
  if (threads < 1 || threads > 256 || rb <= 0 || rows <= 0 || seq <= 0 || reps < 1 || reps > 64) return -1.0;
  uint8_t* emb = malloc((size_t)(rows * rb));
  int32_t* toks = malloc((size_t)seq * 4);
  float* x = malloc((size_t)(seq * cols) * 4);
  double result = -2.0;
  if (!emb || !toks || !x) goto done;
  {
    uint64_t s = 11;
    if (type == ORA_GGML_Q4_K || type == ORA_GGML_Q6_K) {
      fill_quant_table(emb, rows, rb, type, 11);
    } else {
      fill_uniform((float*)emb, rows * rb / 4, 11, -1.f, 1.f);
    }
    for (int64_t t = 0; t < seq; ++t) toks[t] = (int32_t)(splitmix64(&s) % (uint64_t)rows);
    pthread_t tid[256];
    GatherArgs args[256];
    double times[64];
    for (int r = 0; r < reps; ++r) {
      const double t_start = now_s();
      for (int i = 0; i < threads; ++i) {
        GatherArgs g = {type, emb, rows, cols, toks, x, seq * i / threads, seq * (i + 1) / threads};
        args[i] = g;
        pthread_create(&tid[i], NULL, gather_worker, &args[i]);
      }
      for (int i = 0; i < threads; ++i) pthread_join(tid[i], NULL);
      times[r] = now_s() - t_start;
    }
    qsort(times, (size_t)reps, sizeof(double), cmp_double);
    result = times[reps / 2];
  }
done:
  free(emb);
  free(toks);
  free(x);
  return result;
}

/* One thread: the oracle's float64 matmul restatement over a random [rows, cols]
 * matrix of `type` times one fp32 vector; median of `reps` runs, in seconds. */
double ora_bench_matmul(uint32_t type, int64_t rows, int64_t cols, int reps) {
  const int64_t rb = ora_type_row_bytes(type, cols);
  if (rb <= 0 || rows <= 0 || reps < 1 || reps > 64) return -1.0;
  uint8_t* w = malloc((size_t)(rows * rb));
  float* x = malloc((size_t)cols * 4);
  double* out = malloc((size_t)rows * 8);
  double result = -2.0;
  if (!w || !x || !out) goto done;
  {
    uint64_t s = 12;
    for (int64_t i = 0; i < rows * rb; i += 8) {
      const uint64_t r = splitmix64(&s);
      const int64_t m = rows * rb - i < 8 ? rows * rb - i : 8;
      memcpy(w + i, &r, (size_t)m);
    }
    fill_uniform(x, cols, 13, -1.f, 1.f);
    double times[64];
    for (int r = 0; r < reps; ++r) {
      const double t0 = now_s();
      ora_matmul_quant_f64(type, w, rows, cols, x, 1, out, NULL);
      times[r] = now_s() - t0;
    }
    qsort(times, (size_t)reps, sizeof(double), cmp_double);
    result = times[reps / 2];
  }
done:
  free(w);
  free(x);
  free(out);
  return result;
}

double ora_bench_layer_chain(int threads, int64_t n, int64_t hidden, int32_t n_heads, int32_t n_kv_heads,
                             int64_t inter, int reps) {
  return ora_bench_layer_op(0, threads, n, hidden, n_heads, n_kv_heads, inter, reps);
}
