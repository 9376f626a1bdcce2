/*
 * bnr_oracle.c -- CPU restatement of bitnetrs's GQA attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the reported CPU baseline); the
 * product library never links it.
 *
 * Build: gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp (oracle/Makefile).
 * -ffp-contract=off matters: rustc never fuses a*b+c, so the only fused
 * multiply-adds are the explicit _mm256_fmadd_ps of the reference's AVX2
 * kernels.  Transcendentals are glibc powf/cosf/sinf/expf, the libm that a
 * Linux build of the reference links for f32::powf/cos/sin/exp.
 */
#include "bnr_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Errors (bitnet-core/src/error.rs:12-55 Display strings)                  */
/* ------------------------------------------------------------------------ */

static __thread char g_err[512];

const char *bnro_last_error(void) { return g_err; }

static int fail_shape(const char *fmt_expected, const char *got) {
  snprintf(g_err, sizeof g_err, "invalid tensor shape: expected %s, got %s",
           fmt_expected, got);
  return BNRO_INVALID_SHAPE;
}

static int fail_config(const char *fmt, ...) {
  char msg[400];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  snprintf(g_err, sizeof g_err, "invalid model configuration: %s", msg);
  return BNRO_INVALID_CONFIG;
}

static int ok(void) {
  g_err[0] = 0;
  return BNRO_OK;
}

static int fail_quant(const char *msg) {
  snprintf(g_err, sizeof g_err, "quantization error: %s", msg);
  return BNRO_QUANTIZATION_ERROR;
}

/* Rust's Display of an f32: the shortest decimal that reads back to the same
 * value, written positionally ("0.5", "-3", "0.0000001", "NaN", "inf"). */
static void rust_f32(char *buf, size_t cap, float x) {
  if (isnan(x)) { snprintf(buf, cap, "NaN"); return; }
  if (isinf(x)) { snprintf(buf, cap, x < 0 ? "-inf" : "inf"); return; }
  if (x == 0.0f) { snprintf(buf, cap, signbit(x) ? "-0" : "0"); return; }
  char e[64];
  int p = 1;
  for (; p <= 9; ++p) {
    snprintf(e, sizeof e, "%.*e", p - 1, (double)x);
    if ((float)strtod(e, NULL) == x) break;
  }
  /* e = [-]d[.ddd]e[+-]XX */
  char digits[16];
  int nd = 0, neg = e[0] == '-';
  const char *q = e + neg;
  for (; *q && *q != 'e'; ++q)
    if (*q != '.') digits[nd++] = *q;
  const int ex = atoi(q + 1);
  while (nd > 1 && digits[nd - 1] == '0') --nd;
  char out[128];
  int o = 0;
  if (neg) out[o++] = '-';
  if (ex >= nd - 1) {
    for (int i = 0; i < nd; ++i) out[o++] = digits[i];
    for (int i = 0; i < ex - (nd - 1); ++i) out[o++] = '0';
  } else if (ex >= 0) {
    for (int i = 0; i < nd; ++i) {
      out[o++] = digits[i];
      if (i == ex) out[o++] = '.';
    }
  } else {
    out[o++] = '0';
    out[o++] = '.';
    for (int i = 0; i < -ex - 1; ++i) out[o++] = '0';
    for (int i = 0; i < nd; ++i) out[o++] = digits[i];
  }
  out[o] = 0;
  snprintf(buf, cap, "%s", out);
}

/* ------------------------------------------------------------------------ */
/* Seeded generator                                                          */
/* ------------------------------------------------------------------------ */

static uint64_t splitmix64(uint64_t *state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void bnro_fill_normal(uint64_t seed, float *out, size_t n, float scale) {
  uint64_t st = seed;
  for (size_t i = 0; i < n; i += 2) {
    /* u1 in (0,1], u2 in [0,1) from the top 53 bits. */
    double u1 = ((double)(splitmix64(&st) >> 11) + 1.0) * 0x1.0p-53;
    double u2 = (double)(splitmix64(&st) >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    double a = 6.283185307179586476925286766559 * u2;
    out[i] = (float)(r * cos(a)) * scale;
    if (i + 1 < n) out[i + 1] = (float)(r * sin(a)) * scale;
  }
}

/* ------------------------------------------------------------------------ */
/* dot / axpy / softmax                                                      */
/* ------------------------------------------------------------------------ */

static int g_force_scalar = 0;
void bnro_force_scalar(int on) { g_force_scalar = on; }

static int use_avx2_fma(void) {
  static int cached = -1;
  if (cached < 0) {
    __builtin_cpu_init();
    cached = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  }
  return cached && !g_force_scalar;
}

/* hsum_f32_avx2, simd.rs:292-307: ((l0+h0)+(l1+h1)) + ((l2+h2)+(l3+h3)). */
static inline float hsum8(__m256 v) {
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 s4 = _mm_add_ps(lo, hi);
  __m128 sh = _mm_movehdup_ps(s4);
  __m128 s2 = _mm_add_ps(s4, sh);
  __m128 sh2 = _mm_movehl_ps(s2, s2);
  __m128 s1 = _mm_add_ss(s2, sh2);
  return _mm_cvtss_f32(s1);
}

/* dot_f32_f32_avx2, simd.rs:676-704. */
static float dot_avx2(const float *a, const float *b, size_t n) {
  size_t chunks = n / 8, rem = n % 8;
  __m256 acc = _mm256_setzero_ps();
  for (size_t i = 0; i < chunks; i++) {
    __m256 va = _mm256_loadu_ps(a + i * 8);
    __m256 vb = _mm256_loadu_ps(b + i * 8);
    acc = _mm256_fmadd_ps(va, vb, acc);
  }
  float r = hsum8(acc);
  size_t base = chunks * 8;
  for (size_t i = 0; i < rem; i++) r += a[base + i] * b[base + i];
  return r;
}

/* dot_f32_f32_scalar, simd.rs:724-731. */
static float dot_scalar(const float *a, const float *b, size_t n) {
  float acc = 0.0f;
  for (size_t i = 0; i < n; i++) acc += a[i] * b[i];
  return acc;
}

float bnro_dot_f32(const float *a, const float *b, size_t n) {
  return use_avx2_fma() ? dot_avx2(a, b, n) : dot_scalar(a, b, n);
}

/* axpy_f32_avx2, simd.rs:743-766 (FMA body, unfused remainder). */
static void axpy_avx2(float alpha, const float *x, float *out, size_t n) {
  size_t chunks = n / 8, rem = n % 8;
  __m256 va = _mm256_set1_ps(alpha);
  for (size_t i = 0; i < chunks; i++) {
    __m256 vx = _mm256_loadu_ps(x + i * 8);
    __m256 vo = _mm256_loadu_ps(out + i * 8);
    _mm256_storeu_ps(out + i * 8, _mm256_fmadd_ps(va, vx, vo));
  }
  size_t base = chunks * 8;
  for (size_t i = 0; i < rem; i++) out[base + i] += alpha * x[base + i];
}

/* axpy_f32_scalar, simd.rs:786-791 (unfused). */
static void axpy_scalar(float alpha, const float *x, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] += alpha * x[i];
}

void bnro_axpy_f32(float alpha, const float *x, float *out, size_t n) {
  if (use_avx2_fma())
    axpy_avx2(alpha, x, out, n);
  else
    axpy_scalar(alpha, x, out, n);
}

/* softmax_f32, ops.rs:206-226.  f32::max ignores a NaN operand, as fmaxf. */
void bnro_softmax_f32(float *x, size_t n) {
  if (n == 0) return;
  float mx = -INFINITY;
  for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  float inv = 1.0f / sum;
  for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                      */
/* ------------------------------------------------------------------------ */

/* Angle formula shared by RopeCache::new (rope.rs:136-145) and
 * compute_cos_sin (rope.rs:368-382): exponent = (-2*i)/d in f32, evaluated
 * left to right; freq = theta.powf(exponent); angle = pos as f32 * freq. */
static inline void rope_angle(size_t pos, size_t i, size_t head_dim, float theta,
                              float *c, float *s) {
  float exponent = -2.0f * (float)i / (float)head_dim;
  float freq = powf(theta, exponent);
  float angle = (float)pos * freq;
  *c = cosf(angle);
  *s = sinf(angle);
}

/* RopeCache::new validation and tables, rope.rs:100-153. */
int bnro_rope_table(size_t max_seq, size_t head_dim, float theta, float *cos_out,
                    float *sin_out) {
  if (head_dim == 0 || head_dim % 2 != 0)
    return fail_config("head_dim must be even and > 0, got %zu", head_dim);
  if (!(theta > 0.0f) || !isfinite(theta))
    { char tf[64]; rust_f32(tf, sizeof tf, theta); return fail_config("theta must be finite and > 0, got %s", tf); }
  size_t half = head_dim / 2;
  for (size_t pos = 0; pos < max_seq; pos++)
    for (size_t i = 0; i < half; i++)
      rope_angle(pos, i, head_dim, theta, &cos_out[pos * half + i],
                 &sin_out[pos * half + i]);
  return ok();
}

/* apply_rope_to_head_slice, rope.rs:414-430: half-split pairing (i, i+half),
 * two products and one add/sub per output, unfused. */
static void rope_head(float *x, const float *c, const float *s, size_t half) {
  for (size_t i = 0; i < half; i++) {
    float lo = x[i], hi = x[i + half];
    x[i] = lo * c[i] - hi * s[i];
    x[i + half] = hi * c[i] + lo * s[i];
  }
}

static int check_qk_len(size_t q_len, size_t k_len, size_t n_heads, size_t n_kv,
                        size_t head_dim) {
  char e[128], g[64];
  if (q_len != n_heads * head_dim) {
    snprintf(e, sizeof e, "q.len() == %zu * %zu = %zu", n_heads, head_dim,
             n_heads * head_dim);
    snprintf(g, sizeof g, "q.len() = %zu", q_len);
    return fail_shape(e, g);
  }
  if (k_len != n_kv * head_dim) {
    snprintf(e, sizeof e, "k.len() == %zu * %zu = %zu", n_kv, head_dim,
             n_kv * head_dim);
    snprintf(g, sizeof g, "k.len() = %zu", k_len);
    return fail_shape(e, g);
  }
  return BNRO_OK;
}

/* apply_rope, rope.rs:227-292. */
int bnro_apply_rope(float *q, size_t q_len, float *k, size_t k_len, size_t position,
                    size_t head_dim, size_t n_heads, size_t n_kv_heads, float theta) {
  char g[64];
  if (head_dim == 0 || head_dim % 2 != 0) {
    snprintf(g, sizeof g, "head_dim = %zu", head_dim);
    return fail_shape("head_dim must be even and > 0", g);
  }
  if (!(theta > 0.0f) || !isfinite(theta))
    { char tf[64]; rust_f32(tf, sizeof tf, theta); return fail_config("theta must be finite and > 0, got %s", tf); }
  int st = check_qk_len(q_len, k_len, n_heads, n_kv_heads, head_dim);
  if (st) return st;
  size_t half = head_dim / 2;
  float *c = malloc(half * sizeof(float)), *s = malloc(half * sizeof(float));
  for (size_t i = 0; i < half; i++) rope_angle(position, i, head_dim, theta, &c[i], &s[i]);
  for (size_t h = 0; h < n_heads; h++) rope_head(q + h * head_dim, c, s, half);
  for (size_t h = 0; h < n_kv_heads; h++) rope_head(k + h * head_dim, c, s, half);
  free(c);
  free(s);
  return ok();
}

/* apply_rope_cached, rope.rs:312-355 (+ RopeCache::at, rope.rs:165-178). */
int bnro_apply_rope_cached(float *q, size_t q_len, float *k, size_t k_len,
                           size_t position, size_t n_heads, size_t n_kv_heads,
                           const float *cos_tab, const float *sin_tab, size_t max_seq,
                           size_t head_dim) {
  int st = check_qk_len(q_len, k_len, n_heads, n_kv_heads, head_dim);
  if (st) return st;
  if (position >= max_seq) {
    char e[64], g[64];
    snprintf(e, sizeof e, "pos < max_seq = %zu", max_seq);
    snprintf(g, sizeof g, "pos = %zu", position);
    return fail_shape(e, g);
  }
  size_t half = head_dim / 2;
  const float *c = cos_tab + position * half, *s = sin_tab + position * half;
  for (size_t h = 0; h < n_heads; h++) rope_head(q + h * head_dim, c, s, half);
  for (size_t h = 0; h < n_kv_heads; h++) rope_head(k + h * head_dim, c, s, half);
  return ok();
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

static int g_threads = 0;
void bnro_set_threads(int n) { g_threads = n; }
int bnro_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_num_procs(); }

/* masked_attention, attention.rs:97-209: validation order 109-161, scale
 * (sqrt(d) as f32).recip() 165, per q head: scores via dot*scale 185-189,
 * softmax 192, zeroed output then axpy over t 195-204. */
int bnro_masked_attention(const float *q, size_t q_len, const float *k_cache,
                          size_t k_len, const float *v_cache, size_t v_len,
                          float *output, size_t out_len, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, size_t cur_pos) {
  char e[160], g[96];
  if (head_dim == 0) return fail_shape("head_dim > 0", "head_dim = 0");
  if (n_kv_heads == 0) return fail_config("n_kv_heads must be > 0");
  if (n_heads == 0) return fail_config("n_heads must be > 0");
  if (n_heads % n_kv_heads != 0)
    return fail_config("n_heads (%zu) must be divisible by n_kv_heads (%zu)", n_heads,
                       n_kv_heads);
  size_t seq_len = cur_pos + 1;
  size_t head_stride = k_len / n_kv_heads;
  size_t required = n_kv_heads * head_stride;
  size_t q_expected = n_heads * head_dim;
  if (q_len != q_expected) {
    snprintf(e, sizeof e, "q.len() == n_heads * head_dim = %zu * %zu = %zu", n_heads,
             head_dim, q_expected);
    snprintf(g, sizeof g, "q.len() = %zu", q_len);
    return fail_shape(e, g);
  }
  if (k_len < required) {
    snprintf(e, sizeof e, "k_cache.len() >= %zu", required);
    snprintf(g, sizeof g, "k_cache.len() = %zu", k_len);
    return fail_shape(e, g);
  }
  if (v_len < required) {
    snprintf(e, sizeof e, "v_cache.len() >= %zu", required);
    snprintf(g, sizeof g, "v_cache.len() = %zu", v_len);
    return fail_shape(e, g);
  }
  if (head_stride < seq_len * head_dim) {
    snprintf(e, sizeof e, "per-head cache stride >= %zu", seq_len * head_dim);
    snprintf(g, sizeof g, "per-head cache stride = %zu", head_stride);
    return fail_shape(e, g);
  }
  if (out_len != q_expected) {
    snprintf(e, sizeof e, "output.len() == n_heads * head_dim = %zu", q_expected);
    snprintf(g, sizeof g, "output.len() = %zu", out_len);
    return fail_shape(e, g);
  }

  float scale = 1.0f / sqrtf((float)head_dim);
  size_t group = n_heads / n_kv_heads;
  int nthr = bnro_get_threads();
  if ((size_t)nthr > n_heads) nthr = (int)n_heads;

#pragma omp parallel num_threads(nthr)
  {
    float *scores = malloc(seq_len * sizeof(float));
#pragma omp for schedule(static)
    for (long hh = 0; hh < (long)n_heads; hh++) {
      size_t h = (size_t)hh;
      size_t kv = h / group;
      const float *qh = q + h * head_dim;
      float *oh = output + h * head_dim;
      const float *kb = k_cache + kv * head_stride;
      const float *vb = v_cache + kv * head_stride;
      for (size_t t = 0; t < seq_len; t++)
        scores[t] = bnro_dot_f32(qh, kb + t * head_dim, head_dim) * scale;
      bnro_softmax_f32(scores, seq_len);
      for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;
      for (size_t t = 0; t < seq_len; t++)
        bnro_axpy_f32(scores[t], vb + t * head_dim, oh, head_dim);
    }
    free(scores);
  }
  return ok();
}

/* ------------------------------------------------------------------------ */
/* CpuBackend (lazy RoPE table policy)                                       */
/* ------------------------------------------------------------------------ */

struct bnro_backend {
  int has_table;
  size_t max_seq, head_dim;
  float theta;
  float *cos_tab, *sin_tab;
};

bnro_backend *bnro_backend_new(void) { return calloc(1, sizeof(bnro_backend)); }

void bnro_backend_free(bnro_backend *b) {
  if (!b) return;
  free(b->cos_tab);
  free(b->sin_tab);
  free(b);
}

/* CpuBackend::rope_embed, bitnet-cpu/src/lib.rs:289-314: rebuild the table
 * when absent, when head_dim changes, when |theta - cached| > 1e-3 or when
 * position >= max_seq; the new max_seq is max(position + 1, 4096).  A failed
 * rebuild leaves the previous table in place (the `?` returns before the
 * assignment). */
int bnro_backend_rope_embed(bnro_backend *b, float *q, size_t q_len, float *k,
                            size_t k_len, size_t position, size_t head_dim,
                            size_t n_heads, size_t n_kv_heads, float theta) {
  int reinit = !b->has_table || b->head_dim != head_dim ||
               fabsf(b->theta - theta) > 1e-3f || position >= b->max_seq;
  if (reinit) {
    size_t max_seq = position + 1 > 4096 ? position + 1 : 4096;
    size_t n = max_seq * (head_dim / 2);
    float *c = NULL, *s = NULL;
    if (head_dim != 0 && head_dim % 2 == 0) {
      c = malloc((n ? n : 1) * sizeof(float));
      s = malloc((n ? n : 1) * sizeof(float));
    }
    int st = bnro_rope_table(max_seq, head_dim, theta, c, s);
    if (st) {
      free(c);
      free(s);
      return st;
    }
    free(b->cos_tab);
    free(b->sin_tab);
    b->cos_tab = c;
    b->sin_tab = s;
    b->max_seq = max_seq;
    b->head_dim = head_dim;
    b->theta = theta;
    b->has_table = 1;
  }
  return bnro_apply_rope_cached(q, q_len, k, k_len, position, n_heads, n_kv_heads,
                                b->cos_tab, b->sin_tab, b->max_seq, b->head_dim);
}

int bnro_backend_rope_state(const bnro_backend *b, size_t *max_seq, size_t *head_dim,
                            float *theta) {
  if (!b->has_table) return 0;
  *max_seq = b->max_seq;
  *head_dim = b->head_dim;
  *theta = b->theta;
  return 1;
}

/* ------------------------------------------------------------------------ */
/* KVCache                                                                   */
/* ------------------------------------------------------------------------ */

struct bnro_kv_cache {
  size_t n_layers, n_kv, head_dim, max_seq, filled;
  size_t *layer_len;
  float **k, **v;
};

/* KVCache::new, bitnet-model/src/lib.rs:148-169 (zeroed backing buffers). */
bnro_kv_cache *bnro_kv_new(size_t n_layers, size_t n_kv_heads, size_t head_dim,
                           size_t max_seq) {
  bnro_kv_cache *c = calloc(1, sizeof *c);
  c->n_layers = n_layers;
  c->n_kv = n_kv_heads;
  c->head_dim = head_dim;
  c->max_seq = max_seq;
  c->layer_len = calloc(n_layers ? n_layers : 1, sizeof(size_t));
  c->k = calloc(n_layers ? n_layers : 1, sizeof(float *));
  c->v = calloc(n_layers ? n_layers : 1, sizeof(float *));
  size_t cap = max_seq * n_kv_heads * head_dim;
  for (size_t l = 0; l < n_layers; l++) {
    c->k[l] = calloc(cap ? cap : 1, sizeof(float));
    c->v[l] = calloc(cap ? cap : 1, sizeof(float));
  }
  return c;
}

void bnro_kv_free(bnro_kv_cache *c) {
  if (!c) return;
  for (size_t l = 0; l < c->n_layers; l++) {
    free(c->k[l]);
    free(c->v[l]);
  }
  free(c->k);
  free(c->v);
  free(c->layer_len);
  free(c);
}

/* KVCache::store_kv, bitnet-model/src/lib.rs:184-236: validation order
 * k len, v len, position < max_seq, position <= layer length; head-major
 * destination kv_h*max_seq*d + position*d; extends the layer when
 * position == layer length. */
int bnro_kv_store(bnro_kv_cache *c, size_t layer, size_t position, const float *k_vec,
                  size_t k_len, const float *v_vec, size_t v_len) {
  char e[96], g[64];
  size_t stride = c->n_kv * c->head_dim;
  if (k_len != stride) {
    snprintf(e, sizeof e, "k_vec.len() = %zu", stride);
    snprintf(g, sizeof g, "%zu", k_len);
    return fail_shape(e, g);
  }
  if (v_len != stride) {
    snprintf(e, sizeof e, "v_vec.len() = %zu", stride);
    snprintf(g, sizeof g, "%zu", v_len);
    return fail_shape(e, g);
  }
  if (position >= c->max_seq) {
    snprintf(e, sizeof e, "position < max_seq (%zu)", c->max_seq);
    snprintf(g, sizeof g, "position = %zu", position);
    return fail_shape(e, g);
  }
  if (position > c->layer_len[layer]) {
    snprintf(e, sizeof e, "position <= layer_len_positions (%zu)", c->layer_len[layer]);
    snprintf(g, sizeof g, "position = %zu", position);
    return fail_shape(e, g);
  }
  for (size_t h = 0; h < c->n_kv; h++) {
    size_t dst = h * c->max_seq * c->head_dim + position * c->head_dim;
    memcpy(c->k[layer] + dst, k_vec + h * c->head_dim, c->head_dim * sizeof(float));
    memcpy(c->v[layer] + dst, v_vec + h * c->head_dim, c->head_dim * sizeof(float));
  }
  if (position == c->layer_len[layer]) c->layer_len[layer]++;
  return ok();
}

/* KVCache::advance, lib.rs:244-252 (the reference panics on overflow; here
 * the overflow is reported as a backend error so a test can observe it). */
int bnro_kv_advance(bnro_kv_cache *c) {
  if (c->filled >= c->max_seq) {
    snprintf(g_err, sizeof g_err,
             "KVCache::advance overflow: filled_positions=%zu max_seq=%zu", c->filled,
             c->max_seq);
    return BNRO_BACKEND_ERROR;
  }
  c->filled++;
  return ok();
}

/* KVCache::clear, lib.rs:285-292. */
void bnro_kv_clear(bnro_kv_cache *c) {
  size_t cap = c->max_seq * c->n_kv * c->head_dim;
  for (size_t l = 0; l < c->n_layers; l++) {
    memset(c->k[l], 0, cap * sizeof(float));
    memset(c->v[l], 0, cap * sizeof(float));
    c->layer_len[l] = 0;
  }
  c->filled = 0;
}

size_t bnro_kv_len(const bnro_kv_cache *c) { return c->filled; }
size_t bnro_kv_layer_len(const bnro_kv_cache *c, size_t layer) {
  return c->layer_len[layer];
}
float *bnro_kv_k(bnro_kv_cache *c, size_t layer) { return c->k[layer]; }
float *bnro_kv_v(bnro_kv_cache *c, size_t layer) { return c->v[layer]; }
size_t bnro_kv_backing_len(const bnro_kv_cache *c) {
  return c->max_seq * c->n_kv * c->head_dim;
}

/* ------------------------------------------------------------------------ */
/* Per-token call sequence of one layer                                      */
/* ------------------------------------------------------------------------ */

/* BitNetModel::forward hot calls, bitnet-model/src/lib.rs:684-718:
 * rope_embed(q_buf, k_buf, position) -> store_kv(layer, position) ->
 * masked_attention(q_buf, k[layer], v[layer], cur_pos = position). */
int bnro_layer_tokens(bnro_backend *b, bnro_kv_cache *c, size_t layer, float *q_raw,
                      float *k_raw, const float *v_raw, size_t n_tokens,
                      size_t start_pos, size_t n_heads, size_t n_kv_heads,
                      size_t head_dim, float theta, float *out) {
  size_t qd = n_heads * head_dim, kd = n_kv_heads * head_dim;
  size_t backing = bnro_kv_backing_len(c);
  for (size_t i = 0; i < n_tokens; i++) {
    size_t pos = start_pos + i;
    float *q = q_raw + i * qd, *k = k_raw + i * kd;
    const float *v = v_raw + i * kd;
    int st = bnro_backend_rope_embed(b, q, qd, k, kd, pos, head_dim, n_heads,
                                     n_kv_heads, theta);
    if (st) return st;
    st = bnro_kv_store(c, layer, pos, k, kd, v, kd);
    if (st) return st;
    st = bnro_masked_attention(q, qd, c->k[layer], backing, c->v[layer], backing,
                               out + i * qd, qd, n_heads, n_kv_heads, head_dim, pos);
    if (st) return st;
  }
  return ok();
}

/* ------------------------------------------------------------------------ */
/* W2A8 ternary GEMV                                                         */
/* ------------------------------------------------------------------------ */

/* ternary.rs:266-286 */
int bnro_pack_ternary(const int8_t *w, size_t n, uint8_t *out) {
  const size_t nb = (n + 3) / 4;
  memset(out, 0, nb);
  for (size_t i = 0; i < n; ++i) {
    unsigned code;
    switch (w[i]) {
      case 1: code = 0; break;
      case 0: code = 1; break;
      case -1: code = 2; break;
      default:
        return fail_config("ternary value out of range");
    }
    out[i / 4] |= (uint8_t)(code << (2 * (i % 4)));
  }
  return ok();
}

/* DECODE_LUT (simd.rs:390-404): byte -> its four values, code 0b11 -> 0. */
static const int8_t kTernaryCode[4] = {1, 0, -1, 0};
static int8_t g_decode_lut[256][4];
static int g_decode_lut_ready;

static void build_decode_lut(void) {
  for (int b = 0; b < 256; ++b)
    for (int p = 0; p < 4; ++p) g_decode_lut[b][p] = kTernaryCode[(b >> (2 * p)) & 3];
  __atomic_store_n(&g_decode_lut_ready, 1, __ATOMIC_RELEASE);
}

/* unpack_packed_to_i8 (simd.rs:417-446): whole bytes through the LUT, then
 * the remainder of the last byte. */
static void unpack_packed_to_i8(const uint8_t *packed, int8_t *out, size_t n) {
  if (!__atomic_load_n(&g_decode_lut_ready, __ATOMIC_ACQUIRE)) build_decode_lut();
  const size_t full = n / 4, rem = n % 4;
  for (size_t i = 0; i < full; ++i) memcpy(out + 4 * i, g_decode_lut[packed[i]], 4);
  for (size_t j = 0; j < rem; ++j) out[4 * full + j] = g_decode_lut[packed[full]][j];
}

/* dot_ternary_i8_avx2 (simd.rs:118-171): sign-extend to i16, vpsignw,
 * vpmaddwd against ones, i32 lanes, then the scalar tail.  Exact integer
 * arithmetic, so the lane order does not change the result. */
static int32_t dot_ternary_i8_avx2(const int8_t *w, const int8_t *a, size_t len) {
  const size_t chunks = len / 16;
  const __m256i ones = _mm256_set1_epi16(1);
  __m256i acc = _mm256_setzero_si256();
  for (size_t i = 0; i < chunks; ++i) {
    const __m256i w16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + 16 * i)));
    const __m256i a16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + 16 * i)));
    acc = _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_sign_epi16(a16, w16), ones));
  }
  int32_t lanes[8];
  _mm256_storeu_si256((__m256i *)lanes, acc);
  int32_t r = 0;
  for (int i = 0; i < 8; ++i) r += lanes[i];
  for (size_t i = chunks * 16; i < len; ++i) r += (int32_t)w[i] * (int32_t)a[i];
  return r;
}

/* simd.rs:461-500: 64-element chunks decoded into a stack buffer. */
int32_t bnro_dot_packed_ternary_i8(const uint8_t *packed, const int8_t *act, size_t n) {
  int8_t buf[64];
  int32_t total = 0;
  const size_t full = n / 64, rem = n % 64;
  for (size_t c = 0; c < full; ++c) {
    unpack_packed_to_i8(packed + 16 * c, buf, 64);
    total += dot_ternary_i8_avx2(buf, act + 64 * c, 64);
  }
  if (rem) {
    unpack_packed_to_i8(packed + 16 * full, buf, rem);
    for (size_t i = 0; i < rem; ++i) total += (int32_t)buf[i] * (int32_t)act[64 * full + i];
  }
  return total;
}

/* gemv.rs:251-310 (validation order and messages as there). */
int bnro_ternary_gemv_preq(const uint8_t *weight_packed, size_t weight_len, float weight_scale,
                           const int8_t *activation_q, size_t act_len, float act_absmax,
                           float *output, size_t out_len, size_t out_features,
                           size_t in_features) {
  char e[160], g[96], f[64];
  const size_t packed_cols = (in_features + 3) / 4;
  if (packed_cols != 0 && out_features > SIZE_MAX / packed_cols)
    return fail_shape("weight size fits usize", "overflow");
  const size_t expected = out_features * packed_cols;
  if (weight_len != expected) {
    snprintf(e, sizeof e, "weight_packed.len() == %zu * ceil(%zu/4) = %zu", out_features,
             in_features, expected);
    snprintf(g, sizeof g, "weight_packed.len() == %zu", weight_len);
    return fail_shape(e, g);
  }
  if (act_len != in_features) {
    snprintf(e, sizeof e, "activation.len() == %zu", in_features);
    snprintf(g, sizeof g, "activation.len() == %zu", act_len);
    return fail_shape(e, g);
  }
  if (out_len != out_features) {
    snprintf(e, sizeof e, "output.len() == %zu", out_features);
    snprintf(g, sizeof g, "output.len() == %zu", out_len);
    return fail_shape(e, g);
  }
  if (weight_scale <= 0.0f || !isfinite(weight_scale)) {
    rust_f32(f, sizeof f, weight_scale);
    snprintf(e, sizeof e, "weight_scale must be finite > 0, got %s", f);
    return fail_quant(e);
  }
  if (act_absmax <= 0.0f || !isfinite(act_absmax)) {
    rust_f32(f, sizeof f, act_absmax);
    snprintf(e, sizeof e, "act_scale must be finite > 0, got %s", f);
    return fail_quant(e);
  }
  /* combined_scale = weight_scale * act_scale / 127.0 (left to right, f32) */
  const float combined = weight_scale * act_absmax / 127.0f;
  const int nthr = bnro_get_threads();
#pragma omp parallel for num_threads(nthr) schedule(static)
  for (size_t i = 0; i < out_features; ++i) {
    const int32_t acc =
        bnro_dot_packed_ternary_i8(weight_packed + i * packed_cols, activation_q, in_features);
    output[i] = (float)acc * combined;
  }
  return ok();
}

/* ------------------------------------------------------------------------ */
/* LM head with i8 weights                                                   */
/* ------------------------------------------------------------------------ */

/* dot_f32_i8w_avx2 (simd.rs:1213-1246). */
static float dot_i8w_avx2(const int8_t *w, const float *h, size_t n) {
  const size_t chunks = n / 8, rem = n % 8;
  __m256 acc = _mm256_setzero_ps();
  for (size_t i = 0; i < chunks; ++i) {
    const __m128i w8 = _mm_loadl_epi64((const __m128i *)(w + 8 * i));
    const __m256 wf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(w8));
    acc = _mm256_fmadd_ps(wf, _mm256_loadu_ps(h + 8 * i), acc);
  }
  float r = hsum8(acc);
  for (size_t i = 0; i < rem; ++i) r += (float)w[8 * chunks + i] * h[8 * chunks + i];
  return r;
}

/* scalar fallback (simd.rs:1264-1268). */
static float dot_i8w_scalar(const int8_t *w, const float *h, size_t n) {
  float acc = 0.0f;
  for (size_t i = 0; i < n; ++i) acc += (float)w[i] * h[i];
  return acc;
}

float bnro_dot_f32_i8w(const int8_t *w, const float *hidden, size_t n) {
  return use_avx2_fma() ? dot_i8w_avx2(w, hidden, n) : dot_i8w_scalar(w, hidden, n);
}

int bnro_lm_head_matmul_i8(const float *hidden, size_t hidden_len, const int8_t *weights,
                           size_t weights_len, const float *scales, size_t scales_len,
                           float *output, size_t out_len, size_t vocab_size,
                           size_t hidden_size) {
  char e[128], g[96];
  if (hidden_len != hidden_size) {
    snprintf(e, sizeof e, "hidden.len() == %zu", hidden_size);
    snprintf(g, sizeof g, "hidden.len() == %zu", hidden_len);
    return fail_shape(e, g);
  }
  if (hidden_size != 0 && vocab_size > SIZE_MAX / hidden_size)
    return fail_shape("weight size fits usize", "overflow");
  if (weights_len != vocab_size * hidden_size) {
    snprintf(e, sizeof e, "weights_i8.len() == %zu * %zu", vocab_size, hidden_size);
    snprintf(g, sizeof g, "weights_i8.len() == %zu", weights_len);
    return fail_shape(e, g);
  }
  if (scales_len != vocab_size) {
    snprintf(e, sizeof e, "scales.len() == %zu", vocab_size);
    snprintf(g, sizeof g, "scales.len() == %zu", scales_len);
    return fail_shape(e, g);
  }
  if (out_len != vocab_size) {
    snprintf(e, sizeof e, "output.len() == %zu", vocab_size);
    snprintf(g, sizeof g, "output.len() == %zu", out_len);
    return fail_shape(e, g);
  }
  const int nthr = bnro_get_threads();
  /* rayon par_chunks_mut(256): rows are independent, so any split is the same */
#pragma omp parallel for num_threads(nthr) schedule(static, 256)
  for (size_t v = 0; v < vocab_size; ++v)
    output[v] = bnro_dot_f32_i8w(weights + v * hidden_size, hidden, hidden_size) * scales[v];
  return ok();
}

/* ------------------------------------------------------------------------ */
/* Layer glue: RMSNorm, absmax quantisation, squared-ReLU gate               */
/* ------------------------------------------------------------------------ */

/* sum_squares_f32_avx2 (simd.rs:802-828) and the scalar fallback (simd.rs:838). */
float bnro_sum_squares_f32(const float *x, size_t n) {
  if (use_avx2_fma()) {
    const size_t chunks = n / 8, rem = n % 8;
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < chunks; ++i) {
      const __m256 v = _mm256_loadu_ps(x + 8 * i);
      acc = _mm256_fmadd_ps(v, v, acc);
    }
    float r = hsum8(acc);
    for (size_t i = 0; i < rem; ++i) r += x[8 * chunks + i] * x[8 * chunks + i];
    return r;
  }
  float acc = 0.0f;
  for (size_t i = 0; i < n; ++i) acc += x[i] * x[i];
  return acc;
}

/* norm.rs:76-136 */
int bnro_rms_norm(const float *input, size_t in_len, const float *weight, size_t w_len,
                  float eps, float *output, size_t out_len) {
  char e[96], g[96], f[64];
  if (in_len != w_len) {
    snprintf(e, sizeof e, "input.len() == weight.len() = %zu", w_len);
    snprintf(g, sizeof g, "input.len() = %zu", in_len);
    return fail_shape(e, g);
  }
  if (in_len != out_len) {
    snprintf(e, sizeof e, "input.len() == output.len() = %zu", in_len);
    snprintf(g, sizeof g, "output.len() = %zu", out_len);
    return fail_shape(e, g);
  }
  if (eps <= 0.0f || !isfinite(eps)) {
    rust_f32(f, sizeof f, eps);
    snprintf(e, sizeof e, "eps must be finite and > 0, got %s", f);
    return fail_quant(e);
  }
  if (in_len == 0) return ok();
  const float d = (float)in_len;
  const float sum_sq = bnro_sum_squares_f32(input, in_len);
  const float rms = sqrtf(sum_sq / d + eps);
  const float inv = 1.0f / rms;
  for (size_t i = 0; i < in_len; ++i) output[i] = input[i] * inv * weight[i];
  return ok();
}

/* absmax.rs:127-170 */
int bnro_absmax_quantize_row(const float *x, size_t n, int8_t *out, size_t out_len,
                             float *scale) {
  char e[128], f[64];
  if (n == 0) return fail_quant("cannot quantise an empty activation vector");
  if (out_len != n) {
    snprintf(e, sizeof e, "output buffer length %zu != input length %zu", out_len, n);
    return fail_quant(e);
  }
  float max_abs = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    if (!isfinite(x[i])) {
      rust_f32(f, sizeof f, x[i]);
      snprintf(e, sizeof e, "non-finite activation value at index %zu: %s", i, f);
      return fail_quant(e);
    }
    const float a = fabsf(x[i]);
    if (a > max_abs) max_abs = a;
  }
  const float clamped = max_abs > 1e-5f ? max_abs : 1e-5f; /* f32::max(max_abs, 1e-5) */
  *scale = clamped / 127.0f;
  const float inv_scale = 127.0f / clamped;
  for (size_t i = 0; i < n; ++i) {
    float r = roundf(x[i] * inv_scale); /* f32::round: half away from zero */
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    out[i] = (int8_t)r;
  }
  return ok();
}

/* lib.rs:494-509, simd.rs:1135-1185 */
int bnro_sqrelu_gate(const float *gate, size_t g_len, const float *up, size_t u_len,
                     float *out, size_t out_len) {
  char e[96], g[96];
  if (g_len != u_len || g_len != out_len) {
    snprintf(e, sizeof e, "gate.len() == up.len() == out.len() = %zu", g_len);
    snprintf(g, sizeof g, "up.len()=%zu, out.len()=%zu", u_len, out_len);
    return fail_shape(e, g);
  }
  for (size_t i = 0; i < g_len; ++i) {
    const float r = gate[i] > 0.0f ? gate[i] : 0.0f; /* max_ps(g, 0): NaN -> 0 */
    out[i] = r * r * up[i];
  }
  return ok();
}
