/* trait_timer.c -- wall-clock cost of the host-slice (Backend trait) calls
 * as a compiled caller sees them: no Python between the calls, the way the
 * reference's Rust decode loop (bitnet-model/src/lib.rs:1004-1036) drives
 * them through an extern "C" block.  Per token and layer of the 2B shape
 * (20/5 heads, head_dim 128, theta 500000) over host caches of 4096 rows:
 * bnr_rope_embed, the store of the new k/v row into the host cache, then
 * bnr_masked_attention at positions pos_end-steps+1 .. pos_end, after 10
 * untimed ones; then bnr_rms_norm (2560) and bnr_sqrelu_gate (6912) host
 * calls; then the backend-owned cache's one-call decode (bnr_kv_decode:
 * rope_embed, store_kv and masked_attention of a token and layer) at the same
 * positions, after the cache is filled up to them.  Prints one JSON object.
 * Used by bench.py; needs a GPU.
 *
 * usage: trait_timer [steps] [pos_end]
 */
#define _POSIX_C_SOURCE 199309L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "bitnet_hip.h"

enum { HQ = 20, HKV = 5, D = 128, CAP = 4096, HIDDEN = 2560, FFN = 6912, WARM = 10 };

static double now_us(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

/* xorshift64* uniform in [-1, 1) */
static uint64_t rng_state = 0xB17E7091u;
static float urand(void) {
  rng_state ^= rng_state >> 12;
  rng_state ^= rng_state << 25;
  rng_state ^= rng_state >> 27;
  const uint64_t x = rng_state * 0x2545F4914F6CDD1Dull;
  return (float)((x >> 40) * (1.0 / 8388608.0)) - 1.0f;
}

static int die(const char *what) {
  fprintf(stderr, "trait_timer: %s failed: %s\n", what, bnr_last_error());
  return 1;
}

int main(int argc, char **argv) {
  const int steps = argc > 1 ? atoi(argv[1]) : 300;
  const int pos_end = argc > 2 ? atoi(argv[2]) : CAP - 1;
  const int p0 = pos_end - steps + 1;
  if (steps <= 0 || pos_end >= CAP || p0 - WARM - 1 < 0) {
    fprintf(stderr, "trait_timer: need 0 < steps, pos_end < %d, pos_end - steps - %d >= 0\n", CAP,
            WARM);
    return 2;
  }
  float *kc = malloc(sizeof(float) * HKV * CAP * D), *vc = malloc(sizeof(float) * HKV * CAP * D);
  if (!kc || !vc) return 1;
  for (size_t i = 0; i < (size_t)HKV * CAP * D; ++i) {
    kc[i] = urand();
    vc[i] = urand();
  }
  float q0[HQ * D], k0[HKV * D], v0[HKV * D], q[HQ * D], k[HKV * D], out[HQ * D];
  for (int i = 0; i < HQ * D; ++i) q0[i] = urand();
  for (int i = 0; i < HKV * D; ++i) {
    k0[i] = urand();
    v0[i] = urand();
  }
  bnr_ctx *c = NULL;
  if (bnr_create(0, &c) != BNR_OK) return die("bnr_create");
  const float theta = 500000.0f;
  const size_t cl = (size_t)HKV * CAP * D;
  /* first call syncs the mirror of rows 0 .. p0-WARM-1 */
  memcpy(q, q0, sizeof q);
  memcpy(k, k0, sizeof k);
  if (bnr_rope_embed(c, q, HQ * D, k, HKV * D, p0 - WARM - 1, D, HQ, HKV, theta)) return die("rope_embed");
  if (bnr_masked_attention(c, q, HQ * D, kc, cl, vc, cl, out, HQ * D, HQ, HKV, D, p0 - WARM - 1))
    return die("masked_attention");
  double t_rope = 0, t_attn = 0;
  for (int pos = p0 - WARM; pos <= pos_end; ++pos) {
    memcpy(q, q0, sizeof q);
    memcpy(k, k0, sizeof k);
    const double t0 = now_us();
    if (bnr_rope_embed(c, q, HQ * D, k, HKV * D, pos, D, HQ, HKV, theta)) return die("rope_embed");
    const double t1 = now_us();
    for (int h = 0; h < HKV; ++h) { /* store_kv into the head-major host cache */
      memcpy(kc + ((size_t)h * CAP + pos) * D, k + h * D, D * sizeof(float));
      memcpy(vc + ((size_t)h * CAP + pos) * D, v0 + h * D, D * sizeof(float));
    }
    const double t2 = now_us();
    if (bnr_masked_attention(c, q, HQ * D, kc, cl, vc, cl, out, HQ * D, HQ, HKV, D, pos))
      return die("masked_attention");
    const double t3 = now_us();
    if (pos >= p0) {
      t_rope += t1 - t0;
      t_attn += t3 - t2;
    }
  }
  static float x[HIDDEN], g[HIDDEN], y[HIDDEN], gate[FFN], up[FFN], inner[FFN];
  for (int i = 0; i < HIDDEN; ++i) {
    x[i] = urand();
    g[i] = 1.0f + 0.2f * urand();
  }
  for (int i = 0; i < FFN; ++i) {
    gate[i] = urand();
    up[i] = urand();
  }
  const int n_glue = 200;
  for (int i = 0; i < 5; ++i) {
    if (bnr_rms_norm(c, x, HIDDEN, g, HIDDEN, 1e-5f, y, HIDDEN)) return die("rms_norm");
    if (bnr_sqrelu_gate(c, gate, FFN, up, FFN, inner, FFN)) return die("sqrelu_gate");
  }
  const double g0 = now_us();
  for (int i = 0; i < n_glue; ++i)
    if (bnr_rms_norm(c, x, HIDDEN, g, HIDDEN, 1e-5f, y, HIDDEN)) return die("rms_norm");
  const double g1 = now_us();
  for (int i = 0; i < n_glue; ++i)
    if (bnr_sqrelu_gate(c, gate, FFN, up, FFN, inner, FFN)) return die("sqrelu_gate");
  const double g2 = now_us();
  /* backend-owned cache, one layer: fill rows 0 .. p0-1, then time the
   * one-call decode at p0 .. pos_end (KVCache::advance after each token) */
  bnr_kv_cache *kvc = NULL;
  if (bnr_kv_cache_create(c, 1, HKV, D, CAP, &kvc)) return die("kv_cache_create");
  double t_kv = 0;
  for (int pos = 0; pos <= pos_end; ++pos) {
    memcpy(q, q0, sizeof q);
    memcpy(k, k0, sizeof k);
    const double t0 = now_us();
    if (bnr_kv_decode(c, kvc, 0, q, HQ * D, k, HKV * D, v0, HKV * D, pos, HQ, theta, out, HQ * D))
      return die("kv_decode");
    const double t1 = now_us();
    if (bnr_kv_cache_advance(kvc, 1)) return die("kv_cache_advance");
    if (pos >= p0) t_kv += t1 - t0;
  }
  bnr_kv_cache_destroy(kvc);
  printf("{\"steps\": %d, \"pos_end\": %d, \"rope_us\": %.3f, \"attn_us\": %.3f, "
         "\"token_layer_us\": %.3f, \"rms_norm_us\": %.3f, \"sqrelu_gate_us\": %.3f, "
         "\"kv_decode_us\": %.3f, \"out0\": %.6g}\n",
         steps, pos_end, t_rope / steps, t_attn / steps, (t_rope + t_attn) / steps,
         (g1 - g0) / n_glue, (g2 - g1) / n_glue, t_kv / steps, (double)out[0]);
  bnr_destroy(c);
  free(kc);
  free(vc);
  return 0;
}
