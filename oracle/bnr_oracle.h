/*
 * bnr_oracle.h -- CPU restatement of bitnetrs's GQA attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker / the reported CPU baseline.  The product (libbitnet_hip.so) never
 * links or calls it.
 *
 * Every function restates a reference function with the same f32 operation
 * order (AVX2+FMA lanes for dot/axpy, glibc powf/cosf/sinf/expf, no FP
 * contraction); the citation is given beside each declaration.  Status codes
 * are the same as the product's C ABI (include/bitnet_hip.h).
 */
#ifndef BNR_ORACLE_H
#define BNR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: one per BitNetError kind that the path can produce
 * (bitnet-core/src/error.rs:12-55). */
#define BNRO_OK 0
#define BNRO_INVALID_SHAPE 1
#define BNRO_INVALID_CONFIG 2
#define BNRO_BACKEND_ERROR 3
#define BNRO_QUANTIZATION_ERROR 5

/* Last error message of the calling thread ("" after success). */
const char *bnro_last_error(void);

/* Seeded N(0,1) generator: SplitMix64 -> Box-Muller in f64 -> f32.
 * Deterministic and shared by tests and golden-fixture scripts. */
void bnro_fill_normal(uint64_t seed, float *out, size_t n, float scale);

/* simd::dot_f32_f32_fast  bitnet-cpu/src/simd.rs:711-720
 * (AVX2 body simd.rs:676-704, hsum simd.rs:292-307, scalar simd.rs:724-731) */
float bnro_dot_f32(const float *a, const float *b, size_t n);
/* simd::axpy_f32_fast  bitnet-cpu/src/simd.rs:772-782
 * (AVX2 body simd.rs:743-766, scalar simd.rs:786-791) */
void bnro_axpy_f32(float alpha, const float *x, float *out, size_t n);
/* ops::softmax_f32  bitnet-core/src/backend/ops.rs:206-226 */
void bnro_softmax_f32(float *x, size_t n);
/* Set to 1 to force the scalar dot/axpy fallbacks (simd.rs:724-731,786-791)
 * that the reference takes on a CPU without AVX2+FMA. */
void bnro_force_scalar(int on);

/* RopeCache::new  bitnet-cpu/src/rope.rs:100-153.  cos/sin: [max_seq*head_dim/2]. */
int bnro_rope_table(size_t max_seq, size_t head_dim, float theta, float *cos_out,
                    float *sin_out);
/* apply_rope (uncached)  bitnet-cpu/src/rope.rs:227-292, compute_cos_sin 368-382 */
int bnro_apply_rope(float *q, size_t q_len, float *k, size_t k_len, size_t position,
                    size_t head_dim, size_t n_heads, size_t n_kv_heads, float theta);
/* apply_rope_cached  bitnet-cpu/src/rope.rs:312-355, RopeCache::at 165-178 */
int bnro_apply_rope_cached(float *q, size_t q_len, float *k, size_t k_len,
                           size_t position, size_t n_heads, size_t n_kv_heads,
                           const float *cos_tab, const float *sin_tab, size_t max_seq,
                           size_t head_dim);

/* attention::masked_attention  bitnet-cpu/src/attention.rs:97-209 */
int bnro_masked_attention(const float *q, size_t q_len, const float *k_cache,
                          size_t k_len, const float *v_cache, size_t v_len,
                          float *output, size_t out_len, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, size_t cur_pos);

/* CpuBackend: the trait object with its lazily built RoPE table
 * (bitnet-cpu/src/lib.rs:71-80, rope_embed 289-314, masked_attention 333-347). */
typedef struct bnro_backend bnro_backend;
bnro_backend *bnro_backend_new(void);
void bnro_backend_free(bnro_backend *b);
int bnro_backend_rope_embed(bnro_backend *b, float *q, size_t q_len, float *k,
                            size_t k_len, size_t position, size_t head_dim,
                            size_t n_heads, size_t n_kv_heads, float theta);
/* (max_seq, head_dim, theta) of the table currently held, for tests. */
int bnro_backend_rope_state(const bnro_backend *b, size_t *max_seq, size_t *head_dim,
                            float *theta);

/* KVCache  bitnet-model/src/lib.rs:118-292 (one struct, all layers). */
typedef struct bnro_kv_cache bnro_kv_cache;
bnro_kv_cache *bnro_kv_new(size_t n_layers, size_t n_kv_heads, size_t head_dim,
                           size_t max_seq);
void bnro_kv_free(bnro_kv_cache *c);
int bnro_kv_store(bnro_kv_cache *c, size_t layer, size_t position, const float *k_vec,
                  size_t k_len, const float *v_vec, size_t v_len);
int bnro_kv_advance(bnro_kv_cache *c);
void bnro_kv_clear(bnro_kv_cache *c);
size_t bnro_kv_len(const bnro_kv_cache *c);
size_t bnro_kv_layer_len(const bnro_kv_cache *c, size_t layer);
/* Whole backing buffer of a layer (what k_slice/v_slice return, lib.rs:262-280). */
float *bnro_kv_k(bnro_kv_cache *c, size_t layer);
float *bnro_kv_v(bnro_kv_cache *c, size_t layer);
size_t bnro_kv_backing_len(const bnro_kv_cache *c);

/* The per-layer, per-token call sequence of BitNetModel::forward
 * (bitnet-model/src/lib.rs:684-718) and forward_into (lib.rs:1004-1036),
 * for the attention part only: for each token i, rope_embed at position
 * start_pos+i, store_kv, masked_attention(cur_pos = start_pos+i).
 * q_raw/k_raw/v_raw: [n_tokens x heads x head_dim] pre-RoPE projections;
 * q_raw and k_raw are rotated in place (as the model's scratch buffers are).
 * out: [n_tokens x n_heads x head_dim]. */
int bnro_layer_tokens(bnro_backend *b, bnro_kv_cache *c, size_t layer, float *q_raw,
                      float *k_raw, const float *v_raw, size_t n_tokens,
                      size_t start_pos, size_t n_heads, size_t n_kv_heads,
                      size_t head_dim, float theta, float *out);

/* ---- W2A8 ternary GEMV (the next component after attention) ---- */

/* pack_ternary  bitnet-core/src/quant/ternary.rs:266-286: n values in
 * {-1,0,+1} -> ceil(n/4) bytes, value i at bits 2(i%4) of byte i/4,
 * +1 -> 0b00, 0 -> 0b01, -1 -> 0b10, unused positions 0b00. */
int bnro_pack_ternary(const int8_t *w, size_t n, uint8_t *out);
/* simd::dot_packed_ternary_i8_fast  bitnet-cpu/src/simd.rs:511-531
 * (AVX2 body dot_packed_ternary_i8_avx2_chunked 461-500, LUT decode
 * DECODE_LUT 390-404 with code 0b11 -> 0, dot_ternary_i8_avx2 118-171):
 * exact i32 sum of decoded weight x activation over n elements. */
int32_t bnro_dot_packed_ternary_i8(const uint8_t *packed, const int8_t *act, size_t n);
/* gemv::ternary_gemv_quantised  bitnet-cpu/src/gemv.rs:251-310, which is
 * CpuBackend::ternary_gemv_preq (bitnet-cpu/src/lib.rs:519-538):
 * out[i] = (float)dot(W[i], act) * (weight_scale * act_absmax / 127). */
int bnro_ternary_gemv_preq(const uint8_t *weight_packed, size_t weight_len, float weight_scale,
                           const int8_t *activation_q, size_t act_len, float act_absmax,
                           float *output, size_t out_len, size_t out_features,
                           size_t in_features);

/* ---- LM head with i8 weights ---- */

/* simd::dot_f32_i8w_fast  bitnet-cpu/src/simd.rs:1255-1269 (AVX2+FMA body
 * dot_f32_i8w_avx2 1213-1246: 8 lanes, i8 -> f32, fmadd per 8-chunk,
 * hsum_f32_avx2 292-307, unfused scalar tail; scalar fallback 1264-1268). */
float bnro_dot_f32_i8w(const int8_t *w, const float *hidden, size_t n);
/* CpuBackend::lm_head_matmul_i8_into  bitnet-cpu/src/lib.rs:544-575:
 * output[v] = dot_f32_i8w(weights[v*hidden_size ..], hidden) * scales[v].
 * The reference only debug-asserts the lengths; here a mismatch is
 * InvalidShape. */
int bnro_lm_head_matmul_i8(const float *hidden, size_t hidden_len, const int8_t *weights,
                           size_t weights_len, const float *scales, size_t scales_len,
                           float *output, size_t out_len, size_t vocab_size,
                           size_t hidden_size);

/* ---- Layer glue ---- */

/* simd::sum_squares_f32_fast  bitnet-cpu/src/simd.rs:802-839 (AVX2+FMA: 8 FMA
 * lanes, hsum, unfused tail; scalar fallback: sequential sum of x*x). */
float bnro_sum_squares_f32(const float *x, size_t n);
/* norm::rms_norm  bitnet-cpu/src/norm.rs:76-136 (= CpuBackend::rms_norm,
 * bitnet-cpu/src/lib.rs:268-270): rms = sqrt(sum_sq/d + eps), inv = 1/rms,
 * out[i] = (x[i]*inv)*w[i] (mul_scale_f32_fast simd.rs:850-890). */
int bnro_rms_norm(const float *input, size_t in_len, const float *weight, size_t w_len,
                  float eps, float *output, size_t out_len);
/* absmax::absmax_quantize_row_into  bitnet-core/src/quant/absmax.rs:127-170:
 * scale = max(max|x|, 1e-5)/127, q = clamp(round(x*127/max), -128, 127). */
int bnro_absmax_quantize_row(const float *x, size_t n, int8_t *out, size_t out_len,
                             float *scale);
/* CpuBackend::sqrelu_gate  bitnet-cpu/src/lib.rs:494-509 ->
 * simd::sqrelu_gate_f32_fast simd.rs:1135-1185: out = (r*r)*up, r = max(gate, 0). */
int bnro_sqrelu_gate(const float *gate, size_t g_len, const float *up, size_t u_len,
                     float *out, size_t out_len);

/* Number of OpenMP threads the attention head loop uses (Rayon sizes its
 * pool to all logical cores, lib.rs:99-133). 0 = all cores. */
void bnro_set_threads(int n);
int bnro_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
