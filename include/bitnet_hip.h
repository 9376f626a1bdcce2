/*
 * bitnet_hip.h -- C ABI of the MI355X (gfx950) GQA attention hot path of
 * bitnetrs: RoPE (half-split, any theta) on Q/K, KV-cache append into an
 * HBM-resident head-major cache, split-K decode attention and causal
 * flash prefill; and the W2A8 ternary GEMV of the layer projections.
 *
 * Conventions
 *  - Every entry point returns an int status (BNR_OK == 0) and never aborts.
 *    On failure, bnr_last_error() returns the calling thread's message; its
 *    text follows BitNetError's Display strings
 *    (bitnet-core/src/error.rs:12-55).
 *  - "Host" entry points (bnr_rope_embed, bnr_masked_attention,
 *    bnr_ternary_gemv_preq) take host
 *    slices exactly as the reference's Backend trait methods do and are
 *    synchronous: outputs are written when they return.
 *  - "Device" entry points (bnr_dev_*) take device pointers (HBM), are
 *    ordered on the given HIP stream (NULL = the legacy default stream) and
 *    return as soon as the work is enqueued.  Calls that share one context
 *    share its workspace: they must be issued on one stream, or serialised
 *    by the caller.
 *  - Tensors are fp32, row-major.  A KV cache of one layer is head-major
 *    [n_kv_heads x cap x head_dim]: element (h, t, d) lives at
 *    h*cap*head_dim + t*head_dim + d (Backend::masked_attention contract,
 *    bitnet-core/src/backend/mod.rs:278-287; KVCache::store_kv,
 *    bitnet-model/src/lib.rs:218-228).
 */
#ifndef BITNET_HIP_H
#define BITNET_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, one per BitNetError variant the path can return. */
#define BNR_OK 0
#define BNR_INVALID_SHAPE 1      /* BitNetError::InvalidShape            */
#define BNR_INVALID_CONFIG 2     /* BitNetError::InvalidConfig           */
#define BNR_BACKEND_ERROR 3      /* BitNetError::BackendError{"HIP",..}  */
#define BNR_UNSUPPORTED_DEVICE 4 /* BitNetError::UnsupportedDevice       */
#define BNR_QUANTIZATION_ERROR 5 /* BitNetError::QuantizationError       */

typedef struct bnr_ctx bnr_ctx;

/* Message of the last failed call on this thread ("" after a success). */
const char *bnr_last_error(void);

/* The same error as fields, so that a binding rebuilds the BitNetError
 * variant itself rather than wrapping the Display text again
 * (bitnet-core/src/error.rs:12-55).  Returns the status of the error that
 * bnr_last_error() describes (BNR_OK when there is none) and points *first
 * and *second (either may be NULL) at:
 *   BNR_INVALID_SHAPE       expected, got     InvalidShape { expected, got }
 *   BNR_INVALID_CONFIG      message, ""       InvalidConfig(message)
 *   BNR_BACKEND_ERROR       "HIP", message    BackendError { backend, message }
 *   BNR_UNSUPPORTED_DEVICE  message, ""       UnsupportedDevice(message)
 *   BNR_QUANTIZATION_ERROR  message, ""       QuantizationError(message)
 * Display of the variant built from them equals bnr_last_error().  The
 * strings belong to the calling thread and stay valid until its next call
 * into the library. */
int bnr_last_error_parts(const char **first, const char **second);

/* ABI version of this header: (major << 16) | minor. */
uint32_t bnr_abi_version(void);

/* Create a backend bound to HIP device `device_id`; replaces
 * CudaBackend::new(device_id) (bitnet-gpu-cuda/src/lib.rs:94-104).  Fails
 * with BNR_UNSUPPORTED_DEVICE when the device does not exist or is not a
 * gfx950 GPU. */
int bnr_create(int device_id, bnr_ctx **out);
/* Release every device buffer the context owns (mirrors, tables, workspace). */
void bnr_destroy(bnr_ctx *ctx);
/* Backend::device_name (bitnet-core/src/backend/mod.rs:511-516). */
const char *bnr_device_name(const bnr_ctx *ctx);

/* ----------------------------------------------------------------------- */
/* Trait-shaped host entry points                                          */
/* ----------------------------------------------------------------------- */

/* Backend::rope_embed (bitnet-core/src/backend/mod.rs:251-260) as
 * CpuBackend implements it (bitnet-cpu/src/lib.rs:289-314): q
 * [n_heads*head_dim] and k [n_kv_heads*head_dim] are rotated in place at
 * `position` with the half-split pairing (i, i+head_dim/2).  The cos/sin
 * table is built on the host with the reference formula and kept in HBM;
 * it is rebuilt when head_dim changes, |theta - cached| > 1e-3 or
 * position >= its length (new length max(position+1, 4096), at least twice
 * the old one when only the position ran past it; the entries are the same
 * either way).  Errors:
 * zero/odd head_dim or non-positive/non-finite theta -> INVALID_CONFIG;
 * wrong q or k length -> INVALID_SHAPE. */
int bnr_rope_embed(bnr_ctx *ctx, float *q, size_t q_len, float *k, size_t k_len,
                   size_t position, size_t head_dim, size_t n_heads, size_t n_kv_heads,
                   float theta);

/* Backend::masked_attention (bitnet-core/src/backend/mod.rs:301-311) as
 * attention::masked_attention implements it (bitnet-cpu/src/attention.rs:
 * 97-209): out[h] = softmax(q_h . K[h/G, 0..=cur_pos] / sqrt(d)) V[h/G].
 * cap is k_len / n_kv_heads / head_dim, as in the reference (attention.rs:
 * 128).  The context keeps an HBM mirror of each host cache, keyed by
 * (k_cache, v_cache, k_len): when the mirror holds exactly rows
 * 0..cur_pos-1, and rows 0, (cur_pos-1)/2 and cur_pos-1 still begin and end
 * with the floats they held when the mirror was synced (4 of each k and v
 * row of every kv head are compared), only row cur_pos is uploaded;
 * otherwise rows 0..=cur_pos are re-uploaded.  Validation order and error
 * kinds follow attention.rs:109-161. */
int bnr_masked_attention(bnr_ctx *ctx, const float *q, size_t q_len, const float *k_cache,
                         size_t k_len, const float *v_cache, size_t v_len, float *output,
                         size_t out_len, size_t n_heads, size_t n_kv_heads,
                         size_t head_dim, size_t cur_pos);

/* Mirror policy of bnr_masked_attention. */
#define BNR_MIRROR_INCREMENTAL 0 /* upload only the new row when in sync (default) */
#define BNR_MIRROR_FULL 1        /* upload rows 0..=cur_pos on every call          */
int bnr_set_mirror_mode(bnr_ctx *ctx, int mode);
/* Forget every mirror (call after rewriting cached rows in place: the
 * samples above catch rewrites of the three sampled rows only). */
int bnr_mirror_invalidate(bnr_ctx *ctx);

/* Run-to-run reproducible decode, no counterpart in the reference (whose CPU
 * path sums each head in a fixed order, bitnet-cpu/src/attention.rs:
 * 170-206).  on != 0: later decode launches of this context (host-slice and
 * device entry points, single and batched) merge their context splits in a
 * fixed order, so the same inputs give the same output bits on every run;
 * on == 0 (the default): splits add into the merge state with float
 * atomics, faster, and the last bits of an output can differ between runs.
 * Measured at 4096 rows on MI355X: 11.4 against 8.6 us per step. */
int bnr_set_deterministic(bnr_ctx *ctx, int on);

/* Backend::ternary_gemv_preq (bitnet-core/src/backend/mod.rs:445-468), as
 * CpuBackend implements it (bitnet-cpu/src/lib.rs:519-538 ->
 * gemv::ternary_gemv_quantised, bitnet-cpu/src/gemv.rs:251-310):
 *   output[i] = (float)(sum_j W[i][j] * activation_q[j])
 *               * (weight_scale * act_absmax / 127)
 * with W packed 2 bits per weight, row-aligned (ceil(in_features/4) bytes
 * per row; 0b00 -> +1, 0b01 -> 0, 0b10 -> -1, 0b11 -> 0).  The integer sum
 * is exact, so outputs are bit-identical to the reference's.  Validation
 * order and messages follow gemv.rs:260-295 (InvalidShape for lengths,
 * QuantizationError for scales).  The weight matrix is mirrored in HBM on
 * first use, keyed by (weight_packed, weight_len) and a 64-byte sample of
 * its contents: model weights are immutable once loaded.  After rewriting a
 * matrix in place, call bnr_mirror_invalidate (which drops these mirrors). */
int bnr_ternary_gemv_preq(bnr_ctx *ctx, const uint8_t *weight_packed, size_t weight_len,
                          float weight_scale, const int8_t *activation_q, size_t act_len,
                          float act_absmax, float *output, size_t out_len,
                          size_t out_features, size_t in_features);

/* ----------------------------------------------------------------------- */
/* Device entry points (HBM-resident cache, stream-ordered)                */
/* ----------------------------------------------------------------------- */

/* RoPE + KV append for n_tokens consecutive tokens at positions
 * start_pos .. start_pos+n_tokens-1 of one sequence: the per-token
 * rope_embed + KVCache::store_kv pair of BitNetModel::forward
 * (bitnet-model/src/lib.rs:684-699).  q [n_tokens x n_heads x d] and k
 * [n_tokens x n_kv_heads x d] are rotated in place; rotated k rows and v
 * rows are written into k_cache / v_cache rows.  Requires
 * start_pos + n_tokens <= cap.  The rotation is bit-identical to the
 * reference's (same table, unfused products). */
int bnr_dev_rope_append(bnr_ctx *ctx, float *q, float *k, const float *v, size_t n_tokens,
                        size_t start_pos, size_t n_heads, size_t n_kv_heads,
                        size_t head_dim, float theta, float *k_cache, float *v_cache,
                        size_t cap, void *stream);

/* Decode attention of one token over cache rows 0..=cur_pos (q already
 * rotated): the masked_attention call of forward_into's decode path
 * (bitnet-model/src/lib.rs:1022-1036).  out [n_heads x d]. */
int bnr_dev_decode_attention(bnr_ctx *ctx, const float *q, const float *k_cache,
                             const float *v_cache, size_t cap, float *out, size_t n_heads,
                             size_t n_kv_heads, size_t head_dim, size_t cur_pos,
                             void *stream);

/* bnr_dev_decode_attention that allocates nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * split-K merge state lives in a device array of the library (about 4.15
 * MiB, one copy per GPU, set up by bnr_create); calls never allocate, free
 * or synchronise.  Limits: head_dim 128, n_heads / n_kv_heads in {1, 2, 4},
 * n_heads <= 32, 16-byte aligned pointers; anything else is
 * BNR_INVALID_CONFIG / BNR_INVALID_SHAPE.  Every call on a GPU shares that
 * GPU's array, so the array serves one (context, stream) pair at a time:
 * the first call claims it, calls from another context or on another
 * stream fail with BNR_BACKEND_ERROR until the claiming context is
 * destroyed.  Calls of the owning pair from several host threads must
 * still be serialised by the caller (they share the array too). */
int bnr_dev_decode_attention_noalloc(bnr_ctx *ctx, const float *q, const float *k_cache,
                                     const float *v_cache, size_t cap, float *out,
                                     size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                     size_t cur_pos, void *stream);

/* One fused decode step of one layer, in a single kernel launch: rotate q
 * (raw, [n_heads x d]) and k (raw, [n_kv_heads x d]) at `position`, append
 * the rotated k row and the v row at `position`, and attend over rows
 * 0..=position.  q and k are not modified; if q_rot / k_rot are non-NULL
 * the rotated vectors are written there (what rope_embed leaves in its
 * in-place buffers).  Equivalent to rope_embed + store_kv + masked_attention
 * (bitnet-model/src/lib.rs:1004-1036). */
int bnr_dev_decode_step(bnr_ctx *ctx, const float *q, const float *k, const float *v,
                        size_t position, size_t n_heads, size_t n_kv_heads,
                        size_t head_dim, float theta, float *k_cache, float *v_cache,
                        size_t cap, float *out, float *q_rot, float *k_rot, void *stream);

/* Fused decode step for a batch of independent sequences with ragged
 * lengths (no reference counterpart: the reference is single-sequence,
 * bitnet-core/src/backend/mod.rs:301-311 applied per sequence).
 * q [batch x n_heads x d], k/v [batch x n_kv_heads x d] raw projections;
 * positions (HOST array, batch entries) gives each sequence's new-token
 * position; caches are [batch x n_kv_heads x cap x d]; out
 * [batch x n_heads x d]. */
int bnr_dev_decode_step_batched(bnr_ctx *ctx, const float *q, const float *k,
                                const float *v, const int32_t *positions, size_t batch,
                                size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                float theta, float *k_caches, float *v_caches, size_t cap,
                                float *out, void *stream);

/* Causal prefill attention for n_tokens queries at positions
 * start_pos .. start_pos+n_tokens-1 (q already rotated,
 * [n_tokens x n_heads x d]); query i attends to cache rows
 * 0..=start_pos+i, which must already hold the rotated keys.  Equivalent to
 * n_tokens masked_attention calls in BitNetModel::forward's token loop
 * (bitnet-model/src/lib.rs:702-718).  out [n_tokens x n_heads x d]. */
int bnr_dev_prefill_attention(bnr_ctx *ctx, const float *q, const float *k_cache,
                              const float *v_cache, size_t cap, float *out,
                              size_t n_tokens, size_t start_pos, size_t n_heads,
                              size_t n_kv_heads, size_t head_dim, void *stream);

/* Full causal prefill of one layer: bnr_dev_rope_append followed by
 * bnr_dev_prefill_attention (q and k are rotated in place). */
int bnr_dev_prefill(bnr_ctx *ctx, float *q, float *k, const float *v, size_t n_tokens,
                    size_t start_pos, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                    float theta, float *k_cache, float *v_cache, size_t cap, float *out,
                    void *stream);

/* ternary_gemv_preq on device pointers: weight_packed
 * [out_features x ceil(in_features/4)] bytes, activation_q [in_features],
 * output [out_features].  Same arithmetic and scale checks as
 * bnr_ternary_gemv_preq. */
int bnr_dev_ternary_gemv_preq(bnr_ctx *ctx, const uint8_t *weight_packed, float weight_scale,
                              const int8_t *activation_q, float act_absmax, float *output,
                              size_t out_features, size_t in_features, void *stream);

/* Several ternary_gemv_preq calls that share one activation vector, in one
 * launch: the q/k/v projections of BitNetModel::forward
 * (bitnet-model/src/lib.rs:645-680) or gate/up (lib.rs:762-786).  Matrix i
 * is weight_packed[i] [out_features[i] x ceil(in_features/4)] with scale
 * weight_scales[i], written to outputs[i]; 1 <= n <= 8; the three arrays
 * are host memory, the pointers in them device memory.  Results equal n
 * separate bnr_dev_ternary_gemv_preq calls. */
int bnr_dev_ternary_gemv_preq_group(bnr_ctx *ctx, size_t n, const uint8_t *const *weight_packed,
                                    const float *weight_scales, const int8_t *activation_q,
                                    float act_absmax, float *const *outputs,
                                    const size_t *out_features, size_t in_features,
                                    void *stream);

/* Backend::lm_head_matmul_i8_into (bitnet-core/src/backend/mod.rs:470-509)
 * as CpuBackend implements it (bitnet-cpu/src/lib.rs:544-575):
 *   output[v] = (sum_h weights_i8[v*hidden_size + h] * hidden[h]) * scales[v]
 * in fp32 (products and sums in an order of this library's choosing: the
 * results agree with the reference's to rounding, not bit for bit).  Host
 * slices, synchronous; weights and scales are mirrored in HBM as for
 * bnr_ternary_gemv_preq.  Length mismatches (debug assertions in the
 * reference) are InvalidShape. */
int bnr_lm_head_matmul_i8_into(bnr_ctx *ctx, const float *hidden, size_t hidden_len,
                               const int8_t *weights_i8, size_t weights_len, const float *scales,
                               size_t scales_len, float *output, size_t out_len,
                               size_t vocab_size, size_t hidden_size);
/* The same on device pointers: hidden [hidden_size], weights_i8
 * [vocab_size x hidden_size], scales and output [vocab_size]. */
int bnr_dev_lm_head_matmul_i8(bnr_ctx *ctx, const float *hidden, const int8_t *weights_i8,
                              const float *scales, float *output, size_t vocab_size,
                              size_t hidden_size, void *stream);

/* bnr_dev_ternary_gemv_preq_group with the activation scale act_absmax read
 * from device memory (one float, as written by bnr_dev_norm_quant), so that
 * a decode layer runs without a host round trip. */
int bnr_dev_ternary_gemv_preq_group_devscale(bnr_ctx *ctx, size_t n,
                                             const uint8_t *const *weight_packed,
                                             const float *weight_scales,
                                             const int8_t *activation_q, const float *act_absmax,
                                             float *const *outputs, const size_t *out_features,
                                             size_t in_features, void *stream);

/* ---- Layer glue ----------------------------------------------------------- */

/* Backend::rms_norm (bitnet-core/src/backend/mod.rs) as CpuBackend implements
 * it (bitnet-cpu/src/lib.rs:268-270 -> norm::rms_norm, norm.rs:76-136):
 * out[i] = x[i] * (1/sqrt(sum(x^2)/n + eps)) * weight[i].  The sum of squares
 * is reduced as a tree, so outputs agree with the reference's to rounding.
 * Host slices, synchronous; the weight is mirrored in HBM.  Checks and
 * messages as norm.rs:77-97 (InvalidShape, QuantizationError for eps). */
int bnr_rms_norm(bnr_ctx *ctx, const float *input, size_t in_len, const float *weight,
                 size_t w_len, float eps, float *output, size_t out_len);
/* Backend::sqrelu_gate as CpuBackend implements it (bitnet-cpu/src/lib.rs:
 * 494-509): out[i] = max(gate[i], 0)^2 * up[i], bit-identical.  Host slices. */
int bnr_sqrelu_gate(bnr_ctx *ctx, const float *gate, size_t g_len, const float *up,
                    size_t u_len, float *out, size_t out_len);
/* Device forms of the two (n elements each). */
int bnr_dev_rms_norm(bnr_ctx *ctx, const float *input, const float *weight, float eps,
                     float *output, size_t n, void *stream);
int bnr_dev_sqrelu_gate(bnr_ctx *ctx, const float *gate, const float *up, float *out, size_t n,
                        void *stream);
/* h[i] += delta[i]: the residual axpy_f32_fast(1.0, delta, h) of
 * BitNetModel::forward (bitnet-model/src/lib.rs:1061,1130), bit-identical. */
int bnr_dev_residual_add(bnr_ctx *ctx, float *h, const float *delta, size_t n, void *stream);
/* absmax_quantize_row_into (bitnet-core/src/quant/absmax.rs:127-170) on
 * device: q_out [n] int8 and *scale_out (device) = max(max|x|, 1e-5) / 127,
 * bit-identical.  Finite inputs are assumed (the reference's non-finite
 * check is not repeated on the device). */
int bnr_dev_absmax_quantize(bnr_ctx *ctx, const float *x, int8_t *q_out, float *scale_out,
                            size_t n, void *stream);

/* One launch between two projections of a decode layer: form x, RMSNorm it
 * with gamma, quantise the result (absmax int8) for the next ternary GEMV.
 *   BNR_GLUE_PLAIN    x = a                                   (attention and
 *                     sub-norms, bitnet-model/src/lib.rs:628-642, 720-730)
 *   BNR_GLUE_RESIDUAL x = a + b, written to h_out (may be a)  (residual then
 *                     ffn_norm, lib.rs:743-759)
 *   BNR_GLUE_SQRELU   x = max(a,0)^2 * b                      (sqrelu_gate then
 *                     ffn_sub_norm, lib.rs:788-800)
 * q_out [n] int8; *act_absmax (device) = (max|y| / 127) * 127, the value the
 * model passes to ternary_gemv_preq (lib.rs:642). */
#define BNR_GLUE_PLAIN 0
#define BNR_GLUE_RESIDUAL 1
#define BNR_GLUE_SQRELU 2
int bnr_dev_norm_quant(bnr_ctx *ctx, int mode, const float *a, const float *b, const float *gamma,
                       float eps, size_t n, float *h_out, int8_t *q_out, float *act_absmax,
                       void *stream);

/* The glue launch folded into the projection: bnr_dev_norm_quant's x (mode,
 * a, b), RMSNorm with gamma and int8 quantisation computed by every
 * workgroup of the grouped ternary GEMV as its prologue, the int8
 * activations kept in LDS.  One launch instead of two between the layer's
 * norms and projections.  in_features <= 8192; mode BNR_GLUE_RESIDUAL
 * writes a + b to h_out, which must not alias a or b (double-buffer the
 * residual stream).  Outputs agree with norm_quant followed by the
 * devscale GEMV to the rounding of the sum of squares. */
int bnr_dev_ternary_gemv_norm_group(bnr_ctx *ctx, size_t n, const uint8_t *const *weight_packed,
                                    const float *weight_scales, int mode, const float *a,
                                    const float *b, const float *gamma, float eps, float *h_out,
                                    float *const *outputs, const size_t *out_features,
                                    size_t in_features, void *stream);

/* Wait for all work the context enqueued on `stream`. */
int bnr_dev_synchronize(bnr_ctx *ctx, void *stream);

/* ---- Backend-owned KV cache ----------------------------------------------
 * KVCache (bitnet-model/src/lib.rs:118-315) with its buffers in HBM: per
 * layer a K and a V cache, each head-major [n_kv_heads x max_seq x head_dim]
 * fp32, plus the reference's bookkeeping (layer_lengths, filled_positions).
 * Rows are written only by the decode / prefill calls below, which apply
 * store_kv's position rules (lib.rs:204-216): a row either overwrites a
 * stored one or extends its layer by one; position >= max_seq and gaps are
 * BNR_INVALID_SHAPE with the reference's messages.  Calls on one cache are
 * serialised by the cache. */
typedef struct bnr_kv_cache bnr_kv_cache;

/* KVCache::new (lib.rs:148-169): zero-filled caches on the context's device. */
int bnr_kv_cache_create(bnr_ctx *ctx, size_t n_layers, size_t n_kv_heads, size_t head_dim,
                        size_t max_seq, bnr_kv_cache **out);
/* Free the cache's HBM (waits for work in flight on the device). */
void bnr_kv_cache_destroy(bnr_kv_cache *cache);
/* KVCache::clear (lib.rs:285-292): zero every layer, reset lengths and
 * filled_positions.  Waits for all work on the device first. */
int bnr_kv_cache_clear(bnr_kv_cache *cache);
/* KVCache::advance (lib.rs:244-252) by n positions.  Where the reference
 * panics (advancing past max_seq) this returns BNR_BACKEND_ERROR with the
 * panic's message and advances nothing. */
int bnr_kv_cache_advance(bnr_kv_cache *cache, size_t n);
/* KVCache::len (filled_positions, lib.rs:294-298). */
size_t bnr_kv_cache_len(const bnr_kv_cache *cache);
/* Positions stored in `layer` (layer_lengths[layer]). */
int bnr_kv_cache_layer_len(bnr_kv_cache *cache, size_t layer, size_t *len);
/* Device addresses of layer's K and V caches, for the bnr_dev_* calls with
 * cap = max_seq (the k_slice / v_slice backing buffers, lib.rs:262-280). */
int bnr_kv_cache_layer(bnr_kv_cache *cache, size_t layer, float **k, float **v);

/* One token of one layer from host slices: the per-layer sequence of
 * BitNetModel::forward_into (lib.rs:1004-1036) -- rope_embed(q, k,
 * position), store_kv(layer, position, k, v), masked_attention(q, layer's
 * caches, output, cur_pos = position) -- as one kernel launch.  q
 * [n_heads*head_dim] and k [n_kv_heads*head_dim] are rotated in place as
 * rope_embed does; v [n_kv_heads*head_dim]; output [n_heads*head_dim].
 * Validation in the reference's order (rope, store_kv, attention).
 * Synchronous. */
int bnr_kv_decode(bnr_ctx *ctx, bnr_kv_cache *cache, size_t layer, float *q, size_t q_len,
                  float *k, size_t k_len, const float *v, size_t v_len, size_t position,
                  size_t n_heads, float theta, float *output, size_t out_len);
/* bnr_kv_decode on device pointers (q, k, v are read, not rotated in
 * place), ordered on `stream`: bnr_dev_decode_step on the layer's caches. */
int bnr_kv_dev_decode(bnr_ctx *ctx, bnr_kv_cache *cache, size_t layer, const float *q,
                      const float *k, const float *v, size_t position, size_t n_heads,
                      float theta, float *out, void *stream);
/* bnr_dev_prefill on the layer's caches: n_tokens rows from start_pos
 * (store_kv's rules for each row in order); q and k rotated in place. */
int bnr_kv_dev_prefill(bnr_ctx *ctx, bnr_kv_cache *cache, size_t layer, float *q, float *k,
                       const float *v, size_t n_tokens, size_t start_pos, size_t n_heads,
                       float theta, float *out, void *stream);

/* ---- Measurement ---------------------------------------------------------
 * A plain streaming read of two device ranges (a_bytes at a, b_bytes at b;
 * 16-byte aligned, multiples of 16), ordered on `stream`: no counterpart in
 * the reference.  The benchmark times it on the K and V caches a decode step
 * reads, as the floor a single launch of that many bytes can reach. */
int bnr_dev_stream_read(bnr_ctx *ctx, const void *a, size_t a_bytes, const void *b,
                        size_t b_bytes, void *stream);
/* The same read in a chosen shape, no counterpart in the reference:
 * workgroups of `threads` (a multiple of 64 up to 1024), each lane issuing
 * `loads_per_lane` (1, 2, 4, 8 or 16) 16-byte loads before using any, so
 * that many are in flight per lane; non-temporal loads when nontemporal != 0.
 * The benchmark takes the fastest shape as the streaming floor. */
int bnr_dev_stream_read_shape(bnr_ctx *ctx, const void *a, size_t a_bytes, const void *b,
                              size_t b_bytes, int threads, int loads_per_lane, int nontemporal,
                              void *stream);

#ifdef __cplusplus
}
#endif
#endif /* BITNET_HIP_H */
