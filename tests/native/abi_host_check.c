// Drives the C ABI from plain C, with no Python or PyTorch in the process,
// the way an extern "C" block of a Rust backend crate would.  It runs the
// reference's per-token sequence rope_embed -> store_kv -> masked_attention
// (bitnet-model/src/lib.rs:1004-1036) on host slices for 48 tokens of the
// 2B shape (20/5 heads, head_dim 128, theta 500000).  The host caches have
// capacity 64 and are laid out as KVCache's layers (bitnet-model/src/lib.rs:
// 148-169).  The oracle's CpuBackend runs the same calls on its own copies.
// Checks:
//  - rotated q and k bit for bit;
//  - outputs within |gpu - ref| <= 2e-3 + 1e-3 |ref|;
//  - one error of each BitNetError kind the path returns: the variant
//    rebuilt from bnr_last_error_parts() with the reference's Display format
//    (bitnet-core/src/error.rs:17-55) prints bnr_last_error(), and where the
//    oracle has the same call, the oracle's status and message.
// Prints "ok <tokens> <max abs diff>" or the first failure.  Needs a GPU.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "bitnet_hip.h"
#include "bnr_oracle.h"

enum { HQ = 20, HKV = 5, D = 128, CAP = 64, N = 48 };

static int fail(const char *what, int pos) {
  printf("FAIL %s at position %d: %s\n", what, pos, bnr_last_error());
  return 1;
}

// Display of the variant a binding builds from bnr_last_error_parts(); 0 when
// it differs from bnr_last_error() or from want_text (if given), or the kind
// is not want_kind.
static int rebuilt_matches(int want_kind, const char *want_text) {
  const char *a = NULL, *b = NULL;
  const int kind = bnr_last_error_parts(&a, &b);
  char text[1024];
  switch (kind) {
    case BNR_INVALID_SHAPE: snprintf(text, sizeof text, "invalid tensor shape: expected %s, got %s", a, b); break;
    case BNR_INVALID_CONFIG: snprintf(text, sizeof text, "invalid model configuration: %s", a); break;
    case BNR_BACKEND_ERROR: snprintf(text, sizeof text, "backend error (%s): %s", a, b); break;
    case BNR_UNSUPPORTED_DEVICE: snprintf(text, sizeof text, "unsupported device: %s", a); break;
    case BNR_QUANTIZATION_ERROR: snprintf(text, sizeof text, "quantization error: %s", a); break;
    default: return 0;
  }
  if (kind != want_kind || strcmp(text, bnr_last_error()) != 0) return 0;
  if (kind != BNR_INVALID_SHAPE && kind != BNR_BACKEND_ERROR && b[0]) return 0;
  return !want_text || strcmp(text, want_text) == 0;
}

static void store_row(float *cache, const float *row, int pos) {
  for (int h = 0; h < HKV; ++h) memcpy(cache + (h * CAP + pos) * D, row + h * D, D * sizeof(float));
}

int main(void) {
  const float theta = 500000.0f;
  static float kc[HKV * CAP * D], vc[HKV * CAP * D], kc_ref[HKV * CAP * D], vc_ref[HKV * CAP * D];
  float q[HQ * D], k[HKV * D], v[HKV * D], qr[HQ * D], kr[HKV * D];
  float out[HQ * D], out_ref[HQ * D];
  bnr_ctx *ctx = NULL;
  if (bnr_create(0, &ctx) != BNR_OK) return fail("bnr_create", -1);
  bnro_backend *ref = bnro_backend_new();
  double max_abs = 0.0;
  for (int pos = 0; pos < N; ++pos) {
    const uint64_t s = 0xB17E7C00u + 4u * (uint64_t)pos;
    bnro_fill_normal(s, q, HQ * D, 1.0f);
    bnro_fill_normal(s + 1, k, HKV * D, 1.0f);
    bnro_fill_normal(s + 2, v, HKV * D, 1.0f);
    memcpy(qr, q, sizeof q);
    memcpy(kr, k, sizeof k);
    if (bnr_rope_embed(ctx, q, HQ * D, k, HKV * D, pos, D, HQ, HKV, theta) != BNR_OK)
      return fail("bnr_rope_embed", pos);
    if (bnro_backend_rope_embed(ref, qr, HQ * D, kr, HKV * D, pos, D, HQ, HKV, theta) != BNRO_OK)
      return fail("oracle rope_embed", pos);
    if (memcmp(q, qr, sizeof q) || memcmp(k, kr, sizeof k)) return fail("rotated q/k differ", pos);
    store_row(kc, k, pos);
    store_row(vc, v, pos);
    store_row(kc_ref, kr, pos);
    store_row(vc_ref, v, pos);
    if (bnr_masked_attention(ctx, q, HQ * D, kc, HKV * CAP * D, vc, HKV * CAP * D, out, HQ * D, HQ,
                             HKV, D, pos) != BNR_OK)
      return fail("bnr_masked_attention", pos);
    if (bnro_masked_attention(qr, HQ * D, kc_ref, HKV * CAP * D, vc_ref, HKV * CAP * D, out_ref,
                              HQ * D, HQ, HKV, D, pos) != BNRO_OK)
      return fail("oracle masked_attention", pos);
    for (int i = 0; i < HQ * D; ++i) {
      const double d = fabs((double)out[i] - (double)out_ref[i]);
      if (!(d <= 2e-3 + 1e-3 * fabs((double)out_ref[i]))) {
        printf("FAIL output %d at position %d: %.9g vs %.9g\n", i, pos, out[i], out_ref[i]);
        return 1;
      }
      if (d > max_abs) max_abs = d;
    }
  }
  // n_heads not a multiple of n_kv_heads; then a q slice one element short.
  int st = bnr_masked_attention(ctx, q, HQ * D, kc, HKV * CAP * D, vc, HKV * CAP * D, out, HQ * D,
                                HQ, 3, D, 0);
  int st_ref = bnro_masked_attention(qr, HQ * D, kc_ref, HKV * CAP * D, vc_ref, HKV * CAP * D,
                                     out_ref, HQ * D, HQ, 3, D, 0);
  if (st != BNR_INVALID_CONFIG || st != st_ref || !rebuilt_matches(st, bnro_last_error()))
    return fail("masked_attention error kind", -1);
  st = bnr_rope_embed(ctx, q, HQ * D - 1, k, HKV * D, 0, D, HQ, HKV, theta);
  st_ref = bnro_backend_rope_embed(ref, qr, HQ * D - 1, kr, HKV * D, 0, D, HQ, HKV, theta);
  if (st != BNR_INVALID_SHAPE || st != st_ref || !rebuilt_matches(st, bnro_last_error()))
    return fail("rope_embed error kind", -1);
  // QuantizationError: a zero weight scale (checked after the lengths).
  {
    uint8_t w[2] = {0, 0};
    int8_t act[8] = {0};
    float o[1];
    st = bnr_ternary_gemv_preq(ctx, w, 2, 0.0f, act, 8, 1.0f, o, 1, 1, 8);
    st_ref = bnro_ternary_gemv_preq(w, 2, 0.0f, act, 8, 1.0f, o, 1, 1, 8);
    if (st != BNR_QUANTIZATION_ERROR || st != st_ref || !rebuilt_matches(st, bnro_last_error()))
      return fail("ternary_gemv_preq error kind", -1);
  }
  // BackendError and UnsupportedDevice: the library's own (no oracle call).
  if (bnr_create(0, NULL) != BNR_BACKEND_ERROR ||
      !rebuilt_matches(BNR_BACKEND_ERROR, "backend error (HIP): bnr_create: out is NULL"))
    return fail("bnr_create(NULL) error kind", -1);
  {
    bnr_ctx *none = NULL;
    if (bnr_create(1 << 20, &none) != BNR_UNSUPPORTED_DEVICE || none ||
        !rebuilt_matches(BNR_UNSUPPORTED_DEVICE, NULL))
      return fail("bnr_create(missing device) error kind", -1);
  }
  bnro_backend_free(ref);
  bnr_destroy(ctx);
  printf("ok %d %.3g\n", N, max_abs);
  return 0;
}
