"""One decode token of the whole BitNet b1.58 layer stack on the device.

BitNetModel::forward_into's decode path (bitnet-model/src/lib.rs:931-1163)
runs, per layer: RMSNorm + int8 quantisation, the q/k/v ternary GEMVs,
RoPE + KV append + attention, attention sub-norm + quantisation, the o
projection, residual, FFN norm + quantisation, gate/up, squared-ReLU gate +
sub-norm + quantisation, the down projection and the residual; then the
final norm and the i8 LM head.  ``DecodeModel`` keeps weights, KV caches and
activations in HBM.  With ``fused=True`` (the default) a layer is five
launches of this library, each projection computing the RMSNorm and int8
quantisation of its input as its own prologue:

  q/k/v GEMV (attention norm; after the first layer it also adds the
  previous layer's FFN output to the residual stream) -> fused decode step
  -> o GEMV (attention sub-norm) -> gate/up GEMV (residual + FFN norm) ->
  down GEMV (sqrelu gate + FFN sub-norm)

With ``fused=False`` each glue step is its own launch (``bnr_dev_norm_quant``)
and the projection reads the int8 vector and its scale from device memory:
nine launches per layer.  After the last layer: residual, final RMSNorm,
LM head.  A token needs no host round trip and can be captured in one HIP
graph.  Weights are the caller's packed device tensors.
"""
from __future__ import annotations

from dataclasses import dataclass

from ._lib import BNR_GLUE_PLAIN, BNR_GLUE_RESIDUAL, BNR_GLUE_SQRELU
from .backend import DeviceKVCache, HipBackend


@dataclass
class LayerWeights:
    """Packed ternary projections (uint8 device tensors, ceil(in/4) bytes
    per row) with their absmean scales, and the four RMSNorm weights."""
    q: object
    k: object
    v: object
    o: object
    gate: object
    up: object
    down: object
    scales: tuple  # (q, k, v, o, gate, up, down) weight scales
    attention_norm: object
    attn_sub_norm: object
    ffn_norm: object
    ffn_sub_norm: object


@dataclass
class ModelShape:
    hidden: int = 2560
    n_heads: int = 20
    n_kv_heads: int = 5
    head_dim: int = 128
    ffn: int = 6912
    n_layers: int = 30
    vocab: int = 128256
    theta: float = 500000.0
    eps: float = 1e-5


class DecodeModel:
    def __init__(self, backend: HipBackend, shape: ModelShape, layers, final_norm, lm_head_i8,
                 lm_head_scales, max_seq: int, fused: bool = True):
        import torch

        self.be, self.s, self.fused = backend, shape, fused
        self.layers = list(layers)
        assert len(self.layers) == shape.n_layers
        self.final_norm, self.lm_w, self.lm_scales = final_norm, lm_head_i8, lm_head_scales
        self.cache = DeviceKVCache(shape.n_layers, shape.n_kv_heads, shape.head_dim, max_seq)
        s = shape
        dev = lambda n: torch.zeros(n, device="cuda")  # noqa: E731
        self.q_dim, self.kv_dim = s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim
        self.qb, self.kb, self.vb = dev(self.q_dim), dev(self.kv_dim), dev(self.kv_dim)
        self.attn = dev(self.q_dim)
        self.o_out, self.ffn_out = dev(s.hidden), dev(s.hidden)
        self.gate, self.up = dev(s.ffn), dev(s.ffn)
        self.final_normed = dev(s.hidden)
        self.q8 = torch.zeros(max(s.hidden, s.ffn, self.q_dim), dtype=torch.int8, device="cuda")
        self.act_absmax = dev(1)
        self.hbuf = [dev(s.hidden), dev(s.hidden)]  # residual stream, double-buffered

    @property
    def position(self) -> int:
        return self.cache.filled_positions

    def step(self, h, logits, position: int = None, stream=None) -> None:
        """One token: h [hidden] (the embedding; updated in place to the
        residual stream after the last layer), logits [vocab]."""
        pos = self.position if position is None else position
        if self.fused:
            self._step_fused(h, logits, pos, stream)
        else:
            self._step_glue(h, logits, pos, stream)
        if position is None:
            self.cache.advance(1)

    def _step_fused(self, h, logits, pos, stream) -> None:
        be, s = self.be, self.s
        cur, nxt = h, self.hbuf[0]
        for li, w in enumerate(self.layers):
            self.cache.check_store(li, pos, 1)
            if li == 0:
                be.dev_ternary_gemv_norm_group(
                    [w.q, w.k, w.v], w.scales[0:3], BNR_GLUE_PLAIN, cur, None, w.attention_norm,
                    s.eps, None, [self.qb, self.kb, self.vb],
                    [self.q_dim, self.kv_dim, self.kv_dim], s.hidden, stream=stream)
            else:  # previous layer's FFN output joins the residual stream first
                be.dev_ternary_gemv_norm_group(
                    [w.q, w.k, w.v], w.scales[0:3], BNR_GLUE_RESIDUAL, cur, self.ffn_out,
                    w.attention_norm, s.eps, nxt, [self.qb, self.kb, self.vb],
                    [self.q_dim, self.kv_dim, self.kv_dim], s.hidden, stream=stream)
                cur, nxt = nxt, self._other(nxt)
            be.dev_decode_step(self.qb, self.kb, self.vb, pos, s.n_heads, s.n_kv_heads,
                               s.head_dim, s.theta, self.cache.k[li], self.cache.v[li],
                               self.cache.max_seq, self.attn, stream=stream)
            self.cache.mark_stored(li, pos, 1)
            be.dev_ternary_gemv_norm_group(
                [w.o], w.scales[3:4], BNR_GLUE_PLAIN, self.attn, None, w.attn_sub_norm, s.eps,
                None, [self.o_out], [s.hidden], self.q_dim, stream=stream)
            be.dev_ternary_gemv_norm_group(
                [w.gate, w.up], w.scales[4:6], BNR_GLUE_RESIDUAL, cur, self.o_out, w.ffn_norm,
                s.eps, nxt, [self.gate, self.up], [s.ffn, s.ffn], s.hidden, stream=stream)
            cur, nxt = nxt, self._other(nxt)
            be.dev_ternary_gemv_norm_group(
                [w.down], w.scales[6:7], BNR_GLUE_SQRELU, self.gate, self.up, w.ffn_sub_norm,
                s.eps, None, [self.ffn_out], [s.hidden], s.ffn, stream=stream)
        if cur is not h:
            h.copy_(cur)
        be.dev_residual_add(h, self.ffn_out, s.hidden, stream=stream)
        be.dev_rms_norm(h, self.final_norm, s.eps, self.final_normed, s.hidden, stream=stream)
        be.dev_lm_head_matmul_i8(self.final_normed, self.lm_w, self.lm_scales, logits, s.vocab,
                                 s.hidden, stream=stream)

    def _other(self, buf):
        return self.hbuf[1] if buf is self.hbuf[0] else self.hbuf[0]

    def _step_glue(self, h, logits, pos, stream) -> None:
        be, s = self.be, self.s
        for li, w in enumerate(self.layers):
            self.cache.check_store(li, pos, 1)
            if li == 0:
                be.dev_norm_quant(BNR_GLUE_PLAIN, h, None, w.attention_norm, s.eps, s.hidden, None,
                                  self.q8, self.act_absmax, stream=stream)
            else:  # h += previous layer's FFN output, then the attention norm
                be.dev_norm_quant(BNR_GLUE_RESIDUAL, h, self.ffn_out, w.attention_norm, s.eps,
                                  s.hidden, h, self.q8, self.act_absmax, stream=stream)
            be.dev_ternary_gemv_preq_group_devscale(
                [w.q, w.k, w.v], w.scales[0:3], self.q8, self.act_absmax,
                [self.qb, self.kb, self.vb], [self.q_dim, self.kv_dim, self.kv_dim], s.hidden,
                stream=stream)
            be.dev_decode_step(self.qb, self.kb, self.vb, pos, s.n_heads, s.n_kv_heads,
                               s.head_dim, s.theta, self.cache.k[li], self.cache.v[li],
                               self.cache.max_seq, self.attn, stream=stream)
            self.cache.mark_stored(li, pos, 1)
            be.dev_norm_quant(BNR_GLUE_PLAIN, self.attn, None, w.attn_sub_norm, s.eps, self.q_dim,
                              None, self.q8, self.act_absmax, stream=stream)
            be.dev_ternary_gemv_preq_group_devscale(
                [w.o], w.scales[3:4], self.q8, self.act_absmax, [self.o_out], [s.hidden],
                self.q_dim, stream=stream)
            be.dev_norm_quant(BNR_GLUE_RESIDUAL, h, self.o_out, w.ffn_norm, s.eps, s.hidden, h,
                              self.q8, self.act_absmax, stream=stream)
            be.dev_ternary_gemv_preq_group_devscale(
                [w.gate, w.up], w.scales[4:6], self.q8, self.act_absmax, [self.gate, self.up],
                [s.ffn, s.ffn], s.hidden, stream=stream)
            be.dev_norm_quant(BNR_GLUE_SQRELU, self.gate, self.up, w.ffn_sub_norm, s.eps, s.ffn,
                              None, self.q8, self.act_absmax, stream=stream)
            be.dev_ternary_gemv_preq_group_devscale(
                [w.down], w.scales[6:7], self.q8, self.act_absmax, [self.ffn_out], [s.hidden],
                s.ffn, stream=stream)
        be.dev_residual_add(h, self.ffn_out, s.hidden, stream=stream)
        be.dev_rms_norm(h, self.final_norm, s.eps, self.final_normed, s.hidden, stream=stream)
        be.dev_lm_head_matmul_i8(self.final_normed, self.lm_w, self.lm_scales, logits, s.vocab,
                                 s.hidden, stream=stream)
