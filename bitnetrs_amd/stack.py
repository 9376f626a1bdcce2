"""Attention part of BitNetModel's layer loop on HBM-resident caches.

BitNetModel::forward (bitnet-model/src/lib.rs:559-862, hot calls 684-718)
runs, per layer and per token, rope_embed -> store_kv -> masked_attention;
forward_into's decode path (lib.rs:931-1036) does the same for one token.
``AttentionStack`` keeps one HBM cache per layer (``DeviceKVCache``) and
issues the fused device calls: one ``bnr_dev_prefill`` per layer for a
prompt, one ``bnr_dev_decode_step`` per layer for each generated token.
"""
from __future__ import annotations

from .backend import DeviceKVCache, HipBackend


class AttentionStack:
    def __init__(self, backend: HipBackend, n_layers: int, n_heads: int, n_kv_heads: int,
                 head_dim: int, max_seq: int, theta: float):
        self.be = backend
        self.n_layers, self.n_heads, self.n_kv, self.d = n_layers, n_heads, n_kv_heads, head_dim
        self.theta = theta
        self.cache = DeviceKVCache(n_layers, n_kv_heads, head_dim, max_seq)

    @property
    def position(self) -> int:
        return self.cache.filled_positions

    def prefill(self, q, k, v, out, stream=None) -> None:
        """q [L][n][Hq*d], k/v [L][n][Hkv*d] (raw projections, q/k rotated in
        place), out [L][n][Hq*d]; tokens at positions position..position+n-1."""
        n, start = q.shape[1], self.position
        for layer in range(self.n_layers):
            self.cache.check_store(layer, start, n)
            self.be.dev_prefill(q[layer], k[layer], v[layer], n, start, self.n_heads, self.n_kv,
                                self.d, self.theta, self.cache.k[layer], self.cache.v[layer],
                                self.cache.max_seq, out[layer], stream=stream)
            self.cache.mark_stored(layer, start, n)
        self.cache.advance(n)

    def decode(self, q, k, v, out, stream=None) -> None:
        """One token: q [L][Hq*d], k/v [L][Hkv*d] raw, out [L][Hq*d]."""
        pos = self.position
        for layer in range(self.n_layers):
            self.cache.check_store(layer, pos, 1)
            self.be.dev_decode_step(q[layer], k[layer], v[layer], pos, self.n_heads, self.n_kv,
                                    self.d, self.theta, self.cache.k[layer], self.cache.v[layer],
                                    self.cache.max_seq, out[layer], stream=stream)
            self.cache.mark_stored(layer, pos, 1)
        self.cache.advance(1)
