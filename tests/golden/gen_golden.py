"""Write the golden fixtures of this directory from the oracle.

    python tests/golden/gen_golden.py

Fixtures (numpy .npz, arrays only):
  decode_c1.npz   C1 decode step: pos 511, 20/5 heads, d=128, theta 5e5, seeded
                  inputs (SplitMix64 -> Box-Muller; seeds in the file), outputs of
                  rope_embed -> store_kv -> masked_attention.
  prefill_small.npz  16-token causal prefill, 4/2 heads, d=128, theta 5e5
                  (output in full; rotated q/k and the cache as SHA-256).
  rope_rows.npz   cos/sin table rows 0, 1, 511, 4095 for d=128, theta 5e5.
Inputs are regenerated from the seeds by the tests; a SHA-256 of each input
tensor is stored so that a generator change is reported as such.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from common import decode_workload, oracle_decode, oracle_prefill, prefill_workload, seed  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    w = decode_workload(1, 511)
    q_rot, k_rot, _, _, out = oracle_decode(w)
    np.savez(os.path.join(HERE, "decode_c1.npz"), pos=511, seeds=np.array([seed(1, i) for i in range(5)]),
             sha_q=sha(w["q"]), sha_k=sha(w["k"]), sha_v=sha(w["v"]),
             sha_kc=sha(w["k_cache"]), sha_vc=sha(w["v_cache"]), q_rot=q_rot, k_rot=k_rot, out=out)
    p = prefill_workload(36, 16, 4, 2)
    q_r, k_r, cache, o = oracle_prefill(p, cap=16, n_heads=4, n_kv=2)
    np.savez(os.path.join(HERE, "prefill_small.npz"), n_tokens=16, n_heads=4, n_kv=2, cap=16,
             sha_q=sha(p["q"]), sha_k=sha(p["k"]), sha_v=sha(p["v"]), sha_q_rot=sha(q_r),
             sha_k_rot=sha(k_r), sha_k_cache=sha(cache.k(0)), sha_v_cache=sha(cache.v(0)), out=o)
    c, s = oracle.rope_table(4096, 128, 500000.0)
    rows = np.array([0, 1, 511, 4095])
    np.savez(os.path.join(HERE, "rope_rows.npz"), rows=rows, cos=c[rows], sin=s[rows])
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
