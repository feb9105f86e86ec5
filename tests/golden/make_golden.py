"""Writes the golden fixtures of this directory from the numpy oracle.

    python tests/golden/make_golden.py

Fixtures (all derived from seeded inputs; re-running reproduces them):
  rotation_d128_s42.npy      R for head_dim 128, seed 42 (float32, 64 KiB)
  golden.json                sha256 digests: R, QJL projection, config-1 codes/norms,
                             small known-answer vectors
  config1_slice.npz          config-1 (K4/V2, sink 128, window 128) codes / norms of
                             kv heads 0-1, first 32 drained tokens, plus the
                             near-boundary mask of those coordinates
  attn_small.npz             a small mixed-segment decode attention case: query and
                             float64 output (keys/values regenerate from the seed in
                             attn_small_case())

The reference's own numeric data (the shipped codebooks) is checked directly
in tests/test_oracle.py against the values fixed by its .npz files.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config1_inputs():
    rng = np.random.RandomState(0)
    k = rng.randn(1, 8, 1024, 128).astype(np.float16)
    v = rng.randn(1, 8, 1024, 128).astype(np.float16)
    return k, v


def config1_cache():
    k, v = config1_inputs()
    c = O.CacheOracle(head_dim=128, num_kv_heads=8, key_bits=4, value_bits=2,
                      residual_window=128, fp16_sink_size=128)
    c.update(k, v)
    return c


def attn_small_case():
    rng = np.random.RandomState(7)
    B, Hkv, G, D = 1, 2, 4, 128
    c = O.CacheOracle(head_dim=D, num_kv_heads=Hkv, key_bits=4, value_bits=2,
                      residual_window=32, fp16_sink_size=16)
    scale = np.exp(rng.randn(D) * 0.5)
    k = (rng.randn(B, Hkv, 300, D) * scale).astype(np.float16)
    v = rng.randn(B, Hkv, 300, D).astype(np.float16)
    c.update(k, v)
    q = rng.randn(B, Hkv * G, 1, D).astype(np.float16)
    return k, v, q, c.attend(q)


def main():
    out = {}
    R = O.rotation_matrix(128, 42)
    np.save(os.path.join(HERE, "rotation_d128_s42.npy"), R)
    out["rotation_d128_s42"] = sha(R)
    out["projection_d128_m128_s12345"] = sha(O.projection_matrix(128, 128))
    out["projection_d128_m32_s12345"] = sha(O.projection_matrix(128, 32))

    c = config1_cache()
    assert c.drains == [768] and c.compressed_len == 768 and c.fp16_len == 128 and c.sink_len == 128
    kh, _, kn = c.packed("k")
    vh, _, vn = c.packed("v")
    out["config1"] = {"k_codes": sha(kh), "k_norms": sha(kn), "v_codes": sha(vh), "v_norms": sha(vn),
                      "k_near": int(c.comp["k"][0].near.sum()), "v_near": int(c.comp["v"][0].near.sum())}
    np.savez_compressed(os.path.join(HERE, "config1_slice.npz"),
                        k_codes=kh[:, :2, :32], k_norms=kn[:, :2, :32], v_codes=vh[:, :2, :32],
                        v_norms=vn[:, :2, :32], k_near=c.comp["k"][0].near[:, :2, :32],
                        v_near=c.comp["v"][0].near[:, :2, :32])

    k, v, q, o = attn_small_case()
    np.savez_compressed(os.path.join(HERE, "attn_small.npz"), q=q, out=o)
    out["attn_small_out"] = sha(o)

    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
