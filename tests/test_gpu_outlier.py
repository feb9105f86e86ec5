"""Qwen3-8B-shaped outlier stress (36 layers, H_q = 32,
H_kv = 8, D = 128, 65536-token context, K4/V2, fp16_sink_size = 128).

Keys are N(0,1) except in 6 seeded layers, where 4 seeded channels are
scaled x25. apply_turboquant's outlier rule (patch.py:89-133: max key norm of
a 5-token probe > 3 x the median over layers) must keep exactly those layers
uncompressed; decode attention then runs over the mixed fp16 / packed layer
set. Packed layers are checked against the general kernel (all 30) and
against float64 attention over the oracle-dequantised stored codes (one
layer).
"""

import types

import numpy as np
import pytest
import torch

import oracle as O
from gpu_helpers import min_cos, rel_err

pytestmark = pytest.mark.gpu

LAYERS, HQ, HKV, D, T = 36, 32, 8, 128, 65536
SINK, WINDOW = 128, 128


class OutlierModel:
    """Stand-in for the model: a Hugging Face style config and the probe hook
    apply_turboquant uses for outlier detection (one (B, H, T, D) key tensor
    per layer)."""

    def __init__(self, seed):
        rng = np.random.RandomState(seed)
        self.outliers = sorted(rng.choice(LAYERS, 6, replace=False).tolist())
        self.channels = {l: rng.choice(D, 4, replace=False) for l in self.outliers}
        self.config = types.SimpleNamespace(num_hidden_layers=LAYERS, num_key_value_heads=HKV,
                                            num_attention_heads=HQ, hidden_size=HQ * D, head_dim=D)
        self.dev = torch.device("cuda", 0)

    def keys(self, layer, n, g):
        k = torch.randn(1, HKV, n, D, generator=g, device=self.dev)
        if layer in self.channels:
            k[..., torch.as_tensor(self.channels[layer], device=self.dev)] *= 25.0
        return k.half()

    def turboquant_probe(self, tokens):
        g = torch.Generator(device=self.dev).manual_seed(123)
        return [self.keys(l, tokens.shape[1], g) for l in range(LAYERS)]


def test_config3_outlier_layers():
    from turboquant_amd import TurboQuantKVCache, apply_turboquant
    from turboquant_amd.patch import FP16KVCache

    model = OutlierModel(seed=3)
    apply_turboquant(model, key_bits=4, value_bits=2, fp16_sink_size=SINK, residual_window=WINDOW,
                     auto_detect_outliers=True)
    assert model._turboquant_config["skip_layers"] == model.outliers
    caches = model.make_cache()
    assert [isinstance(c, FP16KVCache) for c in caches] == [l in model.outliers for l in range(LAYERS)]

    dev = model.dev
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(1, HQ, 1, D, generator=g, device=dev).half()
    checked_oracle = False
    for l, c in enumerate(caches):
        k = model.keys(l, T, g)
        v = torch.randn(1, HKV, T, D, generator=g, device=dev).half()
        if isinstance(c, FP16KVCache):
            kk, vv = c.update_and_fetch(k, v)
            # the model's own fp16 attention for a kept layer
            kr = kk.float().repeat_interleave(HQ // HKV, dim=1)
            vr = vv.float().repeat_interleave(HQ // HKV, dim=1)
            p = torch.softmax((q.float() @ kr.transpose(-1, -2)) * D ** -0.5, dim=-1)
            assert torch.isfinite(p @ vr).all()
            continue
        assert isinstance(c, TurboQuantKVCache)
        c.update(k, v)
        assert (c._sink_len, c._compressed_len, c._fp16_len) == (SINK, T - SINK - WINDOW, WINDOW)
        fast = c.attend(q)
        general = c.attend(q, general_kernel=True)
        e = rel_err(fast.cpu().numpy(), general.cpu().numpy())
        assert e < 1e-4, f"layer {l}: K4/V2 kernels vs general kernel {e:.3e}"
        if not checked_oracle:
            ks, vs = [], []
            R = O.rotation_matrix(D)
            for side, bits, x, sink in (("k", 4, k, c.sink_keys), ("v", 2, v, c.sink_values)):
                hi, lo, nrm = c.packed(side)
                deq = O.dequantize(hi.cpu().numpy(), None, nrm.cpu().numpy(), R, bits, D)
                parts = [sink[:, :, :SINK].cpu().numpy().astype(np.float64), deq,
                         x[:, :, T - WINDOW:].cpu().numpy().astype(np.float64)]
                (ks if side == "k" else vs).append(np.concatenate(parts, axis=2))
            ref = O.attention(q.cpu().numpy(), ks[0], vs[0])
            got = fast.cpu().numpy()
            e, cs = rel_err(got, ref), min_cos(got, ref)
            print(f"layer {l}: rel {e:.3e} min cos {cs:.7f}")
            assert e < 1e-3 and cs >= 0.9999
            checked_oracle = True
        del k, v
    assert checked_oracle
