"""apply_turboquant's model rules on the CPU (no GPU): the low-KV-head bit
upgrade (patch.py:198-217), explicit skips, and the hybrid / sliding-window
rules (patch.py:228-321) that leave linear-attention and sliding-window
layers on the model's own cache type. Stand-in models carry a Hugging Face
style config and layer modules; no forward pass is run
(auto_detect_outliers=False).
"""

import types
import warnings

import pytest
import torch

from turboquant_amd import TurboQuantKVCache, apply_turboquant
from turboquant_amd.patch import FP16KVCache, SlidingWindowKVCache, linear_attention_layers


def _cfg(layers=4, kv=8, heads=32, **extra):
    return types.SimpleNamespace(num_hidden_layers=layers, num_key_value_heads=kv, num_attention_heads=heads,
                                 hidden_size=heads * 128, head_dim=128, **extra)


class Model:
    def __init__(self, cfg, layers=None):
        self.config = cfg
        self.model = types.SimpleNamespace(layers=layers or [])


def _layer(kind):
    lay = types.SimpleNamespace()
    if kind in ("attn", "both"):
        lay.self_attn = object()
    if kind in ("linear", "both"):
        lay.linear_attn = object()
    return lay


def _kinds(caches):
    return ["tq" if isinstance(c, TurboQuantKVCache) else "fp16" if isinstance(c, FP16KVCache)
            else "swa" if isinstance(c, SlidingWindowKVCache) else type(c).__name__ for c in caches]


def test_plain_model_all_turboquant():
    m = apply_turboquant(Model(_cfg()), auto_detect_outliers=False)
    assert _kinds(m.make_cache()) == ["tq"] * 4
    assert m._turboquant_config["default_cache_layers"] == []


def test_skip_layers_fp16():
    m = apply_turboquant(Model(_cfg()), skip_layers=[1, 3], auto_detect_outliers=False)
    assert _kinds(m.make_cache()) == ["tq", "fp16", "tq", "fp16"]


def test_low_kv_heads_upgrade_warns():
    with pytest.warns(UserWarning, match="upgrading key_bits 3 → 4"):
        m = apply_turboquant(Model(_cfg(kv=2)), key_bits=3, value_bits=3, auto_detect_outliers=False)
    assert m._turboquant_config["key_bits"] == 4 and m._turboquant_config["value_bits"] == 3
    with pytest.warns(UserWarning, match="upgrading value_bits 2 → 3"):
        m = apply_turboquant(Model(_cfg(kv=1)), key_bits=4, value_bits=2, auto_detect_outliers=False)
    assert m._turboquant_config["value_bits"] == 3


def test_hybrid_linear_attention_layers_structural():
    """Layers with linear_attn and no self_attn keep the model's cache; a
    layer holding both modules is treated as self-attention (patch.py:237-251)."""
    layers = [_layer("attn"), _layer("linear"), _layer("attn"), _layer("both")]
    m = Model(_cfg(), layers)
    assert linear_attention_layers(m) == {1}
    with pytest.warns(UserWarning, match="1 linear-attention layers"):
        apply_turboquant(m, auto_detect_outliers=False)
    assert _kinds(m.make_cache()) == ["tq", "NoneType", "tq", "tq"]
    assert m._turboquant_config["default_cache_layers"] == [1]


class _RotatingKVCache:
    """Stand-in for a model's own rotating (sliding-window) cache class."""


class _LinearState:
    pass


class ModelWithCaches(Model):
    """A model class that builds its own per-layer caches (the reference reads
    the class-level make_cache, patch.py:270-300)."""

    def make_cache(self):
        return [FP16KVCache(), _RotatingKVCache(), _LinearState(), FP16KVCache()]


def test_class_level_default_caches():
    layers = [_layer("attn"), _layer("attn"), _layer("linear"), _layer("attn")]
    m = ModelWithCaches(_cfg(), layers)
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        apply_turboquant(m, auto_detect_outliers=False)
    msgs = " ".join(str(r.message) for r in rec)
    assert "1 linear-attention layers" in msgs and "1 sliding-window-attention layers" in msgs
    caches = m.make_cache()  # the instance attribute installed by apply_turboquant
    assert _kinds(caches) == ["tq", "_RotatingKVCache", "_LinearState", "tq"]
    assert m._turboquant_config["default_cache_layers"] == [1, 2]
    # a fresh default object per make_cache call
    assert m.make_cache()[1] is not caches[1]


def test_hf_layer_types_sliding_and_linear():
    cfg = _cfg(layers=6, sliding_window=512,
               layer_types=["sliding_attention", "full_attention", "linear_attention",
                            "sliding_attention", "full_attention", "full_attention"])
    m = Model(cfg)
    with pytest.warns(UserWarning):
        apply_turboquant(m, skip_layers=[4], auto_detect_outliers=False)
    caches = m.make_cache()
    assert _kinds(caches) == ["swa", "tq", "NoneType", "swa", "fp16", "tq"]
    assert caches[0].max_size == 512


@pytest.mark.parametrize("use,first,expect", [
    (True, 2, ["tq", "tq", "swa", "swa"]),   # Qwen2: layers >= max_window_layers slide
    (False, 2, ["tq"] * 4),                  # sliding window configured but off
    (None, None, ["swa"] * 4),               # Mistral-style: every layer slides
])
def test_hf_sliding_window_rules(use, first, expect):
    extra = {"sliding_window": 256}
    if use is not None:
        extra["use_sliding_window"] = use
    if first is not None:
        extra["max_window_layers"] = first
    m = Model(_cfg(**extra))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        apply_turboquant(m, auto_detect_outliers=False)
    assert _kinds(m.make_cache()) == expect


def test_sliding_window_cache_keeps_window_and_masks():
    W = 5
    c = SlidingWindowKVCache(W)
    rng = torch.Generator().manual_seed(0)
    total = []
    for n in (3, 1, 4, 1, 1, 6):
        k = torch.randn(1, 2, n, 8, generator=rng)
        off = c.offset
        mask = c.make_mask(n, return_array=True)
        kk, vv = c.update_and_fetch(k, k + 1)
        total.append(k)
        full = torch.cat(total, dim=2)
        # fetched = kept window + the new tokens, in order
        kept = min(off, W)
        assert torch.equal(kk, full[:, :, off - kept:])
        assert torch.equal(vv, kk + 1)
        assert c.offset == off + n and c.keys.shape[2] == min(off + n, W)
        # mask against brute force over absolute positions
        qpos = [off + i for i in range(n)]
        kpos = [off - kept + j for j in range(kept + n)]
        ref = torch.tensor([[kp <= qp and qp - kp < W for kp in kpos] for qp in qpos])
        assert torch.equal(mask, ref)
    assert c.make_mask(1) is None or c.make_mask(1).shape == (1, W + 1)
    with pytest.raises(ValueError):
        SlidingWindowKVCache(0)
