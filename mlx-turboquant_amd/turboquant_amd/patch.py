"""Model patching for PyTorch models (patch.py of the reference).

``apply_turboquant`` keeps the reference signature and semantics
(patch.py:136-371): low-KV-head bit upgrades, explicit or auto-detected
outlier layers kept uncompressed, and a per-layer cache factory installed as
the instance attribute ``model.make_cache`` plus ``model._turboquant_config``.

Model introspection follows Hugging Face conventions (``model.config`` with
``num_key_value_heads`` / ``head_dim`` / ``num_attention_heads`` /
``hidden_size`` / ``num_hidden_layers``) in place of mlx-lm's ``args``.
Outlier detection runs the reference's 5-token probe (patch.py:89-133)
through ``model.turboquant_probe(tokens)`` when the model defines it (it
returns one (B, H, T, D) key tensor per layer), else through a Hugging Face
forward with ``use_cache=True``.

Hybrid and sliding-window models (patch.py:228-321): layers whose attention
is linear (a ``linear_attn`` / ``linear_attention`` module and no
``self_attn`` / ``attention``, or ``config.layer_types`` entry
``"linear_attention"``) and layers whose model-default cache is a
sliding-window one keep the model's default cache. The defaults come from a
class-level ``make_cache`` when the model class defines one (the reference's
rule), else from the Hugging Face config (``layer_types`` /
``sliding_window`` / ``use_sliding_window`` / ``max_window_layers``):
``SlidingWindowKVCache`` for sliding-window layers, ``None`` for
linear-attention layers (their state belongs to the model), ``FP16KVCache``
otherwise.
"""

from __future__ import annotations

import warnings

import numpy as np
import torch

from .cache import TurboQuantKVCache


class FP16KVCache:
    """Uncompressed cache used for skipped / outlier layers (the reference
    hands those layers mlx-lm's ``KVCache``, patch.py:337-338). Storage grows
    in steps of ``step`` tokens, as mlx-lm's KVCache does; ``keys`` /
    ``values`` are views of the first ``offset`` tokens. ``attend`` runs the
    dense decode-attention kernel over them (fp16 / bf16, head_dim 128)."""

    step = 256

    def __init__(self):
        self._k = self._v = None
        self.offset = 0

    @property
    def keys(self):
        return None if self._k is None else self._k[:, :, :self.offset]

    @property
    def values(self):
        return None if self._v is None else self._v[:, :, :self.offset]

    def update(self, keys, values) -> None:
        """Append (B, H, n, D) keys / values."""
        n, prev = keys.shape[2], self.offset
        if self._k is None or prev + n > self._k.shape[2]:
            B, H, _, D = keys.shape
            cap = (prev + n + self.step - 1) // self.step * self.step
            k = keys.new_empty(B, H, cap, D)
            v = values.new_empty(B, H, cap, values.shape[3])
            if self._k is not None:
                k[:, :, :prev] = self._k[:, :, :prev]
                v[:, :, :prev] = self._v[:, :, :prev]
            self._k, self._v = k, v
        self._k[:, :, prev:prev + n] = keys
        self._v[:, :, prev:prev + n] = values
        self.offset = prev + n

    def update_and_fetch(self, keys, values):
        self.update(keys, values)
        return self.keys, self.values

    def attend(self, queries, scale=None, out=None):
        """Decode attention of one query token per head over the cached tokens:
        float32 (B, Hq, 1, D)."""
        if self._k is None or self.offset == 0:
            raise ValueError("attend() on an empty cache")
        from .cache import dense_attention
        return dense_attention(queries, self.keys, self.values, scale=scale, out=out)

    def make_mask(self, N, offset=0, return_array=False, window_size=None):
        return None if N == 1 and not return_array else "causal"

    def empty(self):
        return self._k is None

    def size(self):
        return self.offset


class SlidingWindowKVCache:
    """fp16 cache of a sliding-window-attention layer: attention sees the last
    ``max_size`` tokens (the role of mlx-lm's ``RotatingKVCache``, which the
    reference leaves on such layers, patch.py:270-321). ``update_and_fetch``
    returns the kept tokens plus the new ones; ``make_mask`` gives the matching
    causal window mask."""

    def __init__(self, max_size: int):
        if max_size <= 0:
            raise ValueError("max_size must be positive")
        self.max_size = max_size
        self.keys = self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        if self.keys is None:
            k, v = keys, values
        else:
            k = torch.cat([self.keys, keys], dim=2)
            v = torch.cat([self.values, values], dim=2)
        self.offset += keys.shape[2]
        self.keys, self.values = k[:, :, -self.max_size:], v[:, :, -self.max_size:]
        return k, v

    def make_mask(self, N, offset=None, return_array=False, window_size=None):
        """Mask of N queries starting at absolute position ``offset`` (default
        the tokens cached so far) over the keys the next ``update_and_fetch``
        returns: True where query i may see key j (causal, within the
        window). None when every key is visible to a single query."""
        off = self.offset if offset is None else offset
        win = window_size or self.max_size
        kept = min(off, self.max_size)
        if N == 1 and kept < win and not return_array:
            return None
        q = off + torch.arange(N).unsqueeze(1)                   # absolute query positions
        kpos = off - kept + torch.arange(kept + N).unsqueeze(0)  # absolute key positions
        return (kpos <= q) & (q - kpos < win)

    def empty(self):
        return self.keys is None

    def size(self):
        return self.offset


def _config_of(model):
    for cand in (model, getattr(model, "model", None), getattr(model, "language_model", None)):
        if cand is None:
            continue
        c = getattr(cand, "config", None) or getattr(cand, "args", None)
        if c is not None:
            return c
    return None


def _model_layers(model) -> list:
    inner = getattr(model, "model", model)
    layers = getattr(inner, "layers", None)
    if layers is None:
        layers = getattr(model, "layers", None)
    return list(layers or [])


def linear_attention_layers(model) -> set[int]:
    """Layers with linear attention (patch.py:228-260): a ``linear_attn`` /
    ``linear_attention`` module and no ``self_attn`` / ``attention`` module,
    or ``"linear_attention"`` in the config's ``layer_types``."""
    out = set()
    for i, layer in enumerate(_model_layers(model)):
        if hasattr(layer, "linear_attn") or hasattr(layer, "linear_attention"):
            if not (hasattr(layer, "self_attn") or hasattr(layer, "attention")):
                out.add(i)
    kinds = getattr(_config_of(model), "layer_types", None)
    if kinds:
        out |= {i for i, t in enumerate(kinds) if t == "linear_attention"}
    return out


def _config_default_caches(model, num_layers: int, linear: set[int]) -> list:
    """The model-default cache of every layer from a Hugging Face config
    (``linear``: the linear-attention layers)."""
    cfg = _config_of(model)
    if cfg is None:
        raise ValueError("no model config")
    window = getattr(cfg, "sliding_window", None)
    kinds = getattr(cfg, "layer_types", None)
    if not kinds:
        use = getattr(cfg, "use_sliding_window", None)
        first = getattr(cfg, "max_window_layers", None)
        if window and use is not False and (use or first is None):
            kinds = ["sliding_attention" if first is None or i >= first else "full_attention"
                     for i in range(num_layers)]
        else:
            kinds = ["full_attention"] * num_layers
    out = []
    for i in range(num_layers):
        t = kinds[i] if i < len(kinds) else "full_attention"
        if i in linear or t == "linear_attention":
            out.append(None)
        elif t == "sliding_attention" and window:
            out.append(SlidingWindowKVCache(int(window)))
        else:
            out.append(FP16KVCache())
    return out


def _is_sliding_cache(c) -> bool:
    """The reference tests for mlx-lm's RotatingKVCache family (patch.py:262-300)."""
    return isinstance(c, SlidingWindowKVCache) or "Rotating" in type(c).__name__


def _get_model_config(model) -> dict:
    """head_dim / num_kv_heads / num_layers from an HF-style config
    (patch.py:13-86 reads mlx-lm ``args`` the same way)."""
    cfg = None
    for cand in (model, getattr(model, "model", None), getattr(model, "language_model", None)):
        if cand is None:
            continue
        c = getattr(cand, "config", None) or getattr(cand, "args", None)
        if c is not None and getattr(c, "hidden_size", None) is not None:
            cfg = c
            break
    if cfg is None:
        raise ValueError("Could not determine model configuration. "
                         "Please specify head_dim and num_kv_heads manually.")
    heads = getattr(cfg, "num_attention_heads", None)
    head_dim = getattr(cfg, "head_dim", None)
    if head_dim is None and heads:
        head_dim = cfg.hidden_size // heads
    nkv = getattr(cfg, "num_key_value_heads", None) or getattr(cfg, "num_kv_heads", None) or heads
    layers = getattr(cfg, "num_hidden_layers", None)
    if layers is None:
        inner = getattr(model, "model", model)
        layers = len(getattr(inner, "layers", []) or [])
    return {"head_dim": head_dim or 128, "num_kv_heads": nkv or 1, "num_layers": layers or 1}


def _probe_layer_keys(model) -> list:
    dev = next((p.device for p in model.parameters()), torch.device("cpu")) if hasattr(model, "parameters") else None
    tokens = torch.tensor([[0, 1, 2, 3, 4]], device=dev)
    if hasattr(model, "turboquant_probe"):
        return list(model.turboquant_probe(tokens))
    out = model(tokens, use_cache=True)
    pkv = getattr(out, "past_key_values", None)
    if pkv is None:
        raise ValueError("model returned no key cache")
    if hasattr(pkv, "layers"):  # transformers >= 4.56 Cache: one layer object per decoder layer
        return [getattr(layer, "keys", None) for layer in pkv.layers]
    if hasattr(pkv, "key_cache"):
        return list(pkv.key_cache)
    return [kv[0] for kv in pkv]


def outlier_layers_from_norms(max_norms, threshold: float = 3.0) -> list[int]:
    """Layers whose max key norm exceeds threshold x the median of the positive
    maxima; empty when none is positive (patch.py:119-133)."""
    m = np.asarray(max_norms, dtype=np.float64)
    pos = m[m > 0]
    if pos.size == 0:
        return []
    med = float(np.median(pos))
    return [i for i, n in enumerate(m) if n > threshold * med]


def detect_outlier_layers(model, threshold: float = 3.0) -> list[int]:
    """Probe forward of tokens [0..4], per-layer max key L2 norm, outlier rule
    (patch.py:89-133)."""
    maxima = []
    for k in _probe_layer_keys(model):
        if k is None or k.numel() == 0:
            maxima.append(0.0)
        else:
            maxima.append(float(torch.linalg.vector_norm(k.float(), dim=-1).max()))
    return outlier_layers_from_norms(maxima, threshold)


def apply_turboquant(model, key_bits: float = 4, value_bits: float = 2, residual_window: int = 128,
                     head_dim: int | None = None, num_kv_heads: int | None = None,
                     num_layers: int | None = None, rotation_seed: int = 42,
                     skip_layers: list[int] | None = None, auto_detect_outliers: bool = True,
                     fp16_sink_size: int = 0, chunk_size: int = 0, qjl_correction: bool = False,
                     qjl_n_proj: int = 32):
    """Install TurboQuant caches on ``model`` (patch.py:136-371)."""
    if head_dim is None or num_kv_heads is None or num_layers is None:
        config = _get_model_config(model)
    else:
        config = {}
    hd = head_dim or config["head_dim"]
    nkv = num_kv_heads or config["num_kv_heads"]
    nl = num_layers or config["num_layers"]

    # few KV heads -> more precision (patch.py:198-217)
    if nkv <= 2 and key_bits < 4:
        old = key_bits
        key_bits = 4
        warnings.warn(f"Model has only {nkv} KV heads — upgrading key_bits {old} → {key_bits} for stability. "
                      f"Effective config: key_bits={key_bits}, value_bits={value_bits}.", UserWarning, stacklevel=2)
    if nkv <= 2 and value_bits < 3:
        old = value_bits
        value_bits = 3
        warnings.warn(f"Model has only {nkv} KV heads — upgrading value_bits {old} → {value_bits} for stability. "
                      f"Effective config: key_bits={key_bits}, value_bits={value_bits}.", UserWarning, stacklevel=2)

    layers_to_skip = set(skip_layers or [])
    if auto_detect_outliers and not skip_layers:
        try:
            layers_to_skip = set(detect_outlier_layers(model))
        except Exception:
            pass  # detection failure compresses every layer (patch.py:221-226)

    # hybrid (linear-attention) and sliding-window layers keep the model's own
    # cache type (patch.py:228-321)
    linear_layers = linear_attention_layers(model)
    if linear_layers:
        warnings.warn(f"Detected {len(linear_layers)} linear-attention layers in model (hybrid architecture, "
                      f"e.g. Qwen3.5). These layers will use the model's default cache type instead of "
                      f"TurboQuantKVCache.", UserWarning, stacklevel=2)
    class_make_cache = getattr(type(model), "make_cache", None)  # captured before the instance attribute

    def default_caches():
        if class_make_cache is not None:
            return list(class_make_cache(model))
        return _config_default_caches(model, nl, linear_layers)

    swa_layers = set()
    try:
        for i, c in enumerate(default_caches()):
            if i not in linear_layers and _is_sliding_cache(c):
                swa_layers.add(i)
    except Exception:
        pass
    if swa_layers:
        warnings.warn(f"Detected {len(swa_layers)} sliding-window-attention layers in model. These layers will "
                      f"use the model's default cache type instead of TurboQuantKVCache.", UserWarning, stacklevel=2)
    default_layers = linear_layers | swa_layers

    def make_cache():
        defaults = default_caches() if default_layers else None
        caches = []
        for i in range(nl):
            if i in default_layers:
                caches.append(defaults[i] if i < len(defaults) else None)
            elif i in layers_to_skip:
                caches.append(FP16KVCache())
            else:
                caches.append(TurboQuantKVCache(
                    head_dim=hd, num_kv_heads=nkv, key_bits=key_bits, value_bits=value_bits,
                    residual_window=residual_window, rotation_seed=rotation_seed,
                    fp16_sink_size=fp16_sink_size, chunk_size=chunk_size,
                    qjl_correction=qjl_correction, qjl_n_proj=qjl_n_proj))
        return caches

    model.make_cache = make_cache
    model._turboquant_config = {
        "head_dim": hd, "num_kv_heads": nkv, "num_layers": nl, "key_bits": key_bits,
        "value_bits": value_bits, "residual_window": residual_window, "fp16_sink_size": fp16_sink_size,
        "chunk_size": chunk_size, "qjl_correction": qjl_correction, "qjl_n_proj": qjl_n_proj,
        "skip_layers": sorted(layers_to_skip), "default_cache_layers": sorted(default_layers),
    }
    return model


def enable_turboquant(model, bits: int = 4, **kwargs):
    """Symmetric bits for keys and values (patch.py:374-385)."""
    return apply_turboquant(model, key_bits=bits, value_bits=bits, **kwargs)
