"""Hugging Face ``transformers`` integration: TurboQuant caches inside a
PyTorch-ROCm decode loop.

The reference installs its caches through mlx-lm's ``model.make_cache``
(patch.py:355-371) and decodes through mlx-lm's attention over the dense K/V
its ``update_and_fetch`` returns (cache.py:620-706). For a ``transformers``
model the same roles are:

- ``TurboQuantCache(model)``: a ``transformers`` ``Cache`` whose layers are
  the caches ``apply_turboquant`` installed: a ``TurboQuantLayer`` per
  compressed layer and per uncompressed full-attention layer (outlier /
  skipped, ``FP16KVCache``), the model's own default layer
  (``DynamicCache(config)``) for sliding-window and linear-attention layers;
- the attention function registered as ``"turboquant"`` (with ``transformers``'
  SDPA mask construction): for a one-token decode step it runs the fused
  decode-attention kernel over the packed codes (``TurboQuantKVCache.attend``,
  never materialising the dense K/V) or the dense decode kernel over an
  ``FP16KVCache`` (fp16 / bf16, head_dim 128); every other call (prefill, the
  model's default layers) is ``transformers``' SDPA over the dense K/V, as in
  the reference. The kernels take no mask, logit soft-capping, sliding window
  or attention sinks: a decode step that carries any of them (a padding mask,
  ``softcap``, a ``sliding_window`` shorter than the context, ``s_aux``
  sinks) attends over the cache's dense K/V instead, with an eager float32
  attention where SDPA cannot express the argument (soft-capping, sinks).

The fused steps run only while the model's attention implementation is
``"turboquant"`` and the layer's shape is one the kernels serve (query heads
per kv head, head_dim); otherwise ``update`` returns the dense K/V for the
model's own attention.

    apply_turboquant(model, key_bits=4, value_bits=2, residual_window=128)
    model.set_attn_implementation("turboquant")
    cache = TurboQuantCache(model)
    out = model(input_ids, past_key_values=cache, use_cache=True)

Batches must hold sequences of equal length (no padding masks), as the
reference's cache does. Beam search reordering and cropping are not
supported by the compressed layers.
"""

from __future__ import annotations

import torch
from transformers import AttentionInterface
from transformers.cache_utils import Cache, CacheLayerMixin, DynamicCache, DynamicLayer
from transformers.integrations.sdpa_attention import sdpa_attention_forward
from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

from .cache import ATTEND_GROUPS, TurboQuantKVCache
from .patch import FP16KVCache

ATTN_IMPLEMENTATION = "turboquant"


def model_heads(config) -> tuple[int, int, int]:
    """(query heads, kv heads, head_dim) of a ``transformers`` config (its
    text config for multimodal models)."""
    text = config.get_text_config() if hasattr(config, "get_text_config") else config
    hq = text.num_attention_heads
    hkv = getattr(text, "num_key_value_heads", None) or hq
    hd = getattr(text, "head_dim", None) or text.hidden_size // hq
    return hq, hkv, hd


def fused_supported(cache, hq: int, hkv: int, head_dim: int) -> bool:
    """Whether the decode kernels serve a layer of this shape: the packed
    route (``TurboQuantKVCache.attend``: any integer query-head ratio) or the
    dense fp16 / bf16 kernel (``FP16KVCache.attend``: head_dim 128, ratios
    1, 2, 4, 8)."""
    if hkv <= 0 or hq % hkv:
        return False
    if isinstance(cache, FP16KVCache):
        return head_dim == 128 and hq // hkv in ATTEND_GROUPS
    return TurboQuantKVCache.attend_head_dim(head_dim)


class TurboQuantLayer(CacheLayerMixin):
    """One attention layer over a ``TurboQuantKVCache`` (compressed) or an
    ``FP16KVCache`` (uncompressed). ``update`` appends the new tokens
    (draining the oldest residual tokens into the packed store) and returns
    the dense K/V in the input dtype, or, for a one-token step with ``fused``,
    the new tokens themselves tagged for the decode kernel."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, cache: TurboQuantKVCache, fused: bool = True, config=None):
        super().__init__()
        self.cache = cache
        self.fused = fused
        self.config = config  # the model's config: fused steps only under its "turboquant" attention

    def lazy_initialization(self, key_states, value_states):
        self.dtype, self.device = key_states.dtype, key_states.device
        if isinstance(self.cache, FP16KVCache):  # the dense kernel's shapes
            self.fused = self.fused and key_states.is_cuda and key_states.shape[-1] == 128 and \
                key_states.dtype in (torch.float16, torch.bfloat16)
        self.is_initialized = True

    def fused_step(self, key_states) -> bool:
        """A one-token step the attention function will run on the kernels."""
        return self.fused and key_states.shape[-2] == 1 and (
            self.config is None or getattr(self.config, "_attn_implementation", None) == ATTN_IMPLEMENTATION)

    def dense_kv(self):
        """The cache's whole dense K/V (B, Hkv, T, D), nothing appended."""
        if isinstance(self.cache, FP16KVCache):
            return self.cache.keys, self.cache.values
        return self.cache.fetch()

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self.fused_step(key_states):
            self.cache.update(key_states, value_states)
            key_states._turboquant_layer = self  # read by turboquant_attention
            return key_states, value_states
        k, v = self.cache.update_and_fetch(key_states, value_states)
        return k.to(key_states.dtype), v.to(value_states.dtype)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        return self.cache.offset

    def get_max_length(self) -> int:
        return -1

    def offload(self):
        pass  # the packed store stays on its device

    def prefetch(self):
        pass

    def reset(self):
        raise NotImplementedError("a TurboQuant layer cannot be reset in place; build a new TurboQuantCache")

    def reorder_cache(self, beam_idx):
        raise NotImplementedError("beam search reordering of a TurboQuant layer")

    def crop(self, *args, **kwargs):
        raise NotImplementedError("cropping a TurboQuant layer")


class TurboQuantCache(Cache):
    """``transformers`` cache over the per-layer caches of
    ``model.make_cache()`` (install them with ``apply_turboquant``)."""

    def __init__(self, model, fused: bool = True):
        make = getattr(model, "make_cache", None)
        if make is None:
            raise ValueError("model has no make_cache: call apply_turboquant(model, ...) first")
        caches = make()
        defaults = DynamicCache(config=model.config).layers
        hq, hkv, hd = model_heads(model.config)
        layers = []
        for i, c in enumerate(caches):
            if isinstance(c, (TurboQuantKVCache, FP16KVCache)):
                layers.append(TurboQuantLayer(c, fused and fused_supported(c, hq, hkv, hd), model.config))
            else:
                layers.append(defaults[i] if i < len(defaults) else DynamicLayer())
        super().__init__(layers=layers)


def eager_attention(query, key, value, attention_mask=None, scaling=None, softcap=None, sinks=None,
                    sliding_window=None):
    """Dense attention in float32 for what SDPA cannot express: logit
    soft-capping (``softcap * tanh(s / softcap)``), attention sinks (a
    per-head logit ``sinks[h]`` that joins every row's softmax and receives
    no value) and a sliding window, with a boolean (True = attend) or
    additive mask, else causal with query i at position T_k - T_q + i.
    query (B, Hq, T_q, D), key / value (B, Hkv, T_k, D); returns (B, T_q,
    Hq, D) in the query's dtype and the weights."""
    B, hq, tq, D = query.shape
    hkv, tk = key.shape[1], key.shape[2]
    g = hq // hkv
    k = key.float().repeat_interleave(g, dim=1)
    v = value.float().repeat_interleave(g, dim=1)
    scale = D ** -0.5 if scaling is None else scaling
    s = torch.matmul(query.float(), k.transpose(-1, -2).contiguous()) * scale
    if softcap:
        s = torch.tanh(s / softcap) * softcap
    pos_q = torch.arange(tq, device=s.device)[:, None] + (tk - tq)
    pos_k = torch.arange(tk, device=s.device)[None, :]
    if attention_mask is None:
        s = s.masked_fill(pos_k > pos_q, float("-inf"))
    else:
        m = attention_mask[..., :tk]
        s = s.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else s + m.float()
    if sliding_window:
        s = s.masked_fill(pos_q - pos_k >= sliding_window, float("-inf"))
    if sinks is not None:
        sk = sinks.float().reshape(1, hq, 1, 1).expand(B, hq, tq, 1)
        s = torch.cat([s, sk], dim=-1)
    p = torch.softmax(s, dim=-1)
    if sinks is not None:
        p = p[..., :-1]
    out = torch.matmul(p, v)
    return out.to(query.dtype).transpose(1, 2).contiguous(), p


def turboquant_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                         scaling: float | None = None, **kwargs):
    """Attention function of ``set_attn_implementation("turboquant")``: the
    decode kernels for a one-token step of a ``TurboQuantLayer`` (packed codes
    or dense fp16 / bf16) that carries no mask, soft-capping, binding sliding
    window or sinks; otherwise ``transformers``' SDPA over the dense K/V, or
    ``eager_attention`` where SDPA cannot express soft-capping or sinks.
    Returns (B, T, Hq, D)."""
    layer = getattr(key, "_turboquant_layer", None)
    softcap = kwargs.get("softcap")
    sinks = kwargs.get("s_aux", kwargs.get("sinks"))
    window = kwargs.get("sliding_window")
    if layer is not None:
        tk = layer.get_seq_length()
        if attention_mask is None and not softcap and sinks is None and not (window and tk > window):
            out = layer.cache.attend(query, scale=scaling)  # (B, Hq, 1, D) float32
            return out.to(query.dtype).transpose(1, 2).contiguous(), None
        # the kernels honour none of these arguments: the cache's dense K/V
        key, value = layer.dense_kv()
        key, value = key.to(query.dtype), value.to(query.dtype)
    if softcap or sinks is not None or (window and key.shape[2] > window and attention_mask is None):
        return eager_attention(query, key, value, attention_mask, scaling, softcap, sinks, window)
    return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                  scaling=scaling, **kwargs)


AttentionInterface.register(ATTN_IMPLEMENTATION, turboquant_attention)
AttentionMaskInterface.register(ATTN_IMPLEMENTATION, sdpa_mask)
