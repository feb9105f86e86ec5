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
- the attention function registered as ``"turboquant"``: for a one-token
  decode step it runs the fused decode-attention kernel over the packed codes
  (``TurboQuantKVCache.attend``, never materialising the dense K/V) or the
  dense decode kernel over an ``FP16KVCache`` (fp16 / bf16, head_dim 128);
  every other call (prefill, the model's default layers) is ``transformers``'
  SDPA over the dense K/V, as in the reference.

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

from .cache import TurboQuantKVCache
from .patch import FP16KVCache

ATTN_IMPLEMENTATION = "turboquant"


class TurboQuantLayer(CacheLayerMixin):
    """One attention layer over a ``TurboQuantKVCache`` (compressed) or an
    ``FP16KVCache`` (uncompressed). ``update`` appends the new tokens
    (draining the oldest residual tokens into the packed store) and returns
    the dense K/V in the input dtype, or, for a one-token step with ``fused``,
    the new tokens themselves tagged for the decode kernel."""

    is_sliding = False
    is_compileable = False
    supports_early_init = False

    def __init__(self, cache: TurboQuantKVCache, fused: bool = True):
        super().__init__()
        self.cache = cache
        self.fused = fused

    def lazy_initialization(self, key_states, value_states):
        self.dtype, self.device = key_states.dtype, key_states.device
        if isinstance(self.cache, FP16KVCache):  # the dense kernel's shapes
            self.fused = self.fused and key_states.is_cuda and key_states.shape[-1] == 128 and \
                key_states.dtype in (torch.float16, torch.bfloat16)
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self.fused and key_states.shape[-2] == 1:
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
        layers = []
        for i, c in enumerate(caches):
            if isinstance(c, (TurboQuantKVCache, FP16KVCache)):
                layers.append(TurboQuantLayer(c, fused))
            else:
                layers.append(defaults[i] if i < len(defaults) else DynamicLayer())
        super().__init__(layers=layers)


def turboquant_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                         scaling: float | None = None, **kwargs):
    """Attention function of ``set_attn_implementation("turboquant")``: the
    decode kernels for a one-token step of a ``TurboQuantLayer`` (packed codes
    or dense fp16 / bf16), ``transformers``' SDPA otherwise. Returns
    (B, T, Hq, D)."""
    layer = getattr(key, "_turboquant_layer", None)
    if layer is None:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                      scaling=scaling, **kwargs)
    out = layer.cache.attend(query, scale=scaling)  # (B, Hq, 1, D) float32
    return out.to(query.dtype).transpose(1, 2).contiguous(), None


AttentionInterface.register(ATTN_IMPLEMENTATION, turboquant_attention)
