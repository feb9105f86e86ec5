"""The transformers integration on the CPU (no GPU): a tiny random-init
Llama (head_dim 128) runs its own forward and decode loop with
TurboQuantCache; the two device calls of the cache are the oracle stand-ins
of test_host_cache.py. Covers the outlier probe on a real forward
(patch.py:89-133), layer placement, exactness while nothing is compressed,
and the compressed cache's state through prefill and decode.
"""

import numpy as np
import pytest
import torch

from test_host_cache import cpu_cache  # noqa: F401  (fixture)

transformers = pytest.importorskip("transformers")


def tiny_llama(seed=0, layers=3):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=97, hidden_size=512, intermediate_size=768, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=1024)
    return LlamaForCausalLM(cfg).eval()


def run(model, cache, ids, steps):
    """Prefill ids, then greedy-decode `steps` tokens; returns the logits of
    every step (prefill's last position first)."""
    out = model(ids, past_key_values=cache, use_cache=True)
    logits = [out.logits[:, -1].float()]
    tok = out.logits[:, -1:].argmax(-1)
    for _ in range(steps):
        out = model(tok, past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1].float())
        tok = out.logits[:, -1:].argmax(-1)
    return torch.stack(logits)


def test_outlier_probe_real_forward():
    from transformers import DynamicCache
    from turboquant_amd.patch import detect_outlier_layers, outlier_layers_from_norms
    m = tiny_llama()
    with torch.no_grad():
        m.model.layers[1].self_attn.k_proj.weight.mul_(40.0)  # one layer with large keys
        pkv = m(torch.tensor([[0, 1, 2, 3, 4]]), past_key_values=DynamicCache(), use_cache=True).past_key_values
        norms = [float(torch.linalg.vector_norm(layer.keys.float(), dim=-1).max()) for layer in pkv.layers]
        assert detect_outlier_layers(m) == outlier_layers_from_norms(norms) == [1]


def test_cache_layers_and_exact_without_compression(cpu_cache):
    from transformers import DynamicCache
    from turboquant_amd import apply_turboquant
    from turboquant_amd.hf import TurboQuantCache, TurboQuantLayer
    m = tiny_llama()
    apply_turboquant(m, key_bits=4, value_bits=2, residual_window=256, skip_layers=[2])
    cache = TurboQuantCache(m, fused=False)
    assert [type(x).__name__ for x in cache.layers] == ["TurboQuantLayer"] * 3
    from turboquant_amd.patch import FP16KVCache
    assert isinstance(cache.layers[2].cache, FP16KVCache)  # the skipped layer: uncompressed
    ids = torch.randint(0, 97, (1, 40), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        got = run(m, cache, ids, 8)
        ref = run(m, DynamicCache(), ids, 8)
    assert torch.equal(got, ref)  # 48 tokens < 2 x window: nothing compressed, same K/V
    # the registered "turboquant" attention (masks built for it, SDPA for untagged K/V) gives the same logits
    m.set_attn_implementation("turboquant")
    with torch.no_grad():
        got2 = run(m, TurboQuantCache(m, fused=False), ids, 8)
    assert torch.equal(got2, ref)
    assert isinstance(cache.layers[0], TurboQuantLayer) and cache.layers[0].cache._compressed_len == 0
    assert cache.get_seq_length() == 48


def test_compressed_decode_loop(cpu_cache):
    from transformers import DynamicCache
    from turboquant_amd import apply_turboquant
    from turboquant_amd.hf import TurboQuantCache
    m = tiny_llama(seed=2)
    apply_turboquant(m, key_bits=4, value_bits=2, residual_window=16, fp16_sink_size=4, auto_detect_outliers=False)
    cache = TurboQuantCache(m, fused=False)
    ids = torch.randint(0, 97, (1, 60), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        got = run(m, cache, ids, 12)
        ref = run(m, DynamicCache(), ids, 12)
    c = cache.layers[0].cache
    # prefill of 60: 4 sink, 56 to the ring, 56 > 2 x 16 drains 40 (cache.py:519-527); then one drain per
    # 16 decode steps on top of the window
    assert c._sink_len == 4 and c.offset == 72 and c._compressed_len + c._fp16_len == 68
    assert c._compressed_len >= 40 and c._fp16_len <= 32
    cos = torch.nn.functional.cosine_similarity(got, ref, dim=-1)
    print("logit cosine per step:", np.round(cos.numpy(), 4))
    assert torch.isfinite(got).all() and cos.min() > 0.9
