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


def test_fused_cache_under_sdpa_and_unsupported_groups(cpu_cache):
    """A fused cache never takes the kernel route unless the model's
    attention is "turboquant" and the layer shape is served: under SDPA every
    step returns the dense K/V, and so does an uncompressed (FP16KVCache)
    layer with 3 query heads per kv head, which the dense decode kernel does
    not serve (the kernels cannot run on this CPU-only box, so a fused step
    would raise). A compressed layer of that shape is fused: the packed
    route takes any ratio."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from turboquant_amd import apply_turboquant
    from turboquant_amd.hf import TurboQuantCache
    ids = torch.randint(0, 97, (1, 50), generator=torch.Generator().manual_seed(7))
    m = tiny_llama(seed=5)
    apply_turboquant(m, key_bits=4, value_bits=2, residual_window=16, auto_detect_outliers=False)
    m.set_attn_implementation("sdpa")
    with torch.no_grad():
        got = run(m, TurboQuantCache(m, fused=True), ids, 6)
        ref = run(m, TurboQuantCache(m, fused=False), ids, 6)
    assert torch.equal(got, ref)

    torch.manual_seed(6)
    cfg = LlamaConfig(vocab_size=97, hidden_size=768, intermediate_size=768, num_hidden_layers=2,
                      num_attention_heads=6, num_key_value_heads=2, head_dim=128, max_position_embeddings=1024)
    m3 = LlamaForCausalLM(cfg).eval()
    apply_turboquant(m3, key_bits=4, value_bits=2, residual_window=16, auto_detect_outliers=False)
    m3.set_attn_implementation("turboquant")
    assert all(layer.fused for layer in TurboQuantCache(m3, fused=True).layers)
    apply_turboquant(m3, key_bits=4, value_bits=2, residual_window=16, auto_detect_outliers=False,
                     skip_layers=[0, 1])
    cache = TurboQuantCache(m3, fused=True)
    assert not any(layer.fused for layer in cache.layers)
    with torch.no_grad():
        got = run(m3, cache, ids, 6)
        ref = run(m3, TurboQuantCache(m3, fused=False), ids, 6)
    assert torch.equal(got, ref)


def test_eager_attention_softcap_sinks_window():
    """eager_attention against closed forms: plain attention equals SDPA;
    soft-capping is s -> c tanh(s / c) before the softmax; a sink logit of
    -inf changes nothing, and a sink logit z scales each row's weights by
    sum(e^s) / (sum(e^s) + e^z); a sliding window w keeps keys with
    0 <= pos_q - pos_k < w."""
    from turboquant_amd.hf import eager_attention
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4, 3, 128, generator=g)
    k = torch.randn(2, 2, 9, 128, generator=g) * 3
    v = torch.randn(2, 2, 9, 128, generator=g)
    kr, vr = k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)
    sdpa = torch.nn.functional.scaled_dot_product_attention
    causal = torch.ones(3, 9, dtype=torch.bool).tril(6)  # query i at position 6 + i
    out, _ = eager_attention(q, k, v)
    ref = sdpa(q, kr, vr, attn_mask=causal).transpose(1, 2)
    assert torch.allclose(out, ref, atol=1e-5)
    out, w = eager_attention(q, k, v, softcap=2.0, scaling=0.5)
    s = 2.0 * torch.tanh(q @ kr.transpose(-1, -2) * 0.5 / 2.0)
    s = s.masked_fill(~causal, float("-inf"))
    assert torch.allclose(w, torch.softmax(s, -1), atol=1e-6)
    out_ninf, _ = eager_attention(q, k, v, sinks=torch.full((4,), float("-inf")))
    base, wb = eager_attention(q, k, v)
    assert torch.allclose(out_ninf, base, atol=1e-6)
    z = torch.tensor([0.5, -1.0, 2.0, 0.0])
    _, wz = eager_attention(q, k, v, sinks=z)
    s = (q @ kr.transpose(-1, -2) * 128 ** -0.5).masked_fill(~causal, float("-inf"))
    den = torch.exp(s).sum(-1, keepdim=True)
    assert torch.allclose(wz, wb * den / (den + torch.exp(z).reshape(1, 4, 1, 1)), atol=1e-6)
    _, ww = eager_attention(q, k, v, sliding_window=4)
    pos_q, pos_k = torch.arange(3)[:, None] + 6, torch.arange(9)[None, :]
    keep = (pos_k <= pos_q) & (pos_q - pos_k < 4)
    assert torch.equal(ww[0, 0] > 0, keep)


def test_softcap_decode_steps_leave_the_kernels(cpu_cache):
    """A Gemma-2-style model (attention logit soft-capping): fused decode
    steps carry softcap, so they attend over the cache's dense K/V with the
    eager float32 attention instead of the kernels (on this CPU-only box a
    kernel call would raise). Nothing is compressed, so the logits match the
    model's own eager attention over a DynamicCache."""
    from transformers import DynamicCache, Gemma2Config, Gemma2ForCausalLM
    from turboquant_amd import apply_turboquant
    from turboquant_amd.hf import TurboQuantCache, TurboQuantLayer
    torch.manual_seed(8)
    cfg = Gemma2Config(vocab_size=97, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128, attn_logit_softcapping=5.0,
                       final_logit_softcapping=30.0, sliding_window=4096, query_pre_attn_scalar=128,
                       max_position_embeddings=1024)
    m = Gemma2ForCausalLM(cfg).eval()
    apply_turboquant(m, key_bits=4, value_bits=2, residual_window=256, auto_detect_outliers=False)
    ids = torch.randint(0, 97, (1, 30), generator=torch.Generator().manual_seed(9))
    m.set_attn_implementation("eager")
    with torch.no_grad():
        ref = run(m, DynamicCache(config=m.config), ids, 6)
    m.set_attn_implementation("turboquant")
    cache = TurboQuantCache(m, fused=True)
    assert any(isinstance(layer, TurboQuantLayer) and layer.fused for layer in cache.layers)
    with torch.no_grad():
        got = run(m, cache, ids, 6)
    assert torch.allclose(got, ref, atol=1e-4, rtol=1e-4)
