"""The transformers integration on the GPU: a tiny random-init Llama (head_dim
128, 8 query heads on 4 kv heads, fp16) runs its own forward and decode loop
with TurboQuantCache and the "turboquant" attention function, so one-token
steps of the compressed layers go through the fused K4/V2 kernel. Decode
tokens are fixed in advance (teacher forcing) so the three runs see the same
inputs:
- fused attention against the same cache's dense path (update_and_fetch +
  SDPA, the reference's route): the same compressed tokens, so the logits
  agree to the kernels' precision;
- against an uncompressed DynamicCache run, the fused path is exactly as far
  off as the reference's dense route over the same compressed tokens (the
  approximation is the quantisation's, not the kernel's);
- while nothing is compressed yet, fused attention over the fp16 residual
  against SDPA.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")

DEV = torch.device("cuda", 0)


def tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=97, hidden_size=1024, intermediate_size=1536, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=4, head_dim=128, max_position_embeddings=2048)
    return LlamaForCausalLM(cfg).to(DEV, torch.float16).eval()


def run(model, cache, prompt, steps):
    """Prefill `prompt`, then feed `steps` (fixed tokens) one at a time;
    returns float32 logits of the prefill's last position and every step."""
    with torch.no_grad():
        out = model(prompt, past_key_values=cache, use_cache=True)
        logits = [out.logits[:, -1].float()]
        for i in range(steps.shape[1]):
            out = model(steps[:, i:i + 1], past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
    return torch.stack(logits)


def _tokens(n, seed):
    return torch.randint(0, 97, (1, n), generator=torch.Generator().manual_seed(seed)).to(DEV)


@pytest.mark.parametrize("prompt_len,window,sink", [(700, 64, 16), (300, 128, 0)])
def test_fused_decode_in_model(prompt_len, window, sink):
    from transformers import DynamicCache
    from turboquant_amd import apply_turboquant
    from turboquant_amd.hf import TurboQuantCache, TurboQuantLayer
    m = tiny_llama()
    apply_turboquant(m, key_bits=4, value_bits=2, residual_window=window, fp16_sink_size=sink,
                     auto_detect_outliers=False)
    prompt, steps = _tokens(prompt_len, 1), _tokens(40, 2)

    m.set_attn_implementation("sdpa")
    ref = run(m, DynamicCache(), prompt, steps)
    dense_cache = TurboQuantCache(m, fused=False)
    dense = run(m, dense_cache, prompt, steps)
    m.set_attn_implementation("turboquant")
    fused_cache = TurboQuantCache(m, fused=True)
    fused = run(m, fused_cache, prompt, steps)

    c = fused_cache.layers[0].cache
    assert isinstance(fused_cache.layers[0], TurboQuantLayer) and c._compressed_len > 0
    assert c.offset == prompt_len + 40 == dense_cache.layers[0].cache.offset
    cos = torch.nn.functional.cosine_similarity
    e_fd = ((fused - dense).norm(dim=-1) / dense.norm(dim=-1)).max().item()
    c_fr = cos(fused, ref, dim=-1)
    c_dr = cos(dense, ref, dim=-1)
    print(f"T={prompt_len}: fused vs dense path rel {e_fd:.2e}; vs uncompressed min cos fused {c_fr.min():.4f} "
          f"dense {c_dr.min():.4f}")
    assert torch.isfinite(fused).all()
    assert e_fd < 2e-2  # the dense path rounds dequantised K/V to fp16 before SDPA
    assert (c_fr - c_dr).abs().max().item() < 5e-3


@pytest.mark.parametrize("skip", [None, [1]], ids=["all_turboquant", "layer1_fp16"])
def test_fused_matches_sdpa_before_compression(skip):
    """Nothing compressed yet (and, with a skipped layer, an uncompressed
    FP16KVCache layer): the one-token steps run the dense decode kernel
    inside the model and match SDPA."""
    from transformers import DynamicCache
    from turboquant_amd import apply_turboquant
    from turboquant_amd.hf import TurboQuantCache, TurboQuantLayer
    from turboquant_amd.patch import FP16KVCache
    m = tiny_llama(seed=4)
    apply_turboquant(m, key_bits=4, value_bits=2, residual_window=512, auto_detect_outliers=False, skip_layers=skip)
    prompt, steps = _tokens(200, 5), _tokens(20, 6)
    m.set_attn_implementation("sdpa")
    ref = run(m, DynamicCache(), prompt, steps)
    m.set_attn_implementation("turboquant")
    cache = TurboQuantCache(m, fused=True)
    got = run(m, cache, prompt, steps)
    assert cache.layers[0].cache._compressed_len == 0
    if skip:
        assert isinstance(cache.layers[1], TurboQuantLayer) and isinstance(cache.layers[1].cache, FP16KVCache)
        assert cache.layers[1].fused and cache.layers[1].cache.offset == 220
    e = ((got - ref).norm(dim=-1) / ref.norm(dim=-1)).max().item()
    print(f"fp16 residual only (skip={skip}): fused vs SDPA rel {e:.2e}")
    assert e < 5e-3
