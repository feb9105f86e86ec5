#!/usr/bin/env python3
"""TurboQuant decode-attention / compress throughput on one MI355X.

Workload: Llama-3.1-8B-shaped single-token decode
attention, 32 layers with per-layer seeds, H_q=32, H_kv=8, D=128, context
T=32768 = 128-token fp16 sink + 32,512 packed K4/V2 tokens + 128-token fp16
residual window. Keys N(0,1) x per-channel LogNormal(0, 0.5), values N(0,1),
queries N(0,1) (fp16). One step = one fused decode-attention call per layer
over its compressed cache (32 calls), captured once in a HIP graph and
replayed; inputs are resident in HBM.

value = algorithmic bytes read per step / time per step (GB/s): packed codes +
norms of every compressed token, the fp16 sink/residual tokens, q and out.

roofline: the dominant kernel is the partials kernel of the two-kernel
K4/V2 path for uniform batches (uniform_decode_kernel<4>); its average duration is timed with events on
the launch stream around graph replays of one partials-only call
(tq_measure_decode_partials) per layer, so its bytes stream from HBM as in the
step (one layer's 28 MB would otherwise stay in the 256 MB last-level cache). traffic = HBM bytes per launch from rocprofv3
FETCH_SIZE / WRITE_SIZE runs of `bench.py --pmc-workload`, scaled by the
same counters on a copy of known size; read from the committed summary.

Also reported: compress throughput on configs[2] (131072-token prefill drained
in 4096-token chunks, K3/V2 and K3.5/V3.5), the roofline of the decode
attention call, the configs[3] 36-layer outlier-stress step (30 packed layers
+ 6 fp16 layers) and the configs[4] ragged layer-step (one-token drains +
attention over 16 sequences, with and without the QJL sketch), and a CPU
baseline (float32 numpy restatement of the reference's per-step path: dense
concat + SDPA) on a bounded sample.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mlx-turboquant_amd")]

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA peak of one MI355X (no sparsity)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "uniform_decode_kernel_k4v2_32k_traffic.md")
METRIC = "fused decode-attn GB/s over packed KV (% HBM peak) + compress vectors/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes_per_layer(c, hq: int) -> int:
    """Algorithmic bytes one decode-attention call reads/writes."""
    D = c.head_dim
    H = c._H * c._B
    per_tok = 0
    for codec in (c._kc, c._vc):
        per_tok += codec.row_hi + codec.row_lo + 4 + (codec.row_sign + 4 if c.qjl_correction else 0)
    packed = H * c._compressed_len * per_tok
    elt = 2 if c._dtype != __import__("torch").float32 else 4
    fp16 = H * (c._sink_len + c._fp16_len) * D * elt * 2
    return packed + fp16 + c._B * hq * D * 2 + c._B * hq * D * 4


def build_decode(layers: int, ctx: int, dev):
    import torch
    from turboquant_amd import TurboQuantKVCache
    caches, qs = [], []
    for l in range(layers):
        g = torch.Generator(device=dev).manual_seed(1000 + l)
        scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
        k = (torch.randn(1, 8, ctx, 128, generator=g, device=dev) * scale).half()
        v = torch.randn(1, 8, ctx, 128, generator=g, device=dev).half()
        c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=4, value_bits=2,
                              residual_window=128, fp16_sink_size=128)
        c.update(k, v)
        del k, v
        caches.append(c)
        qs.append(torch.randn(1, 32, 1, 128, generator=g, device=dev).half())
    torch.cuda.synchronize()
    return caches, qs


def time_graph(fn, reps: int, warmup: int):
    """Capture fn() in a graph, replay warmup + reps times; ms per replay."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    st.record()
    for _ in range(reps):
        g.replay()
    en.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / reps
    return st.elapsed_time(en) / reps, wall, g


def bench_layer_batched(dev, layers: int, ctx: int, reps: int, warmup: int):
    """The 32 layers' decode attention as ONE launch: a cache whose batch
    holds one configs[1]-shaped layer per sequence (same per-layer shapes and
    bytes), attended with one call. Not a decode step a model can take (layer
    l + 1's query needs layer l's output); it shows the per-launch fixed cost
    the per-layer figure pays."""
    import torch
    from turboquant_amd import TurboQuantKVCache
    g = torch.Generator(device=dev).manual_seed(3000)
    scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=4, value_bits=2, residual_window=128,
                          fp16_sink_size=128)
    k = (torch.randn(layers, 8, ctx, 128, generator=g, device=dev) * scale).half()
    v = torch.randn(layers, 8, ctx, 128, generator=g, device=dev).half()
    c.update(k, v)
    del k, v
    q = torch.randn(layers, 32, 1, 128, generator=g, device=dev).half()
    out = torch.empty(layers, 32, 1, 128, dtype=torch.float32, device=dev)
    ms, _, _ = time_graph(lambda: c.attend(q, out=out), reps, warmup)
    nbytes = decode_bytes_per_layer(c, 32)
    del c
    torch.cuda.empty_cache()
    return {"layers": layers, "us_per_launch": round(ms * 1e3, 3), "bytes": nbytes,
            "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel": "uniform_decode_kernel<4> + uniform_merge_kernel<4>, batch = layers"}


def bench_widths(dev, widths=((3, 2), (2, 2), (3, 3), (4, 3), (4, 4), (3.5, 3.5), (3.5, 2), (2.5, 2.5)), layers: int = 12,
                 reps: int = 20,
                 warmup: int = 5):
    """configs[1]'s layer shape (T = 32768: sink 128, 32512 packed, window
    128; Hq = 32, Hkv = 8) at the other widths: the integer ones on the
    uniform-batch MFMA kernels of those widths, the fractional K3.5/V3.5 on
    the split-codebook MFMA kernel; a graph of `layers` attend calls (whole
    call per layer) and of the partials kernel alone (HIP events). 12 layers,
    so the graph's bytes (300-450 MB) exceed the 256 MB last-level cache."""
    import torch
    from turboquant_amd import TurboQuantKVCache
    res = []
    for kb, vb in widths:
        caches, qs = [], []
        for l in range(layers):
            g = torch.Generator(device=dev).manual_seed(int(2000 + 10 * kb + vb + 100 * l))
            scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
            k = (torch.randn(1, 8, 32768, 128, generator=g, device=dev) * scale).half()
            v = torch.randn(1, 8, 32768, 128, generator=g, device=dev).half()
            c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=kb, value_bits=vb,
                                  residual_window=128, fp16_sink_size=128)
            c.update(k, v)
            del k, v
            caches.append(c)
            qs.append(torch.randn(1, 32, 1, 128, generator=g, device=dev).half())
        outs = [torch.empty(1, 32, 1, 128, dtype=torch.float32, device=dev) for _ in caches]

        def step():
            for c, q, o in zip(caches, qs, outs):
                c.attend(q, out=o)

        frac = not (float(kb).is_integer() and float(vb).is_integer())
        mfma = True  # every width of the list has a uniform-batch MFMA kernel
        ms, _, _ = time_graph(step, reps if mfma else 5, warmup if mfma else 2)
        byt = decode_bytes_per_layer(caches[0], 32)
        r = {"key_bits": kb, "value_bits": vb, "route": "split_decode_kernel" if frac else "uniform_decode_kernel",
             "bytes_per_layer": byt, "whole_call_us": round(ms * 1e3 / layers, 3),
             "GBps": round(byt / (ms / layers * 1e-3) / 1e9, 1)}
        if mfma:
            ms_k = time_partials_kernel(caches, qs, outs, reps, warmup)
            r.update({"partials_us": round(ms_k * 1e3, 3), "partials_GBps": round(byt / (ms_k * 1e-3) / 1e9, 1),
                      "partials_frac": round(byt / (ms_k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        res.append(r)
        del caches, qs, outs
        torch.cuda.empty_cache()
    return res


def bench_prefill(dev, ctx: int = 32768, n_qs=(128, 1024), reps: int = 10, warmup: int = 3):
    """Prefill attention at configs[1]'s layer shape (K4/V2, Hq 32, Hkv 8,
    D 128, sink 128, window 128): the cache's last n_q tokens attend causally
    over all ctx tokens (cache.py:722-724), on the query-tiled MFMA kernels
    (preparation + partials + merge, one attend call, in a graph). FLOPs are
    the algorithmic 4 * D per visible (query head, key) pair (QK^T and PV);
    the fraction is against the dense fp16 MFMA peak. One call of the general
    kernel (the route before the query-tiled kernels) is timed beside it."""
    import torch
    from turboquant_amd import TurboQuantKVCache
    g = torch.Generator(device=dev).manual_seed(4000)
    scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=4, value_bits=2, residual_window=128,
                          fp16_sink_size=128)
    k = (torch.randn(1, 8, ctx, 128, generator=g, device=dev) * scale).half()
    v = torch.randn(1, 8, ctx, 128, generator=g, device=dev).half()
    c.update(k, v)
    del k, v
    res = []
    for nq in n_qs:
        q = torch.randn(1, 32, nq, 128, generator=g, device=dev).half()
        out = torch.empty(1, 32, nq, 128, dtype=torch.float32, device=dev)
        ms, _, _ = time_graph(lambda: c.attend(q, out=out), reps, warmup)
        pairs = 32 * sum(ctx - nq + i + 1 for i in range(nq))
        flops = 4 * 128 * pairs
        tf = flops / (ms * 1e-3) / 1e12
        byt = decode_bytes_per_layer(c, 32) - 32 * 128 * 6 + 32 * nq * 128 * 6
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gen = torch.empty_like(out)
        c.attend(q, out=gen, general_kernel=True)
        torch.cuda.synchronize()
        st.record()
        c.attend(q, out=gen, general_kernel=True)
        en.record()
        torch.cuda.synchronize()
        ms_gen = st.elapsed_time(en)
        rel = float((out - gen).norm() / gen.norm())
        res.append({"n_q": nq, "ctx": ctx, "route": "prefill_kernel<4,2> (+ prep, merge)",
                    "ms_per_call": round(ms, 4), "query_tokens_per_s": round(nq / (ms * 1e-3), 1),
                    "algorithmic_TFLOPs": round(tf, 2), "mfma_peak_TFLOPs": MFMA_F16_PEAK_TFLOPS,
                    "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "bytes": byt,
                    "GBps": round(byt / (ms * 1e-3) / 1e9, 1),
                    "general_kernel_ms": round(ms_gen, 3), "speedup_vs_general": round(ms_gen / ms, 1),
                    "rel_diff_vs_general": rel})
        del q, out, gen
    del c
    torch.cuda.empty_cache()
    return res


def bench_compress(dev, kb, vb, total=131072, chunk=4096, reps=3):
    import torch
    from turboquant_amd import TurboQuantKVCache
    g = torch.Generator(device=dev).manual_seed(7)
    scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
    k = (torch.randn(1, 8, total, 128, generator=g, device=dev) * scale).half()
    v = torch.randn(1, 8, total, 128, generator=g, device=dev).half()
    times = []
    for _ in range(reps + 1):
        c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=kb, value_bits=vb,
                              residual_window=128, chunk_size=chunk)
        c._setup(k)
        c._kstore.reserve(total, 0)
        c._vstore.reserve(total, 0)
        torch.cuda.synchronize()
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        c.update(k, v)
        en.record()
        torch.cuda.synchronize()
        times.append(st.elapsed_time(en))
    ms = sorted(times[1:])[len(times[1:]) // 2]
    n_vec = 2 * 8 * c._compressed_len
    per_vec = 256 + (c._kc.row_hi + c._kc.row_lo + 4 + c._vc.row_hi + c._vc.row_lo + 4) / 2
    return {"bits": f"K{kb}/V{vb}", "tokens": c._compressed_len, "vectors": n_vec, "ms": round(ms, 4),
            "vectors_per_s": n_vec / (ms * 1e-3), "GBps": n_vec * per_vec / (ms * 1e-3) / 1e9}


def bench_config3(dev, reps: int = 5, warmup: int = 2):
    """one decode step of a 36-layer Qwen3-8B-shaped model
    (Hq=32, Hkv=8, D=128) at T=65536 where the outlier rule kept 6 seeded
    layers in fp16: 30 fused K4/V2 attend calls (sink 128, window 128) and 6
    dense decode-attention calls over the fp16 K/V of an FP16KVCache (the
    reference hands outlier layers a plain KVCache and runs its SDPA on
    them). Captured in a HIP graph."""
    import numpy as np
    import torch
    from turboquant_amd import TurboQuantKVCache
    from turboquant_amd.patch import FP16KVCache
    layers, T = 36, 65536
    fp16_layers = set(np.random.RandomState(3).choice(layers, 6, replace=False).tolist())
    caches, kvs, qs, outs = [], [], [], []
    for l in range(layers):
        g = torch.Generator(device=dev).manual_seed(2000 + l)
        k = torch.randn(1, 8, T, 128, generator=g, device=dev).half()
        v = torch.randn(1, 8, T, 128, generator=g, device=dev).half()
        if l in fp16_layers:
            f = FP16KVCache()
            f.update(k, v)
            del k, v
            caches.append(None)
            kvs.append(f)
        else:
            c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=4, value_bits=2,
                                  residual_window=128, fp16_sink_size=128)
            c.update(k, v)
            del k, v
            caches.append(c)
            kvs.append(None)
        qs.append(torch.randn(1, 32, 1, 128, generator=g, device=dev).half())
        outs.append(torch.empty(1, 32, 1, 128, dtype=torch.float32, device=dev))

    def run(packed=True, fp16=True):
        def fn():
            for c, kv, q, o in zip(caches, kvs, qs, outs):
                if c is not None and packed:
                    c.attend(q, out=o)
                elif kv is not None and fp16:
                    kv.attend(q, out=o)
        return fn

    ms, _, _ = time_graph(run(), reps, warmup)
    ms_p, _, _ = time_graph(run(fp16=False), reps, warmup)
    ms_f, _, _ = time_graph(run(packed=False), reps, warmup)
    b_packed = sum(decode_bytes_per_layer(c, 32) for c in caches if c is not None)
    b_fp16 = len(fp16_layers) * (2 * 8 * T * 128 * 2 + 32 * 128 * 2 * 2)
    return {"workload": "configs[3]: 36 layers, Hq=32 Hkv=8 D=128, T=65536; 30 K4/V2 layers (sink 128, window "
                        "128) through the fused attend, 6 fp16 outlier layers through the dense decode kernel; "
                        "one graph",
            "ms_per_step": round(ms, 4), "bytes_per_step": b_packed + b_fp16,
            "GBps": round((b_packed + b_fp16) / (ms * 1e-3) / 1e9, 1),
            "packed_layers_ms": round(ms_p, 4), "packed_GBps": round(b_packed / (ms_p * 1e-3) / 1e9, 1),
            "fp16_layers_ms": round(ms_f, 4), "fp16_GBps": round(b_fp16 / (ms_f * 1e-3) / 1e9, 1)}


def bench_config4(dev, steps: int = 12):
    """one layer-step of 16 ragged Llama-3.1-8B-shaped sequences
    (lengths ~ U[4096, 32768], seeded), K4/V2, the reference's defaults
    (window 128, no sink): append one token per sequence, drain one per
    sequence into the packed store (appends and both sides' drains in one
    tq_ragged_step launch), fused decode attention over every sequence in
    one call. With the QJL sketch (m = 128) the K4/V2
    kernels run with the sketch's key and value terms around them; without
    it the K4/V2 kernels alone. Eager launches: one event pair around a
    layer step (it includes the host's launch overhead when the GPU waits
    for it), alternating with steps whose attention call alone is timed;
    then 8 attention calls back to back between two events, the GPU time of
    one call with the host running ahead; then 8 layer steps back to back
    between two events (a decode loop's steady state: the host prepares
    step n + 1 while the GPU runs step n; the stores' capacity is reserved
    beforehand, as their geometric growth leaves it on almost every step)."""
    import numpy as np
    import torch
    from turboquant_amd.ragged import RaggedKVBatch
    lens = np.random.RandomState(4).randint(4096, 32769, size=16)
    res = {"workload": "configs[4]: 16 ragged sequences ~U[4096,32768], Hq=32 Hkv=8 D=128, K4/V2, window 128, "
                       "no sink; per layer-step: one-token drain per sequence + one attention launch"}
    for qjl_m in (128, 0):
        rb = RaggedKVBatch(16, 8, 128, 4, 2, residual_window=128, fp16_sink_size=0, qjl_n_proj=qjl_m, device=dev)
        g = torch.Generator(device=dev).manual_seed(5)
        for b, T in enumerate(lens):
            rb.load(b, torch.randn(8, int(T), 128, generator=g, device=dev).half(),
                    torch.randn(8, int(T), 128, generator=g, device=dev).half())
        q = torch.randn(16, 32, 128, generator=g, device=dev).half()
        out = torch.empty(16, 32, 128, dtype=torch.float32, device=dev)
        kv = [(torch.randn(16, 8, 128, generator=g, device=dev).half(),
               torch.randn(16, 8, 128, generator=g, device=dev).half()) for _ in range(2 * steps + 2)]
        t_step, t_attn = [], []
        for i, (k, v) in enumerate(kv):
            # even iterations time the layer step (one event pair around it),
            # odd ones the attention call alone after an untimed step
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            if i % 2 == 0:
                e0.record()
                rb.step(k, v)
                rb.attend(q, out=out)
                e1.record()
            else:
                rb.step(k, v)
                e0.record()
                rb.attend(q, out=out)
                e1.record()
            torch.cuda.synchronize()
            if i >= 2:
                (t_step if i % 2 == 0 else t_attn).append(e0.elapsed_time(e1))
        rep = 8
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(rep):
            rb.attend(q, out=out)
        e1.record()
        torch.cuda.synchronize()
        ms_b = e0.elapsed_time(e1) / rep
        kv = [(torch.randn(16, 8, 128, generator=g, device=dev).half(),
               torch.randn(16, 8, 128, generator=g, device=dev).half()) for _ in range(rep + 1)]
        for st in (rb.kstore, rb.vstore):
            st.reserve(int(rb.comp_len.max()) + rep + 2, int(rb.comp_len.max()))
        rb.step(*kv[0])
        rb.attend(q, out=out)
        torch.cuda.synchronize()
        e0.record()
        for k, v in kv[1:]:
            rb.step(k, v)
            rb.attend(q, out=out)
        e1.record()
        torch.cuda.synchronize()
        ms_lb = e0.elapsed_time(e1) / rep
        per_tok = sum(c.row_hi + c.row_lo + 4 + (c.row_sign + 4 if qjl_m else 0) for c in (rb.kc, rb.vc))
        byt = 8 * (int(rb.comp_len.sum()) * per_tok + int(rb.res_len.sum()) * 512) + 16 * 32 * 128 * 6
        ms_s, ms_a = float(np.median(t_step)), float(np.median(t_attn))
        res["qjl" if qjl_m else "no_qjl"] = {
            "kernel": ("K4/V2 + sketch (decode_partials_kernel computing S q and the key term from the sketch, "
                       "qjl_value_kernel, merge adding the value term; the step in one tq_ragged_step launch)") if qjl_m
                      else "K4/V2 (decode_partials_kernel + merge; the step in one tq_ragged_step launch)",
            "layer_step_us": round(ms_s * 1e3, 1), "layer_step_back_to_back_us": round(ms_lb * 1e3, 1),
            "attend_us": round(ms_a * 1e3, 1),
            "attend_bytes": byt, "attend_GBps": round(byt / (ms_a * 1e-3) / 1e9, 1),
            "attend_back_to_back_us": round(ms_b * 1e3, 1),
            "attend_back_to_back_GBps": round(byt / (ms_b * 1e-3) / 1e9, 1)}
        del rb
    return res


def cpu_baseline(caches, qs, budget_s: float = 12.0):
    """Reference per-step CPU work for one layer (concat + SDPA, float32
    numpy/OpenBLAS), repeated within a time budget, scaled to a 32-layer step."""
    import numpy as np
    import oracle as O
    c = caches[0]
    kd, vd = c.fetch()
    S, C = c._sink_len, c._compressed_len
    deq_k = kd[:, :, S:S + C].cpu().numpy()
    deq_v = vd[:, :, S:S + C].cpu().numpy()
    sk, sv = c.sink_keys[:, :, :S].cpu().numpy(), c.sink_values[:, :, :S].cpu().numpy()
    rk, rv = [t.cpu().numpy() for t in c._residual_linear()]
    q = qs[0].cpu().numpy()
    del kd, vd
    c._dense_k = c._dense_v = None
    c._dense_comp = c._dense_sink = 0
    O.reference_decode_step_f32(sk, sv, deq_k, deq_v, rk, rv, q)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        O.reference_decode_step_f32(sk, sv, deq_k, deq_v, rk, rv, q)
        times.append(time.perf_counter() - t0)
    per_layer = float(np.median(times))
    try:
        from threadpoolctl import threadpool_info
        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:
        threads = len(os.sched_getaffinity(0))
    # compress sample: 65536 fp16 vectors at 3 bits (configs[2] keys), the
    # median of 5 timed runs after a warm-up
    x = np.random.RandomState(0).randn(65536, 128).astype(np.float16)
    R = O.rotation_matrix(128)
    O.compress_f32(x[:1024], R, 3)
    t_c = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.compress_f32(x, R, 3)
        t_c.append(time.perf_counter() - t0)
    return per_layer, threads, len(times), 65536 / float(np.median(t_c)), len(t_c)


def hbm_reference(dev, bytes_layer: int, layers: int = 32, reps: int = 20):
    """The box's achievable HBM bandwidth, the reference for the decode
    figures: (a) a 268,435,456-byte device-to-device copy (torch copy_, read +
    write bytes counted), median of `reps` timed copies; (b) the library's
    streaming read kernel (tq_measure_read) over one decode layer's worth of
    bytes (bytes_layer), one launch per layer buffer, `layers` distinct buffers
    in one graph (so the bytes come from HBM, not the 256 MB last-level
    cache), HIP events around the replays; (c) the same kernel over one
    268,435,456-byte buffer."""
    import ctypes
    import numpy as np
    import torch
    from turboquant_amd import _lib
    lib = _lib.load()
    fn = lib.tq_measure_read  # measurement hook of the library (not in include/tq_abi.h)
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    t = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        t.append(e0.elapsed_time(e1))
    ms_copy = float(np.median(t))
    del dst
    nwg = 4096
    sink = torch.empty(nwg, dtype=torch.float32, device=dev)
    nb = (bytes_layer + 15) // 16 * 16
    bufs = [torch.ones(nb // 4, dtype=torch.float32, device=dev) for _ in range(layers)]

    def reads():
        for b in bufs:
            _lib.check(fn(b.data_ptr(), nb, sink.data_ptr(), nwg, _lib.stream_ptr(dev)), "tq_measure_read")

    ms_layers, _, _ = time_graph(reads, reps, 5)
    ms_one, _, _ = time_graph(lambda: _lib.check(fn(src.data_ptr(), n, sink.data_ptr(), nwg, _lib.stream_ptr(dev)),
                                                 "tq_measure_read"), reps, 5)
    del bufs, src
    torch.cuda.empty_cache()
    us_layer = ms_layers * 1e3 / layers
    return {"copy_bytes": n, "copy_us": round(ms_copy * 1e3, 2),
            "copy_GBps": round(2 * n / (ms_copy * 1e-3) / 1e9, 1),
            "read_bytes_per_launch": nb, "read_us_per_launch": round(us_layer, 3),
            "read_GBps": round(nb / (us_layer * 1e-6) / 1e9, 1),
            "read_256MB_us": round(ms_one * 1e3, 2), "read_256MB_GBps": round(n / (ms_one * 1e-3) / 1e9, 1),
            "method": "copy: torch copy_ of 256 MiB, median of events, read + write bytes; read: tq_measure_read "
                      "(4096 workgroups x 256 threads, 16-byte nontemporal loads) over one decode layer's bytes, "
                      f"{layers} distinct buffers in one graph, and over one 256 MiB buffer"}


def call_partials_only(c, q, out):
    """One attention call that launches only the partials kernel."""
    import ctypes
    import torch
    from turboquant_amd import _lib
    from turboquant_amd.cache import _workspace
    lib = _lib.load()
    fn = lib.tq_measure_decode_partials  # measurement hook of the library (not in include/tq_abi.h)
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_size_t, ctypes.c_void_p]
    qq = q[:, :, 0].contiguous()
    desc = c.attention_descriptor(qq, out, q.shape[-1] ** -0.5)
    need = lib.tq_decode_workspace_bytes(c._kc.ref(), ctypes.byref(desc))
    ws = _workspace(q.device, need)
    _lib.check(fn(ctypes.addressof(c._kc.struct), ctypes.addressof(c._vc.struct), ctypes.addressof(desc),
                  ws.data_ptr(), ws.numel(), _lib.stream_ptr(q.device)), "tq_measure_decode_partials")


def time_partials_kernel(caches, qs, outs, reps: int, warmup: int):
    """Average duration (ms) of one launch of the partials kernel under the
    step's streaming conditions: a graph of one partials-only call per layer
    (each layer's cache, so the step's bytes come from HBM as in the step),
    replayed `reps` times between two events on the launch stream (torch's
    current stream, which the library is handed)."""
    import torch

    def fn():
        for c, q, o in zip(caches, qs, outs):
            call_partials_only(c, q, o)

    ms, _, _ = time_graph(fn, reps, warmup)
    return ms / len(caches)


def read_traffic():
    """HBM bytes per launch of the partials kernel from the committed counter
    summary (line 'traffic_bytes_per_launch: N'), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def pmc_workload(ctx: int):
    """Short program for the counter runs: a copy of known size (the scale of
    FETCH_SIZE / WRITE_SIZE), then 20 partials-kernel launches of layer 0, then
    10 dense decode calls over a configs[3] fp16 layer (65536 tokens)."""
    import torch
    from turboquant_amd import _lib
    _lib.load()
    dev = torch.device("cuda", 0)
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    caches, qs = build_decode(1, ctx, dev)
    out = torch.empty(1, 32, 1, 128, dtype=torch.float32, device=dev)
    for _ in range(20):
        call_partials_only(caches[0], qs[0], out)
    torch.cuda.synchronize()
    del caches
    from turboquant_amd.patch import FP16KVCache
    g = torch.Generator(device=dev).manual_seed(2000)
    f = FP16KVCache()
    f.update(torch.randn(1, 8, 65536, 128, generator=g, device=dev).half(),
             torch.randn(1, 8, 65536, 128, generator=g, device=dev).half())
    q = torch.randn(1, 32, 1, 128, generator=g, device=dev).half()
    for _ in range(10):
        f.attend(q, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "partials_launches": 20, "dense_launches": 10,
                      "dense_bytes_per_launch": 8 * 65536 * 512 + 32 * 128 * 2}), flush=True)


def pmc_compress_workload():
    """Short program for the compress counter runs: the copy of known size,
    then the configs[2] K3/V2 prefill (131,072 tokens in 4096-token chunks)
    twice, the second on warm codecs."""
    import torch
    from turboquant_amd import _lib
    _lib.load()
    dev = torch.device("cuda", 0)
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst
    r = bench_compress(dev, 3, 2, reps=1)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "compress": r}), flush=True)


def pmc_prefill_workload(n_q: int = 1024):
    """Short program for the prefill kernel trace and counter runs: one
    configs[1]-shaped K4/V2 layer (T = 32768), 5 attend calls of its last n_q
    tokens (causal)."""
    import torch
    from turboquant_amd import TurboQuantKVCache
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(4000)
    scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=4, value_bits=2, residual_window=128,
                          fp16_sink_size=128)
    c.update((torch.randn(1, 8, 32768, 128, generator=g, device=dev) * scale).half(),
             torch.randn(1, 8, 32768, 128, generator=g, device=dev).half())
    q = torch.randn(1, 32, n_q, 128, generator=g, device=dev).half()
    out = torch.empty(1, 32, n_q, 128, dtype=torch.float32, device=dev)
    for _ in range(5):
        c.attend(q, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"prefill_calls": 5, "n_q": n_q, "ctx": 32768}), flush=True)


def pmc_general_workload():
    """Short program for the general kernel's counter runs: one configs[1]-
    shaped K3.5/V3.5 layer (T = 32768) on the general route (chunk_kernel),
    5 decode calls."""
    import torch
    from turboquant_amd import TurboQuantKVCache
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(4100)
    scale = torch.exp(torch.randn(128, generator=g, device=dev) * 0.5)
    c = TurboQuantKVCache(head_dim=128, num_kv_heads=8, key_bits=3.5, value_bits=3.5, residual_window=128,
                          fp16_sink_size=128)
    c.update((torch.randn(1, 8, 32768, 128, generator=g, device=dev) * scale).half(),
             torch.randn(1, 8, 32768, 128, generator=g, device=dev).half())
    q = torch.randn(1, 32, 1, 128, generator=g, device=dev).half()
    out = torch.empty(1, 32, 1, 128, dtype=torch.float32, device=dev)
    for _ in range(5):
        c.attend(q, out=out, general_kernel=True)
    torch.cuda.synchronize()
    print(json.dumps({"general_calls": 5, "ctx": 32768, "bits": 3.5}), flush=True)


def pmc_config4_workload(steps: int = 4, calls: int = 5):
    """Short program for the configs[4] kernel trace and counter runs: the
    16-sequence ragged K4/V2 batch with the 128-projection sketch (lengths
    ~ U[4096, 32768], seeded as in bench_config4), `steps` decode steps, then
    `calls` attention calls."""
    import numpy as np
    import torch
    from turboquant_amd.ragged import RaggedKVBatch
    dev = torch.device("cuda", 0)
    lens = np.random.RandomState(4).randint(4096, 32769, size=16)
    rb = RaggedKVBatch(16, 8, 128, 4, 2, residual_window=128, fp16_sink_size=0, qjl_n_proj=128, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    for b, T in enumerate(lens):
        rb.load(b, torch.randn(8, int(T), 128, generator=g, device=dev).half(),
                torch.randn(8, int(T), 128, generator=g, device=dev).half())
    for _ in range(steps):
        rb.step(torch.randn(16, 8, 128, generator=g, device=dev).half(),
                torch.randn(16, 8, 128, generator=g, device=dev).half())
    q = torch.randn(16, 32, 128, generator=g, device=dev).half()
    out = torch.empty(16, 32, 128, dtype=torch.float32, device=dev)
    for _ in range(calls):
        rb.attend(q, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"config4_calls": calls}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-compress", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the configs[3] / configs[4] timings")
    ap.add_argument("--pmc-workload", action="store_true", help="short program for rocprofv3 --pmc runs")
    ap.add_argument("--pmc-compress", action="store_true", help="short compress program for rocprofv3 --pmc runs")
    ap.add_argument("--pmc-prefill", action="store_true", help="short prefill program for rocprofv3 runs")
    ap.add_argument("--pmc-general", action="store_true", help="short general-kernel program for rocprofv3 runs")
    ap.add_argument("--pmc-config4", action="store_true", help="short configs[4] program for rocprofv3 runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)

    if args.pmc_workload:
        pmc_workload(args.ctx)
        return
    if args.pmc_compress:
        pmc_compress_workload()
        return
    if args.pmc_prefill:
        pmc_prefill_workload()
        return
    if args.pmc_general:
        pmc_general_workload()
        return
    if args.pmc_config4:
        pmc_config4_workload()
        return

    import torch
    from turboquant_amd import _lib
    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    log(f"building {args.layers} layer caches, ctx {args.ctx}")
    caches, qs = build_decode(args.layers, args.ctx, dev)
    outs = [torch.empty(1, 32, 1, 128, dtype=torch.float32, device=dev) for _ in caches]
    bytes_layer = [decode_bytes_per_layer(c, 32) for c in caches]
    bytes_step = sum(bytes_layer)

    def step():
        for c, q, o in zip(caches, qs, outs):
            c.attend(q, out=o)

    log("timing decode step")
    ms_step, wall_step, _ = time_graph(step, args.steps, args.warmup)
    # the partials kernel alone, one launch per layer per replay
    ms_kernel = time_partials_kernel(caches, qs, outs, args.steps, args.warmup)
    gbps = bytes_step / (ms_step * 1e-3) / 1e9
    ach = bytes_layer[0] / (ms_kernel * 1e-3) / 1e9
    traffic = read_traffic()

    result = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (fp16 high part + remainder operands), f32 accumulate",
        "data": "synthetic (seeded N(0,1) keys x LogNormal(0,0.5) channel scale, N(0,1) values/queries)",
        "config": {"workload": "configs[1]: Llama-3.1-8B decode attention, T=32768 = 128 sink + 32512 K4/V2 "
                               "+ 128 residual, 32 layers, Hq=32 Hkv=8 D=128, per-layer fused attend in a HIP graph",
                   "layers": args.layers, "ctx": args.ctx, "key_bits": 4, "value_bits": 2},
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBS, 2),
        "decode_steps_per_s": round(1e3 / ms_step, 2),
        "wall_ms_per_step": round(wall_step, 5),
        "bytes_per_step": bytes_step,
        "roofline": {"kernel": "uniform_decode_kernel<4> (partials of one layer: q rotation, packed K4/V2 + fp16 "
                               "blocks, workgroup combine; the merge kernel applies the inverse rotation)",
                     "bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if traffic else None,
                     "bytes_per_launch": bytes_layer[0], "avg_launch_us": round(ms_kernel * 1e3, 3),
                     "whole_call_us": round(ms_step * 1e3 / len(caches), 3)},
    }
    log("measuring the box's HBM reference bandwidth")
    result["hbm_reference"] = hbm_reference(dev, bytes_layer[0], args.layers, args.steps)
    if not args.no_extra:
        log("timing the layer-batched launch")
        result["layer_batched"] = bench_layer_batched(dev, args.layers, args.ctx, args.steps, args.warmup)
    if not args.no_extra:
        log("timing the other integer widths")
        result["widths"] = bench_widths(dev)
    if not args.no_extra:
        log("timing prefill attention")
        result["prefill"] = bench_prefill(dev)
    if not args.no_compress:
        log("timing compress")
        del outs
        comp = [bench_compress(dev, 3, 2), bench_compress(dev, 3.5, 3.5)]
        result["compress"] = comp
        result["compress_vectors_per_s"] = round(comp[0]["vectors_per_s"], 1)
    if not args.no_extra:
        log("timing configs[3] and configs[4]")
        result["config3"] = bench_config3(dev)
        torch.cuda.empty_cache()
        result["config4"] = bench_config4(dev)
        torch.cuda.empty_cache()
    if not args.no_cpu:
        log("timing CPU baseline")
        per_layer, threads, n, cpu_vps, n_c = cpu_baseline(caches, qs)
        cpu_step = per_layer * args.layers
        result["cpu_baseline"] = {
            "value": round(bytes_step / cpu_step / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"float32 numpy restatement of the reference decode step (concat [sink|dequantised|residual] "
                      f"+ SDPA) for layer 0, median of {n} runs x {args.layers} layers; "
                      f"compress: 65536 vectors K3 f32 norm+GEMM+quantize+pack, median of {n_c} runs",
            "ms_per_step": round(cpu_step * 1e3, 3), "compress_vectors_per_s": round(cpu_vps, 1),
            "cores_note": "cores = OpenBLAS threads the numpy GEMMs ran with (threadpoolctl)",
            "affinity_cores": len(os.sched_getaffinity(0)),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS")}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
