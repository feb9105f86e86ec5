"""tq_ragged_step (one launch per decode step of a ragged batch: the ring
appends and both sides' one-token drains, cache.py:396-427, 529-533, 620-706
per sequence) against the two-call path it replaces (tq_ring_append, then
tq_compress of each side over the rings: with a sketch through the drain
kernel, itself bit-identical to the general compress kernel in
test_gpu_drain.py; without one through the general compress kernel, whose
operations the step's drain performs): rings, codes, norms, signs, gamma and
the post-step length arrays bit for bit, and the attention over the two
batches equal, over steps that fill sinks, fill rings and drain, for a batch
whose ints travel in the kernel arguments and one (72 sequences) whose ints
take the copy.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


class _GeneralCompress:
    """A codec whose tq_compress calls take the general kernel."""

    def __init__(self, codec):
        self._codec = codec

    def ref(self, general_compress: bool = False):
        return self._codec.ref(True)

    def __getattr__(self, name):
        return getattr(self._codec, name)


def _batch(B, H, qjl_m, sink, window, lens, seed, fused, kb=4, vb=2):
    from turboquant_amd.ragged import RaggedKVBatch
    rb = RaggedKVBatch(B, H, 128, kb, vb, residual_window=window, fp16_sink_size=sink, qjl_n_proj=qjl_m, device=DEV)
    rb._fused = fused and rb._fused
    if qjl_m == 0:  # both batches load and (two-call path) drain through the general kernel
        rb.kc, rb.vc = _GeneralCompress(rb.kc), _GeneralCompress(rb.vc)
    g = torch.Generator(device=DEV).manual_seed(seed)
    for b, T in enumerate(lens):
        if T:
            rb.load(b, torch.randn(H, int(T), 128, generator=g, device=DEV).half(),
                    torch.randn(H, int(T), 128, generator=g, device=DEV).half())
    return rb


def _state(rb):
    out = {"ring_k": rb.ring_k, "ring_v": rb.ring_v, "sink_k": rb.sink_k, "sink_v": rb.sink_v}
    for side, st in (("k", rb.kstore), ("v", rb.vstore)):
        for name in ("codes_hi", "codes_lo", "norms", "signs", "gamma"):
            t = getattr(st, name)
            if t is not None:
                out[f"{side}.{name}"] = t
    return {k: v.cpu().numpy().copy() for k, v in out.items()}


@pytest.mark.parametrize("B,H,qjl_m,sink,window,lens,kb,vb", [
    (5, 2, 128, 4, 6, [9, 3, 0, 17, 6], 4, 2),    # sinks filling, rings filling and draining (ints in the arguments)
    (16, 8, 128, 0, 128, None, 4, 2),             # the configs[4] shape (window 128, no sink), shorter contexts
    (72, 1, 64, 2, 5, None, 4, 2),                # 576 ints: the copy path, m = 64
    (16, 8, 0, 0, 128, None, 4, 2),               # configs[4] without a sketch
    (6, 2, 0, 3, 7, [20, 2, 9, 40, 1, 13], 3.5, 2.5),  # fractional widths without a sketch
])
def test_ragged_step_matches_two_call_path(B, H, qjl_m, sink, window, lens, kb, vb):
    rng = np.random.RandomState(B + H)
    if lens is None:
        lens = rng.randint(window + 3, 3 * window + 40, size=B)
    lens = [int(x) for x in lens]
    # sequences start non-empty for attend(); the empty one is loaded with one token
    lens = [max(x, 1) for x in lens]
    a = _batch(B, H, qjl_m, sink, window, lens, 7, fused=True, kb=kb, vb=vb)
    b = _batch(B, H, qjl_m, sink, window, lens, 7, fused=False, kb=kb, vb=vb)
    assert a._fused and not b._fused
    g = torch.Generator(device=DEV).manual_seed(11)
    q = torch.randn(B, 4 * H, 128, generator=g, device=DEV).half()
    n_steps = window + sink + 3
    for s in range(n_steps):
        k = torch.randn(B, H, 128, generator=g, device=DEV).half()
        v = torch.randn(B, H, 128, generator=g, device=DEV).half()
        print(f"B={B} H={H} m={qjl_m} step {s}", flush=True)
        a.step(k, v)
        b.step(k, v)
        assert a._fused, "the fused step fell back"
        for name in ("sink_len", "comp_len", "res_len", "res_start", "offset"):
            assert np.array_equal(getattr(a, name), getattr(b, name)), name
        if s % 4 == 3 or s == n_steps - 1:
            torch.cuda.synchronize()
            sa, sb = _state(a), _state(b)
            for name in sa:
                assert np.array_equal(sa[name], sb[name]), f"step {s}: {name} differs"
            # the device length arrays the next attention call reads
            da, db = a._lens_staged, b._lens_staged
            assert da[0] == a._lens_ver and db[0] == b._lens_ver
            view = lambda staged, p: staged[(p - staged.data_ptr()) // 4:][:B].cpu().numpy()
            for name, pa, pb in zip(("comp_len", "sink_len", "res_len", "res_start"), da[1], db[1]):
                x, y = view(da[2], pa), view(db[2], pb)
                assert np.array_equal(x, y) and np.array_equal(x, getattr(a, name)), name
            oa = a.attend(q)
            ob = b.attend(q)
            torch.cuda.synchronize()
            assert torch.equal(oa, ob), f"step {s}: attention differs"
    assert int(a.comp_len.sum()) > int(sum(max(x - sink - window, 0) for x in lens))  # drains happened


@pytest.mark.parametrize("qjl_m", [128, 0])
def test_back_to_back_steps_match_synchronised_steps(qjl_m):
    """A decode loop with the host running ahead (step + attention per step,
    no synchronisation between steps, as the benchmark's back-to-back layer
    steps): every step's attention output equals that of a batch that
    synchronises after each step, bit for bit (the device length slots the
    step kernel writes alternate between steps and are read in stream order)."""
    B, H, window = 16, 8, 128
    lens = [int(x) for x in np.random.RandomState(5).randint(window + 3, 3 * window + 40, size=B)]
    a = _batch(B, H, qjl_m, 0, window, lens, 9, fused=True)
    b = _batch(B, H, qjl_m, 0, window, lens, 9, fused=True)
    g = torch.Generator(device=DEV).manual_seed(13)
    q = torch.randn(B, 4 * H, 128, generator=g, device=DEV).half()
    kv = [(torch.randn(B, H, 128, generator=g, device=DEV).half(), torch.randn(B, H, 128, generator=g, device=DEV).half())
          for _ in range(12)]
    torch.cuda.synchronize()
    print(f"m={qjl_m} back-to-back steps", flush=True)
    outs = []
    for k, v in kv:
        a.step(k, v)
        outs.append(a.attend(q))
    torch.cuda.synchronize()
    for s, (k, v) in enumerate(kv):
        b.step(k, v)
        ob = b.attend(q)
        torch.cuda.synchronize()
        assert torch.equal(outs[s], ob), f"step {s}: attention differs"
    assert a._fused and b._fused


@pytest.mark.parametrize("qjl_m", [128, 0])
def test_ragged_step_bf16_rings_through_the_abi(qjl_m):
    """tq_ragged_step called through the C ABI with bf16 keys, values and
    rings (RaggedKVBatch keeps fp16 ones): the rings equal a torch append
    (a token going to the sink, slot -1, is not appended), and the stores
    equal the general compress kernel's drain of the same ring slots, bit for
    bit (sequences without a drain write nothing)."""
    from test_gpu_drain import drain
    from turboquant_amd import _codec, _lib
    B, H, cap, D = 5, 3, 12, 128
    g = torch.Generator(device=DEV).manual_seed(23)
    rk = (torch.randn(B, H, cap, D, generator=g, device=DEV) * 2.0).bfloat16()
    rv = torch.randn(B, H, cap, D, generator=g, device=DEV).bfloat16()
    k = torch.randn(B, H, D, generator=g, device=DEV).bfloat16()
    v = torch.randn(B, H, D, generator=g, device=DEV).bfloat16()
    slot = np.array([3, -1, 0, 11, 7], np.int32)
    dr = np.array([1, 1, 0, 1, 1], np.int32)
    src = np.array([4, 9, 0, 2, 6], np.int32)
    dst = np.array([0, 5, 0, 17, 33], np.int32)
    ints = np.ascontiguousarray(np.concatenate([slot, dr, src, dst]))
    ints_dev = torch.zeros(ints.size, dtype=torch.int32, device=DEV)
    kc = _codec.get_codec(D, 4, 42, qjl_m, DEV)
    vc = _codec.get_codec(D, 2, 42, qjl_m, DEV)
    stores = []
    for c in (kc, vc):
        st = _codec.PackedStore(c, B, H, qjl=qjl_m > 0)
        st.reserve(64, 0)
        for name in ("codes_hi", "codes_lo", "norms", "signs", "gamma"):
            t = getattr(st, name)
            if t is not None:
                t.zero_()
        stores.append(st)
    ref_k = drain(kc, rk, dr, src, dst, H, general=True)
    ref_v = drain(vc, rv, dr, src, dst, H, general=True)
    exp_k, exp_v = rk.clone(), rv.clone()
    for b in range(B):
        if slot[b] >= 0:
            exp_k[b, :, slot[b]] = k[b]
            exp_v[b, :, slot[b]] = v[b]
    lib = _lib.load()
    kst, vst = stores[0].struct(0), stores[1].struct(0)
    print(f"m={qjl_m} bf16 ragged step", flush=True)
    _lib.check(lib.tq_ragged_step(kc.ref(), vc.ref(), k.data_ptr(), v.data_ptr(), _lib.TQ_BF16, rk.data_ptr(),
                                  rv.data_ptr(), cap * D, cap, ctypes.byref(kst), ctypes.byref(vst), B, H,
                                  ints.ctypes.data, ints.size, ints_dev.data_ptr(), _lib.stream_ptr(DEV)),
               "tq_ragged_step")
    torch.cuda.synchronize()
    assert torch.equal(rk, exp_k) and torch.equal(rv, exp_v)
    assert np.array_equal(ints_dev.cpu().numpy(), ints)
    for st, ref in zip(stores, (ref_k, ref_v)):
        for name in ("codes_hi", "codes_lo", "norms", "signs", "gamma"):
            t = getattr(st, name)
            if t is not None and t.numel():
                assert np.array_equal(t.cpu().numpy(), ref[name]), name


def test_stream_handle_is_torch_current_stream():
    """Launches go to torch's current stream (the raw handle query agrees with
    torch.cuda.current_stream, also inside a stream context)."""
    from turboquant_amd import _lib
    assert _lib.stream_ptr(DEV) == torch.cuda.current_stream(DEV).cuda_stream
    assert _lib.stream_ptr(torch.device("cuda")) == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(s):
        assert _lib.stream_ptr(DEV) == s.cuda_stream != 0
    assert _lib.stream_ptr(DEV) == torch.cuda.current_stream(DEV).cuda_stream
