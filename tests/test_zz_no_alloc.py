"""The allocation-free entry point gh_qkv_rope_attn_noalloc against
gh_qkv_rope_attn, the entry point it varies: the same kernels on the same
inputs, so the outputs and cache rows must be identical bits.  Two calls in a
row (the second smaller: fewer slots and a smaller head shape) check that the
shared device array carries nothing over, and a captured graph replayed
between eager calls checks the use it exists for."""
import numpy as np
import pytest

import gemma_hip as gh

pytestmark = pytest.mark.gpu


def _case(gpu, nq, nkv, D, slots, S, clock, seed):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    kc, vc = f(slots, nkv * D), f(slots, nkv * D)
    slot = clock % slots
    active = rng.permutation(slots)[:S].astype(np.uint32)
    if slot not in active:
        active[0] = slot
    host = dict(q=f(nq * D), k=f(nkv * D), v=f(nkv * D), qn=1 + 0.1 * f(D), kn=1 + 0.1 * f(D),
                active=active, step=np.array([clock, slot, S, 0], np.uint32))
    dev = {n: gpu.upload(a) for n, a in host.items()}
    return kc, vc, dev


def _run(gpu, fn, kc, vc, dev, nq, nkv, D, rot, theta):
    KC, VC, O = gpu.upload(kc), gpu.upload(vc), gpu.alloc(nq * D * 4)
    fn(dev["q"], dev["k"], dev["v"], dev["qn"], dev["kn"], KC, VC, dev["active"], dev["step"], O,
       nq, nkv, D, rot, False, theta)
    gpu.sync()
    return O.read(np.float32, nq * D), KC.read(np.float32), VC.read(np.float32)


def test_noalloc_matches_allocating_entry(gpu):
    for nq, nkv, D, slots, S, clock, rot, theta in ((16, 8, 256, 640, 544, 600, 256, 1e4),
                                                    (8, 4, 128, 100, 37, 41, 32, 1e6)):
        kc, vc, dev = _case(gpu, nq, nkv, D, slots, S, clock, seed=S)
        ref = _run(gpu, gpu.qkv_rope_attn, kc, vc, dev, nq, nkv, D, rot, theta)
        got = _run(gpu, gpu.qkv_rope_attn_noalloc, kc, vc, dev, nq, nkv, D, rot, theta)
        for a, b in zip(got, ref):
            assert np.array_equal(a, b)
        assert np.all(np.isfinite(got[0]))


def test_noalloc_refuses_oversized_partials(gpu):
    # 16 kv heads of 512 with 4 query heads each: 16 * 16 * 4 * 516 * 4 bytes
    # of partials at 640 slots, above the 1 MiB array
    dummy = gpu.alloc(1 << 16)
    with pytest.raises(gh.GhError, match="1 MiB"):
        gpu.qkv_rope_attn_noalloc(dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                                  dummy, 64, 16, 512, 128, False, 1e4)


def test_noalloc_under_graph_capture(gpu):
    nq, nkv, D, slots, S, clock = 16, 8, 256, 640, 300, 299
    kc, vc, dev = _case(gpu, nq, nkv, D, slots, S, clock, seed=7)
    ref = _run(gpu, gpu.qkv_rope_attn, kc, vc, dev, nq, nkv, D, 64, 1e6)
    KC, VC, O = gpu.upload(kc), gpu.upload(vc), gpu.alloc(nq * D * 4)
    gpu.graph_begin()
    gpu.qkv_rope_attn_noalloc(dev["q"], dev["k"], dev["v"], dev["qn"], dev["kn"], KC, VC,
                              dev["active"], dev["step"], O, nq, nkv, D, 64, False, 1e6)
    g = gpu.graph_end()
    try:
        for rep in range(3):
            gpu.graph_launch(g)
            gpu.sync()
            assert np.array_equal(O.read(np.float32, nq * D), ref[0]), rep
            # eager work on the same array between replays
            kc2, vc2, dev2 = _case(gpu, 8, 4, 128, 100, 37, 41, seed=rep)
            _run(gpu, gpu.qkv_rope_attn_noalloc, kc2, vc2, dev2, 8, 4, 128, 32, 1e6)
    finally:
        gpu.graph_destroy(g)
