"""GPU parity of the norm, RoPE/cache-write, decode-attention and argmax
kernels against the oracle, through the C ABI."""
import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc
from tol import assert_close

pytestmark = pytest.mark.gpu


def bf16_round(a):
    return nr.bf16_to_f32(nr.bf16_rne(a))


# ---------------------------------------------------------------- norms ----
def test_rmsnorm_reference_suite_case(gpu):
    # src/test_gpu_suite.zig:62-101: D = 2048, x = (u - 0.5) * 2, w = 1 + (u - 0.5) * 0.1
    # truncated to bf16; GPU vs CPU abs error < 1e-4.
    rng = np.random.default_rng(202)
    D = 2048
    x = ((rng.random(D, dtype=np.float32) - 0.5) * 2).astype(np.float32)
    wf = (1 + (rng.random(D, dtype=np.float32) - 0.5) * 0.1).astype(np.float32)
    w = ((wf.view(np.uint32) >> 16) << 16).view(np.float32)
    X, W, Y = gpu.upload(x), gpu.upload(w), gpu.alloc(D * 4)
    gpu.rmsnorm(X, W, Y, D, 1e-6)
    y = Y.read(np.float32, D)
    ref = orc.rmsnorm(x, w, 1e-6)
    assert np.max(np.abs(y - ref)) < 1e-4
    assert_close(y, ref, what="rmsnorm")


@pytest.mark.parametrize("dim", [3840, 256, 5])
def test_add_rmsnorm(gpu, dim):
    x = gh.synth_normal(dim, 0, 60, 0.0, 3.0)
    r = gh.synth_normal(dim, 0, 61, 0.0, 1.0)
    w = bf16_round(gh.synth_normal(dim, 0, 62, 1.0, 0.1))
    X, R, W, Y = gpu.upload(x), gpu.upload(r), gpu.upload(w), gpu.alloc(dim * 4)
    gpu.add_rmsnorm(X, R, W, Y, dim, 1e-6, 0.75)
    xn = ((x + r) * np.float32(0.75)).astype(np.float32)
    assert_close(X.read(np.float32, dim), xn, what="add_rmsnorm x")
    assert_close(Y.read(np.float32, dim), orc.rmsnorm(xn, w), what="add_rmsnorm y")


# ------------------------------------------------------------ qkv + RoPE ----
ROPE_CASES = [(64, 10000.0), (256, 10000.0), (64, 1e6)]  # stated case, sliding, full layers
CLOCKS = [0, 31, 32, 543, 544, 639, 1000]


@pytest.mark.parametrize("rot,theta", ROPE_CASES)
@pytest.mark.parametrize("k_eq_v", [False, True])
def test_qkv_rope_and_cache_write(gpu, rot, theta, k_eq_v):
    nq, nkv, D, slots = 16, 8, 256, 640
    ring = orc.Ring(1, nkv * D, 32, 512, 96)
    qn = bf16_round(gh.synth_normal(D, 0, 70, 1.0, 0.1))
    kn = bf16_round(gh.synth_normal(D, 0, 71, 1.0, 0.1))
    QN, KN = gpu.upload(qn), gpu.upload(kn)
    KC, VC = gpu.alloc(slots * nkv * D * 4), gpu.alloc(slots * nkv * D * 4)
    gpu.fill_u32(KC, 0, slots * nkv * D)
    gpu.fill_u32(VC, 0, slots * nkv * D)
    kc_ref = np.zeros((slots, nkv * D), np.float32)
    vc_ref = np.zeros((slots, nkv * D), np.float32)
    for c in CLOCKS:
        q = gh.synth_normal(nq * D, c, 72, 0.0, 1.0)
        k = gh.synth_normal(nkv * D, c, 73, 0.0, 1.0)
        v = gh.synth_normal(nkv * D, c, 74, 0.0, 1.0)
        slot = ring.slot_index(c)
        step = np.array([c, slot, 1, 0], np.uint32)
        Q, K, V, ST = gpu.upload(q), gpu.upload(k), gpu.upload(v), gpu.upload(step)
        gpu.qkv_rope(Q, K, None if k_eq_v else V, QN, KN, Q, KC, VC, ST, nq, nkv, D, rot, k_eq_v,
                     theta, 1e-6)
        q2, k2, v2 = orc.qkv_norm_rope(q, k, v, qn, kn, nq, nkv, D, rot, k_eq_v, theta, 1e-6, c)
        assert_close(Q.read(np.float32, nq * D), q2, what="q clock %d" % c)
        kc_ref[slot] = k2
        vc_ref[slot] = v2
    kc, vc = KC.read(np.float32).reshape(slots, -1), VC.read(np.float32).reshape(slots, -1)
    written = sorted({ring.slot_index(c) for c in CLOCKS})
    for sl in written:
        assert_close(kc[sl], kc_ref[sl], what="K cache slot %d" % sl)
        assert_close(vc[sl], vc_ref[sl], what="V cache slot %d" % sl)
    others = np.setdiff1d(np.arange(slots), written)
    assert not kc[others].any() and not vc[others].any()  # no other slot is touched


# ------------------------------------------------------------- attention ----
def make_cache(slots, nkv, D, seed):
    kc = gh.synth_normal(slots * nkv * D, seed, 80, 0.0, 1.0).reshape(slots, nkv, D)
    v = gh.synth_normal(slots * nkv * D, seed, 81, 0.0, 1.0).reshape(slots, nkv, D)
    v = (v / np.sqrt(np.mean(v.astype(np.float64) ** 2, axis=2, keepdims=True) + 1e-6)).astype(np.float32)
    return kc.reshape(slots, -1).copy(), v.reshape(slots, -1).copy()


@pytest.mark.parametrize("S", [640, 544, 1, 37])
def test_decode_attention(gpu, S):
    # 16 query / 8 kv heads, D = 256, the 640-slot ring; q normalised + roped
    nq, nkv, D, slots = 16, 8, 256, 640
    kc, vc = make_cache(slots, nkv, D, 3)
    qraw = gh.synth_normal(nq * D, 3, 82, 0.0, 1.0)
    qn = bf16_round(gh.synth_normal(D, 3, 83, 1.0, 0.1))
    q, _, _ = orc.qkv_norm_rope(qraw, np.zeros(nkv * D), np.zeros(nkv * D), qn, qn, nq, nkv, D,
                                64, False, 1e4, 1e-6, 700)
    rng = np.random.default_rng(S)
    active = np.arange(slots, dtype=np.uint32) if S == slots else \
        rng.permutation(slots)[:S].astype(np.uint32)
    step = np.array([700, 0, S, 0], np.uint32)
    Q, KC, VC, A, ST, O = (gpu.upload(q), gpu.upload(kc), gpu.upload(vc), gpu.upload(active),
                           gpu.upload(step), gpu.alloc(nq * D * 4))
    gpu.decode_attn(Q, KC, VC, A, O, ST, D, nkv * D, nq // nkv, nq)
    out = O.read(np.float32, nq * D)
    ref = orc.attention(q, kc, vc, active, nq, nkv, D)
    assert_close(out, ref, what="attention S=%d" % S)
    if S == slots:  # the list 0 .. S-1, declared in the step flags: same bits
        ST2 = gpu.upload(np.array([700, 0, S, 2], np.uint32))
        O2 = gpu.alloc(nq * D * 4)
        gpu.decode_attn(Q, KC, VC, A, O2, ST2, D, nkv * D, nq // nkv, nq)
        assert np.array_equal(O2.read(np.float32, nq * D), out)
    # a second launch reuses the self-reset split counters
    gpu.decode_attn(Q, KC, VC, A, O, ST, D, nkv * D, nq // nkv, nq)
    assert np.array_equal(O.read(np.float32, nq * D), out)


@pytest.mark.parametrize("nq,nkv,D", [(8, 2, 128), (4, 4, 512), (8, 8, 64)])
def test_decode_attention_other_shapes(gpu, nq, nkv, D):
    slots, S = 100, 77
    kc, vc = make_cache(slots, nkv, D, 5)
    q = gh.synth_normal(nq * D, 5, 84, 0.0, 0.2)
    active = np.random.default_rng(1).permutation(slots)[:S].astype(np.uint32)
    step = np.array([5, 0, S, 0], np.uint32)
    Q, KC, VC, A, ST, O = (gpu.upload(q), gpu.upload(kc), gpu.upload(vc), gpu.upload(active),
                           gpu.upload(step), gpu.alloc(nq * D * 4))
    gpu.decode_attn(Q, KC, VC, A, O, ST, D, nkv * D, nq // nkv, nq)
    assert_close(O.read(np.float32, nq * D), orc.attention(q, kc, vc, active, nq, nkv, D),
                 what="attention %d/%d/%d" % (nq, nkv, D))


def test_decode_attention_closed_forms(gpu):
    nq, nkv, D, slots = 16, 8, 256, 64
    kc, vc = make_cache(slots, nkv, D, 9)
    active = np.arange(slots, dtype=np.uint32)
    # q = 0: equal scores -> mean of V over the active slots
    Q, KC, VC, A, O = (gpu.upload(np.zeros(nq * D, np.float32)), gpu.upload(kc), gpu.upload(vc),
                       gpu.upload(active), gpu.alloc(nq * D * 4))
    ST = gpu.upload(np.array([0, 0, slots, 0], np.uint32))
    gpu.decode_attn(Q, KC, VC, A, O, ST, D, nkv * D, 2, nq)
    mean = vc.reshape(slots, nkv, D).astype(np.float64).mean(axis=0)
    out = O.read(np.float32, nq * D).reshape(nq, D)
    assert np.allclose(out[0], mean[0], atol=1e-5) and np.allclose(out[15], mean[7], atol=1e-5)
    # S = 1 -> that slot's V
    ST1 = gpu.upload(np.array([0, 0, 1, 0], np.uint32))
    A1 = gpu.upload(np.array([17], np.uint32))
    Q1 = gpu.upload(gh.synth_normal(nq * D, 9, 85, 0.0, 1.0))
    gpu.decode_attn(Q1, KC, VC, A1, O, ST1, D, nkv * D, 2, nq)
    out = O.read(np.float32, nq * D).reshape(nq, D)
    assert np.allclose(out[5], vc[17].reshape(nkv, D)[2], atol=1e-6)


@pytest.mark.parametrize("theta", [1e6, 1e4])
@pytest.mark.parametrize("k_eq_v", [False, True])
@pytest.mark.parametrize("clock,S", [(600, 544), (639, 640), (5, 6)])
def test_qkv_rope_attn_fused(gpu, clock, S, k_eq_v, theta):
    # the decode graph's per-layer attention step: q/k norm + RoPE, the cache
    # write at slot_idx, and attention over the active list that includes it.
    # theta 1e4 with rot 64 over the 32 + 512 + 96 ring, V rows at unit RMS:
    # the GQA attention workload exactly (partial RoPE on the first 64 dims at
    # base 10000, positions with the window wrapped, all 640 slots at 639)
    nq, nkv, D, slots, rot = 16, 8, 256, 640, 64
    kc, vc = make_cache(slots, nkv, D, 11)
    qraw = gh.synth_normal(nq * D, clock, 86, 0.0, 1.0)
    kraw = gh.synth_normal(nkv * D, clock, 87, 0.0, 1.0)
    vraw = gh.synth_normal(nkv * D, clock, 88, 0.0, 1.0)
    qn = bf16_round(gh.synth_normal(D, 11, 89, 1.0, 0.1))
    kn = bf16_round(gh.synth_normal(D, 11, 90, 1.0, 0.1))
    ring = orc.Ring(1, nkv * D, 32, 512, 96)
    slot = ring.slot_index(clock)
    active = np.random.default_rng(S).permutation(slots)[:S].astype(np.uint32)
    if slot not in active:
        active[S // 2] = slot
    step = np.array([clock, slot, S, 0], np.uint32)
    bufs = [gpu.upload(a) for a in (qraw, kraw, vraw, qn, kn, kc, vc, active, step)]
    O = gpu.alloc(nq * D * 4)
    Q, K, V, QN, KN, KC, VC, A, ST = bufs
    gpu.qkv_rope_attn(Q, K, 0 if k_eq_v else V, QN, KN, KC, VC, A, ST, O, nq, nkv, D, rot,
                      k_eq_v, theta)
    q2, k2, v2 = orc.qkv_norm_rope(qraw, kraw, vraw, qn, kn, nq, nkv, D, rot, k_eq_v, theta,
                                   1e-6, clock)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[slot], vc2[slot] = k2, v2
    ref = orc.attention(q2, kc2, vc2, active, nq, nkv, D)
    assert_close(O.read(np.float32, nq * D), ref, what="fused attention S=%d" % S)
    got_k = KC.read(np.float32).reshape(slots, -1)
    got_v = VC.read(np.float32).reshape(slots, -1)
    assert_close(got_k[slot], k2, what="K row")
    assert_close(got_v[slot], v2, what="V row")
    others = np.arange(slots) != slot
    assert np.array_equal(got_k[others], kc[others]) and np.array_equal(got_v[others], vc[others])
    assert np.array_equal(Q.read(np.float32, nq * D), qraw)


@pytest.mark.parametrize("rot,theta", [(256, 1e4), (64, 1e6)])
def test_qkv_rope_attn_table_and_dense_list(gpu, rot, theta):
    # the decode graph's form: RoPE angles from the per-token table and the
    # list declared 0 .. S-1 (step flags bit 1) give the same bits as angles
    # computed in the kernel and the list read from memory
    nq, nkv, D, slots, S, clock = 16, 8, 256, 640, 544, 600
    kc, vc = make_cache(slots, nkv, D, 12)
    raw = [gh.synth_normal(n, clock, 91 + i, 0.0, 1.0) for i, n in enumerate((nq * D, nkv * D, nkv * D))]
    qn = bf16_round(gh.synth_normal(D, 12, 94, 1.0, 0.1))
    kn = bf16_round(gh.synth_normal(D, 12, 95, 1.0, 0.1))
    slot = 32 + (clock - 32) % 512
    Q, K, V, QN, KN, A = (gpu.upload(a) for a in raw + [qn, kn, np.arange(S, dtype=np.uint32)])
    outs = []
    for flags, use_tab in ((0, False), (2, True), (2, False), (0, True)):
        ST = gpu.upload(np.array([clock, slot, S, flags], np.uint32))
        TAB = gpu.alloc(512 * 4)
        if use_tab:
            gpu.rope_table(ST, rot, theta, TAB)
        KC, VC, O = gpu.upload(kc), gpu.upload(vc), gpu.alloc(nq * D * 4)
        gpu.qkv_rope_attn(Q, K, V, QN, KN, KC, VC, A, ST, O, nq, nkv, D, rot, False, theta,
                          table=TAB if use_tab else None)
        outs.append((O.read(np.float32, nq * D), KC.read(np.float32), VC.read(np.float32)))
    for o in outs[1:]:
        for a, b in zip(o, outs[0]):
            assert np.array_equal(a, b)
    q2, k2, v2 = orc.qkv_norm_rope(*raw, qn, kn, nq, nkv, D, rot, False, theta, 1e-6, clock)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[slot], vc2[slot] = k2, v2
    ref = orc.attention(q2, kc2, vc2, np.arange(S, dtype=np.uint32), nq, nkv, D)
    assert_close(outs[0][0], ref, what="fused attention, table + dense list")


def test_rope_table_matches_oracle(gpu):
    # gh_rope_table's angles rotate like applyRopePartial (kernels.zig:132-150)
    for rot, theta, clock in ((256, 1e4, 0), (256, 1e4, 639), (64, 1e6, 1000)):
        ST = gpu.upload(np.array([clock, 0, 1, 0], np.uint32))
        TAB = gpu.alloc(512 * 4)
        gpu.rope_table(ST, rot, theta, TAB)
        tab = TAB.read(np.float32)
        i = np.arange(rot // 2)
        ang = clock / np.float64(theta) ** (2.0 * i / rot)
        assert np.max(np.abs(tab[:rot // 2] - np.cos(ang))) < 2e-4
        assert np.max(np.abs(tab[256:256 + rot // 2] - np.sin(ang))) < 2e-4
        v = np.ones(256, np.float32)
        r = orc.rope_partial(v, clock, 256, rot, theta)
        h = rot // 2
        got = np.concatenate([tab[:h] - tab[256:256 + h], tab[256:256 + h] + tab[:h]])
        # the f32 angle clock * freq: one ulp of powf (device vs the host libm)
        # moves it by up to ~6e-8 * clock radians, ~6e-5 at clock 1000
        assert np.max(np.abs(got - r[:rot])) < 1e-4


# ---------------------------------------------------------------- argmax ----
def test_argmax_bit_exact(gpu):
    V = 262144
    OUT = gpu.alloc(4)
    cases = []
    x = gh.synth_normal(V, 0, 90, 0.0, 1.0)
    cases.append(x)
    t = x.copy()
    t[[1000, 5, 262143]] = 10.0  # ties: lowest index wins
    cases.append(t)
    cases.append(np.zeros(V, np.float32))  # all equal -> 0
    e = np.full(V, -np.inf, np.float32)
    e[262143] = -1.0
    cases.append(e)
    cases.append(np.arange(V, dtype=np.float32))  # maximum at the last index
    for c in cases:
        L = gpu.upload(c)
        gpu.argmax(L, OUT, V)
        assert int(OUT.read(np.uint32, 1)[0]) == orc.argmax(c)
    for n in (1, 7, 1025, 300000):
        c = gh.synth_normal(n, 1, 91, 0.0, 1.0)
        L = gpu.upload(c)
        gpu.argmax(L, OUT, n)
        assert int(OUT.read(np.uint32, 1)[0]) == orc.argmax(c)
