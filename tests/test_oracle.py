"""Pins the C oracle (oracle/liboracle.so) before anything is checked against it.

Each test names what fixes the answer: a known-answer test the reference's own
suite holds, a hand-derived value, a closed form / invariant, or the
independent numpy restatement in tests/numpy_ref.py.
"""
import math
import os

import numpy as np
import pytest

import numpy_ref as nr
import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------- bf16 ----
def test_bf16_roundtrip_reference_kat():
    # src/tensor.zig:30-41
    assert abs(orc.bf16_to_f32(orc.bf16_from_f32(np.float32(3.1415926)))[()] - 3.1415926) < 0.02
    assert orc.bf16_to_f32(orc.bf16_from_f32(np.float32(0.0)))[()] == 0.0
    assert abs(orc.bf16_to_f32(orc.bf16_from_f32(np.float32(-42.5)))[()] + 42.5) < 0.1


def test_bf16_rne_ties():
    # 0x3F808000 is exactly half-way between 0x3F80 and 0x3F81: ties to even.
    v = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF, 0xBF808000], np.uint32).view(np.float32)
    got = orc.bf16_from_f32(v)
    assert list(got) == [0x3F80, 0x3F82, 0x3F81, 0x3F80, 0xBF80]
    rng = np.random.default_rng(7)
    x = rng.standard_normal(100000).astype(np.float32) * 10
    assert np.array_equal(orc.bf16_from_f32(x), nr.bf16_rne(x))


# ------------------------------------------------------------ quantizers ----
def test_q4_known_answers():
    ones = np.full((1, 32), 0x3F80, np.uint16)  # bf16 1.0
    q = orc.quantize_q4(ones)
    assert q[0, 0] == 0x3E124925  # f32 bits of 1/7
    assert list(q[0, 1:]) == [0xFFFFFFFF] * 4  # nibble 15 = 7 + 8
    zeros = np.zeros((1, 32), np.uint16)
    q = orc.quantize_q4(zeros)
    assert q[0, 0] == 0 and list(q[0, 1:]) == [0x88888888] * 4
    # amax 7 -> d = 1, id = 1: values round half away from zero
    v = np.array([7, -7, 3.5, -3.5, 0.5, -0.5, 1.5, -1.5] * 4, np.float32)
    q = orc.quantize_q4(nr.bf16_rne(v)[None, :])
    assert q[0, 0] == np.float32(1.0).view(np.uint32)
    # nibbles 15, 1, 12, 4, 9, 7, 10, 6 packed sequentially from bit 0
    want = 15 | (1 << 4) | (12 << 8) | (4 << 12) | (9 << 16) | (7 << 20) | (10 << 24) | (6 << 28)
    assert list(q[0, 1:]) == [want] * 4


def test_q8_known_answers():
    ones = np.full((1, 32), 0x3F80, np.uint16)
    q = orc.quantize_q8(ones)
    assert q[0, 0] == np.float32(np.float32(1.0) / np.float32(127.0)).view(np.uint32)
    assert list(q[0, 1:]) == [0x7F7F7F7F] * 8
    q = orc.quantize_q8(np.zeros((1, 32), np.uint16))
    assert list(q[0]) == [0] * 9
    v = np.array([127, -127, 0.5, -0.5] * 8, np.float32)
    q = orc.quantize_q8(nr.bf16_rne(v)[None, :])
    # bytes 0x7F, 0x81 (-127), 0x01, 0xFF (-1) little-endian in one word
    assert list(q[0, 1:]) == [0xFF01817F] * 8


def test_quant_matches_numpy_fixtures():
    f = np.load(os.path.join(GOLD, "quant_fixtures.npz"))
    assert np.array_equal(orc.bf16_from_f32(f["w_f32"]), f["w_bf16"])
    assert np.array_equal(orc.quantize_q4(f["w_bf16"]), f["q4"])
    assert np.array_equal(orc.quantize_q8(f["w_bf16"]), f["q8"])


def test_quant_random_rows_match_numpy_and_threads():
    rng = np.random.default_rng(11)
    w = nr.bf16_rne(rng.standard_normal((300, 3840)).astype(np.float32) * 0.02)
    q4 = orc.quantize_q4(w)
    assert np.array_equal(q4, nr.quantize_q4(w))
    assert np.array_equal(orc.quantize_q4(w, nthreads=8), q4)  # threading never changes bytes
    q8 = orc.quantize_q8(w)
    assert np.array_equal(q8, nr.quantize_q8(w))
    assert np.array_equal(orc.quantize_q8(w, nthreads=8), q8)


def test_quant_invariants():
    rng = np.random.default_rng(3)
    wf = rng.standard_normal((64, 256)).astype(np.float32) * 0.02
    w = nr.bf16_rne(wf)
    wn = w ^ np.uint16(0x8000)  # exact negation in bf16
    q, qn = orc.quantize_q4(w), orc.quantize_q4(wn)
    shifts = np.arange(8, dtype=np.uint64) * 4
    nib = lambda a: ((a.reshape(64, 8, 5)[:, :, 1:].astype(np.uint64)[..., None] >> shifts) & 0xF)
    n, nn = nib(q), nib(qn)
    assert np.all(n >= 1) and np.all(n <= 15)  # nibble 0 never occurs
    assert np.array_equal(nn, 16 - n)  # negation maps n -> 16 - n
    # |w - deq(w)| <= d/2 (+ a few ulps)
    deq = nr.dequant_q4(q, 256)
    d = np.repeat(q.reshape(64, 8, 5)[:, :, 0].view(np.float32), 32, axis=1).astype(np.float64)
    err = np.abs(deq - nr.bf16_to_f32(w).astype(np.float64))
    assert np.all(err <= d * 0.5 * (1 + 1e-5) + 1e-12)
    q8, q8n = orc.quantize_q8(w), orc.quantize_q8(wn)
    b = q8.reshape(64, 8, 9)[:, :, 1:].copy().view(np.int8)
    bn = q8n.reshape(64, 8, 9)[:, :, 1:].copy().view(np.int8)
    assert np.all(b != -128)
    assert np.array_equal(bn.astype(np.int32), -b.astype(np.int32))


# ------------------------------------------------------------------ GEMV ----
def test_gemv_bf16_reference_kat():
    # src/kernels.zig:176-183: [[1,2],[3,4]] . [1,2] = [5, 11]
    w = nr.bf16_rne(np.array([[1, 2], [3, 4]], np.float32))
    y = orc.gemv_bf16(w, np.array([1, 2], np.float32))
    assert abs(y[0] - 5) < 0.01 and abs(y[1] - 11) < 0.01


def test_gemv_q4_constant_weight_closed_form():
    # all-ones weights: every dequantized weight is (15-8) * f32(1/7)
    w = np.full((8, 128), 0x3F80, np.uint16)
    x = (np.arange(128) % 5).astype(np.float32) * 0.25  # src/gpu.zig:43 input
    y = orc.gemv_q4(orc.quantize_q4(w), x, 128)
    wv = np.float64(np.float32(7.0) * np.float32(np.float32(1.0) / np.float32(7.0)))
    assert np.allclose(y, wv * x.astype(np.float64).sum(), rtol=1e-6)
    assert np.all(y > 0)  # src/gpu.zig:58


@pytest.mark.parametrize("mode", ["q4", "q8"])
def test_gemv_matches_fp64_brute_force(mode):
    rng = np.random.default_rng(5)
    M, K = 256, 3840
    w = nr.bf16_rne(rng.standard_normal((M, K)).astype(np.float32) * 0.02)
    x = rng.standard_normal(K).astype(np.float32)
    if mode == "q4":
        wq = orc.quantize_q4(w)
        y = orc.gemv_q4(wq, x, K, nthreads=4)
        ref = nr.dequant_q4(wq, K) @ x.astype(np.float64)
    else:
        wq = orc.quantize_q8(w)
        y = orc.gemv_q8(wq, x, K, nthreads=4)
        ref = nr.dequant_q8(wq, K) @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5


# --------------------------------------------------------------- norms -----
def test_rmsnorm_closed_form():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(3840).astype(np.float32) * 3
    y = orc.rmsnorm(x, np.ones(3840, np.float32))
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1) < 1e-5
    w = (1 + rng.standard_normal(3840) * 0.1).astype(np.float32)
    assert np.allclose(orc.rmsnorm(x, w), nr.rmsnorm64(x, w), rtol=1e-5, atol=1e-6)
    u = orc.unit_rmsnorm(x)
    assert abs(np.sqrt(np.mean(u.astype(np.float64) ** 2)) - 1) < 1e-5
    # the norm of an all-zero vector stays zero (eps keeps it finite)
    assert np.all(orc.rmsnorm(np.zeros(16, np.float32), np.ones(16, np.float32)) == 0)


def test_gelu_tanh():
    xs = np.linspace(-8, 8, 161).astype(np.float32)
    got = np.array([orc.gelu_tanh(v) for v in xs])
    assert np.allclose(got, nr.gelu64(xs), rtol=2e-6, atol=1e-7)
    assert orc.gelu_tanh(0.0) == 0.0
    assert abs(orc.gelu_tanh(20.0) - 20.0) < 1e-5 and abs(orc.gelu_tanh(-20.0)) < 1e-5


# ---------------------------------------------------------------- RoPE -----
def test_rope_properties():
    rng = np.random.default_rng(21)
    hd, rot, theta = 256, 64, 10000.0
    v = rng.standard_normal(2 * hd).astype(np.float32)
    assert np.array_equal(orc.rope_partial(v, 0, hd, rot, theta), v)  # pos 0 is identity
    r = orc.rope_partial(v, 1234, hd, rot, theta)
    vh, rh = v.reshape(2, hd), r.reshape(2, hd)
    assert np.array_equal(rh[:, rot:], vh[:, rot:])  # suffix passes through
    n0 = vh[:, :32] ** 2 + vh[:, 32:64] ** 2
    n1 = rh[:, :32] ** 2 + rh[:, 32:64] ** 2
    assert np.allclose(n0, n1, rtol=1e-5)  # each (i, i+rot/2) pair keeps its norm
    assert np.allclose(r, nr.rope64(v, 1234, hd, rot, theta), atol=5e-4)
    # angle additivity R(a) R(b) = R(a + b)
    ab = orc.rope_partial(orc.rope_partial(v, 3, hd, rot, theta), 5, hd, rot, theta)
    assert np.allclose(ab, orc.rope_partial(v, 8, hd, rot, theta), atol=1e-5)
    # full rotation (sliding layers): rot = head_dim
    assert np.allclose(orc.rope_partial(v, 77, hd, hd, theta), nr.rope64(v, 77, hd, hd, theta), atol=5e-5)


# ------------------------------------------------------- softmax / argmax --
def test_softmax_and_argmax():
    rng = np.random.default_rng(2)
    s = rng.standard_normal(640).astype(np.float32) * 16
    p = orc.softmax(s)
    assert abs(p.astype(np.float64).sum() - 1) < 1e-5 and np.all(p >= 0)
    v = np.array([1, 5, 3, 5, 2], np.float32)
    assert orc.argmax(v) == 1  # ties go to the lowest index
    assert orc.argmax(np.zeros(100, np.float32)) == 0
    w = rng.standard_normal(262144).astype(np.float32)
    assert orc.argmax(w) == int(np.argmax(w))


# ---------------------------------------------------------------- ring -----
def test_ring_tiers_and_window_eviction():
    # src/ring_buffer.zig:149-166
    r = orc.Ring(2, 64, 4, 8, 4)
    assert r.total_slots == 16
    k, v = np.ones(64, np.float32), np.full(64, 2.0, np.float32)
    for c in range(20):
        r.write_kv(0, c, k, v)
    s = r.active_slots(0, 19)
    assert len(s) == 12 and s[0] == 0 and s[3] == 3


def test_ring_recall_slots():
    # src/ring_buffer.zig:168-187
    r = orc.Ring(1, 8, 2, 4, 3)
    k, v = np.ones(8, np.float32), np.full(8, 2.0, np.float32)
    r.write_recall_kv(0, 0, k, v, 100)
    r.write_recall_kv(0, 1, k, v, 50)
    assert len(r.active_slots(0, 101)) == 2
    r.clear_recall()
    assert len(r.active_slots(0, 101)) == 0


def test_ring_wraparound():
    r = orc.Ring(1, 4, 32, 512, 96)
    assert r.slot_index(0) == 0 and r.slot_index(31) == 31
    assert r.slot_index(32) == 32 and r.slot_index(543) == 543
    assert r.slot_index(544) == 32 and r.slot_index(1000) == 32 + (1000 - 32) % 512
    for c in range(600):
        r.activate_slot(0, c)
    s = r.active_slots(0, 599)
    # 32 anchors + the 512 newest window clocks (88..599)
    assert len(s) == 544 and list(s[:32]) == list(range(32))
    assert sorted(s[32:]) == list(range(32, 544))


# ----------------------------------------------------------- attention -----
def test_attention_closed_forms():
    rng = np.random.default_rng(4)
    nq, nkv, hd, S = 4, 2, 64, 10
    kc = rng.standard_normal((S, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((S, nkv * hd)).astype(np.float32)
    act = np.arange(S, dtype=np.uint32)
    # equal scores -> mean of V
    out = orc.attention(np.zeros(nq * hd, np.float32), kc, vc, act, nq, nkv, hd).reshape(nq, hd)
    mean = vc.reshape(S, nkv, hd).mean(axis=0)
    assert np.allclose(out[0], mean[0], atol=1e-6) and np.allclose(out[3], mean[1], atol=1e-6)
    # S = 1 -> that V
    out = orc.attention(rng.standard_normal(nq * hd).astype(np.float32), kc, vc,
                        np.array([7], np.uint32), nq, nkv, hd).reshape(nq, hd)
    assert np.allclose(out[1], vc[7].reshape(nkv, hd)[0], atol=1e-6)
    # dominant score -> that slot's V
    q = np.zeros(nq * hd, np.float32)
    q[:hd] = kc[5, :hd] * 50
    out = orc.attention(q, kc, vc, act, nq, nkv, hd).reshape(nq, hd)
    assert np.allclose(out[0], vc[5, :hd], atol=1e-4)


def test_attention_fp64_brute_force():
    rng = np.random.default_rng(8)
    nq, nkv, hd, slots = 16, 8, 256, 640
    kc = rng.standard_normal((slots, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((slots, nkv * hd)).astype(np.float32)
    q = rng.standard_normal(nq * hd).astype(np.float32) * 0.1
    act = rng.permutation(slots)[:300].astype(np.uint32)
    out = orc.attention(q, kc, vc, act, nq, nkv, hd)
    ref = nr.attention64(q, kc, vc, act, nq, nkv, hd)
    assert np.max(np.abs(out - ref)) < 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_qkv_norm_rope_composition():
    rng = np.random.default_rng(6)
    nq, nkv, hd, rot = 4, 2, 256, 64
    q, k, v = (rng.standard_normal(n * hd).astype(np.float32) for n in (nq, nkv, nkv))
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    q2, k2, v2 = orc.qkv_norm_rope(q, k, v, qn, kn, nq, nkv, hd, rot, False, 1e4, 1e-6, 37)
    qref = np.concatenate([nr.rmsnorm64(q[h * hd:(h + 1) * hd], qn) for h in range(nq)])
    assert np.allclose(q2, nr.rope64(qref, 37, hd, rot, 1e4), atol=1e-4)
    for h in range(nkv):
        vh = v[h * hd:(h + 1) * hd].astype(np.float64)
        assert np.allclose(v2[h * hd:(h + 1) * hd], vh / np.sqrt(np.mean(vh ** 2) + 1e-6), atol=1e-5)
    # k_eq_v: V is the raw K, unit-RMS normalised
    _, _, v3 = orc.qkv_norm_rope(q, k, v, qn, kn, nq, nkv, hd, rot, True, 1e4, 1e-6, 37)
    kh = k[:hd].astype(np.float64)
    assert np.allclose(v3[:hd], kh / np.sqrt(np.mean(kh ** 2) + 1e-6), atol=1e-5)


# ------------------------------------------------- MLP, embedding, forward ----
def test_gate_up_and_gated_mlp_fp64():
    # kernels.zig:94-129: act = gelu_tanh(Wg x) * (Wu x), out = Wd act
    rng = np.random.default_rng(21)
    H, I = 256, 384
    wg, wu, wd = (nr.quantize_q4(nr.bf16_rne(rng.standard_normal(s).astype(np.float32) * 0.05))
                  for s in ((I, H), (I, H), (H, I)))
    x = rng.standard_normal(H).astype(np.float32)
    act = orc.gate_up_geglu_q4(x, wg, wu, 3)
    g64 = nr.dequant_q4(wg, H) @ x.astype(np.float64)
    u64 = nr.dequant_q4(wu, H) @ x.astype(np.float64)
    ref = nr.gelu64(g64) * u64
    assert np.max(np.abs(act - ref)) / np.max(np.abs(ref)) < 1e-5
    swapped = nr.gelu64(u64) * g64  # the roles of gate and up matter
    assert np.max(np.abs(act - swapped)) / np.max(np.abs(ref)) > 1e-2
    out, act2 = orc.gated_mlp_q4(x, wg, wu, wd, 4)
    assert np.array_equal(act, act2)
    ref_out = nr.dequant_q4(wd, I) @ ref
    assert np.max(np.abs(out - ref_out)) / np.max(np.abs(ref_out)) < 1e-5


def test_embed_bits():
    # forward.zig:33-37: x = bf16(E[token]) * sqrt(f32(H)), one f32 multiply
    rng = np.random.default_rng(5)
    V, H = 64, 3840
    e = nr.bf16_rne(rng.standard_normal((V, H)).astype(np.float32) * 0.02)
    for t in (0, 17, V - 1):
        want = nr.bf16_to_f32(e[t]) * np.sqrt(np.float32(H))
        assert want.dtype == np.float32
        got = orc.embed(e, t, H)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(orc.embed(e, 1, H), orc.embed(e, 2, H))


def _tiny_forward_model(mode):
    """Three layers covering the shape rules: a sliding layer with v_proj, a
    full-attention layer with attention_k_eq_v (its own head_dim, rotary_dim
    head_dim / 4, one kv head, no post-attention norm, layer_scalar 0.7) and
    a sliding layer without v_proj (the key serves as value) with
    layer_scalar 0.5."""
    rng = np.random.default_rng(99)
    H, I, V, nq, slots = 256, 512, 512, 4, 24
    quant = {"q8": nr.quantize_q8, "q4": nr.quantize_q4,
             "bf16": lambda w: np.ascontiguousarray(w).view(np.uint32)}[mode]
    mat = lambda r, c: quant(nr.bf16_rne(rng.standard_normal((r, c)).astype(np.float32) * 0.05))  # noqa: E731
    vec = lambda n: nr.bf16_to_f32(nr.bf16_rne((1 + 0.1 * rng.standard_normal(n)).astype(np.float32)))  # noqa: E731
    specs = [dict(full=False, head_dim=64, num_kv_heads=2, k_eq_v=False, scalar=1.0, post_attn=True),
             dict(full=True, head_dim=128, num_kv_heads=1, k_eq_v=True, scalar=0.7, post_attn=False),
             dict(full=False, head_dim=64, num_kv_heads=2, k_eq_v=True, scalar=0.5, post_attn=True)]
    layers = []
    for s in specs:
        hd, nkv = s["head_dim"], s["num_kv_heads"]
        qd, kvd = nq * hd, nkv * hd
        d = dict(full=s["full"], head_dim=hd, rotary_dim=hd // 4 if s["full"] else hd,
                 num_kv_heads=nkv, k_eq_v=s["k_eq_v"], layer_scalar=s["scalar"],
                 wq=mat(qd, H), wk=mat(kvd, H), wo=mat(H, qd), wg=mat(I, H), wu=mat(I, H),
                 wd=mat(H, I), input_norm=vec(H), q_norm=vec(hd), k_norm=vec(hd),
                 post_attn_norm=vec(H) if s["post_attn"] else None, pre_ffn_norm=vec(H),
                 post_ffn_norm=vec(H))
        d["wv"] = d["wk"] if s["k_eq_v"] else mat(kvd, H)
        k = rng.standard_normal((slots, kvd)).astype(np.float32)
        v = rng.standard_normal((slots, kvd)).astype(np.float32)
        v /= np.sqrt(np.mean(v.reshape(slots, nkv, hd) ** 2, axis=2, keepdims=True) + 1e-6).repeat(hd, 2).reshape(slots, kvd)
        d["k_cache"], d["v_cache"] = k, v
        layers.append(d)
    head = nr.bf16_rne(rng.standard_normal((V, H)).astype(np.float32) * 0.05)
    head = quant(head) if mode == "bf16" else nr.quantize_q8(head)
    fnorm = vec(H)
    return H, I, V, nq, layers, head, fnorm, rng


_ORC_MODE = {"q4": orc.QUANT_Q4, "q8": orc.QUANT_Q8, "bf16": orc.QUANT_NONE}


def _copy_layers(layers):
    return [dict(d, k_cache=d["k_cache"].copy(), v_cache=d["v_cache"].copy()) for d in layers]


@pytest.mark.parametrize("mode", ["q4", "q8", "bf16"])
def test_forward_token_matches_fp64_restatement(mode):
    # orc_forward_token against tests/numpy_ref.forward64, written separately
    # from forward.zig / model_dispatch.zig: layer order, norm placement, the
    # layer scalar, gate/up roles, k_eq_v / missing v_proj, partial RoPE per
    # layer type, the cache write before attention and the Q8 head.
    H, I, V, nq, layers, head, fnorm, rng = _tiny_forward_model(mode)
    om = orc.Model(H, I, V, nq, layers, head, fnorm, layer_mode=_ORC_MODE[mode])
    ref_layers = _copy_layers(layers)
    for clock in (3, 4, 9, 17):
        slot = clock % 24
        active = np.unique(np.concatenate([[slot], rng.choice(24, 10, replace=False)])).astype(np.uint32)
        x = rng.standard_normal(H).astype(np.float32) * 3
        tok, xo, logits = om.forward(x, clock, slot, active, True, 2)
        rtok, rx, rlog = nr.forward64(ref_layers, x, clock, slot, active, head, fnorm, nq, mode=mode)
        assert np.max(np.abs(logits - rlog)) / np.max(np.abs(rlog)) < 1e-5
        assert np.max(np.abs(xo - rx)) / np.max(np.abs(rx)) < 1e-5
        srt = np.sort(rlog)
        if srt[-1] - srt[-2] > 1e-4 * np.max(np.abs(rlog)):
            assert tok == rtok
        for d, r in zip(layers, ref_layers):
            assert np.max(np.abs(d["k_cache"] - r["k_cache"])) < 1e-5
            assert np.max(np.abs(d["v_cache"] - r["v_cache"])) < 1e-5
    # the prefill graph (no logits) leaves the same residual stream
    x = rng.standard_normal(H).astype(np.float32)
    tok, xo, _ = om.forward(x, 20, 20, np.arange(21, dtype=np.uint32) % 24, False, 1)
    _, rx, _ = nr.forward64(ref_layers, x, 20, 20, np.arange(21) % 24, head, fnorm, nq, mode=mode,
                            want_logits=False)
    assert tok == 0 and np.max(np.abs(xo - rx)) / np.max(np.abs(rx)) < 1e-5


@pytest.mark.parametrize("mistake", ["scalar_both_adds", "swap_gate_up", "skip_post_attn", "rope_v",
                                     "normed_k_as_v", "theta_swap", "attn_scale",
                                     "write_after_attn", "scalar_before_ffn"])
def test_forward_restatement_catches_planted_mistakes(mistake):
    # The comparison above has teeth: each planted mistake in the fp64
    # restatement moves the logits far beyond its 1e-5 bar.
    H, I, V, nq, layers, head, fnorm, rng = _tiny_forward_model("q4")
    om = orc.Model(H, I, V, nq, layers, head, fnorm)
    bad = _copy_layers(layers)
    active = np.array([0, 2, 5, 7, 9, 11], np.uint32)
    x = rng.standard_normal(H).astype(np.float32) * 3
    _, _, logits = om.forward(x, 7, 7, active, True, 1)
    _, _, blog = nr.forward64(bad, x, 7, 7, active, head, fnorm, nq, mistake=mistake)
    assert np.max(np.abs(logits - blog)) / np.max(np.abs(blog)) > 1e-3


# ------------------------------------------------------------- layer gating ----
def test_gate_mean_sq_closed_form_and_update():
    rng = np.random.default_rng(31)
    H = 3840
    x = rng.standard_normal(H).astype(np.float32)
    prev = rng.standard_normal(H).astype(np.float32)
    want = np.mean((x.astype(np.float64) - prev) ** 2)
    p = prev.copy()
    got = orc.gate_mean_sq(x, p)
    assert abs(got - want) < 1e-5 * want
    assert np.array_equal(p, x)  # X_prev <- X_curr (quiescence_gate.wgsl:28)
    assert orc.gate_mean_sq(x, p) == 0.0  # the same input again: no motion


def test_qtracker_reference_kat():
    # src/quiescence.zig:63-77
    t = orc.QTracker(10, split_ratio=0.5, threshold=0.5)
    x = np.ones(2, np.float32)
    for layer in range(5):  # lower layers always execute
        assert t.should_execute(layer, 1, x, x)
    assert not t.should_execute(5, 1, x, x)  # zero delta, off cadence: skip
    assert t.should_execute(5, 4, x, x)  # forced cadence
    assert t.total_evals == 1 and t.skipped_evals == 1
    # relative velocity sqrt(sum d^2 / sum x^2) against the threshold
    t2 = orc.QTracker(4, split_ratio=0.5, threshold=0.1)
    x = np.array([1.0, 0.0], np.float32)
    assert t2.should_execute(3, 1, x, np.array([0.85, 0.0], np.float32))      # 0.15
    assert not t2.should_execute(3, 1, x, np.array([0.95, 0.0], np.float32))  # 0.05
    assert t2.should_execute(0, 1, x, x)  # 0 < split 2
    assert not orc.QTracker(4, threshold=0.1).should_execute(3, 1, np.zeros(2, np.float32),
                                                             np.zeros(2, np.float32))  # velocity 0


def test_forward_gated_matches_ungated_and_skips_whole_layers():
    H, I, V, nq, layers, head, fnorm, rng = _tiny_forward_model("q4")
    L = len(layers)  # 3 layers: layer 0 always runs (3 // 3 = 1), layers 1, 2 gated
    active = np.array([0, 2, 5, 7, 9, 11], np.uint32)
    x = rng.standard_normal(H).astype(np.float32) * 3
    # every gate open (thresh <= 0): the ungated forward, bit for bit
    a, b = _copy_layers(layers), _copy_layers(layers)
    om_a = orc.Model(H, I, V, nq, a, head, fnorm)
    om_b = orc.Model(H, I, V, nq, b, head, fnorm)
    xp = np.zeros((L, H), np.float32)
    ta, xa, la, run = om_a.forward_gated(x, 7, 7, active, xp, 0.0)
    tb, xb, lb = om_b.forward(x, 7, 7, active)
    assert list(run) == [1, 1, 1] and ta == tb
    assert np.array_equal(la, lb) and np.array_equal(xa, xb)
    # x_prev of a gated layer holds that layer's input: layer 1's is layer 0's output
    _, x1, _ = orc.Model(H, I, V, nq, _copy_layers(layers)[:1], head, fnorm).forward(
        x, 7, 7, active, False)
    assert np.array_equal(xp[1], x1) and not np.any(xp[0])
    # the same input again with a threshold: layer 1 sees zero motion and is
    # skipped whole (its cache keeps the slot's old row); that changes layer
    # 2's input, whose gate then opens -- the result is layers 0 and 2 alone
    c = _copy_layers(layers)
    om_c = orc.Model(H, I, V, nq, c, head, fnorm)
    xp2 = xp.copy()
    k_before = [d["k_cache"][7].copy() for d in c]
    tc, xc, lc, run = om_c.forward_gated(x, 7, 7, active, xp2, 1e-3)
    assert list(run) == [1, 0, 1]
    d02 = [d for i, d in enumerate(_copy_layers(layers)) if i != 1]
    td, xd, ld = orc.Model(H, I, V, nq, d02, head, fnorm).forward(x, 7, 7, active)
    assert np.array_equal(lc, ld) and np.array_equal(xc, xd) and tc == td
    assert np.array_equal(c[1]["k_cache"][7], k_before[1])
    assert not np.array_equal(c[0]["k_cache"][7], k_before[0])
    assert not np.array_equal(c[2]["k_cache"][7], k_before[2])
    assert np.array_equal(xp2[1], xp[1])  # a skipped layer still records its input
    # a threshold above every motion skips all gated layers
    e = _copy_layers(layers)
    xp3 = xp.copy()
    xp3[1:] += 1.0
    _, _, _, run = orc.Model(H, I, V, nq, e, head, fnorm).forward_gated(x, 7, 7, active, xp3, 1e9)
    assert list(run) == [1, 0, 0]


@pytest.mark.parametrize("mode", ["q4", "q8", "bf16"])
@pytest.mark.parametrize("case", ["in order", "slot rewritten"])
def test_forward_layer_batch_equals_token_by_token(mode, case):
    # orc_forward_layer_batch is the per-token layer run over T tokens with
    # its GEMVs turned into row x token tiles: every output, and every cache
    # row, must equal T orc_forward_token calls on that layer bit for bit.
    # "slot rewritten": token 5 rewrites slot 2, which tokens 2..4 attend to
    # (the batch must then keep token order through the cache).  T = 37 is not
    # a multiple of the 32-token tile.
    H, I, V, nq, layers, head, fnorm, rng = _tiny_forward_model(mode)
    nslot = 48  # caches of 48 slots: earlier rows random, as _tiny_forward_model fills them
    for d in layers:
        d["k_cache"] = np.concatenate([d["k_cache"], d["k_cache"]])
        d["v_cache"] = np.concatenate([d["v_cache"], d["v_cache"]])
    T = 37 if case == "in order" else 9
    slots = list(range(T)) if case == "in order" else [0, 1, 2, 3, 4, 2, 5, 6, 7]
    clocks = np.arange(100, 100 + T, dtype=np.uint64)
    actives = [np.unique(np.concatenate([[slots[t]], rng.choice(nslot, 7, replace=False)])).astype(np.uint32)
               for t in range(T)]
    X = (rng.standard_normal((T, H)) * 3).astype(np.float32)
    for li in range(len(layers)):
        a = _copy_layers(layers)
        b = _copy_layers(layers)
        om_a = orc.Model(H, I, V, nq, [a[li]], head, fnorm, layer_mode=_ORC_MODE[mode])
        om_b = orc.Model(H, I, V, nq, [b[li]], head, fnorm, layer_mode=_ORC_MODE[mode])
        got = om_a.forward_layer_batch(0, X, clocks, slots, actives, 4)
        want = np.stack([om_b.forward(X[t], int(clocks[t]), slots[t], actives[t], False, 2)[1]
                         for t in range(T)])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (mode, case, li)
        assert np.array_equal(a[li]["k_cache"], b[li]["k_cache"])
        assert np.array_equal(a[li]["v_cache"], b[li]["v_cache"])
