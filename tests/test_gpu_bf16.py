"""The bf16 weight mode (the reference's --gpu flag, quant mode none) on the
device: the bf16 GEMV (shaders/gemv_bf16.wgsl), its normed and gate+up forms
and the bf16 LM head with the fused argmax, through the C ABI, against the
oracle's bf16 rows (dotBf16, src/kernels.zig:25-43) and fp64."""
import os

import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc
from tol import assert_close

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def bf16_rows(M, K, stream, std=0.02):
    return gh.synth_normal(M * K, 0, stream, 0.0, std, bf16=True).reshape(M, K)


def deq64(w):
    return nr.bf16_to_f32(w).astype(np.float64)


def test_gemv_bf16_reference_suite_case(gpu):
    # src/test_gpu_suite.zig:9-52: M=512, K=1024, weights (u-0.5)*0.1 cut to
    # bf16 (the high half), x (u-0.5)*0.5; GPU vs the CPU gemv: max abs error
    # < 1e-3.  (numpy's generator stands in for the Zig one; same shape and
    # distribution.)
    M, K = 512, 1024
    rng = np.random.default_rng(101)
    wf = ((rng.random(M * K, dtype=np.float32) - 0.5) * 0.1).astype(np.float32)
    w = (wf.view(np.uint32) >> 16).astype(np.uint16).reshape(M, K)
    x = ((rng.random(K, dtype=np.float32) - 0.5) * 0.5).astype(np.float32)
    W, X, Y = gpu.upload(w), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_bf16(W, X, Y, M, K)
    y = Y.read(np.float32, M)
    assert np.max(np.abs(y - orc.gemv_bf16(w, x))) < 1e-3
    assert np.max(np.abs(y - deq64(w) @ x.astype(np.float64))) < 1e-4


BF16_SHAPES = [
    (8192, 2048),    # the single-GEMV shape
    (4096, 3840),    # q_proj
    (3840, 4096),    # o_proj
    (3840, 15360),   # down_proj (four 64-weight items per lane)
    (1, 128), (5, 256), (37, 1024), (1000, 3840), (3, 15360),  # ragged rows; chunk tails
    (64, 6144),      # x longer than the staging registers hold
    (17, 16384),     # the longest row a team covers (64 lanes x 4 items x 64)
]


@pytest.mark.parametrize("M,K", BF16_SHAPES)
def test_gemv_bf16_parity(gpu, M, K):
    w = bf16_rows(M, K, 5000 + M + K)
    x = gh.synth_normal(K, 0, 11, 0.0, 1.0)
    W, X, Y = gpu.upload(w), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_bf16(W, X, Y, M, K)
    y = Y.read(np.float32, M)
    assert_close(y, orc.gemv_bf16(w, x), what="gemv_bf16 %dx%d" % (M, K))
    # every weight counts once: the fp64 product of the same bf16 rows
    assert_close(y, deq64(w) @ x.astype(np.float64), what="gemv_bf16 fp64 %dx%d" % (M, K))


def test_gemv_bf16_rejects_rows_beyond_a_team(gpu):
    W, X, Y = gpu.alloc(2 * 32768 * 2), gpu.alloc(32768 * 4), gpu.alloc(8)
    with pytest.raises(gh.GhError):
        gpu.gemv_bf16(W, X, Y, 2, 32768)
    with pytest.raises(gh.GhError):
        gpu.gemv_bf16(W, X, Y, 2, 200)  # K % 128 != 0


def test_gemv_bf16_chunk_order(gpu):
    # one weight at a time: row r has a single 1.0 at column c (all other
    # weights 0), so y[r] = x[c] exactly -- a chunk or lane mapped to the
    # wrong x (or a duplicate of a clamped chunk counted) shows at once
    M, K = 64, 15360
    rng = np.random.default_rng(7)
    cols = rng.choice(K, M, replace=False)
    w = np.zeros((M, K), np.uint16)
    w[np.arange(M), cols] = 0x3F80
    x = gh.synth_normal(K, 0, 12, 0.0, 1.0)
    W, X, Y = gpu.upload(w), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_bf16(W, X, Y, M, K)
    assert np.array_equal(Y.read(np.float32, M), x[cols])


def test_norm_gemv_bf16(gpu):
    # the QKV stream of a later layer: x <- x + RMSNorm(r) * wr, then RMSNorm * w
    M, K = 8192, 3840
    w = bf16_rows(M, K, 5100)
    x = gh.synth_normal(K, 0, 13, 0.0, 1.0)
    r = gh.synth_normal(K, 0, 14, 0.0, 1.0)
    wn = nr.bf16_to_f32(nr.bf16_rne(gh.synth_normal(K, 0, 15, 1.0, 0.1)))
    wr = nr.bf16_to_f32(nr.bf16_rne(gh.synth_normal(K, 0, 16, 1.0, 0.1)))
    X, R, WN, WR, XO, Y = (gpu.upload(x), gpu.upload(r), gpu.upload(wn), gpu.upload(wr),
                           gpu.alloc(K * 4), gpu.alloc(M * 4))
    pro = gpu.prologue(X, 2, norm=WN, r=R, r_norm=WR, x_out=XO, scalar=0.5)
    gpu.norm_gemv(gh.QUANT_NONE, gpu.upload(w), Y, M, K, pro)
    xn = ((x + orc.rmsnorm(r, wr)) * np.float32(0.5)).astype(np.float32)
    assert_close(XO.read(np.float32, K), xn, what="residual stream")
    assert_close(Y.read(np.float32, M), orc.gemv_bf16(w, orc.rmsnorm(xn, wn)),
                 what="norm_gemv bf16")


@pytest.mark.parametrize("normed", [False, True])
def test_gate_up_bf16(gpu, normed):
    M, K = 15360, 3840
    wg, wu = bf16_rows(M, K, 5200), bf16_rows(M, K, 5201)
    x = gh.synth_normal(K, 0, 17, 0.0, 1.0)
    wn = nr.bf16_to_f32(nr.bf16_rne(gh.synth_normal(K, 0, 18, 1.0, 0.1)))
    X, WN, Y = gpu.upload(x), gpu.upload(wn), gpu.alloc(M * 4)
    pro = gpu.prologue(X, 1, norm=WN) if normed else gpu.prologue(X, 0)
    gpu.norm_gate_up_geglu(gh.QUANT_NONE, gpu.upload(wg), gpu.upload(wu), Y, M, K, pro)
    xin = orc.rmsnorm(x, wn) if normed else x
    g = orc.gemv_bf16(wg, xin)
    u = orc.gemv_bf16(wu, xin)
    ref = np.array([orc.gelu_tanh(float(a)) for a in g], np.float32) * u
    assert_close(Y.read(np.float32, M), ref, what="gate_up bf16")
    # gate and up are not interchangeable
    swapped = np.array([orc.gelu_tanh(float(a)) for a in u], np.float32) * g
    assert np.max(np.abs(ref - swapped)) > 1e-2 * np.max(np.abs(ref))


@pytest.mark.parametrize("V", [262144, 1000])
def test_norm_gemv_argmax_bf16(gpu, V):
    # the bf16 head of mode none: the embedding rows themselves
    H = 3840
    E = gpu.alloc(V * H * 2)
    gpu.synth_normal_dev(E, V * H, 0, 5300, 0.0, 0.02, bf16=True)
    e = E.read(np.uint16).reshape(V, H)
    x = gh.synth_normal(H, 0, 19, 0.0, 1.0)
    wn = nr.bf16_to_f32(nr.bf16_rne(gh.synth_normal(H, 0, 20, 1.0, 0.1)))
    X, WN, L, T = gpu.upload(x), gpu.upload(wn), gpu.alloc(V * 4), gpu.alloc(4)
    pro = gpu.prologue(X, 1, norm=WN)
    gpu.norm_gemv_argmax_bf16(E, L, T, V, H, pro)
    logits = L.read(np.float32, V)
    ref = orc.gemv_bf16(e, orc.rmsnorm(x, wn))
    assert_close(logits, ref, what="bf16 head logits")
    tok = int(T.read(np.uint32, 1)[0])
    assert tok == orc.argmax(logits)  # bit-exact pick over the logits it produced
    assert tok == orc.argmax(ref) or ref[tok] >= np.max(ref) - 1e-5 * np.max(np.abs(ref))
    gpu.norm_gemv_argmax_bf16(E, None, T, V, H, pro)  # without materialised logits
    assert int(T.read(np.uint32, 1)[0]) == tok


def test_bf16_model_prompt_then_greedy(gpu):
    # mode none end to end: a 12-token prompt through gh_model_prefill (the
    # batched prefill with bf16 MFMA GEMMs on the bf16 rows) and 6 greedy
    # steps, against the oracle's sequential forward on the same bf16 rows
    # (src/interactive.zig:33-37 prefills token by token)
    from model_ref import oracle_model
    from test_gpu_model import check_token, tiny_cfg
    cfg = tiny_cfg()
    m = gh.Model(gpu, cfg, mode=gh.QUANT_NONE, seed=31)
    try:
        om, layers = oracle_model(m, cfg, gh.QUANT_NONE)
        embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, cfg.hidden_size)
        ring = gh.Ring(1, 4, 16, 4)
        T = 12
        toks = np.random.default_rng(3).integers(0, cfg.vocab_size, T)
        xs = np.stack([orc.embed(embed, int(t), cfg.hidden_size) for t in toks])
        slots = [ring.activate_slot(0, c) for c in range(T)]
        lists = [ring.active_slots(0, c) for c in range(T)]
        tok = m.prefill(xs, np.arange(T), slots, lists, True)
        for c in range(T):
            rtok, _, rlog = om.forward(xs[c], c, slots[c], lists[c], c == T - 1, NT)
        check_token(m, rlog, tok, rtok, "bf16 prompt")
        for c in range(T, T + 6):
            x = orc.embed(embed, tok, cfg.hidden_size)
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            tok = m.forward(x, c, slot, act, True)
            rtok, _, rlog = om.forward(x, c, slot, act, True, NT)
            check_token(m, rlog, tok, rtok, "bf16 greedy step %d" % c)
            tok = rtok
        for l, d in enumerate(layers):
            kvd = d["k_cache"].shape[1]
            kc = m.read(l, gh.T_K_CACHE, np.float32).reshape(cfg.max_slots, kvd)
            assert_close(kc, d["k_cache"], what="K cache layer %d" % l)
    finally:
        m.close()
