"""GPU parity of the batched prefill: the MFMA Q4_0/Q8_0 dequant GEMMs against
an fp64 product of the same dequantized weights, and gh_model_prefill against
the oracle's sequential per-token forward (the reference prefills token by
token, src/interactive.zig:33-37, so that is the semantics to match)."""
import os

import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc
from model_ref import oracle_model
from tol import assert_close

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def quantized(rows, cols, mode, seed):
    """The device rows of mode (Q4_0, Q8_0, or bf16 as is) and their values in fp64."""
    w = nr.bf16_rne(gh.synth_normal(rows * cols, 0, seed, 0.0, 0.02).reshape(rows, cols))
    if mode == gh.QUANT_NONE:
        return w, nr.bf16_to_f32(w).astype(np.float64)
    wq = nr.quantize_q4(w) if mode == gh.QUANT_Q4 else nr.quantize_q8(w)
    deq = nr.dequant_q4(wq, cols) if mode == gh.QUANT_Q4 else nr.dequant_q8(wq, cols)
    return wq, deq


# (T, N, K): single row, ragged T and N, the 12B K, T past one 128-row tile,
# and a long prompt's narrow product (128x128 tiles with K split 3 ways)
# (512, 8192, 256): 256 tiles of 128x128, so the 128x64 tile runs (two per CU);
# (96, 8192, 1024): one 128-row tile of 96 tokens, 64 tiles split 4 ways;
# (300, 128, 1024): 256 tokens on the tiles, the last 44 streamed
GEMM_SHAPES = [(1, 64, 128), (7, 96, 256), (64, 384, 3840), (130, 256, 512), (300, 128, 1024),
               (512, 3840, 1024), (512, 8192, 256), (96, 8192, 1024)]


@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8, gh.QUANT_NONE])
@pytest.mark.parametrize("T,N,K", GEMM_SHAPES)
def test_prefill_gemm(gpu, mode, T, N, K):
    wq, deq = quantized(N, K, mode, 300 + T)
    a = gh.synth_normal(T * K, 1, 301, 0.0, 1.0).reshape(T, K)
    W, A, C = gpu.upload(wq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gemm(mode, W, A, C, T, N, K)
    got = C.read(np.float32, T * N).reshape(T, N)
    assert_close(got, np.asarray(a, np.float64) @ deq.T, what="prefill GEMM")


# (100, 8192, 1024): Q4 takes the 128x64 pair tile with K split (64 tiles of one
# 128-row tile, half the CU count or more); (288, 512, 1024) and (300, 192, 3840):
# the first 256 tokens on the tiles, the rest on the weight-streaming GEMM;
# (352, 192, 1024): the rest of 96 tokens on the tiles
@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8, gh.QUANT_NONE])
@pytest.mark.parametrize("T,N,K", [(1, 64, 128), (45, 192, 512), (256, 512, 3840),
                                   (100, 8192, 1024), (288, 512, 1024), (300, 192, 3840),
                                   (352, 192, 1024)])
def test_prefill_gate_up_geglu(gpu, mode, T, N, K):
    gq, gdeq = quantized(N, K, mode, 310)
    uq, udeq = quantized(N, K, mode, 311)
    a = gh.synth_normal(T * K, 1, 312, 0.0, 1.0).reshape(T, K)
    Wg, Wu, A, act = gpu.upload(gq), gpu.upload(uq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gate_up_geglu(mode, Wg, Wu, A, act, T, N, K)
    got = act.read(np.float32, T * N).reshape(T, N)
    a64 = np.asarray(a, np.float64)
    ref = nr.gelu64(a64 @ gdeq.T) * (a64 @ udeq.T)
    assert_close(got, ref, what="prefill GeGLU")


# The 128x64 gate/up tile (gh_pf_gateup_q{4,8}_m128_n64_k1) runs when
# ceil(N / 64) * ceil(T / 128) reaches the CU count (256): the 12B gate/up of
# a 512-token prompt (960 tiles) and a ragged 129-token batch of exactly 256
# tiles (its second 128-row tile holds one token).
@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8, gh.QUANT_NONE])
@pytest.mark.parametrize("T,N,K", [(512, 15360, 3840), (129, 8192, 512)])
def test_prefill_gate_up_large_tiles(gpu, mode, T, N, K):
    assert -(-N // 64) * -(-T // 128) >= 256
    gq, gdeq = quantized(N, K, mode, 340)
    uq, udeq = quantized(N, K, mode, 341)
    a = gh.synth_normal(T * K, 1, 342, 0.0, 1.0).reshape(T, K)
    Wg, Wu, A, act = gpu.upload(gq), gpu.upload(uq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gate_up_geglu(mode, Wg, Wu, A, act, T, N, K)
    got = act.read(np.float32, T * N).reshape(T, N)
    a64 = np.asarray(a, np.float64)
    ref = nr.gelu64(a64 @ gdeq.T) * (a64 @ udeq.T)
    del gdeq, udeq
    assert_close(got, ref, what="prefill GeGLU, 128x64 tiles")
    for t in (0, T - 1):  # first and last rows, one of them alone in its tile
        assert_close(got[t], ref[t], what="prefill GeGLU row %d" % t)


def test_prefill_gemm_row_range(gpu):
    # rows far outside fp16 range (1e6, 1e-7), a zero row and mixed magnitudes
    # within a row: the per-row power-of-two scale keeps every row exact to
    # the tolerance
    T, N, K = 6, 128, 512
    wq, deq = quantized(N, K, gh.QUANT_Q4, 330)
    a = gh.synth_normal(T * K, 1, 331, 0.0, 1.0).reshape(T, K).astype(np.float64)
    a[0] *= 1e6
    a[1] *= 1e-7
    a[2] = 0.0
    a[3, ::2] *= 1e4
    a = a.astype(np.float32)
    W, A, C = gpu.upload(wq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gemm(gh.QUANT_Q4, W, A, C, T, N, K)
    got = C.read(np.float32, T * N).reshape(T, N)
    ref = np.asarray(a, np.float64) @ deq.T
    for t in range(T):
        if t == 2:
            assert np.all(got[t] == 0.0)
        else:
            assert_close(got[t], ref[t], what="prefill GEMM row %d" % t)


def test_prefill_gemm_weight_scale_range(gpu):
    # Q4 weights enter as two exact fp16 operands per block, (n - 8) times the
    # 8-bit pieces of S d with S a power of two per weight row: rows whose
    # blocks span 2^-24 .. 2^12 of each other, large and tiny rows, all-zero
    # blocks and an all-zero row, against the fp64 product
    T, N, K = 9, 64, 1024
    rng = np.random.default_rng(5)
    w = gh.synth_normal(N * K, 0, 350, 0.0, 0.02).reshape(N, K).astype(np.float64)
    blocks = w.reshape(N, K // 32, 32)
    blocks *= 2.0 ** rng.integers(-24, 13, size=(N, K // 32, 1))
    blocks[1] *= 1e3
    blocks[2] *= 1e-6
    blocks[3, ::3] = 0.0
    blocks[4] = 0.0
    wq = nr.quantize_q4(nr.bf16_rne(w.astype(np.float32)))
    deq = nr.dequant_q4(wq, K)
    a = gh.synth_normal(T * K, 1, 351, 0.0, 1.0).reshape(T, K)
    W, A, C = gpu.upload(wq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gemm(gh.QUANT_Q4, W, A, C, T, N, K)
    got = C.read(np.float32, T * N).reshape(T, N)
    ref = np.asarray(a, np.float64) @ deq.T
    assert np.all(got[:, 4] == 0.0)
    for n in (0, 1, 2, 3, 5, 63):  # each weight row against its own magnitude
        assert_close(got[:, n], ref[:, n], what="prefill GEMM weight row %d" % n)


# Batches of at most 48 tokens with K a multiple of 128 run the
# weight-streaming GEMM (16-token groups on the 16x16x32 MFMA; 8-wave
# workgroups with two groups per wave from 17 tokens and three from 33, where
# their LDS fits; K in slices staged in LDS, the slices' planes added in
# order).  One token; 16; 17 and 32; 33, 40, 45 and 48 (narrower slices); a
# ragged N; the 12B K values (3840, 4096, 15360); K of four quant blocks (one
# slice, a partial weight set).  K = 160 and 49 tokens take the tile GEMM.
STREAM_SHAPES = [(1, 64, 128), (4, 100, 3840), (16, 256, 4096), (13, 96, 15360), (16, 48, 2048),
                 (9, 512, 128), (17, 96, 3840), (32, 200, 4096), (27, 64, 15360), (6, 40, 160),
                 (33, 64, 256), (40, 96, 3840), (48, 200, 4096), (45, 64, 15360), (49, 64, 256)]


@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8, gh.QUANT_NONE])
@pytest.mark.parametrize("T,N,K", STREAM_SHAPES)
def test_prefill_stream_gemm(gpu, mode, T, N, K):
    wq, deq = quantized(N, K, mode, 360 + T)
    a = gh.synth_normal(T * K, 1, 361, 0.0, 1.0).reshape(T, K)
    W, A, C = gpu.upload(wq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gemm(mode, W, A, C, T, N, K)
    got = C.read(np.float32, T * N).reshape(T, N)
    assert_close(got, np.asarray(a, np.float64) @ deq.T, what="streamed prefill GEMM")


@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8, gh.QUANT_NONE])
@pytest.mark.parametrize("T,N,K", [(3, 200, 3840), (16, 64, 1024), (11, 16, 15360),
                                   (24, 300, 3840), (32, 48, 1024), (40, 300, 3840),
                                   (48, 48, 1024)])
def test_prefill_stream_gate_up(gpu, mode, T, N, K):
    gq, gdeq = quantized(N, K, mode, 370)
    uq, udeq = quantized(N, K, mode, 371)
    a = gh.synth_normal(T * K, 1, 372, 0.0, 1.0).reshape(T, K)
    Wg, Wu, A, act = gpu.upload(gq), gpu.upload(uq), gpu.upload(a), gpu.alloc(T * N * 4)
    gpu.prefill_gate_up_geglu(mode, Wg, Wu, A, act, T, N, K)
    got = act.read(np.float32, T * N).reshape(T, N)
    a64 = np.asarray(a, np.float64)
    assert_close(got, nr.gelu64(a64 @ gdeq.T) * (a64 @ udeq.T), what="streamed prefill GeGLU")


@pytest.mark.parametrize("T", [7, 16, 29, 41])
@pytest.mark.parametrize("shape", ["8,1", "16,2", "4,3", "4,8", "24,1", "32,2", "12,2"])
def test_prefill_stream_slices(gpu, monkeypatch, T, shape):
    # forced slice widths (KR quant blocks: 32 blocks of K in 1, 2, 3, 4 or 8
    # slices; 24 and 12 leave an uneven last slice, and 12 and 4 a partial
    # weight set) and row groups per wave (8: waves whose rows all lie past N);
    # at 29 and 41 tokens the widths whose LDS does not fit fall back to the
    # default
    T_, N, K = T, 300, 1024
    monkeypatch.setenv("GH_PF_STREAM", shape)
    gq, gdeq = quantized(N, K, gh.QUANT_Q4, 380)
    uq, udeq = quantized(N, K, gh.QUANT_Q4, 381)
    a = gh.synth_normal(T_ * K, 1, 382, 0.0, 1.0).reshape(T_, K)
    A, C = gpu.upload(a), gpu.alloc(T_ * N * 4)
    a64 = np.asarray(a, np.float64)
    gpu.prefill_gemm(gh.QUANT_Q4, gpu.upload(gq), A, C, T_, N, K)
    assert_close(C.read(np.float32, T_ * N).reshape(T_, N), a64 @ gdeq.T,
                 what="streamed GEMM, slices %s" % shape)
    gpu.prefill_gate_up_geglu(gh.QUANT_Q4, gpu.upload(gq), gpu.upload(uq), A, C, T_, N, K)
    assert_close(C.read(np.float32, T_ * N).reshape(T_, N),
                 nr.gelu64(a64 @ gdeq.T) * (a64 @ udeq.T), what="streamed GeGLU, slices %s" % shape)


@pytest.mark.parametrize("N", [320, 203])
@pytest.mark.parametrize("pair", [False, True])
@pytest.mark.parametrize("split", ["1", "3", "200"])
def test_prefill_split_k(gpu, monkeypatch, pair, split, N):
    # a few tokens on the tile GEMM (the streaming form switched off): the
    # split-K forms (forced 1 = unsplit, 3 = an even split of 120 K steps,
    # 200 = clamped to the 64-split cap, so one or two K steps per split)
    # against the product; N = 203 leaves T N % 4 != 0, so the plane sum
    # takes its one-output-per-thread form
    T, K = 5, 3840
    monkeypatch.setenv("GH_PF_NO_STREAM", "1")
    monkeypatch.setenv("GH_PF_SPLIT", split)
    gq, gdeq = quantized(N, K, gh.QUANT_Q4, 320)
    uq, udeq = quantized(N, K, gh.QUANT_Q4, 321)
    a = gh.synth_normal(T * K, 1, 322, 0.0, 1.0).reshape(T, K)
    A, C = gpu.upload(a), gpu.alloc(T * N * 4)
    a64 = np.asarray(a, np.float64)
    if pair:
        gpu.prefill_gate_up_geglu(gh.QUANT_Q4, gpu.upload(gq), gpu.upload(uq), A, C, T, N, K)
        ref = nr.gelu64(a64 @ gdeq.T) * (a64 @ udeq.T)
    else:
        gpu.prefill_gemm(gh.QUANT_Q4, gpu.upload(gq), A, C, T, N, K)
        ref = a64 @ gdeq.T
    assert_close(C.read(np.float32, T * N).reshape(T, N), ref, what="split-K %s" % split)


def test_prefill_gemm_rejects_bad_shapes(gpu):
    W, A, C = gpu.alloc(4096), gpu.alloc(4096), gpu.alloc(4096)
    with pytest.raises(gh.GhError):
        gpu.prefill_gemm(gh.QUANT_Q4, W, A, C, 4, 8, 100)  # K % 32
    with pytest.raises(gh.GhError):
        gpu.prefill_gemm(3, W, A, C, 4, 8, 128)  # no such weight mode
    with pytest.raises(gh.GhError):  # bf16 rows are read 16 bytes at a time
        gpu.prefill_gemm(gh.QUANT_NONE, W.ptr + 4, A, C, 4, 8, 128)


def tiny_cfg(**kw):
    args = dict(vocab=1024, hidden=256, intermediate=512, layers=3, heads=4, kv_heads=2,
                head_dim=64, max_slots=24, global_kv_heads=2, global_head_dim=128,
                full_layers=(2,))
    args.update(kw)
    return gh.model_config(**args)


def ring_lists(ring, clocks):
    slots, actives = [], []
    for c in clocks:
        slots.append(ring.activate_slot(0, c))
        actives.append(np.array(ring.active_slots(0, c), np.uint32))
    return slots, actives


@pytest.mark.parametrize("mode,T,dup,seq_max", [
    (gh.QUANT_Q4, 12, False, None), (gh.QUANT_Q8, 12, False, None), (gh.QUANT_Q4, 11, False, None),
    (gh.QUANT_Q8, 9, True, None), (gh.QUANT_Q4, 3, False, None), (gh.QUANT_Q8, 2, False, None),
    (gh.QUANT_Q4, 3, False, "0"), (gh.QUANT_Q4, 1, False, "0"), (gh.QUANT_Q4, 3, False, "3"),
    (gh.QUANT_Q8, 1, False, None)])
def test_model_prefill_matches_sequential_oracle(gpu, monkeypatch, mode, T, dup, seq_max):
    # T prompt tokens (4 anchors, then the window), one batch, then decode
    # steps through the per-token graph on the caches the prefill wrote.  T
    # not a multiple of 4 leaves a partial token group in the grouped
    # attention; dup names one slot twice in the last token's list (counted
    # twice, as the reference's loop over the list does), which keeps the
    # batch on the per-token attention kernel.  Batches of 1-2 tokens (Q4;
    # 1 token with Q8 weights) run token by token unless GH_PF_SEQ_MAX=0 keeps
    # them on the batched kernels (GH_PF_SEQ_MAX=3 sends 3 tokens token by
    # token)
    if seq_max is not None:
        monkeypatch.setenv("GH_PF_SEQ_MAX", seq_max)
    cfg = tiny_cfg()
    m = gh.Model(gpu, cfg, mode=mode, seed=11)
    try:
        om, layers = oracle_model(m, cfg, mode)
        ring = gh.Ring(cfg.num_hidden_layers, 4, 16, 4)
        tokens = np.random.default_rng(5).integers(0, cfg.vocab_size, 14)
        xs = np.stack([m.embed(int(t)) for t in tokens])
        slots, actives = ring_lists(ring, range(T))
        if dup:
            actives[-1] = np.append(actives[-1], actives[-1][0])
        tok = m.prefill(xs[:T], np.arange(T), slots, actives, True)
        for c in range(T):
            rtok, _, rlog = om.forward(xs[c], c, slots[c], actives[c], c == T - 1, NT)
        logits = m.read(-1, gh.T_LOGITS, np.float32)
        assert_close(logits, rlog, what="prefill last-token logits")
        assert tok == orc.argmax(logits)
        for l, d in enumerate(layers):
            kvd = d["num_kv_heads"] * d["head_dim"]
            kc = m.read(l, gh.T_K_CACHE, np.float32).reshape(cfg.max_slots, kvd)
            vc = m.read(l, gh.T_V_CACHE, np.float32).reshape(cfg.max_slots, kvd)
            assert_close(kc[slots], d["k_cache"][slots], what="prefill K cache layer %d" % l)
            assert_close(vc[slots], d["v_cache"][slots], what="prefill V cache layer %d" % l)
        for c in range(T, 14):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            tok = m.forward(xs[c], c, slot, act, True)
            rtok, _, rlog = om.forward(xs[c], c, slot, act, True, NT)
            assert_close(m.read(-1, gh.T_LOGITS, np.float32), rlog, what="decode after prefill")
    finally:
        m.close()


def test_model_prefill_norm_forms_bit_identical(gpu, monkeypatch):
    # the row norm runs 512-thread workgroups for rows of up to 4096 and
    # 1024-thread ones above; the extra waves only add zeros to the row sums,
    # so GH_PF_NORM_1024 (the wide form on a narrow row) must change no bit
    cfg = tiny_cfg()
    m = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=13)
    try:
        tokens = np.random.default_rng(6).integers(0, cfg.vocab_size, 12)
        xs = np.stack([m.embed(int(t)) for t in tokens])
        out = []
        for wide in (False, True):
            if wide:
                monkeypatch.setenv("GH_PF_NORM_1024", "1")
            ring = gh.Ring(cfg.num_hidden_layers, 4, 16, 4)
            slots, actives = ring_lists(ring, range(12))
            tok = m.prefill(xs, np.arange(12), slots, actives, True)
            out.append((tok, m.read(-1, gh.T_LOGITS, np.float32).copy(),
                        m.read(0, gh.T_K_CACHE, np.float32).copy()))
        assert out[0][0] == out[1][0]
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
        assert np.array_equal(out[0][2].view(np.uint32), out[1][2].view(np.uint32))
    finally:
        m.close()


@pytest.mark.parametrize("T", [40, 37, 48])
def test_model_prefill_equals_per_token_path(gpu, T):
    # the batched prefill and T per-token calls leave the same caches (to
    # tolerance) and pick the same final token on a 12B-width layer pair
    cfg = gh.model_config(vocab=4096, hidden=3840, intermediate=15360, layers=2, heads=16,
                          kv_heads=8, head_dim=256, max_slots=64, full_layers=(1,))
    a = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=3)
    b = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=3)
    try:
        ring_a, ring_b = gh.Ring(2, 8, 48, 8), gh.Ring(2, 8, 48, 8)
        tokens = np.random.default_rng(9).integers(0, cfg.vocab_size, T)
        xs = np.stack([a.embed(int(t)) for t in tokens])
        slots, actives = ring_lists(ring_a, range(T))
        a.prefill(xs, np.arange(T), slots, actives, True)
        for c in range(T):
            slot = ring_b.activate_slot(0, c)
            b.forward(xs[c], c, slot, ring_b.active_slots(0, c), c == T - 1)
        assert_close(a.read(-1, gh.T_LOGITS, np.float32), b.read(-1, gh.T_LOGITS, np.float32),
                     what="prefill vs per-token logits")
        for l in range(2):
            for t in (gh.T_K_CACHE, gh.T_V_CACHE):
                ka = a.read(l, t, np.float32).reshape(64, -1)[slots]
                kb = b.read(l, t, np.float32).reshape(64, -1)[slots]
                assert_close(ka, kb, what="prefill vs per-token cache %d/%d" % (l, t))
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("shape", ["12b", "tiny", "g4", "g1", "12b-pertoken"])
def test_model_prefill_windowed_lists(gpu, monkeypatch, shape):
    # explicit lists with a sliding window (slot 0 as an anchor plus the last
    # 10 slots): within a token group the later tokens drop slots the earlier
    # ones still attend to, so the grouped attention's token masks decide which
    # union entries each token uses; checked against T per-token calls with the
    # same lists and against the oracle token by token, at 12B width (head_dim
    # 256: the matrix-core kernel, which batches of at most 64 tokens take only
    # with GH_PF_ATTN_MFMA=1; "12b-pertoken" keeps the per-token kernel they
    # take by default) and on the tiny model (head_dim 64/128: the 4-token
    # vector-ALU kernel); g4 and g1
    # are head_dim-256 models with 4 and 1 query heads per kv head, so the
    # matrix-core kernel's 16 columns are 4 tokens x 4 heads and 16 tokens x 1
    if shape in ("12b", "g4", "g1"):
        monkeypatch.setenv("GH_PF_ATTN_MFMA", "1")
    if shape == "12b-pertoken":
        shape = "12b"
    if shape == "g4" or shape == "g1":
        cfg = gh.model_config(vocab=1024, hidden=1024, intermediate=2048, layers=1,
                              heads=8 if shape == "g4" else 4, kv_heads=2 if shape == "g4" else 4,
                              head_dim=256, max_slots=64, full_layers=())
        T = 37
    elif shape == "12b":
        cfg = gh.model_config(vocab=4096, hidden=3840, intermediate=15360, layers=1, heads=16,
                              kv_heads=8, head_dim=256, max_slots=64, full_layers=())
        T = 29
    else:
        cfg = tiny_cfg()
        T = 21
    a = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=4)
    b = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=4)
    try:
        om, layers = oracle_model(a, cfg, gh.QUANT_Q4)
        tokens = np.random.default_rng(13).integers(0, cfg.vocab_size, T)
        xs = np.stack([a.embed(int(t)) for t in tokens])
        slots = list(range(T))
        actives = [np.array(sorted({0} | set(range(max(0, t - 9), t + 1))), np.uint32)
                   for t in range(T)]
        a.prefill(xs, np.arange(T), slots, actives, True)
        for c in range(T):
            b.forward(xs[c], c, slots[c], actives[c], c == T - 1)
            _, _, rlog = om.forward(xs[c], c, slots[c], actives[c], c == T - 1, NT)
        logits = a.read(-1, gh.T_LOGITS, np.float32)
        assert_close(logits, rlog, what="windowed prefill logits vs oracle")
        assert_close(logits, b.read(-1, gh.T_LOGITS, np.float32),
                     what="windowed prefill vs per-token logits")
        for l, d in enumerate(layers):
            for t, ref in ((gh.T_K_CACHE, d["k_cache"]), (gh.T_V_CACHE, d["v_cache"])):
                ka = a.read(l, t, np.float32).reshape(cfg.max_slots, -1)[slots]
                kb = b.read(l, t, np.float32).reshape(cfg.max_slots, -1)[slots]
                assert_close(ka, ref[slots], what="windowed prefill cache %d/%d vs oracle" % (l, t))
                assert_close(ka, kb, what="windowed prefill vs per-token cache %d/%d" % (l, t))
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("splits", [None, "3", "16"])
@pytest.mark.parametrize("case", ["slot twice", "reads a later write", "wrapped window"])
def test_model_prefill_staged_batch_matches_sequential_oracle(gpu, monkeypatch, case, splits):
    # splits: each token's list split over that many workgroups of the
    # per-token attention (as long lists are), merged by gh_pf_attn_merge_k;
    # 16 leaves some splits empty
    if splits is not None:
        monkeypatch.setenv("GH_PF_ATTN_SPLITS", splits)
    # batches whose order the batched kernels cannot keep by writing in place
    # (every token's K/V is written before any token attends): one slot
    # written twice, a token attending to the slot a later token overwrites,
    # and a whole prompt past the window's wraparound.  They write staging
    # rows and move them into the slots after the layers; checked against the
    # oracle run token by token and against the GPU's per-token path
    cfg = tiny_cfg(layers=2, full_layers=(1,))
    m = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=2)
    p = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=2)
    try:
        om, layers = oracle_model(m, cfg, gh.QUANT_Q4)
        xs = np.stack([m.embed(i * 37 % cfg.vocab_size) for i in range(40)])
        if case == "slot twice":
            first, slots = 0, [5, 6, 7, 8, 5]
            lists = [[5], [5, 6], [5, 6, 7], [5, 6, 7, 8], [5, 6, 7, 8]]
        elif case == "reads a later write":
            first, slots = 0, [5, 6, 7, 8, 9]
            lists = [[5, 6], [5, 6], [5, 6, 7], [5, 6, 7, 8], [5, 6, 7, 8, 9]]
        else:  # ring of 4 anchors + 16 window slots: clocks 0..19 one by one, then 20..39
            ring = gh.Ring(1, 4, 16, 4)
            for c in range(20):
                slot = ring.activate_slot(0, c)
                act = ring.active_slots(0, c)
                m.forward(xs[c], c, slot, act, False)
                p.forward(xs[c], c, slot, act, False)
                om.forward(xs[c], c, slot, act, False, NT)
            first = 20
            slots = [ring.activate_slot(0, c) for c in range(20, 40)]
            lists = [ring.active_slots(0, c) for c in range(20, 40)]
        T = len(slots)
        clocks = np.arange(first, first + T)
        tok = m.prefill(xs[first:first + T], clocks, slots, [np.array(a, np.uint32) for a in lists], True)
        for i in range(T):
            want = i == T - 1
            ptok = p.forward(xs[first + i], first + i, slots[i], np.array(lists[i], np.uint32), want)
            rtok, _, rlog = om.forward(xs[first + i], first + i, slots[i], np.array(lists[i], np.uint32),
                                       want, NT)
        logits = m.read(-1, gh.T_LOGITS, np.float32)
        assert_close(logits, rlog, what="staged prefill logits vs oracle")
        assert_close(logits, p.read(-1, gh.T_LOGITS, np.float32), what="staged vs per-token logits")
        assert tok == orc.argmax(logits) and ptok == orc.argmax(p.read(-1, gh.T_LOGITS, np.float32))
        written = sorted(set(slots))
        for l, d in enumerate(layers):
            kvd = d["num_kv_heads"] * d["head_dim"]
            for t, ref in ((gh.T_K_CACHE, d["k_cache"]), (gh.T_V_CACHE, d["v_cache"])):
                got = m.read(l, t, np.float32).reshape(cfg.max_slots, kvd)
                assert_close(got[written], ref[written], what="staged cache %d/%d" % (l, t))
    finally:
        m.close()
        p.close()


@pytest.mark.parametrize("mfma,splits", [(True, None), (False, None), (False, "4")])
@pytest.mark.parametrize("T", [20, 30])
def test_model_ring_prefill_staged_head_dim_256(gpu, monkeypatch, T, mfma, splits):
    # splits "4": the per-token kernel with each list split 4 ways and merged
    if splits is not None:
        monkeypatch.setenv("GH_PF_ATTN_SPLITS", splits)
    # Staged batches on the matrix-core grouped attention (head_dim 256, 16
    # query / 8 kv heads: 8 tokens per group, a K/V staging row named in the
    # union lists; forced by GH_PF_ATTN_MFMA=1 at these batch sizes) and on
    # the per-token kernel: a ring of 4 anchors + 16 window + 4 recall slots, clocks
    # 0..19 token by token, then T tokens from clock 20 in one
    # gh_model_ring_prefill call, every one past the window's wrap.  T = 30
    # exceeds max_slots (24), so the batch runs as two staged chunks (24 + 6
    # tokens).  Checked against the oracle token by token and against the
    # GPU's per-token path: the last token's logits and every cache row.
    if mfma:
        monkeypatch.setenv("GH_PF_ATTN_MFMA", "1")
    cfg = gh.model_config(vocab=1024, hidden=512, intermediate=1024, layers=2, heads=16,
                          kv_heads=8, head_dim=256, max_slots=24, full_layers=(1,))
    m = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=6)
    p = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=6)
    try:
        om, layers = oracle_model(m, cfg, gh.QUANT_Q4)
        for x in (m, p):
            x.ring_init(4, 16, 4)
        ring = gh.Ring(1, 4, 16, 4)
        xs = np.stack([m.embed(i * 53 % cfg.vocab_size) for i in range(20 + T)])
        for c in range(20):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            m.forward_clock(xs[c], c, False)
            p.forward_clock(xs[c], c, False)
            om.forward(xs[c], c, slot, act, False, NT)
        tok = m.ring_prefill(xs[20:], 20, True)
        for c in range(20, 20 + T):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            ptok = p.forward_clock(xs[c], c, c == 20 + T - 1)
            rtok, _, rlog = om.forward(xs[c], c, slot, act, c == 20 + T - 1, NT)
        logits = m.read(-1, gh.T_LOGITS, np.float32)
        plog = p.read(-1, gh.T_LOGITS, np.float32)
        assert_close(logits, rlog, what="staged head_dim-256 prefill logits vs oracle")
        assert_close(logits, plog, what="staged head_dim-256 prefill vs per-token logits")
        assert tok == orc.argmax(logits) and ptok == orc.argmax(plog)
        # the device rings agree with the host ring after the call
        assert np.array_equal(m.read(-1, gh.T_RING_CLOCKS, np.uint32),
                              p.read(-1, gh.T_RING_CLOCKS, np.uint32))
        for l, d in enumerate(layers):
            for t, ref in ((gh.T_K_CACHE, d["k_cache"]), (gh.T_V_CACHE, d["v_cache"])):
                got = m.read(l, t, np.float32).reshape(cfg.max_slots, -1)
                per = p.read(l, t, np.float32).reshape(cfg.max_slots, -1)
                assert_close(got[:20], ref[:20], what="staged cache %d/%d vs oracle" % (l, t))
                assert_close(got[:20], per[:20], what="staged cache %d/%d vs per-token" % (l, t))
    finally:
        m.close()
        p.close()


def test_model_ring_prefill_staged_chunks_below_ring_size(gpu):
    # A 300-slot cache holds 256 staging rows (min(max_slots, 256)), so a
    # staged batch of 270 tokens runs as chunks of 256 and 14.  Ring of 4
    # anchors + 280 window + 16 recall: clocks 0..283 in one batched call (no
    # slot rewritten), then 270 tokens from clock 284, past the wrap.  Checked
    # against the oracle token by token and against the GPU's per-token path.
    cfg = tiny_cfg(layers=2, full_layers=(1,), max_slots=300)
    m = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=8)
    p = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=8)
    try:
        om, layers = oracle_model(m, cfg, gh.QUANT_Q4)
        for x in (m, p):
            x.ring_init(4, 280, 16)
        ring = gh.Ring(1, 4, 280, 16)
        n0, n1 = 284, 270
        xs = np.stack([m.embed(i * 29 % cfg.vocab_size) for i in range(n0 + n1)])
        m.ring_prefill(xs[:n0], 0, False)
        for c in range(n0):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            p.forward_clock(xs[c], c, False)
            om.forward(xs[c], c, slot, act, False, NT)
        tok = m.ring_prefill(xs[n0:], n0, True)
        for c in range(n0, n0 + n1):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            ptok = p.forward_clock(xs[c], c, c == n0 + n1 - 1)
            rtok, _, rlog = om.forward(xs[c], c, slot, act, c == n0 + n1 - 1, NT)
        logits = m.read(-1, gh.T_LOGITS, np.float32)
        plog = p.read(-1, gh.T_LOGITS, np.float32)
        assert_close(logits, rlog, what="chunked staged prefill logits vs oracle")
        assert_close(logits, plog, what="chunked staged prefill vs per-token logits")
        assert tok == orc.argmax(logits) and ptok == orc.argmax(plog)
        for l, d in enumerate(layers):
            kvd = d["num_kv_heads"] * d["head_dim"]
            for t, ref in ((gh.T_K_CACHE, d["k_cache"]), (gh.T_V_CACHE, d["v_cache"])):
                got = m.read(l, t, np.float32).reshape(cfg.max_slots, kvd)
                assert_close(got[:284], ref[:284], what="chunked staged cache %d/%d" % (l, t))
    finally:
        m.close()
        p.close()

