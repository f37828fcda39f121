"""Model-level GPU parity: whole decode steps through gh_dispatch_forward_token
against the oracle's forward (src/gpu/model_dispatch.zig op order) on the
same quantized bytes, plus weight ingest from host bf16 tensors."""
import os

import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc
from model_ref import layer_dims, oracle_model
from tol import assert_close, errors

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def tiny_cfg(**kw):
    # 3 layers, the last a full-attention layer with its own head shape
    args = dict(vocab=1024, hidden=256, intermediate=512, layers=3, heads=4, kv_heads=2,
                head_dim=64, max_slots=24, global_kv_heads=2, global_head_dim=128,
                full_layers=(2,))
    args.update(kw)
    return gh.model_config(**args)


def check_token(m, ref_logits, tok, what):
    logits = m.read(-1, gh.T_LOGITS, np.float32)
    assert_close(logits, ref_logits, what=what)
    assert tok == orc.argmax(logits)  # the fused argmax is bit-exact on its own logits
    top = float(np.max(ref_logits))
    assert ref_logits[tok] >= top - 2e-3 * np.max(np.abs(ref_logits))


@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8])
def test_tiny_model_decode_sequence(gpu, mode):
    cfg = tiny_cfg()
    m = gh.Model(gpu, cfg, mode=mode, seed=7)
    try:
        om, layers = oracle_model(m, cfg, mode)
        embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, cfg.hidden_size)
        ring = gh.Ring(cfg.num_hidden_layers, 4, 16, 4)
        tokens = np.random.default_rng(1).integers(0, cfg.vocab_size, 40)
        for clock, t in enumerate(tokens):
            x = m.embed(int(t))
            assert np.array_equal(x, orc.embed(embed, int(t), cfg.hidden_size))
            slot = ring.activate_slot(0, clock)
            active = ring.active_slots(0, clock)
            want = clock % 3 != 1  # interleave the prefill (no-logits) graph
            tok = m.forward(x, clock, slot, active, want)
            rtok, _, rlog = om.forward(x, clock, slot, active, want, NT)
            if want:
                check_token(m, rlog, tok, "tiny step %d" % clock)
            else:
                assert tok == 0
        for l, d in enumerate(layers):
            kvd = d["num_kv_heads"] * d["head_dim"]
            kc = m.read(l, gh.T_K_CACHE, np.float32).reshape(cfg.max_slots, kvd)
            vc = m.read(l, gh.T_V_CACHE, np.float32).reshape(cfg.max_slots, kvd)
            assert_close(kc, d["k_cache"], what="K cache layer %d" % l)
            assert_close(vc, d["v_cache"], what="V cache layer %d" % l)
    finally:
        m.close()


def test_model_init_from_host_bf16(gpu):
    # gh_model_init quantizes borrowed host bf16 tensors with quantizeMatrix's bytes
    cfg = tiny_cfg(layers=2, full_layers=())
    H, I, V, nq = 256, 512, 1024, 4
    rng = np.random.default_rng(3)
    bf = lambda *s, mean=0.0, std=0.02: nr.bf16_rne((mean + std * rng.standard_normal(s)).astype(np.float32))  # noqa: E731
    layers = []
    for l in range(2):
        d = layer_dims(cfg, l)
        qd, kvd = nq * d["head_dim"], d["num_kv_heads"] * d["head_dim"]
        w = dict(q_proj=bf(qd, H), k_proj=bf(kvd, H), o_proj=bf(H, qd), gate_proj=bf(I, H),
                 up_proj=bf(I, H), down_proj=bf(H, I), input_layernorm=bf(H, mean=1, std=0.1),
                 q_norm=bf(d["head_dim"], mean=1, std=0.1), k_norm=bf(d["head_dim"], mean=1, std=0.1),
                 post_attention_layernorm=bf(H, mean=1, std=0.1),
                 pre_feedforward_layernorm=bf(H, mean=1, std=0.1),
                 post_feedforward_layernorm=bf(H, mean=1, std=0.1), layer_scalar=0.5)
        if l == 0:
            w["v_proj"] = bf(kvd, H)
        layers.append(w)  # layer 1 has no v_proj: the key projection serves as value
    embed = bf(V, H)
    fnorm = bf(H, mean=1, std=0.1)
    m = gh.Model(gpu, cfg, layers=layers, embed=embed, final_norm=fnorm)
    try:
        w0 = layers[0]
        qkv = m.read(0, gh.T_QKV, np.uint32).reshape(-1, (H // 32) * 5)
        assert np.array_equal(qkv, orc.quantize_q4(np.concatenate([w0["q_proj"], w0["k_proj"], w0["v_proj"]])))
        assert np.array_equal(m.read(1, gh.T_QKV, np.uint32).reshape(-1, (H // 32) * 5),
                              orc.quantize_q4(np.concatenate([layers[1]["q_proj"], layers[1]["k_proj"]])))
        assert np.array_equal(m.read(0, gh.T_DOWN, np.uint32).reshape(H, -1), orc.quantize_q4(w0["down_proj"]))
        assert np.array_equal(m.read(-1, gh.T_LM_HEAD, np.uint32).reshape(V, -1), orc.quantize_q8(embed))
        assert np.array_equal(m.read(0, gh.T_Q_NORM, np.float32), nr.bf16_to_f32(w0["q_norm"]))
        om, _ = oracle_model(m, cfg)
        for l in range(2):
            om._layers[l].layer_scalar = 0.5
        ring = gh.Ring(2, 4, 16, 4)
        for clock, t in enumerate([5, 77, 1000, 3, 3, 900]):
            x = orc.embed(embed, t, H)
            slot = ring.activate_slot(0, clock)
            active = ring.active_slots(0, clock)
            tok = m.forward(x, clock, slot, active)
            _, _, rlog = om.forward(x, clock, slot, active, True, NT)
            check_token(m, rlog, tok, "host-weights step %d" % clock)
    finally:
        m.close()


def _12b(layers, full_layers):
    return gh.model_config(vocab=262144, hidden=3840, intermediate=15360, layers=layers,
                           heads=16, kv_heads=8, head_dim=256, max_slots=640,
                           full_layers=full_layers)


def _populated_step(gpu, cfg):
    """A model with every ring cache filled (K ~ N(0,1), V unit-RMS rows) and
    the clock at 600 (S = 544 active slots); returns what both sides need."""
    nl = cfg.num_hidden_layers
    m = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=1)
    ring = gh.Ring(nl, 32, 512, 96)
    for c in range(600):
        ring.activate_slot(0, c)
    clock = 600
    slot = ring.activate_slot(0, clock)
    active = ring.active_slots(0, clock)
    assert len(active) == 544
    rng = np.random.default_rng(600)
    for l in range(nl):
        k = rng.standard_normal((640, 8, 256), dtype=np.float32)
        v = rng.standard_normal((640, 8, 256), dtype=np.float32)
        v /= np.sqrt(np.mean(v * v, axis=2, keepdims=True) + 1e-6)
        m.write(l, gh.T_K_CACHE, k)
        m.write(l, gh.T_V_CACHE, v)
    om, layers = oracle_model(m, cfg)
    return m, om, layers, clock, slot, active


def test_12b_width_two_layers_strict(gpu):
    # 12B widths, one sliding and one full-attention layer, 544 active slots:
    # logits within the 2e-3 bar elementwise and the greedy token bit-exact.
    m, om, layers, clock, slot, active = _populated_step(gpu, _12b(2, [1]))
    try:
        x = m.embed(4242)
        tok = m.forward(x, clock, slot, active)
        rtok, _, rlog = om.forward(x, clock, slot, active, True, NT)
        check_token(m, rlog, tok, "12B-width 2 layers")
        assert tok == rtok
        for l in (0, 1):
            kc = m.read(l, gh.T_K_CACHE, np.float32).reshape(640, -1)
            assert_close(kc[slot], layers[l]["k_cache"][slot], what="K row layer %d" % l)
    finally:
        m.close()


def test_12b_shaped_decode_step(gpu):
    # The full 12B shape: 48 layers (global iff (l+1) % 6 == 0).  A random-init
    # 48-layer stack amplifies rounding differences about 1.2x per layer: the
    # oracle's own logits move by ~3% normwise when its input is perturbed by
    # 1e-6, so the bound here is the greedy token bit-exact and the logit error
    # within 3x that measured sensitivity (the 2e-3 bar is met at 1-2 layers,
    # test above).
    m, om, layers, clock, slot, active = _populated_step(
        gpu, _12b(48, [l for l in range(48) if (l + 1) % 6 == 0]))
    try:
        caches = [(d["k_cache"].copy(), d["v_cache"].copy()) for d in layers]
        x = m.embed(123456)
        tok = m.forward(x, clock, slot, active)
        logits = m.read(-1, gh.T_LOGITS, np.float32)
        rtok, _, rlog = om.forward(x, clock, slot, active, True, NT)
        row_ref = layers[0]["k_cache"][slot].copy()
        for d, (kc, vc) in zip(layers, caches):
            d["k_cache"][:] = kc
            d["v_cache"][:] = vc
        xp = (x * (1 + 1e-6 * np.sign(np.sin(np.arange(x.size))))).astype(np.float32)
        _, _, rlog_p = om.forward(xp, clock, slot, active, True, NT)
        sens = errors(rlog_p, rlog)[0]
        err = errors(logits, rlog)[0]
        assert tok == rtok and tok == orc.argmax(logits)
        assert err <= max(2e-3, 3 * sens), (err, sens)
        kc = m.read(0, gh.T_K_CACHE, np.float32).reshape(640, -1)
        assert_close(kc[slot], row_ref, what="K row layer 0")
    finally:
        m.close()
