"""The 12B workload's prompt phase as a checked run: a 512-token batched
prefill at 12B width (hidden 3840, intermediate 15360, 16/8 heads of 256,
vocab 262144; one sliding and one full-attention layer), ring of 32 anchors +
512 window + 96 recall slots, clocks 0..511, then greedy decode steps.

The reference prefills token by token through its decode graph
(src/interactive.zig:33-48, src/gpu/model_dispatch.zig:144), so the batched
result is checked against the oracle's sequential per-token forward: the last
token's logits and greedy token, every K/V row the prompt writes in both
layers, and 8 greedy steps after it.  Slots and active lists come from the
device ring and are compared with the host ring's bit for bit."""
import os

import numpy as np
import pytest

import gemma_hip as gh
import oracle as orc
from model_ref import oracle_model
from test_gpu_model import check_token
from tol import assert_close

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def test_512_token_prefill_then_greedy_12b_width(gpu):
    cfg = gh.model_config(vocab=262144, hidden=3840, intermediate=15360, layers=2, heads=16,
                          kv_heads=8, head_dim=256, max_slots=640, full_layers=[1])
    m = gh.Model(gpu, cfg, mode=gh.QUANT_Q4, seed=1)
    try:
        om, layers = oracle_model(m, cfg)
        m.ring_init(32, 512, 96)
        ring = gh.Ring(1, 32, 512, 96)
        prompt = gh.synth_uniform_u32(512, 1, 0, cfg.vocab_size)
        xs = np.stack([m.embed(int(t)) for t in prompt])
        tok = m.ring_prefill(xs, 0, True)
        print("prefill done, token", tok, flush=True)
        for c in range(512):
            slot = ring.activate_slot(0, c)
            assert slot == c
            active = ring.active_slots(0, c)
            assert len(active) == c + 1
            rtok, _, rlog = om.forward(xs[c], c, slot, active, c == 511, NT)
        check_token(m, rlog, tok, rtok, "512-token prefill, last token")
        for l, d in enumerate(layers):
            kc = m.read(l, gh.T_K_CACHE, np.float32).reshape(640, -1)
            vc = m.read(l, gh.T_V_CACHE, np.float32).reshape(640, -1)
            assert_close(kc[:512], d["k_cache"][:512], what="prefill K rows layer %d" % l)
            assert_close(vc[:512], d["v_cache"][:512], what="prefill V rows layer %d" % l)
            assert not np.any(kc[512:]) and not np.any(vc[512:])  # untouched slots
        embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, cfg.hidden_size)
        for c in range(512, 520):  # greedy decode after the prompt, the device ring
            x = orc.embed(embed, tok, cfg.hidden_size)
            dtok = m.forward_clock(x, c, True)
            slot = ring.activate_slot(0, c)
            active = ring.active_slots(0, c)
            step = m.read(-1, gh.T_STEP, np.uint32)
            assert list(step[:3]) == [c, slot, len(active)]
            assert np.array_equal(m.read(-1, gh.T_ACTIVE, np.uint32)[:len(active)], active)
            rtok, _, rlog = om.forward(x, c, slot, active, True, NT)
            check_token(m, rlog, dtok, rtok, "greedy step at clock %d" % c)
            tok = rtok
    finally:
        m.close()
