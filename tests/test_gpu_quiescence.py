"""Layer gating ("quiescence", src/gpu/model_dispatch.zig:45-101,
shaders/quiescence_gate.wgsl:16-62) on the GPU against the gated oracle
(oracle.c orc_forward_token_gated): the same layers run or are skipped at
every step, with the same logits, tokens and K/V caches.

The gate compares a mean square with the threshold, and the device and the
oracle sum it in different orders, so the threshold is chosen (from the
oracle's own run) with every gate's value at least 5% away from it."""
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
TOKENS = [5, 5, 5, 5, 9, 9, 9, 100, 100, 7, 7, 7, 7, 7, 300, 300, 41, 41, 41]
PROMPT = 6  # one prefill call, then one step per token


def _cfg():
    # 6 layers: 0 and 1 always run (6 // 3), 2..5 gated; layer 5 full attention
    return gh.model_config(vocab=512, hidden=256, intermediate=512, layers=6, heads=4,
                           kv_heads=2, head_dim=64, max_slots=32, global_kv_heads=2,
                           global_head_dim=128, full_layers=(5,))


def _oracle_run(m, cfg, embed, thr, record=None, mode=gh.QUANT_Q4, prompt=PROMPT):
    """The reference sequence on the oracle: the prompt tokens before the
    last through the prefill graph (gates at threshold 0), then the last
    prompt token, which computes the logits, and the decode steps through the
    decode graph gated at thr (forwardToken's compute_logits selects it,
    src/model/forward.zig:41-45; src/gpu/model_gpu.zig:182-183).  Returns
    per step (token, logits, run, motions, gated at thr)."""
    om, layers = oracle_model(m, cfg, mode)
    ring = gh.Ring(1, 4, 24, 4)
    L, H = cfg.num_hidden_layers, cfg.hidden_size
    xp = np.zeros((L, H), np.float32)
    out = []
    for c, t in enumerate(TOKENS):
        x = orc.embed(embed, t, H)
        slot = ring.activate_slot(0, c)
        act = ring.active_slots(0, c)
        before = xp.copy()
        gated = c >= prompt - 1
        tok, _, lg, run = om.forward_gated(x, c, slot, act, xp, thr if gated else 0.0, gated, NT)
        motion = np.mean((xp.astype(np.float64) - before) ** 2, axis=1)
        out.append((tok, lg, run.copy(), motion, gated))
    return out, layers


@pytest.mark.parametrize("mode,prompt", [(gh.QUANT_Q4, PROMPT), (gh.QUANT_Q8, PROMPT),
                                         (gh.QUANT_NONE, PROMPT), (gh.QUANT_Q4, 3)])
def test_quiescence_gating_matches_oracle(gpu, mode, prompt):
    # every weight mode's gated QKV stream (the gate in its prologue); mode
    # none: bf16 layers and the gated bf16 streams.  The prompt's tokens
    # before the last run every layer (batched, or for a 3-token prompt token
    # by token through the prefill graph); its last token, which computes the
    # logits, runs the gated decode graph
    PROMPT = prompt
    cfg = _cfg()
    m = gh.Model(gpu, cfg, mode=mode, seed=21)
    try:
        embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, cfg.hidden_size)
        dl = cfg.num_hidden_layers // 3
        thr = None
        for cand in (0.1, 0.07, 0.15, 0.2, 0.05, 0.3):
            ref, _ = _oracle_run(m, cfg, embed, cand, mode=mode, prompt=PROMPT)
            motions = np.concatenate([r[3][dl:] for r in ref if r[4]])
            runs = np.concatenate([r[2][dl:] for r in ref if r[4]])
            if np.all(np.abs(motions - cand) > 0.05 * cand) and 0 < runs.sum() < runs.size:
                thr = cand
                break
        assert thr is not None, "no threshold with a 5% margin"
        ref, layers = _oracle_run(m, cfg, embed, thr, mode=mode, prompt=PROMPT)
        m.set_quiescence(thr)
        ring = gh.Ring(1, 4, 24, 4)
        xs = np.stack([orc.embed(embed, t, cfg.hidden_size) for t in TOKENS])
        slots = [ring.activate_slot(0, c) for c in range(PROMPT)]
        lists = [ring.active_slots(0, c) for c in range(PROMPT)]
        tok = m.prefill(xs[:PROMPT], np.arange(PROMPT), slots, lists, True)
        check_token(m, ref[PROMPT - 1][1], tok, ref[PROMPT - 1][0], "prompt")
        flags = m.read(-1, gh.T_GATE_FLAGS, np.uint32)
        assert list(flags) == list(ref[PROMPT - 1][2]), (list(flags), list(ref[PROMPT - 1][2]))
        skipped = int((ref[PROMPT - 1][2] == 0).sum())
        for c in range(PROMPT, len(TOKENS)):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            tok = m.forward(xs[c], c, slot, act, True)
            rtok, rlog, run, _, _ = ref[c]
            flags = m.read(-1, gh.T_GATE_FLAGS, np.uint32)
            assert list(flags) == list(run), (c, list(flags), list(run))
            skipped += int((run == 0).sum())
            check_token(m, rlog, tok, rtok, "gated step %d" % c)
        assert skipped > 0
        # skipped layers wrote no K/V: every cache row matches the oracle's
        for l, d in enumerate(layers):
            kvd = d["k_cache"].shape[1]
            kc = m.read(l, gh.T_K_CACHE, np.float32).reshape(cfg.max_slots, kvd)
            assert_close(kc[:len(TOKENS)], d["k_cache"][:len(TOKENS)], what="K cache layer %d" % l)
    finally:
        m.close()


def test_quiescence_off_and_threshold_zero_paths(gpu):
    # threshold 0 = ungated graph; a negative threshold gates with every gate
    # open: both give the ungated logits, and the gated graph records x_prev
    cfg = _cfg()
    ma, mb = gh.Model(gpu, cfg, seed=22), gh.Model(gpu, cfg, seed=22)
    try:
        mb.set_quiescence(-1.0)
        ring = gh.Ring(1, 4, 24, 4)
        for c, t in enumerate((3, 3, 17)):
            slot = ring.activate_slot(0, c)
            act = ring.active_slots(0, c)
            x = ma.embed(t)
            assert ma.forward(x, c, slot, act) == mb.forward(x, c, slot, act)
            assert_close(mb.read(-1, gh.T_LOGITS, np.float32), ma.read(-1, gh.T_LOGITS, np.float32),
                         rtol=1e-4, what="gated, all open")
            assert np.all(mb.read(-1, gh.T_GATE_FLAGS, np.uint32) == 1)
        prev = mb.read(-1, gh.T_GATE_PREV, np.float32).reshape(6, -1)
        assert not np.any(prev[:2]) and np.all(np.any(prev[2:], axis=1))
        mb.set_quiescence(0.0)  # off again: x_prev reset
        assert not np.any(mb.read(-1, gh.T_GATE_PREV, np.float32))
    finally:
        ma.close()
        mb.close()
