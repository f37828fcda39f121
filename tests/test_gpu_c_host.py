"""The C ABI from a compiled C host (tests/c_host/decode_host.c), driven the
way the Zig engine drives its GPU backend: borrowed bf16 host tensors into
GpuModelContext.init, the host ring for slot numbers and active lists, and
gpuDispatchForwardToken per token -- the prompt token by token without
logits except for its last token, then greedy decode (src/interactive.zig:
33-48, src/gpu/model_dispatch.zig:131-147).  Its tokens must equal the
oracle's, teacher-forced on the same sequence, and those of the same model
driven through the Python binding.  It then runs the engine's --bench
sequence (src/model/bench.zig:12-21) through gh_model_submit_prerecorded."""
import os
import struct
import subprocess

import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc
from model_ref import layer_dims, oracle_model
from tol import assert_close

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)
HOST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_host", "decode_host")
TENSORS = ("input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
           "post_attention_layernorm", "pre_feedforward_layernorm", "gate_proj", "up_proj",
           "down_proj", "post_feedforward_layernorm")


def _weights(cfg, seed):
    rng = np.random.default_rng(seed)
    bf = lambda *s, mean=0.0, std=0.02: nr.bf16_rne((mean + std * rng.standard_normal(s)).astype(np.float32))  # noqa: E731
    H, I, nq = cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads
    layers = []
    for l in range(cfg.num_hidden_layers):
        d = layer_dims(cfg, l)
        qd, kvd = nq * d["head_dim"], d["num_kv_heads"] * d["head_dim"]
        w = dict(q_proj=bf(qd, H), k_proj=bf(kvd, H), o_proj=bf(H, qd), gate_proj=bf(I, H),
                 up_proj=bf(I, H), down_proj=bf(H, I), input_layernorm=bf(H, mean=1, std=0.1),
                 q_norm=bf(d["head_dim"], mean=1, std=0.1), k_norm=bf(d["head_dim"], mean=1, std=0.1),
                 post_attention_layernorm=bf(H, mean=1, std=0.1),
                 pre_feedforward_layernorm=bf(H, mean=1, std=0.1),
                 post_feedforward_layernorm=bf(H, mean=1, std=0.1),
                 layer_scalar=0.5 if l == 1 else 1.0)
        if l != 1:  # layer 1 has no v_proj: the key projection serves as value
            w["v_proj"] = bf(kvd, H)
        layers.append(w)
    return layers, bf(cfg.vocab_size, H), bf(H, mean=1, std=0.1)


def _write_model(path, cfg, mode, ring, layers, embed, fnorm, prompt, n_decode):
    with open(path, "wb") as f:
        f.write(b"GHH1")
        f.write(struct.pack("<17I", cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size,
                            cfg.num_hidden_layers, cfg.num_attention_heads,
                            cfg.num_key_value_heads, cfg.num_global_key_value_heads,
                            cfg.head_dim, cfg.global_head_dim, cfg.attention_k_eq_v,
                            cfg.max_slots, mode, ring[0], ring[1], ring[2], len(prompt), n_decode))
        f.write(struct.pack("<3f", cfg.rms_norm_eps, cfg.rope_theta, cfg.rope_theta_full))
        f.write(bytes(cfg.layer_types))
        for w in layers:
            f.write(struct.pack("<13I", *[w[t].size if t in w else 0 for t in TENSORS]))
            f.write(struct.pack("<f", w["layer_scalar"]))
            for t in TENSORS:
                if t in w:
                    f.write(np.ascontiguousarray(w[t], np.uint16).tobytes())
        f.write(np.ascontiguousarray(embed, np.uint16).tobytes())
        f.write(np.ascontiguousarray(fnorm, np.uint16).tobytes())
        f.write(np.asarray(prompt, np.uint32).tobytes())


@pytest.mark.parametrize("mode", [gh.QUANT_Q4, gh.QUANT_Q8, gh.QUANT_NONE])
def test_c_host_prompt_then_greedy_decode(gpu, tmp_path, mode):
    assert os.path.exists(HOST), "tests/c_host/decode_host is not built (__graft_entry__.build())"
    cfg = gh.model_config(vocab=1024, hidden=256, intermediate=512, layers=3, heads=4,
                          kv_heads=2, head_dim=64, max_slots=24, global_kv_heads=2,
                          global_head_dim=128, full_layers=(2,))
    ring_shape = (4, 16, 4)
    layers, embed, fnorm = _weights(cfg, 11)
    prompt = [5, 77, 1000, 3, 3, 900, 42]
    n_decode = 12
    path = str(tmp_path / "model.bin")
    _write_model(path, cfg, mode, ring_shape, layers, embed, fnorm, prompt, n_decode)
    print("c host: mode %d, %d prompt tokens, %d decode steps" % (mode, len(prompt), n_decode),
          flush=True)
    run = subprocess.run([HOST, path], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    line = [ln for ln in run.stdout.splitlines() if ln.startswith("tokens:")][0]
    ctoks = [int(t) for t in line.split()[1:]]
    assert len(ctoks) == n_decode + 1

    # the same model and sequence through the Python binding, and the oracle
    m = gh.Model(gpu, cfg, mode=mode, layers=layers, embed=embed, final_norm=fnorm)
    try:
        om, _ = oracle_model(m, cfg, mode)
        for l, w in enumerate(layers):
            om._layers[l].layer_scalar = w["layer_scalar"]
        ring = gh.Ring(cfg.num_hidden_layers, *ring_shape)
        seq = prompt + ctoks[:-1]  # teacher-forced on the C host's own tokens
        ptoks = []
        for clock, t in enumerate(seq):
            want = clock >= len(prompt) - 1
            x = orc.embed(embed, t, cfg.hidden_size)
            slot = ring.activate_slot(0, clock)
            active = ring.active_slots(0, clock)
            tok = m.forward(x, clock, slot, active, want)
            rtok, _, rlog = om.forward(x, clock, slot, active, want, NT)
            if want:
                ptoks.append(tok)
                logits = m.read(-1, gh.T_LOGITS, np.float32)
                assert_close(logits, rlog, what="C-host sequence step %d" % clock)
                assert tok == rtok, "step %d: token %d vs oracle %d" % (clock, tok, rtok)
        assert ptoks == ctoks, "C host %s vs Python binding %s" % (ctoks, ptoks)
        # the --bench replays (src/model/bench.zig:12-15) recompute the last
        # decode step: its token again
        bench = [ln for ln in run.stdout.splitlines() if ln.startswith("bench:")][0].split()
        assert float(bench[1]) > 0.0
        assert int(bench[-1]) == ctoks[-1], bench
    finally:
        m.close()
