"""Builds the oracle's model (oracle.Model) from a GPU model's own tensors, so
the CPU restatement and the device run the same quantized bytes (or, in
mode none, the same bf16 rows)."""
import numpy as np

import gemma_hip as gh
import oracle as orc


def layer_dims(cfg, l):
    # src/model/loader.zig:36-42
    full = bool(cfg.layer_types[l])
    hd = cfg.global_head_dim if full else cfg.head_dim
    return dict(full=full, head_dim=hd, rotary_dim=hd // 4 if full else hd,
                num_kv_heads=cfg.num_global_key_value_heads if full else cfg.num_key_value_heads,
                k_eq_v=full and bool(cfg.attention_k_eq_v))


# uint32 words per 32 weights of a row, and the oracle's mode, per weight mode
WORDS = {gh.QUANT_Q4: 5, gh.QUANT_Q8: 9, gh.QUANT_NONE: 16}
ORC_MODE = {gh.QUANT_Q4: orc.QUANT_Q4, gh.QUANT_Q8: orc.QUANT_Q8, gh.QUANT_NONE: orc.QUANT_NONE}


def oracle_model(m, cfg, mode=gh.QUANT_Q4):
    H, I, V, nq = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_attention_heads
    words = WORDS[mode]
    layers = []
    for l in range(cfg.num_hidden_layers):
        d = layer_dims(cfg, l)
        qd, kvd = nq * d["head_dim"], d["num_kv_heads"] * d["head_dim"]
        qkv = m.read(l, gh.T_QKV, np.uint32).reshape(-1, (H // 32) * words)
        k_eq_v = d["k_eq_v"] or qkv.shape[0] == qd + kvd
        d["k_eq_v"] = k_eq_v
        d["wq"], d["wk"] = qkv[:qd], qkv[qd:qd + kvd]
        d["wv"] = d["wk"] if k_eq_v else qkv[qd + kvd:qd + 2 * kvd]
        d["wo"] = m.read(l, gh.T_O_PROJ, np.uint32).reshape(H, -1)
        d["wg"] = m.read(l, gh.T_GATE, np.uint32).reshape(I, -1)
        d["wu"] = m.read(l, gh.T_UP, np.uint32).reshape(I, -1)
        d["wd"] = m.read(l, gh.T_DOWN, np.uint32).reshape(H, -1)
        d["input_norm"] = m.read(l, gh.T_INPUT_NORM, np.float32)
        d["q_norm"] = m.read(l, gh.T_Q_NORM, np.float32)
        d["k_norm"] = m.read(l, gh.T_K_NORM, np.float32)
        d["post_attn_norm"] = m.read(l, gh.T_POST_ATTN_NORM, np.float32)
        d["pre_ffn_norm"] = m.read(l, gh.T_PRE_FFN_NORM, np.float32)
        d["post_ffn_norm"] = m.read(l, gh.T_POST_FFN_NORM, np.float32)
        d["k_cache"] = m.read(l, gh.T_K_CACHE, np.float32).reshape(cfg.max_slots, kvd)
        d["v_cache"] = m.read(l, gh.T_V_CACHE, np.float32).reshape(cfg.max_slots, kvd)
        layers.append(d)
    head = m.read(-1, gh.T_LM_HEAD, np.uint32).reshape(V, -1)
    fn = m.read(-1, gh.T_FINAL_NORM, np.float32)
    return orc.Model(H, I, V, nq, layers, head, fn, cfg.rms_norm_eps, cfg.rope_theta,
                     cfg.rope_theta_full, ORC_MODE[mode]), layers
