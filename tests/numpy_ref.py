"""Independent numpy restatements used to pin the C oracle.

These are written from the reference's source semantics, separately from
oracle/oracle.c, and use different arithmetic where that is possible (fp64
half-away rounding, fp64 brute force), so that a transcription mistake in
either one shows up as a mismatch.

  bf16_rne          src/tensor.zig:7-13
  quantize_q4/q8    src/quant.zig:20-90
  dequant_q4/q8     src/test_q4_exec.zig:62-67, shaders/gemv_q8.wgsl:23-37
"""
import numpy as np


def bf16_rne(x):
    """fp32 -> bf16 bits with round-to-nearest-even (no NaN handling)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _round_half_away(p32):
    p = p32.astype(np.float64)  # exact widening; |p| + 0.5 is exact in fp64
    return np.sign(p) * np.floor(np.abs(p) + 0.5)


def _blocks(w_bf16):
    w = bf16_to_f32(w_bf16)
    rows, cols = w.shape
    assert cols % 32 == 0
    return w.reshape(rows, cols // 32, 32)


def quantize_q4(w_bf16):
    v = _blocks(w_bf16)
    amax = np.abs(v).max(axis=2)  # float32
    with np.errstate(divide="ignore"):
        d = (amax / np.float32(7.0)).astype(np.float32)
        idv = np.where(amax > 0, np.float32(7.0) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    p = (v * idv[..., None]).astype(np.float32)
    q = np.clip(_round_half_away(p), -8, 7).astype(np.int64) + 8
    rows, nb = amax.shape
    out = np.zeros((rows, nb, 5), np.uint32)
    out[:, :, 0] = d.view(np.uint32)
    q = q.reshape(rows, nb, 4, 8).astype(np.uint64)
    shifts = (np.arange(8, dtype=np.uint64) * 4)
    out[:, :, 1:] = (q << shifts).sum(axis=3).astype(np.uint32)
    return out.reshape(rows, nb * 5)


def quantize_q8(w_bf16):
    v = _blocks(w_bf16)
    amax = np.abs(v).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    idv = np.where(amax > 0, np.float32(127.0) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    p = (v * idv[..., None]).astype(np.float32)
    q = np.clip(_round_half_away(p), -128, 127).astype(np.int64)
    rows, nb = amax.shape
    out = np.zeros((rows, nb, 9), np.uint32)
    out[:, :, 0] = d.view(np.uint32)
    qb = (q & 0xFF).astype(np.uint64).reshape(rows, nb, 8, 4)
    shifts = np.arange(4, dtype=np.uint64) * 8
    out[:, :, 1:] = (qb << shifts).sum(axis=3).astype(np.uint32)
    return out.reshape(rows, nb * 9)


def dequant_q4(wq, cols):
    rows = wq.shape[0]
    nb = cols // 32
    blk = wq.reshape(rows, nb, 5)
    d = blk[:, :, 0].view(np.float32).astype(np.float64)
    words = blk[:, :, 1:].astype(np.uint64)
    shifts = np.arange(8, dtype=np.uint64) * 4
    nib = ((words[..., None] >> shifts) & 0xF).reshape(rows, nb, 32).astype(np.float64)
    return ((nib - 8.0) * d[..., None]).reshape(rows, cols)


def dequant_q8(wq, cols):
    rows = wq.shape[0]
    nb = cols // 32
    blk = wq.reshape(rows, nb, 9)
    d = blk[:, :, 0].view(np.float32).astype(np.float64)
    q = blk[:, :, 1:].copy().view(np.int8).reshape(rows, nb, 32).astype(np.float64)
    return (q * d[..., None]).reshape(rows, cols)


def rmsnorm64(x, w, eps=1e-6):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def gelu64(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def rope64(vec, pos, head_dim, rot, theta):
    v = np.array(vec, np.float64, copy=True).reshape(-1, head_dim)
    half = rot // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos * theta ** (-2.0 * i / rot)
    c, s = np.cos(ang), np.sin(ang)
    v0, v1 = v[:, :half].copy(), v[:, half:rot].copy()
    v[:, :half] = v0 * c - v1 * s
    v[:, half:rot] = v0 * s + v1 * c
    return v.reshape(-1)


def attention64(q, k_cache, v_cache, active, nq, nkv, hd):
    q = np.asarray(q, np.float64).reshape(nq, hd)
    kc = np.asarray(k_cache, np.float64).reshape(k_cache.shape[0], nkv, hd)
    vc = np.asarray(v_cache, np.float64).reshape(v_cache.shape[0], nkv, hd)
    act = np.asarray(active, np.int64)
    out = np.zeros((nq, hd))
    g = nq // nkv
    for h in range(nq):
        kh = h // g
        s = kc[act, kh, :] @ q[h]
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ vc[act, kh, :]
    return out.reshape(-1)


# ---------------------------------------------------------------------------
# One decode step in fp64, written from src/model/forward.zig:49-70,106-161
# (forwardAttentionCpu, runAttentionHeads, forwardMlpCpu, the tail) with the
# GPU graph's quantized weights and Q8_0 LM head (src/gpu/model_dispatch.zig:
# 10-43,121-127).  It shares no code with oracle/oracle.c: dequantized fp64
# matrices, fp64 norms/RoPE/softmax, and numpy's argmax.
#
# `mistake` plants one plausible transcription error (for the tests that show
# a comparison against this restatement would catch it):
#   "scalar_both_adds"  layer_scalar applied after the attention add too
#   "swap_gate_up"      gelu on the up projection instead of the gate
#   "skip_post_attn"    post-attention norm left out
#   "rope_v"            RoPE applied to v as well
#   "normed_k_as_v"     k_eq_v takes the normed k instead of the raw k
#   "theta_swap"        full layers rotate with the sliding theta
#   "attn_scale"        scores scaled by 1/sqrt(head_dim)
#   "write_after_attn"  this token's K/V written after its attention
#   "scalar_before_ffn" layer_scalar applied before the FFN add
# ---------------------------------------------------------------------------
def _deq(w, cols, mode):
    if mode == "bf16":  # mode none: the bf16 rows themselves, two per uint32 word
        return bf16_to_f32(np.ascontiguousarray(w).view(np.uint16)).astype(np.float64).reshape(-1, cols)
    return dequant_q8(w, cols) if mode == "q8" else dequant_q4(w, cols)


def _rms64(v, w=None, eps=1e-6):
    v = np.asarray(v, np.float64)
    y = v / np.sqrt(np.mean(v * v) + eps)
    return y if w is None else y * np.asarray(w, np.float64)


def _rope_heads(vec, pos, hd, rot, theta):
    v = np.array(vec, np.float64).reshape(-1, hd)
    half = rot // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos / theta ** (2.0 * i / rot)
    c, s = np.cos(ang), np.sin(ang)
    a, b = v[:, :half].copy(), v[:, half:rot].copy()
    v[:, :half] = a * c - b * s
    v[:, half:rot] = a * s + b * c
    return v.reshape(-1)


def forward64(layers, x, clock, slot, active, head_q8, final_norm, nq, eps=1e-6,
              theta=10000.0, theta_full=1e6, mode="q4", want_logits=True, mistake=None):
    """layers: dicts as oracle.Model takes them (k_cache / v_cache are updated
    in place, as ring.writeKV does).  Returns (token, x, logits) in fp64."""
    x = np.asarray(x, np.float64).copy()
    H = x.size
    act_slots = np.asarray(active, np.int64)
    for L in layers:
        hd, rot, nkv = L["head_dim"], L["rotary_dim"], L["num_kv_heads"]
        full = bool(L["full"])
        th = theta_full if full and mistake != "theta_swap" else theta
        qd, kvd = nq * hd, nkv * hd
        # forwardAttentionCpu (forward.zig:106-146)
        xn = _rms64(x, L["input_norm"], eps)
        q = _deq(L["wq"], H, mode) @ xn
        k = _deq(L["wk"], H, mode) @ xn
        if L["k_eq_v"]:
            v = k.copy()
        else:
            v = _deq(L["wv"], H, mode) @ xn
        q = np.concatenate([_rms64(h, L["q_norm"], eps) for h in q.reshape(nq, hd)])
        q = _rope_heads(q, clock, hd, rot, th)
        kn = np.concatenate([_rms64(h, L["k_norm"], eps) for h in k.reshape(nkv, hd)])
        if L["k_eq_v"] and mistake == "normed_k_as_v":
            v = kn.copy()
        v = np.concatenate([_rms64(h, None, eps) for h in v.reshape(nkv, hd)])
        k = _rope_heads(kn, clock, hd, rot, th)
        if mistake == "rope_v":
            v = _rope_heads(v, clock, hd, rot, th)
        kc, vc = L["k_cache"], L["v_cache"]
        if mistake != "write_after_attn":
            kc[slot], vc[slot] = k, v
        # runAttentionHeads (forward.zig:77-104): scale 1.0, kv head h / group
        K = kc[act_slots].astype(np.float64).reshape(len(act_slots), nkv, hd)
        Vv = vc[act_slots].astype(np.float64).reshape(len(act_slots), nkv, hd)
        scale = 1.0 / np.sqrt(hd) if mistake == "attn_scale" else 1.0
        out = np.zeros((nq, hd))
        g = nq // nkv
        for h in range(nq):
            s = K[:, h // g, :] @ q[h * hd:(h + 1) * hd] * scale
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ Vv[:, h // g, :]
        if mistake == "write_after_attn":
            kc[slot], vc[slot] = k, v
        o = _deq(L["wo"], qd, mode) @ out.reshape(-1)
        if L.get("post_attn_norm") is not None and mistake != "skip_post_attn":
            o = _rms64(o, L["post_attn_norm"], eps)
        x = x + o
        s_l = float(L.get("layer_scalar", 1.0))
        if mistake == "scalar_both_adds":
            x = x * s_l
        if mistake == "scalar_before_ffn":
            x = x * s_l
        # forwardMlpCpu (forward.zig:148-154) with kernels.gatedMlp
        xn = _rms64(x, L["pre_ffn_norm"], eps)
        gt = _deq(L["wg"], H, mode) @ xn
        up = _deq(L["wu"], H, mode) @ xn
        a = gelu64(up) * gt if mistake == "swap_gate_up" else gelu64(gt) * up
        m = _deq(L["wd"], a.size, mode) @ a
        if L.get("post_ffn_norm") is not None:
            m = _rms64(m, L["post_ffn_norm"], eps)
        x = x + m
        if mistake != "scalar_before_ffn":
            x = x * s_l  # forward.zig:61-63
    if not want_logits:
        return 0, x, None
    # forward.zig:62-70 with the GPU's Q8_0 head (model_dispatch.zig:121-127),
    # or the bf16 embedding in mode none (model_gpu.zig:160-161)
    head = _deq(head_q8, H, "bf16") if mode == "bf16" else dequant_q8(head_q8, H)
    logits = head @ _rms64(x, final_norm, eps)
    return int(np.argmax(logits)), x, logits
