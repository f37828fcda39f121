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
