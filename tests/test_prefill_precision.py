"""Why the prefill GEMM feeds its activations through the matrix cores twice.

The batched prefill computes C = A . deq(W)^T with fp16 MFMA operands.  The
Q4_0 weights enter exactly (the integers n - 8, with the block scale applied
to each block's fp32 sum); the activations are split per row into
hi = fp16(a / s) and lo = fp16(a / s - hi), s a power of two, and both
halves go through the MFMA.  The cheaper alternative, one fp16 pass over
fp16 activations and weights rounded to fp16 as d (n - 8), halves the matrix
work and drops the per-block scale FMAs, but it does not meet the parity bar
at the 12B width: this module shows both on the CPU (numpy, fp64 sums, so
only the operand rounding differs), at K = 3840 with N(0, 0.02) Q4_0 weights.
"""
import numpy as np

from tol import RTOL, errors

T, K, N = 64, 3840, 1024


def _q4(w):
    """Q4_0 of each 32-element block (src/quant.zig:55-90): d = signed max / -8,
    n = clamp(floor(w / d + 8.5), 0, 15); returns d [N][K/32] and n - 8."""
    b = w.reshape(w.shape[0], -1, 32)
    idx = np.argmax(np.abs(b), axis=2)
    mx = np.take_along_axis(b, idx[..., None], 2)[..., 0]
    d = (mx / -8.0).astype(np.float32)
    inv = np.where(d != 0, 1.0 / d.astype(np.float64), 0.0)
    n = np.clip(np.floor(b * inv[..., None] + 8.5), 0, 15)
    return d, n - 8.0


def _operands():
    rng = np.random.default_rng(0)
    a = (rng.standard_normal((T, K)) * (1.0 + 0.1 * rng.standard_normal(K))).astype(np.float32)
    a[:, :8] *= 20.0  # a few large channels, as a residual stream has
    d, q = _q4((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    return a.astype(np.float64), d.astype(np.float64), q


def _row_scale(a):
    e = np.frexp(np.max(np.abs(a), axis=1))[1] - 14
    return np.ldexp(1.0, e)[:, None]


def _blockwise(a, d, q):
    """sum_b d[n][b] * (a_b . q[n]_b): the block scales applied to block sums."""
    ab = a.reshape(a.shape[0], -1, 32)
    return np.einsum("tbk,nbk,nb->tn", ab, q, d)


def test_split_activations_meet_the_bar():
    a, d, q = _operands()
    ref = _blockwise(a, d, q)
    s = _row_scale(a)
    hi = (a / s).astype(np.float16).astype(np.float64)
    lo = (a / s - hi).astype(np.float16).astype(np.float64)
    got = (_blockwise(hi, d, q) + _blockwise(lo, d, q)) * s
    nw, ew = errors(got, ref)
    assert nw < RTOL / 100 and ew < RTOL / 100, (nw, ew)


def test_one_fp16_pass_misses_the_bar():
    a, d, q = _operands()
    ref = _blockwise(a, d, q)
    s = _row_scale(a)
    a16 = (a / s).astype(np.float16).astype(np.float64) * s
    w16 = (d[..., None] * q).reshape(N, K).astype(np.float16).astype(np.float64)
    nw, ew = errors(a16 @ w16.T, ref)
    # normwise it would pass; element by element it does not
    assert nw < RTOL
    assert ew > 2 * RTOL, ew
