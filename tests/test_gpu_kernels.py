"""GPU parity of the engine kernels against the oracle, through the C ABI.

Integer work (synthetic bits, quantized bytes) must be bit-exact; float
outputs must meet tests/tol.py (normwise and floored elementwise relative
error <= 2e-3, fp32 accumulation).
"""
import os

import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc
from tol import assert_close

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NT = min(16, os.cpu_count() or 1)


def q4_weights(M, K, seed, stream, std=0.02):
    w = gh.synth_normal(M * K, seed, stream, 0.0, std, bf16=True).reshape(M, K)
    return orc.quantize_q4(w, NT)


# ---------------------------------------------------------------- data ----
def test_synth_device_matches_host_bits(gpu):
    n = 3_000_001
    for bf16 in (False, True):
        host = gh.synth_normal(n, 17, 3, 0.5, 0.02, bf16=bf16, offset=12345)
        buf = gpu.alloc(n * host.itemsize)
        gpu.synth_normal_dev(buf, n, 17, 3, 0.5, 0.02, bf16=bf16, offset=12345)
        dev = buf.read(host.dtype, n)
        assert np.array_equal(dev.view(np.uint16 if bf16 else np.uint32),
                              host.view(np.uint16 if bf16 else np.uint32))


def test_quantize_device_matches_oracle(gpu):
    f = np.load(os.path.join(ROOT, "tests", "golden", "quant_fixtures.npz"))
    for mode, key in ((gh.QUANT_Q4, "q4"), (gh.QUANT_Q8, "q8")):
        src = gpu.upload(f["w_bf16"])
        dst = gpu.alloc(f[key].nbytes)
        gpu.quantize_dev(dst, src, f["w_bf16"].shape[0], f["w_bf16"].shape[1], mode)
        assert np.array_equal(dst.read(np.uint32).reshape(f[key].shape), f[key])
    M, K = 2048, 3840
    w = gh.synth_normal(M * K, 0, 40, 0.0, 0.02, bf16=True).reshape(M, K)
    src = gpu.upload(w)
    for mode, ref in ((gh.QUANT_Q4, orc.quantize_q4(w, NT)), (gh.QUANT_Q8, orc.quantize_q8(w, NT))):
        dst = gpu.alloc(ref.nbytes)
        gpu.quantize_dev(dst, src, M, K, mode)
        assert np.array_equal(dst.read(np.uint32).reshape(ref.shape), ref)


# ---------------------------------------------------------------- Q4 GEMV -
Q4_SHAPES = [
    (8192, 2048),    # single Q4_0 GEMV, batch 1
    (4096, 3840),    # q_proj
    (2048, 3840),    # k_proj / v_proj
    (3840, 4096),    # o_proj
    (3840, 15360),   # down_proj
    (1, 128), (5, 256), (37, 1024), (1000, 3840), (3, 15360),  # ragged row tails
    # x longer than the staging registers hold (K > 16 x threads): the workgroup
    # splits into x stagers and first streamers (256 and 1024 threads)
    (64, 6144), (40, 32768),
]


@pytest.mark.parametrize("M,K", Q4_SHAPES)
def test_gemv_q4_parity(gpu, M, K):
    wq = q4_weights(M, K, 0, 1000 + M + K)
    x = gh.synth_normal(K, 0, 7, 0.0, 1.0)
    ref = orc.gemv_q4(wq, x, K, NT)
    W, X, Y = gpu.upload(wq), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_q4(W, X, Y, M, K)
    assert_close(Y.read(np.float32, M), ref, what="gemv_q4 %dx%d" % (M, K))


def test_gemv_q4_reference_exec_case(gpu):
    # src/test_q4_exec.zig:16-95: M=3840, K=15360, weights (u-0.5)*0.2 cut to
    # bf16, x (u-0.5)*0.5, GPU vs the scalar CPU loop: max abs error < 1e-3.
    M, K = 3840, 15360
    rng = np.random.default_rng(42)
    wf = ((rng.random(M * K, dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
    wb = (wf.view(np.uint32) >> 16).astype(np.uint16).reshape(M, K)  # truncation, as :27
    x = ((rng.random(K, dtype=np.float32) - 0.5) * 0.5).astype(np.float32)
    wq = orc.quantize_q4(wb, NT)
    ref = orc.gemv_q4(wq, x, K, NT)
    W, X, Y = gpu.upload(wq), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_q4(W, X, Y, M, K)
    assert np.max(np.abs(Y.read(np.float32, M) - ref)) < 1e-3


def test_gemv_q4_all_ones(gpu):
    # src/gpu.zig:30-59: 64 x 128 all-1.0 bf16 weights, x = (i % 5) * 0.25: all y > 0
    M, K = 64, 128
    wq = orc.quantize_q4(np.full((M, K), 0x3F80, np.uint16))
    x = (np.arange(K) % 5).astype(np.float32) * 0.25
    W, X, Y = gpu.upload(wq), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_q4(W, X, Y, M, K)
    y = Y.read(np.float32, M)
    assert np.all(y > 0)
    assert_close(y, orc.gemv_q4(wq, x, K), what="all-ones")


def test_gemv_rejects_unsupported_shapes(gpu):
    W, X, Y = gpu.alloc(4096), gpu.alloc(4096), gpu.alloc(4096)
    with pytest.raises(gh.GhError, match="multiple of 128"):
        gpu.gemv_q4(W, X, Y, 4, 96)
    with pytest.raises(gh.GhError):
        gpu.gemv_q4(W, X, Y, 0, 128)


# ---------------------------------------------------------------- Q8 GEMV -
@pytest.mark.parametrize("M,K", [(4096, 3840), (777, 1024), (1, 128), (3840, 15360), (64, 6144)])
def test_gemv_q8_parity(gpu, M, K):
    w = gh.synth_normal(M * K, 0, 2000 + M, 0.0, 0.02, bf16=True).reshape(M, K)
    wq = orc.quantize_q8(w, NT)
    x = gh.synth_normal(K, 0, 8, 0.0, 1.0)
    W, X, Y = gpu.upload(wq), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gemv_q8(W, X, Y, M, K)
    assert_close(Y.read(np.float32, M), orc.gemv_q8(wq, x, K, NT), what="gemv_q8")


def test_gemv_q8_vocab_full_size(gpu):
    # Q8_0 vocab projection 262144 x 3840: weights generated and quantized on
    # the device (both bit-exact with the host routines, tested above), then
    # read back for the oracle.
    V, H = 262144, 3840
    wb = gpu.alloc(V * H * 2)
    gpu.synth_normal_dev(wb, V * H, 0, 4, 0.0, 0.02, bf16=True)
    wq = gpu.alloc(V * (H // 32) * 36)
    gpu.quantize_dev(wq, wb, V, H, gh.QUANT_Q8)
    wb.free()
    x = gh.synth_normal(H, 0, 5, 0.0, 1.0)
    X, Y = gpu.upload(x), gpu.alloc(V * 4)
    gpu.gemv_q8(wq, X, Y, V, H)
    y = Y.read(np.float32, V)
    host_q = wq.read(np.uint32).reshape(V, -1)
    # spot-check the device bytes against the host quantizer on a slice
    rows = gh.synth_normal(64 * H, 0, 4, 0.0, 0.02, bf16=True, offset=1000 * H).reshape(64, H)
    assert np.array_equal(host_q[1000:1064], orc.quantize_q8(rows))
    ref = orc.gemv_q8(host_q, x, H, NT)
    assert_close(y, ref, what="vocab q8")
    assert int(np.argmax(y)) == orc.argmax(ref)


# ------------------------------------------------------ fused gate + up ----
@pytest.mark.parametrize("M,K", [(15360, 3840), (96, 256), (1, 128)])
def test_gate_up_geglu_q4_parity(gpu, M, K):
    wg = q4_weights(M, K, 0, 3000 + M)
    wu = q4_weights(M, K, 0, 3001 + M)
    x = gh.synth_normal(K, 0, 9, 0.0, 1.0)
    ref = orc.gate_up_geglu_q4(x, wg, wu, NT)
    Wg, Wu, X, Y = gpu.upload(wg), gpu.upload(wu), gpu.upload(x), gpu.alloc(M * 4)
    gpu.gate_up_geglu_q4(Wg, Wu, X, Y, M, K)
    assert_close(Y.read(np.float32, M), ref, what="gate_up %dx%d" % (M, K))


# ------------------------------------------------ fused prologue / epilogue --
def _bf16r(a):
    return nr.bf16_to_f32(nr.bf16_rne(a))


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("with_rnorm", [True, False])
def test_norm_gemv_prologues(gpu, mode, with_rnorm):
    # mode 1: input RMSNorm fused in; mode 2: post-FFN norm of r, residual add
    # with layer_scalar, then the next input norm (model_dispatch.zig:39-41, 21)
    M, K = 2048, 3840
    wq = q4_weights(M, K, 0, 4000)
    x = gh.synth_normal(K, 0, 41, 0.0, 2.0)
    r = gh.synth_normal(K, 0, 42, 0.0, 1.0)
    wn = _bf16r(gh.synth_normal(K, 0, 43, 1.0, 0.1))
    wr = _bf16r(gh.synth_normal(K, 0, 44, 1.0, 0.1))
    s = np.float32(0.875)
    X, R, WN, WR, XO, Y = (gpu.upload(x), gpu.upload(r), gpu.upload(wn), gpu.upload(wr),
                           gpu.alloc(K * 4), gpu.alloc(M * 4))
    if mode == 1:
        pro = gpu.prologue(X, 1, norm=WN)
        xin = orc.rmsnorm(x, wn)
    else:
        pro = gpu.prologue(X, 2, norm=WN, r=R, r_norm=WR if with_rnorm else None, x_out=XO,
                           scalar=float(s))
        rr = orc.rmsnorm(r, wr) if with_rnorm else r
        xn = ((x + rr) * s).astype(np.float32)
        xin = orc.rmsnorm(xn, wn)
    gpu.norm_gemv(gh.QUANT_Q4, gpu.upload(wq), Y, M, K, pro)
    assert_close(Y.read(np.float32, M), orc.gemv_q4(wq, xin, K, NT), what="norm_gemv mode %d" % mode)
    if mode == 2:
        assert_close(XO.read(np.float32, K), xn, what="residual stream")


@pytest.mark.parametrize("with_rnorm", [True, False])
def test_norm_gemv_residual_cancellation(gpu, with_rnorm):
    # x + r' nearly cancels: the prologue's one-pass sum of squares (expanded
    # from sum x^2, sum x r', sum r'^2) would lose the result, so it reduces
    # the residual itself; the output must still match the oracle
    M, K = 512, 3840
    wq = q4_weights(M, K, 0, 4050)
    r = gh.synth_normal(K, 0, 51, 0.0, 1.0)
    wr = _bf16r(gh.synth_normal(K, 0, 52, 1.0, 0.1))
    wn = _bf16r(gh.synth_normal(K, 0, 53, 1.0, 0.1))
    rr = orc.rmsnorm(r, wr) if with_rnorm else r
    x = (-rr + 1e-3 * gh.synth_normal(K, 0, 54, 0.0, 1.0)).astype(np.float32)
    X, R, WN, WR, XO, Y = (gpu.upload(x), gpu.upload(r), gpu.upload(wn), gpu.upload(wr),
                           gpu.alloc(K * 4), gpu.alloc(M * 4))
    pro = gpu.prologue(X, 2, norm=WN, r=R, r_norm=WR if with_rnorm else None, x_out=XO, scalar=1.0)
    gpu.norm_gemv(gh.QUANT_Q4, gpu.upload(wq), Y, M, K, pro)
    xn = (x + rr).astype(np.float32)
    assert_close(XO.read(np.float32, K), xn, what="residual stream")
    assert_close(Y.read(np.float32, M), orc.gemv_q4(wq, orc.rmsnorm(xn, wn), K, NT),
                 what="norm_gemv under cancellation")


def test_norm_gate_up_matches_oracle(gpu):
    M, K = 15360, 3840
    wg, wu = q4_weights(M, K, 0, 4100), q4_weights(M, K, 0, 4101)
    x = gh.synth_normal(K, 0, 45, 0.0, 1.0)
    r = gh.synth_normal(K, 0, 46, 0.0, 1.0)
    wn = _bf16r(gh.synth_normal(K, 0, 47, 1.0, 0.1))
    wr = _bf16r(gh.synth_normal(K, 0, 48, 1.0, 0.1))
    X, R, WN, WR, XO, Y = (gpu.upload(x), gpu.upload(r), gpu.upload(wn), gpu.upload(wr),
                           gpu.alloc(K * 4), gpu.alloc(M * 4))
    pro = gpu.prologue(X, 2, norm=WN, r=R, r_norm=WR, x_out=XO, scalar=1.0)
    gpu.norm_gate_up_geglu(gh.QUANT_Q4, gpu.upload(wg), gpu.upload(wu), Y, M, K, pro)
    xn = (x + orc.rmsnorm(r, wr)).astype(np.float32)
    ref = orc.gate_up_geglu_q4(orc.rmsnorm(xn, wn), wg, wu, NT)
    assert_close(Y.read(np.float32, M), ref, what="norm gate_up")


@pytest.mark.parametrize("V", [262144, 50000, 1000])
def test_norm_gemv_argmax_q8(gpu, V):
    H = 3840
    w = gh.synth_normal(V * H, 0, 4200, 0.0, 0.02, bf16=True).reshape(V, H)
    wq = orc.quantize_q8(w, NT)
    x = gh.synth_normal(H, 0, 49, 0.0, 1.0)
    wn = _bf16r(gh.synth_normal(H, 0, 50, 1.0, 0.1))
    W, X, WN, L, T = gpu.upload(wq), gpu.upload(x), gpu.upload(wn), gpu.alloc(V * 4), gpu.alloc(4)
    pro = gpu.prologue(X, 1, norm=WN)
    gpu.norm_gemv_argmax_q8(W, L, T, V, H, pro)
    logits = L.read(np.float32, V)
    ref = orc.gemv_q8(wq, orc.rmsnorm(x, wn), H, NT)
    assert_close(logits, ref, what="head logits")
    tok = int(T.read(np.uint32, 1)[0])
    assert tok == orc.argmax(logits)  # bit-exact pick over the logits it produced
    assert tok == orc.argmax(ref) or ref[tok] >= np.max(ref) - 1e-5 * np.max(np.abs(ref))
    gpu.norm_gemv_argmax_q8(W, None, T, V, H, pro)  # without materialised logits
    assert int(T.read(np.uint32, 1)[0]) == tok
