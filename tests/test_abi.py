"""CPU-side checks of the C-ABI library: it loads without a GPU, exports every
function include/gemma_hip.h declares, and its host routines (quantizer,
synthetic generator) match the oracle bit for bit.  No device calls."""
import os
import re

import numpy as np
import pytest

import gemma_hip as gh
import numpy_ref as nr
import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    txt = open(os.path.join(ROOT, "include", "gemma_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(gh_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_function():
    L = gh.lib()
    names = header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the binding's signature table covers the header exactly
    assert sorted(gh.exported_symbols()) == names


def header_arities():
    """Parameter count of every function the header declares."""
    txt = open(os.path.join(ROOT, "include", "gemma_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(gh_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", txt):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_arity_matches_header():
    # the ctypes table passes exactly the header's parameters
    L = gh.lib()
    ar = header_arities()
    assert len(ar) == len(header_functions())
    bad = {n: (k, len(getattr(L, n).argtypes)) for n, k in ar.items()
           if len(getattr(L, n).argtypes) != k}
    assert not bad, bad


def test_device_count_without_gpu_is_not_an_error():
    assert gh.device_count() >= 0


def test_row_word_helpers_match_quant_zig():
    L = gh.lib()
    for cols in (32, 64, 100, 3840, 15360):
        for mode in (gh.QUANT_Q4, gh.QUANT_Q8):
            assert L.gh_quantized_row_words(cols, mode) == orc.row_words(cols, mode)
    assert L.gh_quantized_size_bytes(8192, 2048, gh.QUANT_Q4) == 10485760  # config 1 weights
    assert L.gh_quantized_size_bytes(262144, 3840, gh.QUANT_Q8) == 1132462080  # LM head


def test_host_quantizer_matches_oracle_and_fixtures():
    f = np.load(os.path.join(ROOT, "tests", "golden", "quant_fixtures.npz"))
    assert np.array_equal(gh.quantize_matrix(f["w_bf16"], gh.QUANT_Q4), f["q4"])
    assert np.array_equal(gh.quantize_matrix(f["w_bf16"], gh.QUANT_Q8), f["q8"])
    w = gh.synth_normal(512 * 3840, 0, 99, 0.0, 0.02, bf16=True).reshape(512, 3840)
    assert np.array_equal(gh.quantize_matrix(w, gh.QUANT_Q4, 8), orc.quantize_q4(w))
    assert np.array_equal(gh.quantize_matrix(w, gh.QUANT_Q8, 8), orc.quantize_q8(w))


def test_synth_generator_is_deterministic_and_normal():
    a = gh.synth_normal(1 << 20, 0, 1, 0.0, 1.0)
    b = gh.synth_normal(1 << 20, 0, 1, 0.0, 1.0)
    assert np.array_equal(a, b)
    # offset addresses the same sequence
    assert np.array_equal(gh.synth_normal(100, 0, 1, 0.0, 1.0, offset=500), a[500:600])
    assert not np.array_equal(a[:1000], gh.synth_normal(1000, 0, 2, 0.0, 1.0))
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1) < 5e-3
    # tail mass of a normal: P(|z| > 3) = 0.0027
    assert abs(np.mean(np.abs(a) > 3) - 0.0027) < 4e-4
    bf = gh.synth_normal(4096, 5, 7, 0.0, 0.02, bf16=True)
    assert np.array_equal(bf, nr.bf16_rne(gh.synth_normal(4096, 5, 7, 0.0, 0.02)))
    t = gh.synth_uniform_u32(100000, 1, 0, 262144)
    assert t.max() < 262144 and len(np.unique(t)) > 80000


def test_gpu_calls_fail_loudly_without_device():
    if gh.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(gh.GhError):
        gh.Context()
