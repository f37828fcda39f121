"""The float tolerance used by every parity test.

The stated bar is "max relative error 2e-3 (fp32 accumulation)".  A plain
elementwise relative error is ill-posed for outputs near zero, so both of
these must hold, with RTOL = 2e-3:
  normwise     max|got - ref| / max|ref|                     <= RTOL
  elementwise  |got - ref| <= RTOL * max(|ref|, floor)         for every element
               floor = max(1e-2 * max|ref|, 0.1 * rms(ref))
The floor keeps the elementwise test meaningful for elements that happen to
sit near zero: RoPE at clocks in the hundreds turns one-ulp differences
between two f32 pow/cos/sin implementations into ~1e-4 absolute errors.
"""
import numpy as np

RTOL = 2e-3


def errors(got, ref):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    scale = max(np.max(np.abs(ref)), 1e-30)
    rms = float(np.sqrt(np.mean(ref * ref)))
    d = np.abs(got - ref)
    floor = np.maximum(np.abs(ref), max(1e-2 * scale, 0.1 * rms))
    return float(np.max(d) / scale), float(np.max(d / floor))


def assert_close(got, ref, rtol=RTOL, what=""):
    assert np.all(np.isfinite(got)), "%s: non-finite output" % what
    nw, ew = errors(got, ref)
    assert nw <= rtol and ew <= rtol, "%s: normwise %.3g, elementwise %.3g > %.3g" % (what, nw, ew, rtol)
    return nw, ew
