"""Writes tests/golden/quant_fixtures.npz: bf16 rows and their Q4_0 / Q8_0
bytes as computed by the independent numpy restatement in tests/numpy_ref.py
(src/quant.zig:20-90 semantics).  The C oracle and the GPU quantizer are both
checked against these bytes.

Run:  python tests/golden/make_quant_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import numpy_ref as nr  # noqa: E402


def rows():
    cols = 64
    out = []
    out.append(np.full(cols, 1.0, np.float32))
    out.append(np.zeros(cols, np.float32))
    out.append(np.full(cols, -1.0, np.float32))
    # exact half-way products: amax 7 -> id 1, so v itself is rounded
    ties = np.array([7, -7, 3.5, -3.5, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 4.5, -4.5, 5.5,
                     -5.5, 6.5, -6.5] * 4, np.float32)
    out.append(ties)
    # amax 3.5 -> id 2: 1.25 * 2 = 2.5 (half away -> 3, half even would give 2)
    t2 = np.array([3.5, 1.25, -1.25, 0.75, -0.75, 0.25, -0.25, 2.75] * 8, np.float32)
    out.append(t2)
    one = np.zeros(cols, np.float32)
    one[5] = -0.0625
    one[40] = 3.0
    out.append(one)
    out.append(np.full(cols, 1e-30, np.float32))
    out.append(np.linspace(-1e30, 1e30, cols).astype(np.float32))
    # Q8 half-way: amax 127 -> id 1
    out.append(np.array([127, -127, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5] * 8, np.float32))
    rng = np.random.default_rng(1234)
    for _ in range(23):
        out.append((rng.standard_normal(cols) * 0.02).astype(np.float32))
    return np.stack(out)


def main():
    w = rows()
    wb = nr.bf16_rne(w)
    np.savez(os.path.join(HERE, "quant_fixtures.npz"), w_f32=w, w_bf16=wb,
             q4=nr.quantize_q4(wb), q8=nr.quantize_q8(wb))
    print("wrote", wb.shape[0], "rows")


if __name__ == "__main__":
    main()
