"""HBM traffic of the decode kernels from rocprofv3 counters.

Two rocprofv3 passes, one counter each (FETCH_SIZE, then WRITE_SIZE, KiB per
dispatch), over `python traffic.py run`, which launches:
  * a device-to-device copy of COPY_BYTES (the calibration kernel: it reads
    and writes exactly COPY_BYTES),
  * the Q4_0 fused gate+up GeGLU, 15360 x 3840, and the down projection,
    3840 x 15360, over 6 rotated weight copies (so every launch streams from
    HBM, not from the 256 MB Infinity Cache).
`python traffic.py summarize FETCH_CSV WRITE_CSV OUT_JSON` then scales each
kernel's average counter by (bytes the copy moved / what the counter read
for the copy) and writes the per-launch HBM bytes next to the algorithmic
bytes.  Command lines: see the header of the committed summary.
"""
import csv
import json
import os
import sys
from collections import defaultdict

H, I = 3840, 15360
COPY_BYTES = 512 << 20
Q4_ROW = lambda k: (k // 32) * 20  # noqa: E731

ALGORITHMIC = {  # bytes one launch must move: weights + x in + y out
    "gh_gateup_q4": 2 * I * Q4_ROW(H) + H * 4 + I * 4,
    "gh_gemv_q4": H * Q4_ROW(I) + I * 4 + H * 4,
}


def run(launches=30):
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import gemma_hip as gh

    ctx = gh.Context()
    src, dst = ctx.alloc(COPY_BYTES), ctx.alloc(COPY_BYTES)
    ctx.fill_u32(src, 0x3F800000, COPY_BYTES // 4)
    for _ in range(5):
        ctx.copy(dst, src, COPY_BYTES)
    ctx.sync()
    staging = ctx.alloc(I * H * 2)
    copies = []
    for c in range(6):
        mats = []
        for rows, cols, s in ((I, H, 0), (I, H, 1), (H, I, 2)):
            ctx.synth_normal_dev(staging, rows * cols, 0, 100 + 3 * c + s, 0.0, 0.02, bf16=True)
            m = ctx.alloc(rows * Q4_ROW(cols))
            ctx.quantize_dev(m, staging, rows, cols, gh.QUANT_Q4)
            mats.append(m)
        copies.append(mats)
    staging.free()
    X = ctx.upload(gh.synth_normal(H, 0, 1, 0.0, 1.0))
    ACT, OUT = ctx.alloc(I * 4), ctx.alloc(H * 4)
    for i in range(launches):
        wg, wu, wd = copies[i % 6]
        ctx.gate_up_geglu_q4(wg, wu, X, ACT, I, H)
        ctx.gemv_q4(wd, ACT, OUT, H, I)
    ctx.sync()
    print("traffic workload done: %d copies of %d B, %d MLP steps" % (5, COPY_BYTES, launches),
          flush=True)


def _family(name):
    for fam in ("gh_gateup_q4", "gh_gemv_q4"):
        if name.startswith(fam + "_") or name.startswith(fam + "n_"):
            return fam
    if "copyBuffer" in name:
        return "copy"
    return None


def _averages(path, counter):
    vals = defaultdict(list)
    with open(path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            fam = _family(row["Kernel_Name"])
            if fam:
                vals[fam].append(float(row["Counter_Value"]))
    # the copy family also catches small host-upload blits: keep the
    # COPY_BYTES dispatches (the largest by far)
    if "copy" in vals:
        top = max(vals["copy"])
        vals["copy"] = [v for v in vals["copy"] if v >= 0.5 * top]
    return {k: sum(v) / len(v) for k, v in vals.items()}


def summarize(fetch_csv, write_csv, out_json):
    fetch = _averages(fetch_csv, "FETCH_SIZE")
    write = _averages(write_csv, "WRITE_SIZE")
    kib = COPY_BYTES / 1024.0
    f_scale, w_scale = kib / fetch["copy"], kib / write["copy"]
    out = {"calibration": {"copy_bytes": COPY_BYTES,
                           "copy_fetch_kib": fetch["copy"], "copy_write_kib": write["copy"],
                           "fetch_scale": f_scale, "write_scale": w_scale}}
    for fam, alg in ALGORITHMIC.items():
        rd = fetch[fam] * f_scale * 1024
        wr = write[fam] * w_scale * 1024
        out[fam] = {"hbm_read_bytes": round(rd), "hbm_write_bytes": round(wr),
                    "hbm_bytes": round(rd + wr), "algorithmic_bytes": alg,
                    "ratio": round((rd + wr) / alg, 4)}
    with open(out_json, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    if len(sys.argv) >= 2 and sys.argv[1] == "run":
        run()
    elif len(sys.argv) == 5 and sys.argv[1] == "summarize":
        summarize(sys.argv[2], sys.argv[3], sys.argv[4])
    else:
        sys.exit("usage: traffic.py run | summarize FETCH_CSV WRITE_CSV OUT_JSON")
