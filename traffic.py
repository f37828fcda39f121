"""HBM traffic of the decode kernels from rocprofv3 counters.

Two rocprofv3 passes, one counter each (FETCH_SIZE, then WRITE_SIZE, KiB per
dispatch), over `python traffic.py run`, which launches:
  * a device-to-device copy of COPY_BYTES (the calibration kernel: it reads
    and writes exactly COPY_BYTES),
  * the Q4_0 fused gate+up GeGLU, 15360 x 3840, and the down projection,
    3840 x 15360, over 6 rotated weight copies (so every launch streams from
    HBM, not from the 256 MB Infinity Cache),
  * the Q4_0 GEMV 8192 x 2048 over 40 rotated copies (421 MB),
  * the decode attention step at 544 active slots (q/k norm + RoPE + cache
    write + split-K attention, then the split merge; 16 query / 8 kv heads
    of 256) over 48 rotated 640-slot caches (503 MB),
  * the final norm + Q8_0 LM head 262144 x 3840 + block argmax (1.13 GB).
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

V, S, NQ, NKV, D, SLOTS = 262144, 544, 16, 8, 256, 640
ALGORITHMIC = {  # bytes one launch must move: weights + x in + y out
    "gh_gateup_q4": 2 * I * Q4_ROW(H) + H * 4 + I * 4,
    "gh_gemv_q4": H * Q4_ROW(I) + I * 4 + H * 4,  # the down projection
    "gemv_q4_8192x2048": 8192 * Q4_ROW(2048) + 2048 * 4 + 8192 * 4,
    # K and V rows of the S slots, q, the new k and v, the output, the list
    # (attention and merge kernels together)
    "attention_544": S * NKV * D * 4 * 2 + 2 * NQ * D * 4 + 2 * NKV * D * 4 + S * 4,
    # Q8_0 rows, x and the norm weight in, the logits out, the token
    "lm_head_q8": V * (H // 32) * 36 + 2 * H * 4 + V * 4 + 4,
}
# kernel-name prefix -> ALGORITHMIC key (each dispatch's counters are summed
# per key: the attention step is two kernels)
FAMILIES = (
    ("gh_gateup_q4_", "gh_gateup_q4"),
    ("gh_gateup_q4n_", "gh_gateup_q4"),
    ("gh_gemv_q4_t64_g2_d1_w", "gh_gemv_q4"),
    ("gh_gemv_q4_t16_g1_d1", "gemv_q4_8192x2048"),
    ("gh_attn_d4_k", "attention_544"),
    ("gh_attn_merge_k", "attention_544"),
    ("gh_argmax_q8n_", "lm_head_q8"),
    ("gh_argmax_final_k", "lm_head_q8"),
)


def run(launches=30):
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "ai-research_amd"))
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
    for mats in copies:
        for m in mats:
            m.free()
    # config-1 GEMV: 40 rotated 8192 x 2048 copies
    staging = ctx.alloc(8192 * 2048 * 2)
    gcopies = []
    for c in range(40):
        ctx.synth_normal_dev(staging, 8192 * 2048, 0, 400 + c, 0.0, 0.02, bf16=True)
        m = ctx.alloc(8192 * Q4_ROW(2048))
        ctx.quantize_dev(m, staging, 8192, 2048, gh.QUANT_Q4)
        gcopies.append(m)
    staging.free()
    x2 = ctx.upload(gh.synth_normal(2048, 0, 2, 0.0, 1.0))
    y2 = ctx.alloc(8192 * 4)
    for i in range(launches):
        ctx.gemv_q4(gcopies[i % 40], x2, y2, 8192, 2048)
    ctx.sync()
    for m in gcopies:
        m.free()
    # decode attention at S = 544 over 48 rotated caches, as the decode graph
    # runs it (list 0 .. S-1 declared dense, RoPE angles from the table)
    import numpy as np
    caches = []
    for l in range(48):
        kc, vc = ctx.alloc(SLOTS * NKV * D * 4), ctx.alloc(SLOTS * NKV * D * 4)
        ctx.synth_normal_dev(kc, SLOTS * NKV * D, 7, 2 * l, 0.0, 1.0)
        ctx.synth_normal_dev(vc, SLOTS * NKV * D, 7, 2 * l + 1, 0.0, 1.0)
        caches.append((kc, vc))
    q, k, v = (ctx.upload(gh.synth_normal(n, 7, 200 + i, 0.0, 1.0))
               for i, n in enumerate((NQ * D, NKV * D, NKV * D)))
    qn = ctx.upload(gh.synth_normal(D, 7, 210, 1.0, 0.1))
    kn = ctx.upload(gh.synth_normal(D, 7, 211, 1.0, 0.1))
    out = ctx.alloc(NQ * D * 4)
    clock = 600
    act = ctx.upload(np.arange(S, dtype=np.uint32))
    st = ctx.upload(np.array([clock, 32 + (clock - 32) % 512, S, 2], np.uint32))
    tab = ctx.alloc(512 * 4)
    ctx.rope_table(st, D, 1e4, tab)
    for i in range(launches):
        kc, vc = caches[i % 48]
        ctx.qkv_rope_attn(q, k, v, qn, kn, kc, vc, act, st, out, NQ, NKV, D, D, False, 1e4,
                          table=tab)
    ctx.sync()
    for kc, vc in caches:
        kc.free()
        vc.free()
    # final norm + Q8_0 LM head + argmax (one 1.13 GB copy exceeds the cache)
    staging = ctx.alloc(V * H * 2)
    ctx.synth_normal_dev(staging, V * H, 0, 999, 0.0, 0.02, bf16=True)
    W = ctx.alloc(V * (H // 32) * 36)
    ctx.quantize_dev(W, staging, V, H, gh.QUANT_Q8)
    staging.free()
    nw = ctx.upload(gh.synth_normal(H, 0, 5, 1.0, 0.1))
    logits, tok = ctx.alloc(V * 4), ctx.alloc(4)
    pro = ctx.prologue(X, mode=1, norm=nw)
    for i in range(10):
        ctx.norm_gemv_argmax_q8(W, logits, tok, V, H, pro)
    ctx.sync()
    print("traffic workload done: %d copies of %d B, %d MLP steps, GEMV, attention and LM-head "
          "launches" % (5, COPY_BYTES, launches), flush=True)


def _kernel_key(name):
    for prefix, key in FAMILIES:
        if name.startswith(prefix):
            return key
    if "copyBuffer" in name:
        return "copy"
    return None


def _averages(path, counter):
    """Per key: the sum over its kernels of each kernel's average counter
    value per dispatch."""
    vals = defaultdict(list)
    with open(path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            name = row["Kernel_Name"]
            if _kernel_key(name):
                vals[name].append(float(row["Counter_Value"]))
    per_key = defaultdict(float)
    for name, v in vals.items():
        if "copyBuffer" in name:
            # small host-upload blits share the name: keep the COPY_BYTES
            # dispatches (the largest by far)
            top = max(v)
            v = [x for x in v if x >= 0.5 * top]
        per_key[_kernel_key(name)] += sum(v) / len(v)
    return dict(per_key)


def summarize(fetch_csv, write_csv, out_json):
    fetch = _averages(fetch_csv, "FETCH_SIZE")
    write = _averages(write_csv, "WRITE_SIZE")
    kib = COPY_BYTES / 1024.0
    f_scale, w_scale = kib / fetch["copy"], kib / write["copy"]
    out = {"calibration": {"copy_bytes": COPY_BYTES,
                           "copy_fetch_kib": fetch["copy"], "copy_write_kib": write["copy"],
                           "fetch_scale": f_scale, "write_scale": w_scale}}
    for fam, alg in ALGORITHMIC.items():
        if fam not in fetch or fam not in write:
            continue
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
