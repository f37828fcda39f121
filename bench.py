"""Benchmark of the Q4_0 decode hot path on one MI355X.

Headline workload (one "step"): the fused gate+up GeGLU MLP in Q4_0 at batch
1 -- hidden 3840, intermediate 15360: act = gelu_tanh(Wg x) * (Wu x), then
out = Wd act, fp32 accumulation, weights random N(0, 0.02) -> bf16 -> Q4_0.
Weights are rotated over several distinct copies so every step streams its
110.6 MB from HBM rather than from the 256 MB Infinity Cache.

Printed as one JSON line: value = MLP HBM GB/s (algorithmic bytes / wall time
of the K timed steps, recorded once as a HIP graph and replayed, as the decode
step runs), plus the dominant kernel's roofline (gate+up, its duration from
HIP events around K back-to-back launches of it alone), the CPU baseline (the
oracle's restatement of the reference CPU path, timed on this host) and
secondary figures: the single Q4_0 GEMV 8192 x 2048, the decode attention at
S = 544 / 640, the Q8_0 LM head + argmax and the 12B-shaped decode, each with
its own CPU baseline on the same bytes (--no-cpu skips the CPU legs).  The
`traffic` figures are read from the committed counter passes
(profiles/traffic.json), not measured in the run.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ai-research_amd"))

import numpy as np  # noqa: E402

import gemma_hip as gh  # noqa: E402

METRIC = "Q4_0 GEMV/fused-MLP HBM GB/s (% peak); 12B-shape Q4_0 decode tokens/s"
HBM_PEAK_GBS = 8000.0
H, I = 3840, 15360
Q4_ROW = lambda k: (k // 32) * 20  # noqa: E731  bytes per Q4_0 row (quant.zig:164-175)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_q4(ctx, rows, cols, seed, stream, staging):
    """Random N(0, 0.02) weights drawn, rounded to bf16 and quantized on the device."""
    ctx.synth_normal_dev(staging, rows * cols, seed, stream, 0.0, 0.02, bf16=True)
    out = ctx.alloc(rows * Q4_ROW(cols))
    ctx.quantize_dev(out, staging, rows, cols, gh.QUANT_Q4)
    return out


CLOCK_WARM_S = 0.15  # untimed replays before the warm-up steps of the MLP leg


def bench_mlp(ctx, steps, warmup):
    ncopy = 6  # 6 x 110.6 MB = 664 MB > 2.5 x the 256 MB Infinity Cache
    staging = ctx.alloc(I * H * 2)
    copies = []
    for c in range(ncopy):
        copies.append((make_q4(ctx, I, H, 0, 100 + 3 * c, staging),
                       make_q4(ctx, I, H, 0, 101 + 3 * c, staging),
                       make_q4(ctx, H, I, 0, 102 + 3 * c, staging)))
    # The per-kernel timings rotate over at least 640 MB of that kernel's own
    # weights too (gate+up: 9 pairs, down: 18 matrices), so neither reads
    # from the Infinity Cache; the extra copies serve only those timings.
    gu_copies = [(c[0], c[1]) for c in copies]
    dn_copies = [c[2] for c in copies]
    for c in range(3):
        gu_copies.append((make_q4(ctx, I, H, 0, 200 + 2 * c, staging),
                          make_q4(ctx, I, H, 0, 201 + 2 * c, staging)))
    for c in range(12):
        dn_copies.append(make_q4(ctx, H, I, 0, 300 + c, staging))
    staging.free()
    # x = RMSNorm(x_raw) * (1 + N(0, 0.1)), eps 1e-6 (input prep, not timed)
    xr = gh.synth_normal(H, 0, 1, 0.0, 1.0).astype(np.float64)
    w = gh.synth_normal(H, 0, 2, 1.0, 0.1).astype(np.float64)
    x = (xr / np.sqrt(np.mean(xr * xr) + 1e-6) * w).astype(np.float32)
    X, ACT, OUT = ctx.upload(x), ctx.alloc(I * 4), ctx.alloc(H * 4)

    def gate_up(i):
        wg, wu, _ = copies[i % ncopy]
        ctx.gate_up_geglu_q4(wg, wu, X, ACT, I, H)

    def down(i):
        ctx.gemv_q4(copies[i % ncopy][2], ACT, OUT, H, I)

    def gate_up_alone(i):
        wg, wu = gu_copies[i % len(gu_copies)]
        ctx.gate_up_geglu_q4(wg, wu, X, ACT, I, H)

    def down_alone(i):
        ctx.gemv_q4(dn_copies[i % len(dn_copies)], ACT, OUT, H, I)

    def record(n, parts):
        def launch(i):
            for f in parts:
                f(i)
        return record_graph(ctx, launch, n)

    # The K steps are recorded once as a HIP graph (how the decode step runs
    # them) and replayed; the warmup is a replay of W steps.
    g_warm = record(max(1, warmup), (gate_up, down))
    g_step = record(steps, (gate_up, down))
    g_gu = record(steps, (gate_up_alone,))
    g_dn = record(steps, (down_alone,))
    # Steady clocks first: the GPU idles while the graphs are recorded, and
    # the first tens of milliseconds of work after that run slower (measured
    # 4070 GB/s after 20 warm-up steps, 4290 after 2000).  So the warm-up
    # graph is replayed, untimed, for CLOCK_WARM_S before the W warm-up steps.
    t_end = time.perf_counter() + CLOCK_WARM_S
    while time.perf_counter() < t_end:
        replay(ctx, g_warm)
        ctx.sync()
    replay(ctx, g_warm)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    # timed region: K steps, synchronized on both sides
    t0 = time.perf_counter()
    ctx.record(e0)
    replay(ctx, g_step)
    ctx.record(e1)
    ctx.sync()
    wall = time.perf_counter() - t0
    step_ms = ctx.elapsed_ms(e0, e1)
    # per-kernel durations for the roofline: the same K launches of one
    # kernel alone, events on the context stream around the replay
    per_kernel = []
    for g in (g_gu, g_dn):
        replay(ctx, g)
        ctx.sync()
        ctx.record(e0)
        replay(ctx, g)
        ctx.record(e1)
        ctx.sync()
        per_kernel.append(ctx.elapsed_ms(e0, e1) / steps)
    for g in (g_warm, g_step, g_gu, g_dn):
        drop_graph(ctx, g)
    ctx.destroy_event(e0)
    ctx.destroy_event(e1)
    out = OUT.read(np.float32, H)
    assert np.all(np.isfinite(out))
    host_w = [b.read(np.uint32) for b in copies[0]]
    return wall, step_ms, per_kernel[0], per_kernel[1], x, host_w


def bench_gemv(ctx, reps=256):
    """Single Q4_0 GEMV, 8192 x 2048, rotated over 64 weight copies (671 MB).
    The copies are consecutive in one arena, so the same bytes also serve as
    256 matrices of 2048 rows and 16 of 32768: the three sizes give the
    per-launch fixed cost and the marginal read rate of the stream (a line
    t = a + bytes / b through the 2048- and 32768-row points)."""
    M, K, ncopy = 8192, 2048, 64
    mat = M * Q4_ROW(K)
    arena = ctx.alloc(ncopy * mat)
    staging = ctx.alloc(M * K * 2)
    for c in range(ncopy):
        ctx.synth_normal_dev(staging, M * K, 0, 500 + c, 0.0, 0.02, bf16=True)
        ctx.quantize_dev(arena.ptr + c * mat, staging, M, K, gh.QUANT_Q4)
    staging.free()
    x = gh.synth_normal(K, 0, 3, 0.0, 1.0)
    X = ctx.upload(x)
    Y = ctx.alloc(32768 * 4)
    host_w = arena.read(np.uint32, mat // 4).reshape(M, -1)  # copy 0, for the CPU baseline
    sizes = {}
    for rows in (8192, 2048, 32768):
        nb = rows * Q4_ROW(K)
        n = ncopy * mat // nb
        ms = timed_graph(ctx, lambda i: ctx.gemv_q4(arena.ptr + (i % n) * nb, X, Y, rows, K), reps)
        sizes[rows] = (ms * 1e3, rows * Q4_ROW(K) + K * 4 + rows * 4)
    arena.free()
    us, nbytes = sizes[M]
    (t0, b0), (t1, b1) = sizes[2048], sizes[32768]
    marginal = (b1 - b0) / ((t1 - t0) * 1e-6) / 1e9
    fit = {"us_2048_rows": round(t0, 3), "us_8192_rows": round(us, 3), "us_32768_rows": round(t1, 3),
           "marginal_gbs": round(marginal, 1),
           "fixed_us": round(t0 - b0 / (marginal * 1e9) * 1e6, 3)}
    return nbytes / (us * 1e-6) / 1e9, us, fit, (host_w, x)


def bench_gemv_bf16(ctx, reps=96):
    """The bf16 GEMV of mode none (shaders/gemv_bf16.wgsl), 8192 x 2048 bf16
    rows, rotated over 24 weight copies (805 MB)."""
    M, K, ncopy = 8192, 2048, 24
    ws = []
    for c in range(ncopy):
        w = ctx.alloc(M * K * 2)
        ctx.synth_normal_dev(w, M * K, 0, 600 + c, 0.0, 0.02, bf16=True)
        ws.append(w)
    X = ctx.upload(gh.synth_normal(K, 0, 3, 0.0, 1.0))
    Y = ctx.alloc(M * 4)
    ms = timed_graph(ctx, lambda i: ctx.gemv_bf16(ws[i % ncopy], X, Y, M, K), reps)
    for w in ws:
        w.free()
    nbytes = M * K * 2 + K * 4 + M * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 3), "bytes": nbytes, "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


# --eager: every "graph" below is replayed by launching its kernels again
# instead of recording a HIP graph.  For kernel tracing only (rocprofv3's
# kernel tracing of graph replays ends in a segfault inside the profiler);
# the timings then include the host's launch overhead and are not results.
EAGER = False


def record_graph(ctx, launch, n):
    """launch(0) .. launch(n - 1) recorded once as a HIP graph (or, with
    --eager, kept to be launched again at each replay)."""
    if EAGER:
        return (launch, n)
    ctx.graph_begin()
    for i in range(n):
        launch(i)
    return ctx.graph_end()


def replay(ctx, g):
    if EAGER:
        launch, n = g
        for i in range(n):
            launch(i)
    else:
        ctx.graph_launch(g)


def drop_graph(ctx, g):
    if not EAGER:
        ctx.graph_destroy(g)


def timed_graph(ctx, launch, reps):
    """Average ms of one launch: `reps` launches recorded once as a graph,
    replayed once untimed, then timed with HIP events on the context stream.
    One eager launch first: an entry point's first call may allocate its
    scratch, which a capture refuses."""
    launch(0)
    ctx.sync()
    g = record_graph(ctx, launch, reps)
    replay(ctx, g)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    replay(ctx, g)
    ctx.record(e1)
    ctx.sync()
    ms = ctx.elapsed_ms(e0, e1) / reps
    drop_graph(ctx, g)
    ctx.destroy_event(e0)
    ctx.destroy_event(e1)
    return ms


def bench_read_ceiling(ctx):
    """Attainable HBM read rate (gh_read_probe, a plain 16-byte load stream):
    1 GiB read once per launch (4x the Infinity Cache) over a sweep of loads
    in flight per lane, grid sizes and access orders; then, with the best
    shape, reads of 72 MiB and 36 MiB windows rotated over the same GiB -- the
    MLP kernels' sizes, where the per-launch ramp shows."""
    GiB = 1 << 30
    buf = ctx.alloc(GiB)
    ctx.fill_u32(buf, 0x3C000000, GiB // 4)  # 2^-7: sums stay finite
    sums = ctx.alloc(4 * 4096)
    ncu = 256
    sweep = []
    for grid_per_cu in (1, 2, 4, 8):
        for u in (1, 2, 4, 8):
            for contig in (0, 1):
                g = ncu * grid_per_cu
                ms = timed_graph(ctx, lambda i: ctx.read_probe(buf, GiB, u, contig, g, sums), 8)
                sweep.append((GiB / (ms * 1e-3) / 1e9, g, u, contig))
    sweep.sort(reverse=True)
    best_gbs, g, u, contig = sweep[0]
    windows = {}
    chunk = 16 * 256 * u * g  # a launch reads a whole number of grid rounds
    for mib in (72, 36):
        nb = max(chunk, (mib << 20) // chunk * chunk)
        nwin = GiB // nb
        ms = timed_graph(ctx, lambda i: ctx.read_probe(buf.ptr + nb * (i % nwin), nb, u, contig, g, sums), 64)
        windows["%dMiB" % mib] = {"bytes": nb, "us": round(ms * 1e3, 3),
                                  "gbs": round(nb / (ms * 1e-3) / 1e9, 1)}
    buf.free()
    sums.free()
    return {"gbs_1GiB": round(best_gbs, 1), "frac_of_8TBs": round(best_gbs / HBM_PEAK_GBS, 4),
            "best_shape": {"grid": g, "loads_in_flight_per_lane": u, "contiguous": contig},
            "windows": windows,
            "sweep_top5": [{"gbs": round(s[0], 1), "grid": s[1], "u": s[2], "contiguous": s[3]}
                           for s in sweep[:5]],
            "sweep_worst": round(sweep[-1][0], 1)}


def bench_attention(ctx, reps=96):
    """The decode graph's per-layer attention step (q/k norm + RoPE, the cache
    write, split-K attention and the split merge; gh_qkv_rope_attn): 16 query /
    8 kv heads of 256, 48 rotated per-layer 640-slot caches (503 MB, beyond
    the Infinity Cache), S = 544 (the steady decode context) and 640 (the
    whole ring).  Algorithmic bytes: K + V rows of the S slots, q, the new
    k/v, the output and the list."""
    nq, nkv, D, slots, nl = 16, 8, 256, 640, 48
    caches = []
    for l in range(nl):
        kc, vc = ctx.alloc(slots * nkv * D * 4), ctx.alloc(slots * nkv * D * 4)
        ctx.synth_normal_dev(kc, slots * nkv * D, 7, 2 * l, 0.0, 1.0)
        ctx.synth_normal_dev(vc, slots * nkv * D, 7, 2 * l + 1, 0.0, 1.0)
        caches.append((kc, vc))
    q, k, v = (ctx.upload(gh.synth_normal(n, 7, 200 + i, 0.0, 1.0))
               for i, n in enumerate((nq * D, nkv * D, nkv * D)))
    qn = ctx.upload(gh.synth_normal(D, 7, 210, 1.0, 0.1))
    kn = ctx.upload(gh.synth_normal(D, 7, 211, 1.0, 0.1))
    out = ctx.alloc(nq * D * 4)
    res = {}
    tab = ctx.alloc(512 * 4)
    # (S, clock, cache capacity): the capacity sets the launch's grid of splits
    # (32 per kv head at 1024, 23 at 640), S the splits that run (20 at 544)
    for S, clock, cap in ((544, 600, 640), (640, 639, 640), (544, 600, 1024)):
        slot = 32 + (clock - 32) % 512
        act = ctx.upload(np.arange(S, dtype=np.uint32))
        # as the decode graph runs it: the list 0 .. S-1 declared in the step
        # flags, the RoPE angles from the per-token table (built untimed; the
        # step kernel builds it once per token for all 48 layers)
        st = ctx.upload(np.array([clock, slot, S, 2], np.uint32))
        ctx.rope_table(st, 256, 1e4, tab)
        st_plain = ctx.upload(np.array([clock, slot, S, 0], np.uint32))

        def launch(i):
            kc, vc = caches[i % nl]
            ctx.qkv_rope_attn(q, k, v, qn, kn, kc, vc, act, st, out, nq, nkv, D, 256, False, 1e4,
                              table=tab, max_slots=cap)

        def launch_plain(i):
            kc, vc = caches[i % nl]
            ctx.qkv_rope_attn(q, k, v, qn, kn, kc, vc, act, st_plain, out, nq, nkv, D, 256, False,
                              1e4, max_slots=cap)

        ms = timed_graph(ctx, launch, reps)
        nbytes = S * nkv * D * 4 * 2 + 2 * nq * D * 4 + 2 * nkv * D * 4 + S * 4
        row = {"us": round(ms * 1e3, 3), "bytes": nbytes,
               "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
               "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if cap == 640:
            row["us_list_read_angles_computed"] = round(timed_graph(ctx, launch_plain, reps) * 1e3, 3)
            res["S%d" % S] = row
        else:
            res["S%d_capacity%d" % (S, cap)] = row
    # what the CPU baseline runs: the same inputs and layer 0's caches
    sample = {"q": q.read(np.float32, nq * D), "k": k.read(np.float32, nkv * D),
              "v": v.read(np.float32, nkv * D), "q_norm": qn.read(np.float32, D),
              "k_norm": kn.read(np.float32, D),
              "k_cache": caches[0][0].read(np.float32).reshape(slots, nkv * D),
              "v_cache": caches[0][1].read(np.float32).reshape(slots, nkv * D)}
    for kc, vc in caches:
        kc.free()
        vc.free()
    return res, sample


def bench_lm_head(ctx, reps=20):
    """Final norm -> Q8_0 LM head 262144 x 3840 -> greedy argmax (one fused
    stream plus the partial reduction), the decode step's tail.  1.13 GB of
    weights: one copy already exceeds the Infinity Cache."""
    V = 262144
    staging = ctx.alloc(V * H * 2)
    ctx.synth_normal_dev(staging, V * H, 0, 999, 0.0, 0.02, bf16=True)
    W = ctx.alloc(V * (H // 32) * 36)
    ctx.quantize_dev(W, staging, V, H, gh.QUANT_Q8)
    staging.free()
    X = ctx.upload(gh.synth_normal(H, 0, 4, 0.0, 1.0))
    NW = ctx.upload(gh.synth_normal(H, 0, 5, 1.0, 0.1))
    L, TOK = ctx.alloc(V * 4), ctx.alloc(4)
    pro = ctx.prologue(X, mode=1, norm=NW)
    ms = timed_graph(ctx, lambda i: ctx.norm_gemv_argmax_q8(W, L, TOK, V, H, pro), reps)
    # what the CPU baseline runs: the same head, input, norm and the token
    sample = {"w": W.read(np.uint32).reshape(V, -1), "x": X.read(np.float32, H),
              "norm": NW.read(np.float32, H), "token": int(TOK.read(np.uint32, 1)[0])}
    W.free()
    nbytes = V * (H // 32) * 36 + 2 * H * 4 + V * 4 + 4
    return {"us": round(ms * 1e3, 2), "bytes": nbytes, "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}, sample


def decode_step_bytes(S):
    """Algorithmic HBM bytes of one 12B-shaped decode step at S active slots:
    layer weights, the Q8 LM head, K/V rows of the S slots in 48 layers, the
    f32 norms and the 1 MiB of logits."""
    layers = 48 * (8192 * Q4_ROW(H) + H * Q4_ROW(4096) + 2 * I * Q4_ROW(H) + H * Q4_ROW(I))
    head = 262144 * (H // 32) * 36
    kv = S * 8 * 256 * 4 * 2 * 48
    norms = 48 * (4 * H + 2 * 256) * 4 + H * 4
    return layers + head + kv + norms + 262144 * 4


def cpu_decode_baseline(m, cfg, clock, nt, steps=2):
    """The oracle's restatement of the reference CPU forward
    (src/model/forward.zig:49-70, quantized weights as the GPU graph runs
    them) for whole 12B decode steps on this host: weights and caches read
    back from the device, `steps` timed steps after one untimed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from model_ref import oracle_model

    om, _ = oracle_model(m, cfg)
    ring = gh.Ring(1, 32, 512, 96)
    for c in range(clock):
        ring.activate_slot(0, c)
    x = gh.synth_normal(H, 0, 6, 0.0, 1.0)
    times = []
    for i in range(steps + 1):
        c = clock + i
        slot = ring.activate_slot(0, c)
        act = ring.active_slots(0, c)
        t0 = time.perf_counter()
        om.forward(x, c, slot, act, True, nt)
        times.append(time.perf_counter() - t0)
    dt = sum(times[1:]) / steps
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": nt,
            "host_cpus": os.cpu_count(), "kind": "port",
            "sample": "%d full 12B decode steps (48 layers + Q8 head, S = %d) after one untimed, "
                      "%.2f s each" % (steps, len(act), dt)}


def bench_decode_bf16(ctx, n_prompt=512, n_decode=32):
    """The 12B shape in mode none (the reference's --gpu): bf16 layers and the
    bf16 262144 x 3840 head (24.2 GB of weights per token).  The prompt goes
    through the batched prefill (bf16 MFMA GEMMs on the bf16 rows; median of
    2 calls after one untimed), then n_decode greedy steps on the device
    ring."""
    cfg = gh.model_config(vocab=262144, hidden=H, intermediate=I, layers=48, heads=16,
                          kv_heads=8, head_dim=256, max_slots=640,
                          full_layers=[l for l in range(48) if (l + 1) % 6 == 0])
    m = gh.Model(ctx, cfg, mode=gh.QUANT_NONE, seed=0)
    embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, H)
    scale = np.sqrt(np.float32(H))

    def emb(t):
        return (embed[t].astype(np.uint32) << 16).view(np.float32) * scale

    m.ring_init(32, 512, 96)
    prompt = gh.synth_uniform_u32(n_prompt, 1, 0, cfg.vocab_size)
    xs = np.stack([emb(int(t)) for t in prompt])
    m.ring_prefill(xs, 0, True)  # allocates the prefill buffers
    times = []
    for _ in range(2):
        t0 = time.perf_counter()
        tok = m.ring_prefill(xs, 0, True)
        times.append(time.perf_counter() - t0)
    prefill_s = min(times)
    t0 = time.perf_counter()
    for i in range(n_decode):
        tok = m.forward_clock(emb(tok), n_prompt + i, True)
    decode_s = time.perf_counter() - t0
    m.close()
    layers = 48 * (8192 * H + H * 4096 + 2 * I * H + H * I) * 2
    head = 262144 * H * 2
    norms = 48 * (4 * H + 2 * 256) * 4 + H * 4
    ideal_s = sum(layers + head + norms + 262144 * 4 + min(c + 1, 544) * 8 * 256 * 4 * 2 * 48
                  for c in range(n_prompt, n_prompt + n_decode)) / (HBM_PEAK_GBS * 1e9)
    return {"decode_tok_s": round(n_decode / decode_s, 2),
            "decode_ms_per_token": round(decode_s / n_decode * 1e3, 3),
            "weight_bytes_per_token": layers + head,
            "decode_weight_gbs": round((layers + head) * n_decode / decode_s / 1e9, 1),
            "decode_roofline_frac": round(ideal_s / decode_s, 4),
            "prefill_ms": round(prefill_s * 1e3, 2),
            "prefill_path": "batched (bf16 MFMA GEMM on the bf16 rows), best of 2 calls after 1"}


def bench_decode_q8(ctx, n_prompt=512, n_decode=64):
    """The 12B shape with Q8_0 layers (the reference's --q8) and the Q8_0 head:
    the 512-token prompt in one batched call (best of 2 after one untimed),
    then n_decode greedy steps on the device ring."""
    cfg = gh.model_config(vocab=262144, hidden=H, intermediate=I, layers=48, heads=16,
                          kv_heads=8, head_dim=256, max_slots=640,
                          full_layers=[l for l in range(48) if (l + 1) % 6 == 0])
    m = gh.Model(ctx, cfg, mode=gh.QUANT_Q8, seed=0)
    embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, H)
    scale = np.sqrt(np.float32(H))

    def emb(t):
        return (embed[t].astype(np.uint32) << 16).view(np.float32) * scale

    m.ring_init(32, 512, 96)
    prompt = gh.synth_uniform_u32(n_prompt, 1, 0, cfg.vocab_size)
    xs = np.stack([emb(int(t)) for t in prompt])
    m.ring_prefill(xs, 0, True)  # allocates the prefill buffers
    times = []
    for _ in range(2):
        t0 = time.perf_counter()
        tok = m.ring_prefill(xs, 0, True)
        times.append(time.perf_counter() - t0)
    prefill_s = min(times)
    t0 = time.perf_counter()
    for i in range(n_decode):
        tok = m.forward_clock(emb(tok), n_prompt + i, True)
    decode_s = time.perf_counter() - t0
    m.close()
    q8 = lambda k: (k // 32) * 36  # noqa: E731
    layers = 48 * (8192 * q8(H) + H * q8(4096) + 2 * I * q8(H) + H * q8(I))
    head = 262144 * q8(H)
    norms = 48 * (4 * H + 2 * 256) * 4 + H * 4
    ideal_s = sum(layers + head + norms + 262144 * 4 + min(c + 1, 544) * 8 * 256 * 4 * 2 * 48
                  for c in range(n_prompt, n_prompt + n_decode)) / (HBM_PEAK_GBS * 1e9)
    return {"decode_tok_s": round(n_decode / decode_s, 2),
            "decode_ms_per_token": round(decode_s / n_decode * 1e3, 3),
            "weight_bytes_per_token": layers + head,
            "decode_weight_gbs": round((layers + head) * n_decode / decode_s / 1e9, 1),
            "decode_roofline_frac": round(ideal_s / decode_s, 4),
            "prefill_ms": round(prefill_s * 1e3, 2),
            "prefill_path": "batched (MFMA Q8 dequant GEMM), best of 2 calls after 1"}


def bench_decode(ctx, n_prompt=512, n_decode=128, cpu=False):
    """12B-shaped decode: 48 layers (global iff (l+1) % 6 == 0), hidden 3840,
    16/8 heads of 256, intermediate 15360, vocab 262144, Q4_0 layers and Q8_0
    tied head, 640-slot ring (32 anchors, 512 window, 96 recall).  A prompt of
    512 token ids uniform over the vocabulary (seed 1) is prefilled in one
    batched call (MFMA GEMMs), then 128 greedy steps run, each one host round
    trip like gpuDispatchForwardToken: embedding on the host, slot
    bookkeeping, graph replay, token read back."""
    cfg = gh.model_config(vocab=262144, hidden=H, intermediate=I, layers=48, heads=16,
                          kv_heads=8, head_dim=256, max_slots=640,
                          full_layers=[l for l in range(48) if (l + 1) % 6 == 0])
    t0 = time.perf_counter()
    m = gh.Model(ctx, cfg, mode=gh.QUANT_Q4, seed=0)
    init_s = time.perf_counter() - t0
    embed = m.read(-1, gh.T_EMBED, np.uint16).reshape(cfg.vocab_size, H)
    scale = np.sqrt(np.float32(H))

    def emb(t):  # src/model/forward.zig:33-37
        return (embed[t].astype(np.uint32) << 16).view(np.float32) * scale

    m.ring_init(32, 512, 96)  # device-resident ring: a token uploads x and its clock
    ring = gh.Ring(1, 32, 512, 96)  # host ring, for the host-list steps at the end
    prompt = gh.synth_uniform_u32(n_prompt, 1, 0, cfg.vocab_size)
    xs = np.stack([emb(int(t)) for t in prompt])
    # Two untimed calls (the first allocates the prefill buffers; the GPU comes
    # up to clock after the idle embedding read), then the median of three
    # timed calls, each rewriting the same K/V.
    for _ in range(2):
        m.ring_prefill(xs, 0, True)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        tok = m.ring_prefill(xs, 0, True)
        times.append(time.perf_counter() - t0)
    prefill_s = sorted(times)[1]
    for c in range(n_prompt):
        ring.activate_slot(0, c)
    toks = []
    t0 = time.perf_counter()
    for i in range(n_decode):
        c = n_prompt + i
        tok = m.forward_clock(emb(tok), c, True)
        toks.append(tok)
    decode_s = time.perf_counter() - t0
    for i in range(n_decode):
        ring.activate_slot(0, n_prompt + i)
    # the same per-token work with the host's slot bookkeeping and list upload
    # (gpuDispatchForwardToken's interface): 32 more steps
    n_host = 32
    t0 = time.perf_counter()
    for i in range(n_host):
        c = n_prompt + n_decode + i
        slot = ring.activate_slot(0, c)
        tok = m.forward(emb(tok), c, slot, ring.active_slots(0, c), True)
    host_s = time.perf_counter() - t0
    # layer gating at the reference CLI's default threshold (--quiescence:
    # 0.001, src/main.zig:56): 32 more steps timed, then 8 whose run flags
    # are read back for the skip fraction
    m.set_quiescence(0.001)
    n_q = 32
    c0 = n_prompt + n_decode + n_host
    t0 = time.perf_counter()
    for i in range(n_q):
        tok = m.forward_clock(emb(tok), c0 + i, True)
    q_s = time.perf_counter() - t0
    gated, skipped = 0, 0
    for i in range(8):
        tok = m.forward_clock(emb(tok), c0 + n_q + i, True)
        flags = m.read(-1, gh.T_GATE_FLAGS, np.uint32)[48 // 3:]
        gated += flags.size
        skipped += int((flags == 0).sum())
    m.set_quiescence(0.0)
    for i in range(n_q + 8):
        ring.activate_slot(0, c0 + i)
    n_host += n_q + 8
    cpu_dec = None
    if cpu:
        cpu_dec = cpu_decode_baseline(m, cfg, n_prompt + n_decode + n_host,
                                      max(1, min(16, os.cpu_count() or 1)))
    # later-turn prompts past the window's wraparound (fresh clocks after the
    # run): batched through staging rows, median of 3 calls each
    wrapped = {}
    c = n_prompt + n_decode + n_host
    for T in (16, 64, 128):
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            m.ring_prefill(xs[:T], c, True)
            times.append(time.perf_counter() - t0)
            c += T
        wrapped[str(T)] = round(sorted(times)[1] * 1e3, 2)
    # short first-turn prompts (clocks from 0, after the run): 1-2 tokens go
    # token by token through the decode graphs, longer ones to the batched
    # kernels (the weight-streaming GEMMs up to 48 tokens); median of 3 calls
    # each
    short = {}
    for T in (1, 2, 3, 4, 8, 16, 32, 48, 64):
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            m.ring_prefill(xs[:T], 0, True)
            times.append(time.perf_counter() - t0)
        short[str(T)] = round(sorted(times)[1] * 1e3, 2)
    m.close()
    clocks = range(n_prompt, n_prompt + n_decode)
    ideal_s = sum(decode_step_bytes(min(c + 1, 544)) for c in clocks) / (HBM_PEAK_GBS * 1e9)
    step_bytes = (48 * (8192 * Q4_ROW(H) + H * Q4_ROW(4096) + 2 * I * Q4_ROW(H) + H * Q4_ROW(I))
                  + 262144 * (H // 32) * 36)
    gemm_flop = 2 * n_prompt * 48 * (8192 * H + H * 4096 + 2 * I * H + H * I)
    return {"decode_tok_s": round(n_decode / decode_s, 2),
            "decode_ms_per_token": round(decode_s / n_decode * 1e3, 3),
            "decode_weight_gbs": round(step_bytes * n_decode / decode_s / 1e9, 1),
            "decode_roofline_ms_per_token": round(ideal_s / n_decode * 1e3, 4),
            "decode_roofline_frac": round(ideal_s / decode_s, 4),
            "decode_path": "device ring (gh_model_forward_clock): x and the clock go up, the "
                           "token comes back, one host round trip per token",
            "decode_tok_s_host_lists": round(32 / host_s, 2),
            "decode_tok_s_quiescence_0.001": round(n_q / q_s, 2),
            "quiescence_skip_fraction": round(skipped / max(1, gated), 4),
            "prefill_tok_s": round(n_prompt / prefill_s, 1),
            "prefill_ms": round(prefill_s * 1e3, 2),
            "prefill_path": "batched (MFMA Q4 dequant GEMM), one call; median of 3 after 2 warm-up calls",
            "prefill_gemm_tflops": round(gemm_flop / prefill_s / 1e12, 1),
            "prefill_short_ms": short,
            "prefill_wrapped_ms": wrapped,
            "model_init_s": round(init_s, 2),
            "decode_tokens_head": [int(t) for t in toks[:8]],
            "cpu_decode_baseline": cpu_dec}


def _median_time(fn, budget_s, min_runs=3):
    """Median seconds of fn() over at least min_runs runs and budget_s
    seconds, after one untimed run."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_kernel_baselines(gemv_sample, attn_sample, head_sample, budget_s=2.0):
    """The oracle's restatement of the reference CPU path for the other
    workloads, timed on this host on the same bytes the GPU legs read, each
    the median of at least 3 runs after one untimed:
      * Q4_0 GEMV 8192 x 2048: the src/test_q4_exec.zig:56-74 dequant loop
        inside gemvParallel's 16-job row split (src/kernels.zig:76-92), on
        16 threads (or the host's count) and on one;
      * decode attention at S = 544 and 640: q/k RMSNorm + RoPE and the cache
        write, then runAttentionHeads (src/model/forward.zig:77-104,125-143),
        which the reference runs on one thread;
      * the Q8_0 LM head + argmax: final RMSNorm, the Q8_0 GEMV
        (shaders/gemv_q8.wgsl's dequant order; the reference CPU path is
        bf16-only) split 16 ways, and sampleArgmax (src/kernels.zig:164-174).
    GB/s on the same algorithmic bytes as the GPU figures."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    nt = max(1, min(16, os.cpu_count() or 1))
    res = {}
    w, x = gemv_sample
    M, K = w.shape[0], x.size
    nbytes = M * Q4_ROW(K) + K * 4 + M * 4
    t16, n16 = _median_time(lambda: orc.gemv_q4(w, x, K, nt), budget_s)
    t1, n1 = _median_time(lambda: orc.gemv_q4(w, x, K, 1), budget_s)
    res["gemv_q4_8192x2048"] = {
        "value": round(nbytes / t16 / 1e9, 3), "unit": "GB/s", "cores": nt,
        "host_cpus": os.cpu_count(), "kind": "port",
        "sample": "%d calls, median %.3f ms, 16-job row split" % (n16, t16 * 1e3),
        "one_thread": {"value": round(nbytes / t1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                       "sample": "%d calls, median %.3f ms" % (n1, t1 * 1e3)}}
    a = attn_sample
    nq, nkv, D = 16, 8, 256
    for S, clock in ((544, 600), (640, 639)):
        slot = 32 + (clock - 32) % 512
        active = np.arange(S, dtype=np.uint32)
        kc, vc = a["k_cache"].copy(), a["v_cache"].copy()

        def step():
            q, k, v = orc.qkv_norm_rope(a["q"], a["k"], a["v"], a["q_norm"], a["k_norm"], nq, nkv,
                                        D, 256, False, 1e4, 1e-6, clock)
            kc[slot], vc[slot] = k, v
            return orc.attention(q, kc, vc, active, nq, nkv, D)

        t, n = _median_time(step, budget_s)
        nb = S * nkv * D * 4 * 2 + 2 * nq * D * 4 + 2 * nkv * D * 4 + S * 4
        res["attention_S%d" % S] = {
            "value": round(nb / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "us": round(t * 1e6, 1),
            "sample": "%d calls (q/k norm + RoPE, cache write, 16 heads over %d slots), median "
                      "%.3f ms" % (n, S, t * 1e3)}
    h = head_sample
    V = h["w"].shape[0]

    def head():
        xn = orc.rmsnorm(h["x"], h["norm"])
        return orc.argmax(orc.gemv_q8(h["w"], xn, H, nt))

    tok = head()
    t, n = _median_time(head, budget_s * 1.5)
    nb = V * (H // 32) * 36 + 2 * H * 4 + V * 4 + 4
    res["lm_head_q8_argmax"] = {
        "value": round(nb / t / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
        "ms": round(t * 1e3, 2), "token": tok, "token_equals_gpu": tok == h["token"],
        "sample": "%d calls (RMSNorm, Q8_0 GEMV 262144 x 3840 split 16 ways, argmax), median "
                  "%.1f ms" % (n, t * 1e3)}
    return res


def cpu_baseline(x, host_w, budget_s=10.0, threads=None):
    """The oracle's restatement of the reference CPU path (src/test_q4_exec.zig
    dequant loop inside gatedMlp's 16-job row split, src/kernels.zig:100-129)
    timed on this host over whole MLP steps (threads: 16 or the host's count
    if lower, unless given)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    nt = threads or max(1, min(16, os.cpu_count() or 1))
    wg, wu, wd = (w.reshape(r, -1) for w, r in zip(host_w, (I, I, H)))
    orc.gated_mlp_q4(x, wg, wu, wd, nt)  # warm-up
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        orc.gated_mlp_q4(x, wg, wu, wd, nt)
        n += 1
    dt = time.perf_counter() - t0
    return n, dt, nt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the 12B decode leg")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the 12B decode leg and print its figures (for profiling)")
    ap.add_argument("--prompt", type=int, default=512, help="decode leg: prompt tokens")
    ap.add_argument("--decode", type=int, default=128, help="decode leg: greedy steps")
    ap.add_argument("--eager", action="store_true",
                    help="launch kernels directly instead of replaying HIP graphs (for kernel "
                         "tracing; the timings then include launch overhead and are not results)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print("bench.py measures one MI355X: the decode backend has no multi-GPU path "
              "(--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    ctx = gh.Context()
    log("device:", ctx.device_name)
    if args.decode_only:
        print(json.dumps({"decode_12b": bench_decode(ctx, args.prompt, args.decode)}), flush=True)
        ctx.close()
        return
    wall, step_ms, gu_ms, dn_ms, x, host_w = bench_mlp(ctx, args.steps, args.warmup)
    gu_bytes = 2 * I * Q4_ROW(H) + H * 4 + I * 4
    dn_bytes = H * Q4_ROW(I) + I * 4 + H * 4
    step_bytes = gu_bytes + dn_bytes
    value = step_bytes * args.steps / wall / 1e9
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
    gemv_gbs, gemv_us, gemv_fit, gemv_sample = bench_gemv(ctx)
    ceiling = bench_read_ceiling(ctx)
    attn, attn_sample = bench_attention(ctx)
    head, head_sample = bench_lm_head(ctx)
    gemv_bf16 = bench_gemv_bf16(ctx)
    dec = bench_decode(ctx, args.prompt, args.decode, cpu=not args.no_cpu) if not args.no_decode else None
    dec_bf16 = bench_decode_bf16(ctx, args.prompt) if not args.no_decode else None
    dec_q8 = bench_decode_q8(ctx, args.prompt) if not args.no_decode else None
    if dec:
        log("decode %.1f tok/s (%.3f ms/token), prefill %.1f tok/s"
            % (dec["decode_tok_s"], dec["decode_ms_per_token"], dec["prefill_tok_s"]))
    log("mlp %.1f GB/s, gate_up %.2f us, down %.2f us, gemv8192x2048 %.2f us"
        % (value, gu_ms * 1e3, dn_ms * 1e3, gemv_us))

    # HBM bytes per launch: not measured in this run, but read from the
    # committed counter passes (traffic.py: rocprofv3 --pmc FETCH_SIZE, then
    # WRITE_SIZE, scaled by a copy kernel's reading; profiles/traffic.json)
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    trec = json.load(open(tpath)) if os.path.exists(tpath) else {}
    tbytes = lambda k: trec[k]["hbm_bytes"] if k in trec else None  # noqa: E731
    traffic = tbytes("gh_gateup_q4")
    attn["S544"]["traffic"] = tbytes("attention_544")
    head["traffic"] = tbytes("lm_head_q8")

    cpu = cpu1 = cpu_kernels = None
    if not args.no_cpu:
        cpu_kernels = cpu_kernel_baselines(gemv_sample, attn_sample, head_sample)
        attn["S544"]["cpu_baseline"] = cpu_kernels["attention_S544"]
        attn["S640"]["cpu_baseline"] = cpu_kernels["attention_S640"]
        head["cpu_baseline"] = cpu_kernels["lm_head_q8_argmax"]
    del gemv_sample, attn_sample, head_sample
    if not args.no_cpu:
        n, dt, nt = cpu_baseline(x, host_w)
        cpu = {"value": round(step_bytes * n / dt / 1e9, 3), "unit": "GB/s", "cores": nt,
               "host_cpus": os.cpu_count(), "kind": "port",
               "sample": "%d full MLP steps (3840/15360 Q4_0, copy 0 of the weights) in %.1f s "
                         "with the oracle's 16-way row split" % (n, dt)}
        n1, dt1, _ = cpu_baseline(x, host_w, budget_s=4.0, threads=1)
        cpu1 = {"value": round(step_bytes * n1 / dt1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                "sample": "%d full MLP steps in %.1f s on one thread" % (n1, dt1)}

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "fused gate+up GeGLU + down projection, Q4_0, batch 1",
                   "hidden": H, "intermediate": I, "weight_copies_rotated": 6,
                   "bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "gh_gateup_q4",
                     "avg_launch_us": round(gu_ms * 1e3, 3),
                     "traffic_source": "committed counter pass (profiles/traffic.json), "
                                       "not measured in this run"},
        "cpu_baseline": cpu,
        "extra": {"mlp_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
                  "clock_warmup_ms": round(CLOCK_WARM_S * 1e3),
                  "mlp_gbs_event_timed": round(step_bytes * args.steps / (step_ms * 1e-3) / 1e9, 1),
                  "down_proj_us": round(dn_ms * 1e3, 3),
                  "down_proj_gbs": round(dn_bytes / (dn_ms * 1e-3) / 1e9, 1),
                  "gemv_q4_8192x2048_gbs": round(gemv_gbs, 1),
                  "gemv_q4_8192x2048_us": round(gemv_us, 3),
                  "gemv_q4_8192x2048_roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1),
                                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                 "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                                                 "bytes": 10526720,
                                                 "traffic": tbytes("gemv_q4_8192x2048")},
                  "gemv_q4_8192x2048_cpu_baseline": cpu_kernels and cpu_kernels["gemv_q4_8192x2048"],
                  "traffic_source": "every traffic figure: the committed counter passes in "
                                    "profiles/traffic.json (traffic.py), not this run",
                  "down_proj_traffic": tbytes("gh_gemv_q4"),
                  "gemv_q4_k2048_size_fit": gemv_fit,
                  "hbm_read_ceiling": ceiling,
                  "attention_640_slots": attn,
                  "lm_head_q8_argmax": head,
                  "gemv_bf16_8192x2048": gemv_bf16,
                  "decode_12b_bf16": dec_bf16,
                  "decode_12b_q8": dec_q8,
                  "cpu_baseline_1thread": cpu1,
                  "decode_12b": dec},
    }
    ctx.close()
    if EAGER:
        line["extra"]["timings"] = "eager launches for kernel tracing: not results"
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
