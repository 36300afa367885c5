"""Benchmark of the quantized MoE expert path on one MI355X.

Workload (N=1): a Qwen3-30B-A3B-shaped MoE layer at decode batch 1 -- 128
SwiGLU experts in q4_0 (H 2048, I 768), f32 router [128 x 2048], softmax,
top-8 renormalised, weighted combine.  One step is one token through one
MoE layer.  48 such layers (the model's depth, 16.3 GB) stay resident in HBM
and consecutive steps visit consecutive layers with fresh inputs, so every
step reads weights that are not in the 256 MB last-level cache.  The steps
run --warmup eager steps first (each layer's scratch is sized beforehand by
MoeLayer.reserve, which runs nothing), then exactly --steps steps in one
region timed with HIP events on the library's stream: replays of a captured
graph of one pass over the 48 layers, then a graph of the remaining steps
(graphs are uploaded when captured).  `value` and `ms_per_step` come from
that region; `timing` gives the median, min and max per step over 20 more
passes timed one at a time, after it.

value: algorithmic bytes per step (8 routed experts x 2,654,208 B + the
1,048,576 B router) x steps / time, in GB/s.  roofline: the dominant
kernel's algorithmic bytes per launch / its average duration, timed with
HIP events on the library's stream during a second (eager) pass.
roofline.traffic: HBM bytes per launch of that kernel from the FETCH_SIZE and
WRITE_SIZE counter passes, each scaled by what the counter reads for the
plain copy kernel, as committed in profiles/traffic_decode_q4_qwen3_30b.txt.
cpu_baseline: the oracle (C restatement of the reference CPU algorithm)
on one layer of the same shape on this host, built -march=x86-64 and
-march=native, each on all threads and on one; medians of at least 20 tokens.
expert: one q8_0 Qwen3-30B expert (Expert::forward, 1 token), 128 distinct
experts in turn (cold weights).
decode_more: Mixtral-8x7B- and Qwen3-235B-shaped decode layers, same timing,
and 8 (Mixtral) or 16 (Qwen3-235B) tokens per step on each path.
float_matvec: WeightMatrix::matvec over float weights (a bf16 vocabulary
projection and a dense f32 matrix), GB/s of weight bytes.
attention: RMSNorm + Attention::forward of one token with 4096 cached
positions (Qwen3-30B-A3B shape, bf16 projections), per-kernel times.
reference_kernel_bench: the reference's `hale bench kernels` (a 4096 x 4096
WeightMatrix::matvec per dtype: f32, bf16, f16, q8_0, q4_0) on the GPU, cold
(rotated copies) and warm (one matrix, as the reference loops), with the
oracle at the same shape on the host in cpu_baseline.
strict_dropin: the decode workload through the unchanged provider surface
(route, fetch, k x Expert::forward, host combine), microseconds per token.
decode_few_tokens / decode_band: the same layers with 2 to 64 tokens per
step (graph replay): the default path (one decode pass below the layer's
grouped threshold, from it the expert-grouped row-chain kernels up to the
band threshold, the grouped int8 matrix products above) and, from 16
tokens, each of the three forced.
stream_read_ceiling: each decode kernel beside the library's plain read of
the same bytes in one launch.
prefill: the two multi-token workloads (512 tokens q8_0 H 2048 I 768, and
2048 tokens q4_0 H 4096 I 1536; 128 experts, top-8, Zipf-skewed routing)
with tokens/s, TOPS, the fraction of the int8 MFMA peak and a roofline
block for the dominant grouped kernel (HBM for the 512-token workload,
int8 MFMA for the 2048-token one).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--no-prefill] [--prefill-only] [--decode-eager]
                       [--eager-leg kernels|float|expert|band|attention]
                       [--copy-calibration BYTES]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hale-token_amd"))

import numpy as np  # noqa: E402

import hale_moe as H  # noqa: E402

METRIC = "expert FFN GB/s (% HBM peak) decode; MoE-layer tokens/s + MFMA % prefill"
HBM_PEAK_GBS = 8000.0

E, HID, INTER, TOPK = 128, 2048, 768, 8
DTYPE = H.Q4_0
INT8_PEAK_OPS = 5.0e15  # MI355X dense int8 MFMA

# tokens per step of the batched decode_more measurement
MORE_BATCH = {"mixtral-8x7b decode q4_0": 8, "qwen3-235b-a22b decode q4_0": 16}
# further decode workloads: (name, dtype, hidden, inter, experts, top_k, layers)
DECODE_MORE = [
    ("mixtral-8x7b decode q4_0", H.Q4_0, 4096, 14336, 8, 2, 4),
    ("qwen3-235b-a22b decode q4_0", H.Q4_0, 4096, 1536, 128, 8, 6),
]

# prefill workloads: (name, dtype, hidden, inter, experts, top_k, tokens, roofline bound)
PREFILL = [
    ("qwen3-30b-a3b prefill 512 tok q8_0", H.Q8_0, 2048, 768, 128, 8, 512, "hbm"),
    ("qwen3-235b-a22b prefill 2048 tok q4_0", H.Q4_0, 4096, 1536, 128, 8, 2048, "mfma"),
]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(dtype, hidden, inter):
    return 2 * inter * H.row_bytes(dtype, hidden) + hidden * H.row_bytes(dtype, inter)


def build_layers(ctx, nlayers, seed=1234, dtype=DTYPE, hid=HID, inter=INTER, experts=E,
                 topk=TOPK, router=True):
    """nlayers MoE layers with N(0, 0.02^2) weights quantized on the GPU."""
    ng = inter * H.row_bytes(dtype, hid)
    nd = hid * H.row_bytes(dtype, inter)
    chunk = min(experts, 32)  # experts generated per pass (bounds the f32 staging)
    vals = ctx.malloc(chunk * inter * hid * 4)
    aos = [ctx.malloc(chunk * ng), ctx.malloc(chunk * ng), ctx.malloc(chunk * nd)]
    rbuf = ctx.malloc(experts * hid * 4) if router else None
    layers = []
    for l in range(nlayers):
        rm = None
        if router:
            rbuf.fill_normal(seed + 7919 * l, experts * hid, 0.0, 0.02)
            rmat = H._vp()
            ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, H.F32, experts, hid,
                                                        H._vp(rbuf.address), experts * hid * 4,
                                                        H.C.byref(rmat)), "router")
            rm = H.WeightMatrix(ctx, rmat, experts, hid, H.F32)
        moe = H.MoeLayer(ctx, l, experts, hid, inter, dtype, topk, True, rm)
        for e0 in range(0, experts, chunk):
            n = min(chunk, experts - e0)
            for j, (rows, cols) in enumerate(((inter, hid), (inter, hid), (hid, inter))):
                vals.fill_normal(seed + 7919 * l + 101 * (j + 1) + 1000003 * e0, n * rows * cols, 0.0, 0.02)
                ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dtype, n * rows, cols,
                                                          H._vp(vals.address), H._vp(aos[j].address)),
                          "encode")
            moe.set_experts_device(e0, n, aos[0].address, aos[1].address, aos[2].address)
        layers.append(moe)
    for b in (vals, rbuf, *aos):
        if b is not None:
            b.free()
    return layers


PREFILL_WARMUP = 30  # untimed forwards before each prefill timing


def gpu_prefill(name, dtype, hid, inter, experts, topk, tokens, reps, bound="mfma", router=True):
    """One MoE layer forward over `tokens` tokens with Zipf-skewed routing
    (and, with `router`, the same forward through the layer's router)."""
    from hale_moe.synth import zipf_logits

    ctx = H.Context(0)
    # the layer has a router too: the workload's logits are given (Zipf), and
    # one more timing runs the same forward through the router instead
    moe = build_layers(ctx, 1, seed=4321, dtype=dtype, hid=hid, inter=inter, experts=experts,
                       topk=topk, router=True)[0]
    logits = zipf_logits(tokens, experts, 1.1, seed=7)
    dl = ctx.malloc(logits.nbytes)
    dl.upload(logits)
    dx = ctx.malloc(tokens * hid * 4)
    dx.fill_normal(17, tokens * hid, 0.0, 1.0)
    dout = ctx.malloc(tokens * hid * 4)
    didx = ctx.malloc(tokens * topk * 4)
    # untimed forwards first: a GPU that has not been busy runs the first
    # forwards up to about 10 % slower (2048 tokens q4_0: 1.49 ms in the
    # first five, 1.32-1.36 ms from about the twenty-fifth on)
    for _ in range(PREFILL_WARMUP):
        moe.forward_device(tokens, dx.address, dout.address, dl.address, didx.address)
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        moe.forward_device(tokens, dx.address, dout.address, dl.address)
    ms = ctx.timer_stop() / reps
    ctx.profile(True)
    ctx.profile_reset()
    for _ in range(reps):
        moe.forward_device(tokens, dx.address, dout.address, dl.address)
    prof = ctx.profile_read()
    ctx.profile(False)
    # the same forward with the layer's router computing the logits
    router_ms, rprof = None, None
    if router:
        for _ in range(PREFILL_WARMUP // 3):
            moe.forward_device(tokens, dx.address, dout.address)
        ctx.synchronize()
        ctx.timer_start()
        for _ in range(reps):
            moe.forward_device(tokens, dx.address, dout.address)
        router_ms = ctx.timer_stop() / reps
        ctx.profile(True)
        ctx.profile_reset()
        for _ in range(reps):
            moe.forward_device(tokens, dx.address, dout.address)
        rprof = ctx.profile_read()
        ctx.profile(False)
    # the opt-in FMA fold of the grouped down projection: its time, and its
    # relative L2 distance from the exact output on the same input
    moe.forward_device(tokens, dx.address, dout.address, dl.address)
    exact = dout.download(np.float32, tokens * hid).astype(np.float64)
    moe.set_down_fold("fma")
    for _ in range(PREFILL_WARMUP // 3):
        moe.forward_device(tokens, dx.address, dout.address, dl.address)
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        moe.forward_device(tokens, dx.address, dout.address, dl.address)
    fma_ms = ctx.timer_stop() / reps
    ctx.profile(True)
    ctx.profile_reset()
    for _ in range(reps):
        moe.forward_device(tokens, dx.address, dout.address, dl.address)
    fma_prof = ctx.profile_read()
    ctx.profile(False)
    fma_out = dout.download(np.float32, tokens * hid).astype(np.float64)
    moe.set_down_fold("exact")
    fma_rel = float(np.linalg.norm(fma_out - exact) / max(np.linalg.norm(exact), 1e-30))
    idx = didx.download(np.int32, tokens * topk)
    touched = len(np.unique(idx))
    groups = np.bincount(idx, minlength=experts)
    ops = 2.0 * tokens * topk * 3 * hid * inter
    wbytes = touched * expert_bytes(dtype, hid, inter)
    sec = ms / 1000.0
    res = {
        "workload": name, "tokens": tokens, "ms": round(ms, 4), "warmup_forwards": PREFILL_WARMUP,
        "timed_forwards": reps,
        "tokens_per_s": round(tokens / sec, 1),
        "tops": round(ops / sec / 1e12, 2),
        "pct_int8_mfma_peak": round(100 * ops / sec / INT8_PEAK_OPS, 2),
        "weight_bytes": wbytes, "pct_hbm_peak": round(100 * wbytes / sec / 1e9 / HBM_PEAK_GBS, 2),
        "experts_touched": touched, "group_sizes": {"max": int(groups.max()),
                                                      "median": float(np.median(groups)),
                                                      "min": int(groups.min())},
        "kernels": {k: {"avg_us": round(1000 * v[0] / v[1], 2), "launches": v[1]} for k, v in prof.items()},
        "fma_down_fold": {"ms": round(fma_ms, 4), "tokens_per_s": round(tokens / (fma_ms / 1000.0), 1),
                          "pct_int8_mfma_peak": round(100 * ops / (fma_ms / 1000.0) / INT8_PEAK_OPS, 2),
                          "grouped_down_avg_us": round(1000 * fma_prof["grouped_down"][0] / fma_prof["grouped_down"][1], 2),
                          "rel_l2_vs_exact": float(f"{fma_rel:.3e}")},
        "with_router": None if router_ms is None else {
            "ms": round(router_ms, 4), "tokens_per_s": round(tokens / (router_ms / 1000.0), 1),
            "route_avg_us": round(1000 * rprof["route"][0] / rprof["route"][1], 2),
            "note": "the same forward, logits from the layer's f32 router (routes differ from the Zipf workload's)"},
    }
    # roofline of the dominant grouped kernel: algorithmic weight bytes (every
    # touched expert's planes once) against HBM, or int8 ops against the MFMA
    A = tokens * topk
    per_launch = {"grouped_gate_up": (touched * 2 * inter * H.row_bytes(dtype, hid), 2.0 * A * 2 * hid * inter),
                  "grouped_down": (touched * hid * H.row_bytes(dtype, inter), 2.0 * A * hid * inter)}
    dom = max((k for k in prof if k in per_launch), key=lambda k: prof[k][0])
    dom_s = prof[dom][0] / prof[dom][1] / 1000.0
    nbytes, nops = per_launch[dom]
    if bound == "hbm":
        ach, peak, unit = nbytes / dom_s / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        ach, peak, unit = nops / dom_s / 1e12, INT8_PEAK_OPS / 1e12, "TOP/s"
    res["roofline"] = {"bound": bound, "kernel": dom, "achieved": round(ach, 1), "peak": peak,
                       "unit": unit, "frac": round(ach / peak, 4),
                       "traffic": measured_traffic(PREFILL_TRAFFIC[name]).get(dom),
                       "bytes_per_launch": nbytes, "ops_per_launch": nops}
    for b in (dl, dx, dout, didx):
        b.free()
    moe.close()
    ctx.close()
    return res


def copy_calibration(nbytes, reps=5):
    """The library's plain copy kernel over nbytes, reps times: the yardstick
    for the FETCH_SIZE / WRITE_SIZE counters (each launch reads and writes
    nbytes)."""
    ctx = H.Context(0)
    a, b = ctx.malloc(nbytes), ctx.malloc(nbytes)
    a.fill_normal(1, nbytes // 4)
    b.copy_from(a, nbytes)
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        b.copy_from(a, nbytes)
    ms = ctx.timer_stop() / reps
    a.free()
    b.free()
    ctx.close()
    return {"copy_bytes": nbytes, "launches": reps + 1, "ms": round(ms, 4),
            "GB_per_s": round(2 * nbytes / ms / 1e6, 1)}


STREAM_POOL = 768 << 20          # three times the 256 MB last-level cache: every read is cold
STREAM_WORKGROUPS = (512, 1024, 2048)


def stream_ceiling(named_bytes, reps=12):
    """What one launch can stream from HBM: the library's plain read kernel
    over each kernel's bytes, each launch timed like the decode kernels'
    (events around the launch, eager), cold (consecutive reads walk a pool
    three times the last-level cache); the best of three work-group counts.
    {name: {"bytes", "us", "GB_per_s", "workgroups"}}."""
    ctx = H.Context(0)
    pool = ctx.malloc(STREAM_POOL)
    pool.fill_normal(5, STREAM_POOL // 4)
    out = ctx.malloc(4 * max(STREAM_WORKGROUPS))
    pool.stream_read(1 << 20, 512, out)  # first launch of the kernel, untimed
    ctx.synchronize()
    res, off = {}, 0
    for name, nbytes in named_bytes.items():
        n = (nbytes + 4095) // 4096 * 4096
        best = None
        for wg in STREAM_WORKGROUPS:
            ctx.profile(True)
            ctx.profile_reset()
            for _ in range(reps):
                if off + n > STREAM_POOL:
                    off = 0
                pool.stream_read(n, wg, out, offset=off)
                off += n
            tot_ms, cnt = ctx.profile_read()["stream_read"]
            ctx.profile(False)
            us = 1000 * tot_ms / cnt
            if best is None or us < best[0]:
                best = (us, wg)
        res[name] = {"bytes": n, "us": round(best[0], 2), "GB_per_s": round(n / best[0] / 1e3, 1),
                     "workgroups": best[1]}
    pool.free()
    out.free()
    ctx.close()
    return res


def decode_eager(args):
    """Two eager passes over the resident layers (no graph): the run the
    per-dispatch counter passes profile.  --decode-workload picks one of the
    larger decode layers instead of the headline one."""
    ctx = H.Context(0)
    hid = HID
    if args.decode_workload:
        spec = {w[0]: w for w in DECODE_MORE}.get(args.decode_workload)
        if spec is None:
            raise SystemExit(f"unknown decode workload {args.decode_workload!r}: "
                             f"one of {[w[0] for w in DECODE_MORE]}")
        _, dt, hid, inter, ex, k, nl = spec
        layers = build_layers(ctx, nl, dtype=dt, hid=hid, inter=inter, experts=ex, topk=k)
    else:
        layers = build_layers(ctx, args.layers)
    xs = ctx.malloc(64 * hid * 4)
    xs.fill_normal(99, 64 * hid, 0.0, 1.0)
    out = ctx.malloc(hid * 4)
    L = len(layers)
    for s in range(2 * L):
        layers[s % L].forward_device(1, xs.offset((s % 64) * hid * 4), out.address)
    ctx.synchronize()
    for m in layers:
        m.close()
    ctx.close()
    return 2 * L


# token counts of the eager `band` leg (the headline layers on their default
# grouped row-chain path)
BAND_EAGER_T = (16, 48)


def eager_leg(name, passes=3):
    """One secondary workload launched eagerly (no graph), for kernel traces
    and counter runs: `kernels` (the reference's 4096 x 4096 matvec per
    dtype, rotated copies), `float` (the bf16 vocabulary projection and the
    dense f32 matrix), `expert` (the q8_0 Qwen3-30B expert, 128 copies in
    turn), `band` (the 48 headline layers in turn, two passes at 16 and at
    48 tokens per call: the grouped row-chain kernels) or `attention`
    (RMSNorm + attention decode).  Returns the number of calls."""
    ctx = H.Context(0)
    calls = 0
    if name in ("kernels", "float"):
        specs = ([(n, dt, KB_ROWS, KB_COLS, c) for n, dt, _, c in KBENCH] if name == "kernels"
                 else [(n, dt, r, c, k) for n, dt, r, c, k in FLOAT_MATVEC])
        for label, dt, rows, cols, copies in specs:
            nbytes = rows * H.row_bytes(dt, cols)
            vals = ctx.malloc(rows * cols * 4)
            if name == "kernels":
                vals.upload(kbench_values())
            else:
                vals.fill_normal(900, rows * cols, 0.0, 0.02)
            enc = ctx.malloc(nbytes)
            ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dt, rows, cols, H._vp(vals.address),
                                                      H._vp(enc.address)), "encode")
            vals.free()
            mats = []
            for _ in range(copies):
                h = H._vp()
                ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, dt, rows, cols, H._vp(enc.address),
                                                            nbytes, H.C.byref(h)), "upload")
                mats.append(H.WeightMatrix(ctx, h, rows, cols, dt))
            enc.free()
            x = ctx.malloc(cols * 4)
            x.upload(np.full(cols, 0.5, np.float32))
            out = ctx.malloc(rows * 4)
            for _ in range(passes):
                for m in mats:
                    ctx.check(H.lib().hale_matvec_device(ctx.handle, m.handle, H._vp(x.address),
                                                         H._vp(out.address)), "matvec")
                    calls += 1
            ctx.synchronize()
            for m in mats:
                m.close()
            x.free()
            out.free()
            log(f"eager {name}: {label} done")
    elif name == "expert":
        hid, inter, dt = 2048, 768, H.Q8_0
        vals = ctx.malloc(inter * hid * 4)
        enc = ctx.malloc(inter * H.row_bytes(dt, hid))
        experts = []
        for c in range(128):
            mats = []
            for j, (rows, cols) in enumerate(((inter, hid), (inter, hid), (hid, inter))):
                vals.fill_normal(31 + 3 * c + j, rows * cols, 0.0, 0.02)
                ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dt, rows, cols, H._vp(vals.address),
                                                          H._vp(enc.address)), "encode")
                h = H._vp()
                ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, dt, rows, cols, H._vp(enc.address),
                                                            rows * H.row_bytes(dt, cols), H.C.byref(h)), "upload")
                mats.append(H.WeightMatrix(ctx, h, rows, cols, dt))
            experts.append(H.Expert(*mats))
        vals.free()
        enc.free()
        xs = ctx.malloc(16 * hid * 4)
        xs.fill_normal(8, 16 * hid, 0.0, 1.0)
        out = ctx.malloc(hid * 4)
        for s in range(passes * 128):
            experts[s % 128].forward_device(xs.offset((s % 16) * hid * 4), out.address)
            calls += 1
        ctx.synchronize()
        for e in experts:
            for m in (e.gate, e.up, e.down):
                m.close()
    elif name == "band":
        layers = build_layers(ctx, 48)
        xs = ctx.malloc((max(BAND_EAGER_T) + 8) * HID * 4)
        xs.fill_normal(98, (max(BAND_EAGER_T) + 8) * HID, 0.0, 1.0)
        out = ctx.malloc(max(BAND_EAGER_T) * HID * 4)
        for T in BAND_EAGER_T:
            for s in range(2 * len(layers)):
                layers[s % len(layers)].forward_device(T, xs.offset((s % 8) * HID * 4), out.address)
                calls += 1
            ctx.synchronize()
            log(f"eager band: {T} tokens done")
        for m in layers:
            m.close()
        xs.free()
        out.free()
    elif name == "attention":
        ctx.close()
        for spec in ATTENTION:
            r = gpu_attention(*spec)
            calls += r.get("calls", 64)
        return calls
    else:
        raise SystemExit(f"unknown eager leg {name!r}: kernels, float, expert or attention")
    ctx.close()
    return calls


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_decode_q4_qwen3_30b.txt")
PREFILL_TRAFFIC = {
    "qwen3-30b-a3b prefill 512 tok q8_0": os.path.join(ROOT, "profiles", "traffic_prefill_q8_512.txt"),
    "qwen3-235b-a22b prefill 2048 tok q4_0": os.path.join(ROOT, "profiles", "traffic_prefill_q4_2048.txt"),
}


def measured_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch by kernel, from a committed counter summary
    (lines `traffic <kernel> <bytes>`), or {} when it is absent."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                p = line.split()
                if len(p) == 3 and p[0] == "traffic":
                    out[p[1]] = int(p[2])
    except OSError:
        pass
    return out


def gpu_decode_more(name, dtype, hid, inter, experts, topk, nlayers, reps=20, batch=0):
    """One-token MoE layer decode over nlayers resident layers visited in
    turn (cold weights), replayed from a graph; GB/s of routed expert bytes
    plus router bytes.  batch > 0: also `batch` tokens per step, on the
    default path and with each of the decode pass, the grouped row chains
    and the grouped matrix products forced (graph replay, us per step)."""
    ctx = H.Context(0)
    layers = build_layers(ctx, nlayers, seed=555, dtype=dtype, hid=hid, inter=inter,
                          experts=experts, topk=topk)
    nx = 16 + batch
    xs = ctx.malloc(nx * hid * 4)
    xs.fill_normal(7, nx * hid, 0.0, 1.0)
    out = ctx.malloc(max(batch, 1) * hid * 4)

    def step(s):
        layers[s % nlayers].forward_device(1, xs.offset((s % 16) * hid * 4), out.address)

    for s in range(2 * nlayers):
        step(s)
    ctx.synchronize()
    graph = ctx.capture(lambda: [step(s) for s in range(nlayers)])
    graph.launch()
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        graph.launch()
    ms = ctx.timer_stop()
    steps = reps * nlayers
    ctx.profile(True)
    ctx.profile_reset()
    for s in range(2 * nlayers):
        step(s)
    prof = ctx.profile_read()
    ctx.profile(False)
    graph.close()
    batched = None
    if batch:
        gmin0, bmax0 = layers[0].grouped_min_tokens, layers[0].band_max_tokens

        def time_t(gmin, bmax):
            for m in layers:
                m.set_grouped_min_tokens(gmin)
                m.set_band_max_tokens(bmax)

            def step_t(s):
                layers[s % nlayers].forward_device(batch, xs.offset((s % 16) * hid * 4), out.address)
            for s in range(nlayers):
                step_t(s)
            ctx.synchronize()
            g = ctx.capture(lambda: [step_t(s) for s in range(nlayers)])
            g.launch()
            ctx.synchronize()
            t = time_replays(ctx, g, 10)
            g.close()
            return round(1000 * float(np.median(t)) / nlayers, 2)

        path = "decode pass" if batch < gmin0 else ("row chains" if batch <= bmax0 else "matrix products")
        batched = {"tokens": batch, "path": path, "us_per_step": time_t(gmin0, bmax0),
                   "decode_pass_us": time_t(min(batch + 1, 257), bmax0),
                   "row_chains_us": time_t(2, 1 << 20), "matrix_products_us": time_t(2, 0)}
        log(f"{name} at {batch} tokens per step: {batched}")
    for m in layers:
        m.close()
    ctx.close()
    bytes_step = topk * expert_bytes(dtype, hid, inter) + experts * hid * 4
    us = 1000 * ms / steps
    r = {"workload": name, "bytes_per_step": bytes_step, "us_per_step": round(us, 2),
         "GB_per_s": round(bytes_step / us / 1e3, 1),
         "pct_hbm_peak": round(100 * bytes_step / us / 1e3 / HBM_PEAK_GBS, 2),
         "layers_resident": nlayers,
         "kernels": {k: {"avg_us": round(1000 * v[0] / v[1], 2), "launches": v[1]} for k, v in prof.items()}}
    if batched:
        r["batched"] = batched
    return r


def gpu_expert(copies=128, reps=20):
    """Expert::forward of one q8_0 Qwen3-30B-shaped expert (H 2048, I 768):
    `copies` distinct experts (5 MB each, 640 MB in all) visited in turn so
    the weights are cold, replayed from a graph; GB/s of expert bytes."""
    ctx = H.Context(0)
    hid, inter, dt = 2048, 768, H.Q8_0
    vals = ctx.malloc(inter * hid * 4)
    enc = ctx.malloc(inter * H.row_bytes(dt, hid))
    experts = []
    for c in range(copies):
        mats = []
        for j, (rows, cols) in enumerate(((inter, hid), (inter, hid), (hid, inter))):
            vals.fill_normal(31 + 3 * c + j, rows * cols, 0.0, 0.02)
            ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dt, rows, cols, H._vp(vals.address),
                                                      H._vp(enc.address)), "encode")
            h = H._vp()
            ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, dt, rows, cols, H._vp(enc.address),
                                                        rows * H.row_bytes(dt, cols), H.C.byref(h)), "upload")
            mats.append(H.WeightMatrix(ctx, h, rows, cols, dt))
        experts.append(H.Expert(*mats))
    vals.free()
    enc.free()
    xs = ctx.malloc(16 * hid * 4)
    xs.fill_normal(8, 16 * hid, 0.0, 1.0)
    out = ctx.malloc(hid * 4)

    def step(s):
        experts[s % copies].forward_device(xs.offset((s % 16) * hid * 4), out.address)

    for s in range(copies):
        step(s)
    ctx.synchronize()
    graph = ctx.capture(lambda: [step(s) for s in range(copies)])
    graph.launch()
    ctx.synchronize()
    times = time_replays(ctx, graph, reps)
    ctx.profile(True)
    ctx.profile_reset()
    for s in range(copies):
        step(s)
    prof = ctx.profile_read()
    ctx.profile(False)
    graph.close()
    for x in experts:
        for m in (x.gate, x.up, x.down):
            m.close()
    ctx.close()
    nbytes = expert_bytes(dt, hid, inter)
    us = 1000 * float(np.median(times)) / copies
    return {"workload": "Qwen3-30B-A3B expert forward q8_0 (H 2048, I 768), 1 token, "
                        f"{copies} distinct experts in turn (cold)",
            "bytes_per_step": nbytes, "us_per_step": round(us, 3),
            "GB_per_s": round(nbytes / us / 1e3, 1),
            "pct_hbm_peak": round(100 * nbytes / us / 1e3 / HBM_PEAK_GBS, 2),
            "timing": replay_stats(times, copies),
            "kernels": {k: {"avg_us": round(1000 * v[0] / v[1], 2), "launches": v[1]} for k, v in prof.items()}}


# (workload, dtype, rows, cols, distinct copies rotated so the weights stay cold)
FLOAT_MATVEC = [
    ("lm_head bf16 [151936 x 2048] (Qwen3 vocabulary)", H.BF16, 151936, 2048, 2),
    ("dense f32 [4096 x 4096]", H.F32, 4096, 4096, 8),
]


def gpu_float_matvec(name, dtype, rows, cols, copies, reps=20):
    """WeightMatrix::matvec over float weights, the 8-lane dot of the
    reference; GB/s of weight bytes, graph-replayed over `copies` distinct
    matrices visited in turn."""
    ctx = H.Context(0)
    nbytes = rows * H.row_bytes(dtype, cols)
    vals = ctx.malloc(rows * cols * 4)
    enc = ctx.malloc(nbytes)
    mats = []
    for c in range(copies):
        vals.fill_normal(900 + c, rows * cols, 0.0, 0.02)
        ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dtype, rows, cols, H._vp(vals.address),
                                                  H._vp(enc.address)), "encode")
        h = H._vp()
        ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, dtype, rows, cols, H._vp(enc.address),
                                                    nbytes, H.C.byref(h)), "upload")
        mats.append(H.WeightMatrix(ctx, h, rows, cols, dtype))
    enc.free()
    vals.free()
    x = ctx.malloc(cols * 4)
    x.fill_normal(5, cols, 0.0, 1.0)
    out = ctx.malloc(rows * 4)

    def step(s):
        ctx.check(H.lib().hale_matvec_device(ctx.handle, mats[s % copies].handle, H._vp(x.address),
                                             H._vp(out.address)), "matvec")

    for s in range(2 * copies):
        step(s)
    ctx.synchronize()
    graph = ctx.capture(lambda: [step(s) for s in range(copies)])
    graph.launch()
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        graph.launch()
    ms = ctx.timer_stop()
    ctx.profile(True)
    ctx.profile_reset()
    for s in range(2 * copies):
        step(s)
    prof = ctx.profile_read()
    ctx.profile(False)
    graph.close()
    for m in mats:
        m.close()
    ctx.close()
    us = 1000 * ms / (reps * copies)
    k = prof.get("gemv")
    kus = 1000 * k[0] / k[1] if k else None
    return {"workload": name, "bytes_per_call": nbytes, "us_per_call": round(us, 2),
            "GB_per_s": round(nbytes / us / 1e3, 1),
            "pct_hbm_peak": round(100 * nbytes / us / 1e3 / HBM_PEAK_GBS, 2),
            "kernel_avg_us": round(kus, 2) if kus else None,
            "kernel_GB_per_s": round(nbytes / kus / 1e3, 1) if kus else None}


# The reference's own kernel benchmark (`hale bench kernels`,
# src/cli/bench.rs:73-85 -> matvec_gflops, src/hardware/bench.rs:72-87): a
# 4096 x 4096 WeightMatrix::matvec for each of f32, bf16, f16, q8_0 and q4_0,
# values ((i % 97) - 48) / 97 in f32, x = 0.5, GFLOP/s = 2 rows cols / time
# and GB/s of weights = GFLOP/s / 2 x bits per weight / 8.
# (name, dtype, bits per weight, distinct copies rotated so the weights stay cold)
KBENCH = [("f32", H.F32, 32.0, 8), ("bf16", H.BF16, 16.0, 16), ("f16", H.F16, 16.0, 16),
          ("q8_0", H.Q8_0, 8.5, 32), ("q4_0", H.Q4_0, 4.5, 64)]
KB_ROWS = KB_COLS = 4096


def kbench_values():
    """The reference benchmark's matrix: ((i % 97) as f32 - 48.0) / 97.0."""
    i = np.arange(KB_ROWS * KB_COLS, dtype=np.int64)
    return ((i % 97).astype(np.float32) - np.float32(48.0)) / np.float32(97.0)


def gpu_kernel_bench(reps=20):
    """hale bench kernels on the GPU: per dtype, `copies` matrices holding
    the benchmark's values, visited in turn (cold weights), and one matrix
    called repeatedly as the reference's loop does (warm: the matrix stays
    in the GPU's caches).  Graph-replayed; the outputs are returned for the
    CPU leg to compare with the oracle's."""
    ctx = H.Context(0)
    vals = kbench_values()
    dv = ctx.malloc(vals.nbytes)
    dv.upload(vals)
    x = ctx.malloc(KB_COLS * 4)
    x.upload(np.full(KB_COLS, 0.5, np.float32))
    out = ctx.malloc(KB_ROWS * 4)
    res, outs = [], {}
    for name, dt, bits, copies in KBENCH:
        nbytes = KB_ROWS * H.row_bytes(dt, KB_COLS)
        enc = ctx.malloc(nbytes)
        ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dt, KB_ROWS, KB_COLS, H._vp(dv.address),
                                                  H._vp(enc.address)), "encode")
        mats = []
        for _ in range(copies):
            h = H._vp()
            ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, dt, KB_ROWS, KB_COLS,
                                                        H._vp(enc.address), nbytes, H.C.byref(h)), "upload")
            mats.append(H.WeightMatrix(ctx, h, KB_ROWS, KB_COLS, dt))
        enc.free()

        def call(m):
            ctx.check(H.lib().hale_matvec_device(ctx.handle, m.handle, H._vp(x.address),
                                                 H._vp(out.address)), "matvec")

        for m in mats:
            call(m)
        ctx.synchronize()
        outs[name] = out.download(np.float32, KB_ROWS)
        timed = {}
        for mode, seq in (("cold", mats), ("warm", [mats[0]] * copies)):
            g = ctx.capture(lambda: [call(m) for m in seq])
            g.launch()
            ctx.synchronize()
            t = time_replays(ctx, g, reps)
            g.close()
            timed[mode] = 1000 * float(np.median(t)) / copies
        for m in mats:
            m.close()
        flops = 2.0 * KB_ROWS * KB_COLS
        row = {"dtype": name, "bytes_per_call": nbytes, "copies": copies}
        for mode, us in timed.items():
            gflops = flops / us / 1e3
            row[mode] = {"us_per_call": round(us, 3), "GFLOP_per_s": round(gflops, 1),
                         "GB_per_s": round(gflops / 2 * bits / 8, 1),
                         "pct_hbm_peak": round(100 * gflops / 2 * bits / 8 / HBM_PEAK_GBS, 2)}
        res.append(row)
        log(f"matvec 4096x4096 {name:>5}: cold {row['cold']['GFLOP_per_s']} GFLOP/s "
            f"({row['cold']['GB_per_s']} GB/s), warm {row['warm']['GFLOP_per_s']} GFLOP/s")
    for b in (dv, x, out):
        b.free()
    ctx.close()
    return res, outs


def cpu_kernel_bench(gpu_outs, nthreads):
    """The same benchmark on the host through the oracle (the C restatement
    of WeightMatrix::matvec, row-parallel like the reference's rayon loop):
    a warm-up call, then 20 timed calls, as matvec_gflops does, on all
    threads and on one.  Also checks the GPU's outputs against the oracle's,
    bit for bit."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    vals = kbench_values().reshape(KB_ROWS, KB_COLS)
    xv = np.full(KB_COLS, 0.5, np.float32)
    res = {}
    for name, dt, bits, _ in KBENCH:
        data = O.encode_matrix(dt, vals)
        ref = O.matvec(dt, KB_ROWS, KB_COLS, data, xv, nthreads=nthreads)
        got = gpu_outs.get(name)
        row = {"bit_exact_gpu_vs_oracle": None if got is None else bool(
            (got.view(np.uint32) == ref.view(np.uint32)).all())}
        for nt in (nthreads, 1):
            O.matvec(dt, KB_ROWS, KB_COLS, data, xv, nthreads=nt)  # warm-up
            t0 = time.perf_counter()
            for _ in range(20):
                O.matvec(dt, KB_ROWS, KB_COLS, data, xv, nthreads=nt)
            sec = (time.perf_counter() - t0) / 20
            gflops = 2.0 * KB_ROWS * KB_COLS / sec / 1e9
            row[f"{nt}_threads"] = {"GFLOP_per_s": round(gflops, 2),
                                    "GB_per_s": round(gflops / 2 * bits / 8, 2),
                                    "us_per_call": round(1e6 * sec, 1)}
        res[name] = row
        log(f"cpu matvec 4096x4096 {name:>5}: {row[f'{nthreads}_threads']['GFLOP_per_s']} GFLOP/s "
            f"({nthreads} threads), {row['1_threads']['GFLOP_per_s']} (1); "
            f"GPU bit-exact: {row['bit_exact_gpu_vs_oracle']}")
    return res


def strict_dropin(layers, xs, ntok=96):
    """MoeLayer::forward through the provider surface left as the reference
    has it (src/model/moe.rs:56-70, src/expert/mod.rs:91-103): per token
    MoeLayer::route (hale_moe_route), ExpertProvider::fetch (hale_moe_fetch),
    then per route Expert::forward (hale_expert_forward, host slices in and
    out, synchronous) and the combine out = out + w * y on the host in route
    order.  Wall-clock per token over the resident layers in turn (cold), with
    the time of each part, and whether the outputs equal the fused layer
    forward's bit for bit."""
    lib = H.lib()
    L = len(layers)
    m0 = layers[0]
    k, hid = m0.top_k, m0.hidden
    idx = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    g, u, d = ((H._vp * k)() for _ in range(3))
    tmp = np.zeros((k, hid), np.float32)
    out = np.zeros(hid, np.float32)
    ptr = lambda a, t: a.ctypes.data_as(t)  # noqa: E731
    fp, u32p = H.C.POINTER(H.C.c_float), H.C.POINTER(H.C.c_uint32)
    parts = {"route": 0.0, "fetch": 0.0, "expert_forward": 0.0, "combine": 0.0}
    per_tok, exact = [], True
    for s in range(ntok + L):
        m = layers[s % L]
        x = xs[s % xs.shape[0]]
        t0 = time.perf_counter()
        m.ctx.check(lib.hale_moe_route(m.handle, ptr(x, fp), ptr(idx, u32p), ptr(w, fp)), "route")
        t1 = time.perf_counter()
        m.ctx.check(lib.hale_moe_fetch(m.handle, ptr(idx, u32p), k, g, u, d), "fetch")
        t2 = time.perf_counter()
        for r in range(k):
            m.ctx.check(lib.hale_expert_forward(m.ctx.handle, g[r], u[r], d[r], ptr(x, fp),
                                                ptr(tmp[r], fp)), "Expert::forward")
        t3 = time.perf_counter()
        out[:] = 0.0
        for r in range(k):
            out[:] = out + w[r] * tmp[r]  # f32: the product rounded, then the sum
        t4 = time.perf_counter()
        if s < L:
            continue  # first visit of each layer: untimed
        per_tok.append(t4 - t0)
        for key, dt_ in zip(parts, (t1 - t0, t2 - t1, t3 - t2, t4 - t3)):
            parts[key] += dt_
        if s < L + 8:
            fused = m.forward(x)
            exact = exact and bool((fused.view(np.uint32) == out.view(np.uint32)).all())
    n = len(per_tok)
    us = 1e6 * float(np.median(per_tok))
    return {"workload": "the decode workload's layers through route, fetch, k x Expert::forward "
                        "and a host combine (the reference's provider surface unchanged)",
            "tokens": n, "us_per_token": round(us, 1), "tokens_per_s": round(1e6 / us, 1),
            "parts_us_per_token": {k2: round(1e6 * v / n, 1) for k2, v in parts.items()},
            "same_bits_as_fused_forward": exact,
            "note": "wall clock including the Python ctypes calls; each Expert::forward copies x in "
                    "and its output out and synchronizes, as the infallible host-slice API requires"}


# (workload, projection dtype, hidden, heads, kv heads, head dim, QK-norm, cached positions)
ATTENTION = [
    ("qwen3-30b-a3b attention decode bf16, 4096 cached positions", H.BF16, 2048, 32, 4, 128, True, 4096),
]


def gpu_attention(name, dtype, hid, nh, nkv, hd, qk, positions, timed=64):
    """Attention::forward for one token after `positions - timed` cached
    positions, timed over the last `timed` positions (each appends its k/v),
    plus the RMSNorm before it.  Bytes per call: the four projections plus the
    keys and values read."""
    ctx = H.Context(0)
    shapes = ((nh * hd, hid), (nkv * hd, hid), (nkv * hd, hid), (hid, nh * hd))
    vals = ctx.malloc(max(r * c for r, c in shapes) * 4)
    enc = ctx.malloc(max(r * H.row_bytes(dtype, c) for r, c in shapes))
    mats = []
    for j, (r, c) in enumerate(shapes):
        vals.fill_normal(700 + j, r * c, 0.0, 0.02)
        ctx.check(H.lib().hale_encode_rows_device(ctx.handle, dtype, r, c, H._vp(vals.address),
                                                  H._vp(enc.address)), "encode")
        h = H._vp()
        ctx.check(H.lib().hale_matrix_upload_device(ctx.handle, dtype, r, c, H._vp(enc.address),
                                                    r * H.row_bytes(dtype, c), H.C.byref(h)), "upload")
        mats.append(H.WeightMatrix(ctx, h, r, c, dtype))
    enc.free()
    vals.free()
    norm_w = np.ones(hd, np.float32) if qk else None
    att = H.Attention(ctx, *mats, norm_w, norm_w, nh, nkv, hd, 1e-6, max_len=positions)
    x = ctx.malloc(hid * 4)
    x.fill_normal(3, hid, 0.0, 1.0)
    w = ctx.malloc(hid * 4)
    w.fill_normal(4, hid, 1.0, 0.1)
    xn = ctx.malloc(hid * 4)
    out = ctx.malloc(hid * 4)
    cs = ctx.malloc(hd * 4)
    cs.fill_normal(5, hd, 0.0, 0.5)

    def call(pos):
        ctx.check(H.lib().hale_rms_norm_device(ctx.handle, H._vp(x.address), None, H._vp(w.address), 1,
                                               hid, np.float32(1e-6), H._vp(xn.address)), "rms_norm")
        ctx.check(H.lib().hale_attention_forward_device(att.handle, H._vp(xn.address), pos,
                                                        H._vp(cs.address), H._vp(cs.address + hd * 2),
                                                        H._vp(out.address)), "attention")

    for pos in range(positions - timed):
        call(pos)
    ctx.synchronize()
    ctx.profile(True)
    ctx.profile_reset()
    ctx.timer_start()
    for pos in range(positions - timed, positions):
        call(pos)
    ms = ctx.timer_stop()
    prof = ctx.profile_read()
    ctx.profile(False)
    att.close()
    for m in mats:
        m.close()
    for b in (x, w, xn, out, cs):
        b.free()
    ctx.close()
    wbytes = sum(r * H.row_bytes(dtype, c) for r, c in shapes)
    kv = 2 * (positions - timed // 2) * nkv * hd * 4
    us = 1000 * ms / timed
    return {"workload": name, "us_per_token": round(us, 2), "weight_bytes": wbytes,
            "kv_bytes": kv, "GB_per_s": round((wbytes + kv) / us / 1e3, 1),
            "kernels": {k: {"avg_us": round(1000 * v[0] / v[1], 2), "launches": v[1]} for k, v in prof.items()}}


def time_replays(ctx, graph, reps):
    """Times `reps` graph replays one by one (HIP events on the library's
    stream around each launch); returns the per-replay times in ms."""
    out = []
    for _ in range(reps):
        ctx.timer_start()
        graph.launch()
        out.append(ctx.timer_stop())
    return out


def replay_stats(times_ms, steps_per_replay):
    t = np.asarray(times_ms)
    return {"replays": int(t.size), "steps_per_replay": steps_per_replay,
            "us_per_step_median": round(1000 * float(np.median(t)) / steps_per_replay, 3),
            "us_per_step_min": round(1000 * float(t.min()) / steps_per_replay, 3),
            "us_per_step_max": round(1000 * float(t.max()) / steps_per_replay, 3)}


def gpu_decode(args):
    ctx = H.Context(0)
    t0 = time.time()
    layers = build_layers(ctx, args.layers)
    log(f"{args.layers} layers resident ({args.layers * (E * expert_bytes(DTYPE, HID, INTER) + E * HID * 4) / 1e9:.1f} GB) in {time.time() - t0:.1f}s")
    nx = 64
    xs = ctx.malloc(nx * HID * 4)
    xs.fill_normal(99, nx * HID, 0.0, 1.0)
    out = ctx.malloc(8 * HID * 4)
    L = len(layers)

    def step(s):
        layers[s % L].forward_device(1, xs.offset((s % nx) * HID * 4), out.address)

    for m in layers:  # size each layer's scratch without running a step
        m.reserve(1)
    warm = args.warmup
    for s in range(warm):   # the eager warm-up steps
        step(s)
    ctx.synchronize()
    # The timed region is exactly `steps` steps (layers s % L for s = warm ..
    # warm + steps - 1): replays of a graph of one pass over all layers, then
    # a graph of the remaining steps.  Graphs are uploaded when captured, so
    # no first-launch work falls inside the region.
    steps = args.steps
    s0 = warm % L
    graph = ctx.capture(lambda: [step(s0 + s) for s in range(L)])
    full, rest = divmod(steps, L)
    tail = ctx.capture(lambda: [step(s0 + s) for s in range(rest)]) if rest else None
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(full):
        graph.launch()
    if tail is not None:
        tail.launch()
    ms = ctx.timer_stop()
    log(f"timed {steps} steps ({full} passes over {L} layers + {rest}): "
        f"{1000 * ms / steps:.2f} us/step")
    # per-pass spread, after the timed region: one pass timed at a time
    times = time_replays(ctx, graph, 20)
    if tail is not None:
        tail.close()

    # per-kernel durations: eager pass with events around every launch
    ctx.profile(True)
    ctx.profile_reset()
    for s in range(2 * L):
        step(s)
    prof = ctx.profile_read()
    ctx.profile(False)
    graph.close()

    # a few tokens per step (the decode path up to 7 tokens: one gate/up and
    # one down launch for all of them), same layers, graph-replayed
    few = []
    if not args.no_prefill:
        for T in (2, 4, 7):
            def step_t(s, T=T):
                layers[s % L].forward_device(T, xs.offset((s % (nx - 8)) * HID * 4), out.address)
            for s in range(L):
                step_t(s)
            ctx.synchronize()
            g = ctx.capture(lambda: [step_t(s) for s in range(L)])
            g.launch()
            ctx.synchronize()
            t = time_replays(ctx, g, 20)
            g.close()
            us = 1000 * float(np.median(t)) / L
            few.append({"tokens": T, "us_per_step": round(us, 2), "us_per_token": round(us / T, 2),
                        "tokens_per_s": round(1e6 * T / us, 1), "timing": replay_stats(t, L)})
            log(f"decode {T} tokens per step: {us:.2f} us/step ({us / T:.2f} us/token)")
    # 8 to 64 tokens per step: the default path (the decode pass below the
    # layer's grouped threshold, from it the grouped row-chain kernels up to
    # the band threshold, the grouped matrix products above) and, from 16
    # tokens, each path forced
    band = []
    if not args.no_prefill:
        band_t = (8, 12, 16, 24, 32, 48, 64)
        xb = ctx.malloc((max(band_t) + 8) * HID * 4)  # step inputs start up to 7 rows in
        xb.fill_normal(98, (max(band_t) + 8) * HID, 0.0, 1.0)
        ob = ctx.malloc(max(band_t) * HID * 4)
        gmin0 = layers[0].grouped_min_tokens
        bmax0 = layers[0].band_max_tokens

        def time_band(T):
            def step_b(s):
                layers[s % L].forward_device(T, xb.offset((s % 8) * HID * 4), ob.address)
            for s in range(L):  # sizes each layer's scratch for T tokens
                step_b(s)
            ctx.synchronize()
            g = ctx.capture(lambda: [step_b(s) for s in range(L)])
            g.launch()
            ctx.synchronize()
            t = time_replays(ctx, g, 10)
            g.close()
            return round(1000 * float(np.median(t)) / L, 2)

        def forced(gmin, bmax):
            for m in layers:
                m.set_grouped_min_tokens(gmin)
                m.set_band_max_tokens(bmax)

        for T in band_t:
            path = "decode pass" if T < gmin0 else ("row chains" if T <= bmax0 else "matrix products")
            row = {"tokens": T, "path": path, "us_per_step": time_band(T)}
            if T >= 16:
                forced(T + 1, bmax0)
                row["decode_pass_us"] = time_band(T)
                forced(2, 1 << 20)
                row["row_chains_us"] = time_band(T)
                forced(2, 0)
                row["matrix_products_us"] = time_band(T)
                forced(gmin0, bmax0)
            band.append(row)
            log(f"band {T} tokens: {row}")
        xb.free()
        ob.free()
    dropin = None
    if not args.no_prefill:
        xs_host = np.random.default_rng(99).standard_normal((64, HID), dtype=np.float32)
        dropin = strict_dropin(layers, xs_host)
        log(f"strict drop-in (route, fetch, k x Expert::forward, host combine): "
            f"{dropin['us_per_token']} us/token")
    for m in layers:
        m.close()
    ctx.close()
    return steps, ms, prof, warm, replay_stats(times, L), few, dropin, band


def cpu_info():
    """The host CPU as lscpu reports it (model name, sockets, physical cores
    per socket, threads per core) and the CPUs this process may run on."""
    import subprocess

    info = {"model": cpu_model()}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, check=True).stdout
        kv = {a.strip(): b.strip() for a, b in (ln.split(":", 1) for ln in txt.splitlines() if ":" in ln)}
        info["model"] = kv.get("Model name", info["model"])
        sockets = int(kv.get("Socket(s)", "0") or 0)
        cps = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets
        info["physical_cores"] = sockets * cps if sockets and cps else None
        info["threads_per_core"] = int(kv.get("Thread(s) per core", "0") or 0) or None
        info["logical_cpus"] = int(kv.get("CPU(s)", "0") or 0) or None
    except (OSError, subprocess.CalledProcessError, ValueError):
        pass
    try:
        info["cpus_available_to_process"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    return info


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s):
    """The oracle (the C restatement of the reference's CPU algorithm) on one
    layer of the decode workload's shape, one token per iteration: built at
    -march=x86-64 (what a default cargo build targets) and at -march=native
    (compiled here for this host), each on all host threads and on one.  At
    least 20 timed iterations per variant after a warm-up; medians."""
    import shutil
    import subprocess
    import tempfile

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    nall = os.cpu_count() or 1
    L = O.OracleMoe.synthetic(O.Q4_0, HID, INTER, E, TOPK, normalize_topk=True, seed=77,
                              nthreads=nall)
    xs = O.normal(5, 16 * HID).reshape(16, HID)
    variants = [("x86-64", "")]
    tmp = tempfile.mkdtemp(prefix="hale_oracle_native_")
    try:
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "native",
                        f"NATIVE_OUT={tmp}"], check=True, capture_output=True)
        variants.append(("native", os.path.join(tmp, "libhale_oracle_native.so")))
    except (subprocess.CalledProcessError, OSError) as e:
        log(f"cpu baseline: -march=native build failed ({e}); reporting x86-64 only")
    res = {}
    for name, variant in variants:
        for nt in (nall, 1):
            L.forward(xs[0], nthreads=nt, variant=variant)
            times, t0 = [], time.perf_counter()
            while len(times) < 20 or time.perf_counter() - t0 < budget_s:
                a = time.perf_counter()
                L.forward(xs[len(times) % 16], nthreads=nt, variant=variant)
                times.append(time.perf_counter() - a)
            med = float(np.median(times))
            res[(name, nt)] = (med, len(times))
            log(f"cpu {name} {nt} threads: {1e3 * med:.2f} ms/token over {len(times)} tokens")
    shutil.rmtree(tmp, ignore_errors=True)
    return nall, res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=960)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="minimum timed seconds per CPU-baseline variant (4 variants)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill workloads (for counter runs)")
    ap.add_argument("--decode-eager", action="store_true",
                    help="only two eager decode passes over the layers (for counter runs)")
    ap.add_argument("--decode-workload", default="", metavar="NAME",
                    help="with --decode-eager: one of the larger decode layers")
    ap.add_argument("--eager-leg", default="", metavar="NAME",
                    help="only one secondary workload, launched eagerly (for counter and trace runs): "
                         "kernels, float, expert, band or attention")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only time the plain copy kernel over BYTES (counter yardstick)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        print(json.dumps(copy_calibration(args.copy_calibration)), flush=True)
        return
    if args.decode_eager:
        print(json.dumps({"decode_eager_steps": decode_eager(args)}), flush=True)
        return
    if args.eager_leg:
        print(json.dumps({"eager_leg": args.eager_leg, "calls": eager_leg(args.eager_leg)}), flush=True)
        return
    if args.prefill_only:
        res = [gpu_prefill(name, dt, hid, inter, ex, k, tok, reps=3, bound=bound, router=False)
               for (name, dt, hid, inter, ex, k, tok, bound) in PREFILL]
        print(json.dumps({"prefill": res}), flush=True)
        return

    bytes_step = TOPK * expert_bytes(DTYPE, HID, INTER) + E * HID * 4
    steps, ms, prof, warm, rstats, few, dropin, band = gpu_decode(args)
    sec = ms / 1000.0
    gbs = bytes_step * steps / sec / 1e9

    kernels = {k: {"avg_us": round(1000 * v[0] / v[1], 3), "launches": v[1]} for k, v in prof.items()}
    dom = max(prof, key=lambda k: prof[k][0])
    dom_avg_s = prof[dom][0] / prof[dom][1] / 1000.0
    launch_bytes = {
        "gate_up": TOPK * 2 * INTER * H.row_bytes(DTYPE, HID),
        "down": TOPK * HID * H.row_bytes(DTYPE, INTER),
        "route": E * HID * 4,
    }
    achieved = launch_bytes.get(dom, 0) / dom_avg_s / 1e9 if dom in launch_bytes else None
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1) if achieved else None,
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
                "traffic": measured_traffic().get(dom), "bytes_per_launch": launch_bytes.get(dom)}

    expert = None
    if not args.no_prefill:
        expert = gpu_expert()
        log(f"expert q8_0 2048x768: {expert['us_per_step']} us, {expert['GB_per_s']} GB/s")

    more = []
    if not args.no_prefill:
        for (name, dt, hid, inter, ex, k, nl) in DECODE_MORE:
            more.append(gpu_decode_more(name, dt, hid, inter, ex, k, nl, batch=MORE_BATCH.get(name, 0)))
            log(f"decode {name}: {more[-1]['us_per_step']} us/step, {more[-1]['GB_per_s']} GB/s")

    fmv = []
    if not args.no_prefill:
        for (name, dt, rows, cols, copies) in FLOAT_MATVEC:
            fmv.append(gpu_float_matvec(name, dt, rows, cols, copies))
            log(f"matvec {name}: {fmv[-1]['us_per_call']} us, {fmv[-1]['GB_per_s']} GB/s")

    kb, kb_outs = [], {}
    if not args.no_prefill:
        kb, kb_outs = gpu_kernel_bench()

    attn = []
    if not args.no_prefill:
        for (name, dt, hid, nh, nkv, hd, qk, npos) in ATTENTION:
            attn.append(gpu_attention(name, dt, hid, nh, nkv, hd, qk, npos))
            log(f"attention {name}: {attn[-1]['us_per_token']} us/token, {attn[-1]['GB_per_s']} GB/s")

    ceiling = None
    if not args.no_prefill:
        # each decode kernel beside a plain read of its bytes in one launch
        sizes, kernel_us = {}, {}
        for (name, dt, hid, inter, ex, k, nl), r in [(("qwen3-30b-a3b decode q4_0", DTYPE, HID, INTER, E,
                                                        TOPK, args.layers), {"kernels": kernels})] + \
                [(spec, m) for spec, m in zip(DECODE_MORE, more)]:
            short = name.split(" decode")[0]
            per = {"route": ex * hid * 4, "gate_up": k * 2 * inter * H.row_bytes(dt, hid),
                   "down": k * hid * H.row_bytes(dt, inter)}
            for kern, nbytes in per.items():
                if kern in r["kernels"]:
                    sizes[f"{short} {kern}"] = nbytes
                    kernel_us[f"{short} {kern}"] = r["kernels"][kern]["avg_us"]
        ceiling = stream_ceiling(sizes)
        for key, c in ceiling.items():
            c["kernel_us"] = kernel_us[key]
            c["kernel_over_ceiling"] = round(kernel_us[key] / c["us"], 3)
            log(f"{key}: {kernel_us[key]} us vs one-launch read of {c['bytes'] / 1e6:.1f} MB "
                f"{c['us']} us ({c['GB_per_s']} GB/s)")

    prefill = []
    if not args.no_prefill:
        for (name, dt, hid, inter, ex, k, tok, bound) in PREFILL:
            prefill.append(gpu_prefill(name, dt, hid, inter, ex, k, tok, reps=20, bound=bound))
            f = prefill[-1]["fma_down_fold"]
            log(f"prefill {name}: {prefill[-1]['ms']} ms, {prefill[-1]['tokens_per_s']} tok/s, "
                f"{prefill[-1]['pct_int8_mfma_peak']}% int8 MFMA; FMA down fold {f['ms']} ms "
                f"(rel-L2 {f['rel_l2_vs_exact']:.1e}); with the router {prefill[-1]['with_router']['ms']} ms")

    cpu = None
    if not args.no_cpu:
        nall, res = cpu_baseline(args.cpu_seconds)
        kb_cpu = cpu_kernel_bench(kb_outs, nall) if kb else None
        host = cpu_info()
        med, n = res[("x86-64", nall)]
        cpu = {"value": round(bytes_step / med / 1e9, 3), "unit": "GB/s", "cores": nall,
               "kind": "port",
               "sample": f"oracle MoeLayer::forward (q4_0, 128 experts, top-8, H 2048, I 768; one "
                         f"340 MB layer, one token per iteration), median of {n} tokens, built "
                         f"-O3 -march=x86-64, {nall} threads on {host['model']}",
               "tokens_per_s": round(1.0 / med, 1),
               "cpu_model": host["model"],
               "host": host,
               "threads_used": nall,
               "reference_kernel_bench": kb_cpu,
               "variants": {f"{name} {nt} thread{'s' if nt > 1 else ''}":
                            {"GB_per_s": round(bytes_step / m / 1e9, 3), "ms_per_token": round(1e3 * m, 3),
                             "tokens": c}
                            for (name, nt), (m, c) in res.items()}}

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi8->i32, f32 scales",
        "data": "synthetic: seeded N(0,0.02) weights quantized on the GPU, N(0,1) inputs",
        "config": {"workload": "Qwen3-30B-A3B MoE layer decode, batch 1: 128 q4_0 experts "
                               "(H 2048, I 768), f32 router, top-8 renormalised; 48 resident "
                               "layers visited in turn (cold weights)",
                   "global_batch": 1, "bytes_per_step": bytes_step, "layers_resident": args.layers,
                   "parallelism": "single GPU"},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "moe_layer_tokens_per_s": round(steps / sec, 1),
        "roofline": roofline,
        "timing": rstats,
        "kernels": kernels,
        "expert": expert,
        "decode_few_tokens": few,
        "decode_band": band,
        "decode_more": more,
        "stream_read_ceiling": ceiling,
        "float_matvec": fmv,
        "reference_kernel_bench": {"workload": "hale bench kernels: WeightMatrix::matvec 4096 x 4096, "
                                               "values ((i % 97) - 48) / 97, x = 0.5",
                                   "gpu": kb},
        "strict_dropin": dropin,
        "attention": attn,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
