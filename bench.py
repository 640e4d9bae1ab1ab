#!/usr/bin/env python3
"""bench.py -- Q4_0 decode matvec throughput on one MI355X.

Workload ("config 2"): the SmolLM2-135M Llama
shape's Q4_0 matvec set at batch 1 -- per token 30 layers of merged qkv
[960, 576], o [576, 576], merged gate_up [3072, 576], down [576, 1536], plus
the tied head [49152, 576]: 121 products, 75,644,928 weight bytes. Weights
~N(0, 0.02) quantised to Q4_0 (host quantiser), activations ~N(0, 1), all
resident in HBM before timing. One step = one token's 121 products as ONE
launch (tmh_plan_run). Steps rotate through enough distinct copies of the
weights (>= 512 MB) that the 256 MB Infinity Cache cannot serve them.

value = algorithmic bytes per step (weights + f32 x + f32 y) / wall time
per step, in GB/s. The roofline object prices the launch against 8 TB/s
from the median per-launch time over at least 100 groups of 20 back-to-back
launches (HIP events between groups on the library's stream). The CPU baseline times the oracle's
restatement of tensomite's CPU path (Quant.matmul on every host core, in its
portable and native builds) on the same bytes, and checks the GPU's output
bits against it.

Beside it, in the same line:
  config1      BASELINE configs[0], the Q8_0 GPT-2 c_attn matvec (2304 x 768):
               one product a launch, and 128 products (distinct weight
               copies) a launch; >= 1024 copies rotated; its CPU baseline.
  decode_1p7b  config 5: greedy decode of a SmolLM2-1.7B-shaped Llama with
               W ~ N(0, 0.02) quantised to Q4_0, after a 128-token prompt, at
               batch 1 and 8 through the device-resident decoder (every op on
               the GPU with the host's bits); the CPU oracle's time per token
               after the same prompt, and its tokens against the GPU's.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-decode]
  config3      config 3: Q4_1 batched-decode products, both shapes, B = 1..16,
               each point with its roofline and CPU baseline.
  config4      config 4: the Q8_0 prefill GEMM, N = 2048 and 8192, ordered
               (AUTO) and UNORDERED, each with its MFMA roofline; CPU baseline.
  host_memory  the host's STREAM-style copy rate (numpy, every core), beside
               the CPU baselines.

    python bench.py --batched     # config 3 alone, its own line
    python bench.py --gemm        # config 4 alone, its own line
    python bench.py --decode-only # config 5, its own line
    python bench.py --write-gguf DIR   # the configs' weights as GGUF files
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "tensomite.cr_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20
ROOFLINE_GROUPS = 100  # per-launch figures: the median over this many groups of launches
GROUP = 20             # launches a group

# config 2: (name, n, k) per layer, then the head
LAYER = [("qkv", 960, 576), ("o", 576, 576), ("gate_up", 3072, 576), ("down", 576, 1536)]
LAYERS = 30
HEAD = ("head", 49152, 576)

# config 1: GPT-2-small c_attn
C_ATTN = (2304, 768)


def products_135m():
    out = []
    for layer in range(LAYERS):
        for name, n, k in LAYER:
            out.append((f"{name}.{layer}", n, k))
    out.append(HEAD)
    return out


def q4_0_bytes(n, k):
    return n * (k // 32) * 18


def q8_0_bytes(n, k):
    return n * (k // 32) * 34


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """The host's core count (the threads the CPU baselines use), model and
    NUMA nodes."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    model = "?"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        numa = len([d for d in os.listdir("/sys/devices/system/node") if d.startswith("node")])
    except OSError:
        numa = None
    return {"cores": cores, "nproc": os.cpu_count(), "model": model, "numa_nodes": numa}


def traffic_from_profiles(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by a copy kernel's reading), if the committed summary has them."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def time_launches(dev, launch, count, group=1):
    """Runs launch(i) for i < count, back to back on the library's stream,
    with a HIP event after every `group` launches: the mean launch time of
    each group in ms, and the wall time of the whole (host clock, from the
    first enqueue to the end of the GPU's work). An event between every two
    launches costs ~2.5 us of its own on MI355X (config 2: 18.0 us a launch
    against 15.5 back to back), so groups of 20 keep that under 1%."""
    groups = count // group
    events = [dev.event() for _ in range(groups + 1)]
    t0 = time.perf_counter()
    dev.record(events[0])
    for g in range(groups):
        for j in range(group):
            launch(g * group + j)
        dev.record(events[g + 1])
    dev.sync()
    wall = time.perf_counter() - t0
    per = [dev.elapsed_ms(events[g], events[g + 1]) / group for g in range(groups)]
    for ev in events:
        dev.destroy_event(ev)
    return per, wall


def warm_up(dev, launch, count, seconds=0.05):
    """`count` launches, continued until the GPU has been kept busy for
    `seconds`: after the host-side set-up the GPU's clocks need that long to
    settle (20 launches of config 2 left the mean ~1 us high)."""
    done = 0
    t0 = time.perf_counter()
    while done < count or time.perf_counter() - t0 < seconds:
        for _ in range(100 if done >= count else 1):
            launch(done)
            done += 1
        if done >= count:
            dev.sync()
    dev.sync()
    return done


def launch_stats(per_ms, algorithmic_bytes, group=1):
    med = statistics.median(per_ms)
    mean = sum(per_ms) / len(per_ms)
    return {"launches": len(per_ms) * group, "groups": len(per_ms), "launches_per_group": group,
            "median_us": round(med * 1e3, 3), "mean_us": round(mean * 1e3, 3),
            "min_us": round(min(per_ms) * 1e3, 3), "max_us": round(max(per_ms) * 1e3, 3),
            "GB_per_s_median": round(algorithmic_bytes / (med * 1e-3) / 1e9, 1)}


# ---------------------------------------------------------------- CPU baselines

def cpu_products(kind, weights, xs, shapes, gpu_out, seconds, variant, cores):
    """The oracle's Quant.matmul restatement over a set of one-row products
    (`variant` build, `cores` threads), timed over whole sets for about
    `seconds`; with gpu_out, also counts the products whose GPU bits differ."""
    from oracle import oracle

    oracle.set_threads(cores, variant)
    mismatched = None
    if gpu_out is not None:
        mismatched = 0
        for i, (n, k) in enumerate(shapes):
            want = oracle.matmul(kind, xs[i], weights[i], 1, n, k, variant)[0]
            if not np.array_equal(want.view(np.uint32), gpu_out[i].view(np.uint32)):
                mismatched += 1
    sets, start = 0, time.perf_counter()
    while True:
        for i, (n, k) in enumerate(shapes):
            oracle.matmul(kind, xs[i], weights[i], 1, n, k, variant)
        sets += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds:
            break
    return sets, elapsed, mismatched


def cpu_baseline_config2(weights, xs, prods, gpu_out, seconds):
    """Config 2 on the host: the portable build and the widest native build
    the CPU runs (the reference's --mcpu=native analogue), every core each;
    `value` is the faster."""
    from oracle import oracle

    host = host_cpu()
    algorithmic = sum(q4_0_bytes(n, k) + 4 * k + 4 * n for _, n, k in prods)
    shapes = [(n, k) for _, n, k in prods]
    builds = {}
    for variant in dict.fromkeys(["portable", oracle.best_variant()]):
        sets, elapsed, mismatched = cpu_products("Q4_0", weights, xs, shapes, gpu_out, seconds, variant,
                                                 host["cores"])
        builds[variant] = {"GB_per_s": round(algorithmic * sets / elapsed / 1e9, 2),
                           "ms_per_token": round(elapsed / sets * 1e3, 3), "tokens": sets,
                           "seconds": round(elapsed, 2), "parity_mismatched_products": mismatched}
    best = max(builds, key=lambda v: builds[v]["GB_per_s"])
    return {
        "value": builds[best]["GB_per_s"],
        "unit": "GB/s",
        "cores": host["cores"],
        "kind": "port",
        "sample": f"whole tokens of the config-2 set (121 one-row products each) for ~{seconds:.0f} s per build; "
                  f"the oracle's Quant.matmul restatement with the reference's span rule and spin pool, "
                  f"{host['cores']} threads; value from the {best} build",
        "ms_per_token": builds[best]["ms_per_token"],
        "builds": builds,
        "host": host,
        "parity_mismatched_products": builds[best]["parity_mismatched_products"],
    }


# ---------------------------------------------------------------- config 2

def build_config2(dev, copies):
    """Config 2's inputs on the device: the 121 products' Q4_0 weights (W ~
    N(0, 0.02) quantised, seed 0x5EED0002 + i) packed into one buffer per
    copy at 256-byte offsets, x ~ N(0, 1) per product, outputs, and one plan
    per copy (the launch bench.py times)."""
    import quant_host

    prods = products_135m()
    rng = np.random.default_rng(0x5EED0002)
    weights, xs = [], []
    for i, (name, n, k) in enumerate(prods):
        weights.append(quant_host.synthetic_weights("Q4_0", n, k, seed=0x5EED0002 + i))
        xs.append(rng.standard_normal(k, dtype=np.float32))
    offsets, off = [], 0
    for w in weights:
        offsets.append(off)
        off += (w.nbytes + 255) // 256 * 256
    packed = np.zeros(off, np.uint8)
    for w, o in zip(weights, offsets):
        packed[o:o + w.nbytes] = w
    # One upload, then device-to-device copies (a copy kernel of known size,
    # which also calibrates the HBM byte counters of a profile run).
    wbufs = [dev.from_array(packed, asynchronous=True)]
    for _ in range(copies - 1):
        buf = dev.alloc(packed.nbytes)
        dev.copy(buf, wbufs[0], packed.nbytes)
        wbufs.append(buf)
    xbufs = [dev.from_array(x) for x in xs]
    ybufs = [dev.alloc(4 * n) for _, n, _ in prods]
    plans = []
    for c in range(copies):
        items = [(_View(wbufs[c], offsets[i]), 0, xbufs[i], ybufs[i], None, n, k)
                 for i, (name, n, k) in enumerate(prods)]
        plans.append(dev.plan("Q4_0", items))
    dev.sync()
    return {"prods": prods, "weights": weights, "xs": xs, "offsets": offsets, "wbufs": wbufs, "xbufs": xbufs,
            "ybufs": ybufs, "plans": plans, "packed_bytes": int(packed.nbytes)}


def config2(dev, args):
    import tensomite_hip as th

    prods = products_135m()
    weight_bytes = sum(q4_0_bytes(n, k) for _, n, k in prods)
    algorithmic = sum(q4_0_bytes(n, k) + 4 * k + 4 * n for _, n, k in prods)
    copies = max(2, math.ceil(2 * MALL_BYTES / weight_bytes))
    t0 = time.perf_counter()
    c2 = build_config2(dev, copies)
    plans, wbufs, xbufs, ybufs, offsets = (c2[key] for key in ("plans", "wbufs", "xbufs", "ybufs", "offsets"))
    log(f"config 2 built in {time.perf_counter() - t0:.1f} s; {weight_bytes / 1e6:.1f} MB per token, "
        f"{copies} copies = {copies * weight_bytes / 1e6:.0f} MB")

    run = lambda i: plans[i % copies].run()
    warm = warm_up(dev, run, args.warmup)
    # The timed region: K launches back to back, an event every GROUP.
    group = GROUP if args.steps >= GROUP else 1
    per, wall = time_launches(dev, run, args.steps, group)
    ms_per_step = wall * 1e3 / args.steps
    value = algorithmic / (ms_per_step * 1e-3) / 1e9
    # The roofline: the median over at least ROOFLINE_GROUPS groups of
    # GROUP back-to-back launches (per-launch time = the group's / GROUP).
    if len(per) < ROOFLINE_GROUPS:
        group = GROUP
        per, _ = time_launches(dev, run, ROOFLINE_GROUPS * GROUP, GROUP)
    stats = launch_stats(per, algorithmic, group)
    achieved = stats["GB_per_s_median"]
    gpu_out = [dev.to_array(y, np.float32, n) for y, (_, n, _) in zip(ybufs, prods)]

    # The same launch in UNORDERED (each row's contributions as four running
    # sums instead of the host's block order; measurement only): the price
    # of the host's order.
    for plan in plans:
        plan.set_mode("unordered")
    warm_up(dev, run, args.warmup)
    per_u, _ = time_launches(dev, run, ROOFLINE_GROUPS * GROUP, GROUP)
    u_stats = launch_stats(per_u, algorithmic, GROUP)
    for plan in plans:
        plan.set_mode("auto")

    # Per-product launches (the reference's one launch per product), for comparison.
    def per_product(s):
        for i, (name, n, k) in enumerate(prods):
            th.check("tmh_block_matmul", dev.lib.tmh_block_matmul(
                th.Q4_0, wbufs[s % copies].pointer, offsets[i], xbufs[i].pointer, k, ybufs[i].pointer, 0, 1, n, k,
                0))
    warm_up(dev, per_product, 3, seconds=0.0)
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for s in range(20):
        per_product(s)
    dev.record(e1)
    dev.sync()
    per_product_ms = dev.elapsed_ms(e0, e1) / 20

    result = {
        "metric": "Q4_0 matvec HBM GB/s (% peak); decode tokens/sec at 1.7B Llama shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot + f32 fold",
        "data": "synthetic: W ~ N(0,0.02) quantised to Q4_0, x ~ N(0,1); random init, no checkpoint",
        "config": {
            "workload": "config 2: SmolLM2-135M Q4_0 matvec set at batch 1 (30 x [qkv 960x576, o 576x576, "
                        "gate_up 3072x576, down 576x1536] + head 49152x576), one launch per token",
            "products_per_step": len(prods),
            "weight_bytes_per_step": weight_bytes,
            "algorithmic_bytes_per_step": algorithmic,
            "weight_copies_rotated": copies,
            "rotated_bytes": copies * weight_bytes,
            "copy_bytes": c2["packed_bytes"],
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 1),
        "roofline": {
            "kernel": plans[0].describe() + " (Q4_0; one launch = the 121 products of a token)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("traffic_q4_0_set_135m.json"),
            "algorithmic_bytes_per_launch": algorithmic,
            "launch_us_median": stats["median_us"],
            "launch_us_mean": stats["mean_us"],
            "launch_us_min": stats["min_us"],
            "launch_us_max": stats["max_us"],
            "launches": stats["launches"],
            "groups": stats["groups"],
            "launches_per_group": stats["launches_per_group"],
            "warmup_launches": warm,
        },
        "unordered": {
            "launch_us_median": u_stats["median_us"], "GB_per_s": u_stats["GB_per_s_median"],
            "frac": round(u_stats["GB_per_s_median"] / HBM_PEAK_GBS, 4),
            "note": "the same plan in BlockMatMulMode UNORDERED (tmh_plan_set_mode): each row's contributions "
                    "summed as four running sums instead of in block order; measurement only",
        },
        "per_product_launches": {
            "ms_per_token": round(per_product_ms, 4),
            "GB_per_s": round(algorithmic / (per_product_ms * 1e-3) / 1e9, 1),
            "note": "the same 121 products as 121 tmh_block_matmul calls",
        },
    }
    if not args.no_cpu:
        log("cpu baseline (config 2) ...")
        result["cpu_baseline"] = cpu_baseline_config2(c2["weights"], c2["xs"], prods, gpu_out, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    for plan in plans:
        plan.destroy()
    for buf in wbufs + xbufs + ybufs:
        buf.release()
    dev.sync()
    return result


# ---------------------------------------------------------------- config 1

def config1(dev, args, batch=128, min_copies=1024):
    """W [2304, 768] ~ N(0, 0.02) quantised to Q8_0, x
    ~ N(0, 1), y = W·x. Two figures, both rotating through >= 1024 distinct
    weight copies (1.9 GB, past the 256 MB Infinity Cache):
      single   one tmh_block_matmul a launch (the one-row kernel), the median
               of >= 100 per-launch event times;
      batched  `batch` products a launch (a plan over distinct copies and
               outputs, the same x), as the median per launch.
    Bytes a product: weights + 4·K of x + 4·N of y (1,892,352 B)."""
    import quant_host
    import tensomite_hip as th

    n, k = C_ATTN
    wbytes = q8_0_bytes(n, k)
    algorithmic = wbytes + 4 * k + 4 * n
    copies = max(min_copies, math.ceil(2 * MALL_BYTES / wbytes))
    copies = (copies + batch - 1) // batch * batch
    host = quant_host.synthetic_weights("Q8_0", n, k, seed=0x5EED0001)
    x_host = np.random.default_rng(0x5EED0001 + 1).standard_normal(k, dtype=np.float32)
    stride = (wbytes + 255) // 256 * 256
    per_buffer = 256  # copies a device buffer holds
    buffers, views = [], []
    first = dev.from_array(host)
    for b in range(copies // per_buffer):
        buf = dev.alloc(stride * per_buffer)
        for j in range(per_buffer):
            dev.copy(buf, first, wbytes, dst_offset=j * stride)
            views.append(_View(buf, j * stride))
        buffers.append(buf)
    x = dev.from_array(x_host)
    y = dev.alloc(4 * n)
    ys = [dev.alloc(4 * n) for _ in range(batch)]
    dev.sync()

    def single(i):
        th.check("tmh_block_matmul", dev.lib.tmh_block_matmul(th.Q8_0, views[i % copies].pointer, 0, x.pointer, k,
                                                               y.pointer, 0, 1, n, k, 0))
    warm_up(dev, single, args.warmup)
    per, wall = time_launches(dev, single, ROOFLINE_GROUPS * GROUP, GROUP)
    s_stats = launch_stats(per, algorithmic, GROUP)
    gpu_y = dev.to_array(y, np.float32, n)

    plans = [dev.plan("Q8_0", [(views[p * batch + j], 0, x, ys[j], None, n, k) for j in range(batch)])
             for p in range(copies // batch)]
    run = lambda i: plans[i % len(plans)].run()
    warm_up(dev, run, args.warmup)
    per_b, _ = time_launches(dev, run, ROOFLINE_GROUPS * 4, 4)
    b_stats = launch_stats(per_b, algorithmic * batch, 4)
    batched_y = dev.to_array(ys[batch - 1], np.float32, n)
    out = {
        "workload": "config 1: GPT-2-small c_attn, Q8_0 W [2304, 768] x f32 [768] -> [2304]",
        "algorithmic_bytes_per_product": algorithmic,
        "weight_copies_rotated": copies,
        "rotated_bytes": copies * wbytes,
        "single": dict(s_stats, kernel="one tmh_block_matmul (k_matvec_row) a launch",
                       roofline={"bound": "hbm", "achieved": s_stats["GB_per_s_median"], "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(s_stats["GB_per_s_median"] / HBM_PEAK_GBS, 4),
                                 "traffic": traffic_from_profiles("traffic_q8_0_c_attn.json")}),
        "batched": dict(b_stats, products_per_launch=batch, kernel=plans[0].describe(),
                        roofline={"bound": "hbm", "achieved": b_stats["GB_per_s_median"], "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(b_stats["GB_per_s_median"] / HBM_PEAK_GBS, 4)}),
    }
    if not args.no_cpu:
        from oracle import oracle
        hostinfo = host_cpu()
        builds = {}
        for variant in dict.fromkeys(["portable", oracle.best_variant()]):
            sets, elapsed, mismatched = cpu_products("Q8_0", [host], [x_host], [(n, k)], [gpu_y],
                                                     args.cpu_seconds / 2, variant, hostinfo["cores"])
            builds[variant] = {"GB_per_s": round(algorithmic * sets / elapsed / 1e9, 2),
                               "us_per_product": round(elapsed / sets * 1e6, 2), "products": sets,
                               "parity_mismatched": mismatched}
        want = oracle.matmul("Q8_0", x_host, host, 1, n, k)[0]
        best = max(builds, key=lambda v: builds[v]["GB_per_s"])
        out["cpu_baseline"] = {
            "value": builds[best]["GB_per_s"], "unit": "GB/s", "cores": hostinfo["cores"], "kind": "port",
            "sample": f"the one product repeated for ~{args.cpu_seconds / 2:.0f} s per build (weights stay in the "
                      f"host's caches: 1.9 MB); oracle Quant.matmul restatement, {hostinfo['cores']} threads; "
                      f"value from the {best} build",
            "builds": builds,
            "batched_parity_ok": bool(np.array_equal(batched_y.view(np.uint32), want.view(np.uint32)))}
    for plan in plans:
        plan.destroy()
    for buf in buffers + [first, x, y] + ys:
        buf.release()
    dev.sync()
    return out


# ---------------------------------------------------------------- config 5

def decode_1p7b(dev, steps, cpu_seconds, with_cpu, graph=True):
    """Config 5: greedy decode of a SmolLM2-1.7B-shaped Llama, every matrix
    W ~ N(0, 0.02) quantised to Q4_0 (quant_host.synthetic_llama, tied head),
    through the device-resident decoder, after a 128-token prompt, at batch 1
    and batch 8 (f32 KV capacity 2048). A step is one token per row, replayed
    from a captured HIP graph, timed with HIP events on the library's stream.
    The CPU figure is the oracle's forward (the restatement of tensomite's
    host path) per decoded token after the same 128-token prompt as the
    GPU's batch 1, on a bounded sample; its tokens are compared with the
    GPU's."""
    import quant_host
    import tensomite_hip as th

    config = dict(quant_host.SMOLLM2_1P7B)
    t0 = time.perf_counter()
    weights = quant_host.synthetic_llama(config, seed=0x5EED0005)
    log(f"1.7B weights in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(0x5EED0005 + 1)
    prompts = [[int(t) for t in rng.integers(0, config["vocab"], 128)] for _ in range(8)]
    out = {"model": "SmolLM2-1.7B shape, Q4_0, tied head; W ~ N(0, 0.02) quantised (synthetic_llama), norms 1",
           "prompt": 128, "capacity": 2048}
    weight_bytes = sum(w.nbytes for key in ("qkv", "o", "gate_up", "down") for w in weights[key]) + \
        weights["embed"].nbytes
    out["weight_bytes_per_token"] = weight_bytes
    gpu_tokens = None
    for rows in (1, 8):
        model = th.HIPLlama(dev, config, weights, rows=rows, capacity=2048, max_tokens=128)
        prefill = []
        for r in range(rows):
            t = time.perf_counter()
            model.forward(prompts[r], row=r, last_only=True)
            prefill.append(time.perf_counter() - t)
        tokens = model.generate(steps, graph=graph)  # the graph is captured on first use
        if rows == 1:
            gpu_tokens = [int(t) for t in tokens[0]]
        # The timed run: the same prompts again, then the `steps` greedy
        # tokens (steps - 1 decode forwards at positions 128..126 + steps,
        # each one graph launch), HIP events around the generate call.
        model.reset()
        for r in range(rows):
            model.forward(prompts[r], row=r, last_only=True)
        e0, e1 = dev.event(), dev.event()
        dev.record(e0)
        again = model.generate(steps, graph=graph)
        dev.record(e1)
        dev.sync()
        ms = dev.elapsed_ms(e0, e1) / (steps - 1)
        out[f"batch{rows}"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(rows * 1e3 / ms, 1), "graph": graph,
                               "steps": steps, "positions": f"128..{126 + steps}",
                               "repeat_tokens_equal": bool(np.array_equal(again, tokens)),
                               "prefill_128_ms": round(1e3 * float(np.median(prefill)), 2),
                               "weight_GB_per_s": round(weight_bytes / (ms * 1e-3) / 1e9, 1)}
        # The same steps with the products in UNORDERED (tmh_llama_set_mode;
        # each product's contributions as four running sums, measurement
        # only): what the host's order costs a step. Its tokens may differ.
        model.set_mode("unordered")
        model.reset()
        for r in range(rows):
            model.forward(prompts[r], row=r, last_only=True)
        model.generate(2, graph=graph)  # the UNORDERED step graph captured
        model.reset()
        for r in range(rows):
            model.forward(prompts[r], row=r, last_only=True)
        dev.record(e0)
        model.generate(steps, graph=graph)
        dev.record(e1)
        dev.sync()
        out[f"batch{rows}"]["unordered_ms_per_step"] = round(dev.elapsed_ms(e0, e1) / (steps - 1), 4)
        model.destroy()
        log(f"decode batch {rows}: {ms * 1e3:.0f} us/step")
    if with_cpu:
        # The same steps the GPU's batch 1 times: the 128-token prompt
        # (untimed), then `steps` - 1 decode forwards at positions
        # 128..126 + steps, each timed; the median and mean a token.
        from oracle import oracle
        host = host_cpu()
        variant = oracle.best_variant()
        oracle.set_threads(host["cores"], variant)
        cpu = oracle.Llama(config, weights, variant)
        logits = cpu.forward(prompts[0], last_only=True)[0]
        cpu_tokens, per = [oracle.argmax(logits)], []
        start = time.perf_counter()
        while len(cpu_tokens) < steps and time.perf_counter() - start < cpu_seconds:
            t = time.perf_counter()
            logits = cpu.forward([cpu_tokens[-1]], last_only=True)[0]
            per.append(time.perf_counter() - t)
            cpu_tokens.append(oracle.argmax(logits))
        decoded = len(per)
        ms = statistics.median(per) * 1e3 if per else None
        out["cpu_baseline"] = {
            "value": round(1e3 / ms, 2) if ms else None, "unit": "tokens/s", "cores": host["cores"], "kind": "port",
            "ms_per_token": round(ms, 2) if ms else None,
            "ms_per_token_mean": round(sum(per) / decoded * 1e3, 2) if per else None,
            "weight_GB_per_s": round(weight_bytes / (ms * 1e-3) / 1e9, 1) if ms else None,
            "sample": f"{decoded} greedy decode steps at positions 128..{127 + decoded} (the GPU's batch-1 timed "
                      f"steps are 128..{126 + steps}), after the same 128-token prompt (prefill excluded); the "
                      f"oracle's Llama forward ({variant} build, {host['cores']} threads); median a token",
            "tokens_equal_gpu": gpu_tokens is not None and cpu_tokens == gpu_tokens[:len(cpu_tokens)],
            "tokens_compared": len(cpu_tokens)}
    return out


def host_memory_rate(cores, mbytes=1024, seconds=1.0):
    """The host's STREAM-style copy rate: `cores` threads each copying its
    share of a `mbytes` MB array (numpy releases the GIL while copying);
    GB/s counts the bytes read plus written. It bounds what a CPU baseline
    that streams weights from DRAM can reach on this host."""
    from concurrent.futures import ThreadPoolExecutor

    n = (mbytes << 20) // 8
    src = np.ones(n, np.float64)
    dst = np.empty_like(src)
    bounds = [(i * n // cores, (i + 1) * n // cores) for i in range(cores)]

    def part(i):
        a, b = bounds[i]
        np.copyto(dst[a:b], src[a:b])

    rates = []
    with ThreadPoolExecutor(cores) as pool:
        list(pool.map(part, range(cores)))  # pages touched
        start = time.perf_counter()
        while time.perf_counter() - start < seconds or len(rates) < 3:
            t = time.perf_counter()
            list(pool.map(part, range(cores)))
            rates.append(2 * src.nbytes / (time.perf_counter() - t) / 1e9)
    return {"copy_GB_per_s": round(max(rates), 1), "copy_GB_per_s_median": round(statistics.median(rates), 1),
            "threads": cores, "array_bytes": int(src.nbytes),
            "method": "numpy copyto of a 1 GiB float64 array split over the threads; read + write bytes"}


# ---------------------------------------------------------------- config 3

C3_SHAPES = ((8192, 2048), (2048, 8192))
C3_ROWS = (1, 2, 4, 8, 16)


def cpu_rate(kind, x, w, rows, n, k, seconds, variant, cores):
    """The oracle's Quant.matmul (`variant` build, `cores` threads) repeated
    for about `seconds` (at least twice): seconds a call, and the last output."""
    from oracle import oracle

    oracle.set_threads(cores, variant)
    out = oracle.matmul(kind, x, w, rows, n, k, variant)  # warm: pages, pool
    calls, start = 0, time.perf_counter()
    while True:
        out = oracle.matmul(kind, x, w, rows, n, k, variant)
        calls += 1
        elapsed = time.perf_counter() - start
        if calls >= 2 and elapsed >= seconds:
            break
    return elapsed / calls, calls, out


def config3(dev, warmup, cpu_seconds=None):
    """Config 3: Q4_1 batched-decode products, W [8192, 2048] and [2048, 8192]
    (W ~ N(0, 0.02) quantised, seed 0x5EED0003 + n) against B = 1, 2, 4, 8,
    16 f32 activation rows (x ~ N(0, 1)). One call is tmh_block_matmul in
    AUTO mode (whatever kernels it takes: one launch below 8 rows of K =
    2048, the quantise pass and a product otherwise). Calls rotate through
    enough weight copies (>= 512 MB) that the 256 MB Infinity Cache cannot
    serve them; HIP events every 10 calls, the median over 100 groups.
    Bytes a call: weights + 4·B·K of x + 4·B·N of y (HBM-bound at every B).
    Every point's output bits are checked against the oracle; with
    cpu_seconds, the oracle's Quant.matmul restatement is timed on the same
    bytes (portable and native builds, every host core)."""
    import quant_host
    from oracle import oracle

    host = host_cpu()
    variants = list(dict.fromkeys(["portable", oracle.best_variant()]))
    out = {"workload": "config 3: Q4_1 batched-decode products, [8192, 2048] and [2048, 8192] x B f32 rows",
           "unit": "GB/s", "points": {}}
    rng = np.random.default_rng(0x5EED0003)
    for n, k in C3_SHAPES:
        wq = quant_host.synthetic_weights("Q4_1", n, k, seed=0x5EED0003 + n)
        copies = max(2, math.ceil(2 * MALL_BYTES / wq.nbytes))
        first = dev.from_array(wq)
        ws = [first] + [dev.alloc(wq.nbytes) for _ in range(copies - 1)]
        for w in ws[1:]:
            dev.copy(w, first, wq.nbytes)
        for b in C3_ROWS:
            xh = rng.standard_normal((b, k), dtype=np.float32)
            x = dev.from_array(xh)
            dst = dev.alloc(4 * b * n)
            call = lambda i: dev.block_matmul("Q4_1", ws[i % copies], x, b, n, k, dst=dst)
            warm_up(dev, call, warmup)
            per, _ = time_launches(dev, call, ROOFLINE_GROUPS * 10, 10)
            nbytes = wq.nbytes + 4 * b * k + 4 * b * n
            st = launch_stats(per, nbytes, 10)
            got = dev.to_array(dst, np.float32, b * n).reshape(b, n)
            point = {"us_per_call_median": st["median_us"], "us_per_call_mean": st["mean_us"],
                     "algorithmic_bytes": nbytes, "weight_copies_rotated": copies,
                     "roofline": {"bound": "hbm", "achieved": st["GB_per_s_median"], "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(st["GB_per_s_median"] / HBM_PEAK_GBS, 4)}}
            want = oracle.matmul("Q4_1", xh, wq, b, n, k, oracle.best_variant())
            point["bit_exact_vs_oracle"] = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
            ucall = lambda i: dev.block_matmul("Q4_1", ws[i % copies], x, b, n, k, dst=dst, mode="unordered")
            warm_up(dev, ucall, warmup)
            per_u, _ = time_launches(dev, ucall, ROOFLINE_GROUPS * 10, 10)
            point["unordered_us_per_call_median"] = round(statistics.median(per_u) * 1e3, 3)
            if cpu_seconds:
                builds = {}
                for variant in variants:
                    sec, calls, _ = cpu_rate("Q4_1", xh, wq, b, n, k, cpu_seconds, variant, host["cores"])
                    builds[variant] = {"GB_per_s": round(nbytes / sec / 1e9, 2), "us_per_call": round(sec * 1e6, 1),
                                       "calls": calls}
                best = max(builds, key=lambda v: builds[v]["GB_per_s"])
                point["cpu_baseline"] = {"value": builds[best]["GB_per_s"], "unit": "GB/s", "cores": host["cores"],
                                         "kind": "port", "build": best, "builds": builds}
            out["points"][f"{n}x{k} B={b}"] = point
            x.release()
            dst.release()
        for w in ws:
            w.release()
    pts = out["points"]
    out["value"] = pts["8192x2048 B=1"]["roofline"]["achieved"]
    out["roofline_frac_min"] = min(p["roofline"]["frac"] for p in pts.values())
    out["roofline_frac_max"] = max(p["roofline"]["frac"] for p in pts.values())
    out["bit_exact_vs_oracle"] = all(p["bit_exact_vs_oracle"] for p in pts.values())
    if cpu_seconds:
        head = pts["8192x2048 B=1"]["cpu_baseline"]
        out["cpu_baseline"] = {
            "value": head["value"], "unit": "GB/s", "cores": host["cores"], "kind": "port",
            "sample": f"each of the 10 points (2 shapes x B = 1..16) repeated for ~{cpu_seconds:g} s per build "
                      f"(portable and {oracle.best_variant()}), the oracle's Quant.matmul restatement with the "
                      f"reference's span rule and spin pool, {host['cores']} threads; value: 8192x2048 B=1, "
                      f"each point's own figure under points[].cpu_baseline (weights 10.5 MB: the host's caches "
                      f"hold part of them between calls)",
            "host": host}
    return out


# ---------------------------------------------------------------- heads

HEADS = (("135m", 49152, 576), ("1p7b", 49152, 2048))


def heads(dev, warmup, cpu_seconds=None):
    """The two tied heads as single one-row Q4_0 products (W ~ N(0, 0.02)
    quantised, seed 0x5EED0006 + k; x ~ N(0, 1)): SmolLM2-135M's [49152, 576]
    (15.9 MB) and the 1.7B shape's [49152, 2048] (56.6 MB), the largest
    single products of configs 2 and 5. Two routes each: one
    tmh_block_matmul call in AUTO mode, and a plan of that one product (the
    streamed kernel). Calls rotate through >= 512 MB of weight copies; HIP
    events every 20 calls, the median over 100 groups. Bytes a call:
    weights + 4·K of x + 4·N of y. Both routes' output bits are checked
    against the oracle; with cpu_seconds, the oracle's Quant.matmul
    restatement is timed on the same product (portable and native builds,
    every host core)."""
    import quant_host
    from oracle import oracle

    host = host_cpu()
    variants = list(dict.fromkeys(["portable", oracle.best_variant()]))
    out = {"workload": "the tied heads as single one-row Q4_0 products: [49152, 576] (SmolLM2-135M, 15.9 MB) and "
                       "[49152, 2048] (1.7B shape, 56.6 MB)", "unit": "GB/s", "points": {}}
    rng = np.random.default_rng(0x5EED0006)
    for name, n, k in HEADS:
        wq = quant_host.synthetic_weights("Q4_0", n, k, seed=0x5EED0006 + k)
        xh = rng.standard_normal(k, dtype=np.float32)
        copies = max(2, math.ceil(2 * MALL_BYTES / wq.nbytes))
        first = dev.from_array(wq)
        ws = [first] + [dev.alloc(wq.nbytes) for _ in range(copies - 1)]
        for w in ws[1:]:
            dev.copy(w, first, wq.nbytes)
        x = dev.from_array(xh)
        dst = dev.alloc(4 * n)
        nbytes = wq.nbytes + 4 * k + 4 * n
        want = oracle.matmul("Q4_0", xh, wq, 1, n, k, oracle.best_variant())[0]
        point = {"n": n, "k": k, "weight_bytes": int(wq.nbytes), "algorithmic_bytes": nbytes,
                 "weight_copies_rotated": copies}
        plans = [dev.plan("Q4_0", [(w, 0, x, dst, None, n, k)]) for w in ws]
        routes = (("auto", lambda i: dev.block_matmul("Q4_0", ws[i % copies], x, 1, n, k, dst=dst)),
                  ("plan", lambda i: plans[i % copies].run()))
        for route, call in routes:
            warm_up(dev, call, warmup)
            per, _ = time_launches(dev, call, ROOFLINE_GROUPS * GROUP, GROUP)
            st = launch_stats(per, nbytes, GROUP)
            got = dev.to_array(dst, np.float32, n)
            point[route] = {"us_per_call_median": st["median_us"], "us_per_call_mean": st["mean_us"],
                            "roofline": {"bound": "hbm", "achieved": st["GB_per_s_median"], "peak": HBM_PEAK_GBS,
                                         "unit": "GB/s", "frac": round(st["GB_per_s_median"] / HBM_PEAK_GBS, 4)},
                            "bit_exact_vs_oracle": bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))}
        point["auto"]["route"] = "tmh_block_matmul, AUTO"
        point["plan"]["route"] = plans[0].describe()
        if cpu_seconds:
            builds = {}
            for variant in variants:
                sec, calls, _ = cpu_rate("Q4_0", xh, wq, 1, n, k, cpu_seconds, variant, host["cores"])
                builds[variant] = {"GB_per_s": round(nbytes / sec / 1e9, 2), "us_per_call": round(sec * 1e6, 1),
                                   "calls": calls}
            best = max(builds, key=lambda v: builds[v]["GB_per_s"])
            point["cpu_baseline"] = {"value": builds[best]["GB_per_s"], "unit": "GB/s", "cores": host["cores"],
                                     "kind": "port", "build": best, "builds": builds,
                                     "sample": f"the product repeated for ~{cpu_seconds:g} s per build"}
        out["points"][name] = point
        for plan in plans:
            plan.destroy()
        for buf in ws + [x, dst]:
            buf.release()
    out["bit_exact_vs_oracle"] = all(p[r]["bit_exact_vs_oracle"] for p in out["points"].values()
                                     for r in ("auto", "plan"))
    return out


# ---------------------------------------------------------------- config 4

def config4(dev, warmup, cpu_seconds=None):
    """Config 4: the Q8_0 prefill GEMM at the Llama-1.7B shape, 512 tokens x
    K = 2048 against N = 2048 (attention projections) and N = 8192 (MLP
    up/gate), W ~ N(0, 0.02) quantised (seed 0x5EED0004 + N), x ~ N(0, 1).
    One call is tmh_block_matmul over f32 x (the activation quantiser, then
    the matrix-core kernel k_matmul_mx); HIP events every 4 calls, the median
    over 100 groups. int8 work: 2 · 512 · 2048 · N ops a call; bytes: weights
    + 4·512·K of x + 4·512·N of y. Each N runs in AUTO (the host's ordered,
    separately rounded fold; its bits checked against the oracle) and in
    UNORDERED (one fused multiply-add per output and block: measurement
    only, the price of the host's order). With cpu_seconds, the oracle's
    Quant.matmul restatement on the same bytes (portable and native builds,
    every host core)."""
    import quant_host
    from oracle import oracle

    host = host_cpu()
    variants = list(dict.fromkeys(["portable", oracle.best_variant()]))
    rows, k = 512, 2048
    rng = np.random.default_rng(0x5EED0004)
    xh = rng.standard_normal((rows, k), dtype=np.float32)
    x = dev.from_array(xh)
    out = {"workload": "config 4: Q8_0 prefill GEMM, 512 tokens x K=2048 -> N = 2048 and 8192", "unit": "TOP/s",
           "points": {}}
    for n in (2048, 8192):
        wq = quant_host.synthetic_weights("Q8_0", n, k, seed=0x5EED0004 + n)
        w = dev.from_array(wq)
        dst = dev.alloc(4 * rows * n)
        ops = 2.0 * rows * k * n
        nbytes = wq.nbytes + 4 * rows * k + 4 * rows * n
        want = oracle.matmul("Q8_0", xh, wq, rows, n, k, oracle.best_variant())
        for mode in ("auto", "unordered"):
            call = lambda i: dev.block_matmul("Q8_0", w, x, rows, n, k, dst=dst, mode=mode)
            warm_up(dev, call, warmup)
            per, _ = time_launches(dev, call, ROOFLINE_GROUPS * 4, 4)
            med = statistics.median(per)
            tops = ops / (med * 1e-3) / 1e12
            got = dev.to_array(dst, np.float32, rows * n).reshape(rows, n)
            point = {"us_per_call_median": round(med * 1e3, 2), "us_per_call_mean": round(sum(per) / len(per) * 1e3, 2),
                     "int8_ops": ops, "algorithmic_bytes": nbytes,
                     "GB_per_s": round(nbytes / (med * 1e-3) / 1e9, 1),
                     "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                                  "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4)}}
            if mode == "auto":
                point["bit_exact_vs_oracle"] = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
            else:
                rel = float(np.linalg.norm((got - want).astype(np.float64)) / np.linalg.norm(want.astype(np.float64)))
                point["relative_l2_vs_oracle"] = rel
            out["points"][f"N={n} {mode}"] = point
        if cpu_seconds:
            builds = {}
            for variant in variants:
                sec, calls, _ = cpu_rate("Q8_0", xh, wq, rows, n, k, cpu_seconds, variant, host["cores"])
                builds[variant] = {"TOP_per_s": round(ops / sec / 1e12, 3), "ms_per_call": round(sec * 1e3, 2),
                                   "calls": calls}
            best = max(builds, key=lambda v: builds[v]["TOP_per_s"])
            out["points"][f"N={n} auto"]["cpu_baseline"] = {
                "value": builds[best]["TOP_per_s"], "unit": "TOP/s", "cores": host["cores"], "kind": "port",
                "build": best, "builds": builds}
        w.release()
        dst.release()
    x.release()
    pts = out["points"]
    out["value"] = pts["N=8192 auto"]["roofline"]["achieved"]
    out["bit_exact_vs_oracle"] = all(p.get("bit_exact_vs_oracle", True) for p in pts.values())
    if cpu_seconds:
        out["cpu_baseline"] = {
            "value": pts["N=8192 auto"]["cpu_baseline"]["value"], "unit": "TOP/s", "cores": host["cores"],
            "kind": "port",
            "sample": f"each N repeated for ~{cpu_seconds:g} s (at least 2 calls) per build (portable and "
                      f"{oracle.best_variant()}), the oracle's Quant.matmul restatement, {host['cores']} threads; "
                      f"value: N=8192",
            "host": host}
    return out


# ---------------------------------------------------------------- ceilings

def ceilings(dev, warmup):
    """The box's own ceilings beside the vendor peaks: the HBM read rate of a
    grid-stride read kernel (tmh_debug_read: 16 B a lane a load, four in
    flight, non-temporal) at 15.9 and 56.6 MB (the heads' single products),
    77 MB (config 2's bytes) and 1 GiB, by workgroup count; the device-to-device copy rate (tmh_copy: bytes read +
    written); each the median over >= 100 launches rotating through >= 512
    MB so the 256 MB Infinity Cache cannot serve them; and what rocminfo
    and amd-smi report of the device."""
    import subprocess
    import tensomite_hip as th

    out = {"device": {"name": dev.name, "arch": dev.arch, "compute_units": dev.compute_units}, "read": {},
           "copy": {}}
    info = th.DeviceInfo()
    th.check("tmh_device_info_get", dev.lib.tmh_device_info_get(0, ctypes_byref(info)))
    out["device"].update({"memory_bytes": info.memory, "clock_khz": info.clock_khz,
                          "memory_clock_khz": info.memory_clock_khz, "memory_bus_width": info.memory_bus_width,
                          "l2_bytes": info.l2_bytes})
    tools = {}
    for cmd in (["rocminfo"], ["amd-smi", "static", "--gpu", "0"], ["amd-smi", "metric", "--gpu", "0", "--clock"]):
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=60)
            keep = [ln.strip() for ln in r.stdout.splitlines()
                    if any(key in ln for key in ("Marketing Name", "gfx950", "Compute Unit", "Max Clock", "MARKET_NAME",
                                                 "MAX_SCLK", "MAX_MCLK", "VRAM", "SIZE", "TYPE", "BUS", "CLK",
                                                 "SCLK", "MCLK", "Memory"))]
            tools[" ".join(cmd)] = keep[:40]
        except (OSError, subprocess.SubprocessError) as e:
            tools[" ".join(cmd)] = [f"unavailable: {e}"]
    out["tools"] = tools
    sink = dev.alloc(4 * 8192)
    sizes = [(f"head_{name}", (q4_0_bytes(n, k) + 4 * k + 4 * n) // 16 * 16) for name, n, k in HEADS]
    for label, size in sizes + [("77MB", 76_857_600 // 16 * 16), ("1GiB", 1 << 30)]:
        copies = max(2, math.ceil(2 * MALL_BYTES / size))
        bufs = [dev.alloc(size) for _ in range(copies)]  # contents do not matter to a read rate
        dev.sync()
        groups = 100 if size < (1 << 28) else 20
        per_group = 10 if size < (1 << 28) else 2
        for wgs in (256, 512, 1024, 1536, 2048, 4096):
            call = lambda i: th.check("tmh_debug_read", dev.lib.tmh_debug_read(bufs[i % copies].pointer, size, wgs,
                                                                              sink.pointer))
            warm_up(dev, call, warmup)
            per, _ = time_launches(dev, call, groups * per_group, per_group)
            st = launch_stats(per, size, per_group)
            out["read"][f"{label} wgs={wgs}"] = {"us_median": st["median_us"], "GB_per_s": st["GB_per_s_median"],
                                                 "frac_of_8TBs": round(st["GB_per_s_median"] / HBM_PEAK_GBS, 4)}
        half = size // 2
        call = lambda i: dev.copy(bufs[i % copies], bufs[(i + 1) % copies], half, dst_offset=half)
        warm_up(dev, call, warmup)
        per, _ = time_launches(dev, call, groups * per_group, per_group)
        st = launch_stats(per, 2 * half, per_group)
        out["copy"][label] = {"bytes_copied": half, "us_median": st["median_us"], "GB_per_s_read_plus_write":
                              st["GB_per_s_median"], "frac_of_8TBs": round(st["GB_per_s_median"] / HBM_PEAK_GBS, 4)}
        for b in bufs:
            b.release()
        dev.sync()
    sink.release()
    best = max(out["read"].items(), key=lambda kv: kv[1]["GB_per_s"])
    out["best_read"] = {"where": best[0], **best[1]}
    return out


def ctypes_byref(obj):
    import ctypes
    return ctypes.byref(obj)


class _View:
    """A buffer seen from a byte offset (a product's weights inside a packed buffer)."""

    def __init__(self, buf, offset):
        self.buffer = buf
        self.pointer = buf.pointer + offset
        self.bytesize = buf.bytesize - offset


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="CPU baseline sample for configs 1, 2 and 5 (config 5 stops at the GPU's step count)")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decode measurement")
    ap.add_argument("--no-config1", action="store_true", help="skip the config-1 (GPT-2 c_attn) measurement")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--batched", action="store_true",
                    help="config 3 instead (Q4_1 batched-decode products, B = 1..16); its own JSON line")
    ap.add_argument("--gemm", action="store_true",
                    help="config 4 instead (Q8_0 prefill GEMM on the matrix cores); its own JSON line")
    ap.add_argument("--no-config3", action="store_true", help="skip the config-3 (Q4_1 batched) measurement")
    ap.add_argument("--no-config4", action="store_true", help="skip the config-4 (Q8_0 prefill GEMM) measurement")
    ap.add_argument("--no-heads", action="store_true", help="skip the single-product head measurement")
    ap.add_argument("--heads", action="store_true",
                    help="the two heads as single products instead (AUTO and a one-product plan); its own JSON line")
    ap.add_argument("--cpu-point-seconds", type=float, default=0.4,
                    help="CPU baseline sample per config-3/4 point and build")
    ap.add_argument("--ceilings", action="store_true",
                    help="the box's read and copy rates and device facts instead; its own JSON line")
    ap.add_argument("--decode-only", action="store_true",
                    help="config 5 only (decode at batch 1 and 8); its own JSON line")
    ap.add_argument("--decode-eager", action="store_true",
                    help="launch decode steps one kernel at a time, not from a captured graph (for kernel tracers)")
    ap.add_argument("--write-gguf", metavar="DIR",
                    help="write the configs' weights as GGUF files (the bytes measured here, for the reference's own "
                         "timing where Crystal exists) into DIR, then exit; needs no GPU")
    args = ap.parse_args()
    if args.write_gguf:
        import gguf_export
        for path in gguf_export.export_configs(args.write_gguf):
            log(f"wrote {path} ({os.path.getsize(path)} bytes)")
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path runs on one GPU's share only (asked for --gpus {args.gpus}); "
              "a product shards by output rows across GPUs, each GPU running this kernel on its share",
              file=sys.stderr)
        sys.exit(1)

    import tensomite_hip as th

    dev = th.HIPDevice(0)
    log(f"device {dev.name or '?'} {dev.arch} CUs={dev.compute_units}")
    cpu_points = None if args.no_cpu else args.cpu_point_seconds
    if args.ceilings:
        print(json.dumps(ceilings(dev, args.warmup)), flush=True)
        return
    if args.gemm:
        print(json.dumps(config4(dev, args.warmup, cpu_points)), flush=True)
        return
    if args.batched:
        print(json.dumps(config3(dev, args.warmup, cpu_points)), flush=True)
        return
    if args.heads:
        print(json.dumps(heads(dev, args.warmup, cpu_points)), flush=True)
        return
    if args.decode_only:
        print(json.dumps(decode_1p7b(dev, args.decode_steps, args.cpu_seconds, not args.no_cpu,
                                     graph=not args.decode_eager)), flush=True)
        return
    result = config2(dev, args)
    if not args.no_cpu:
        result["host_memory"] = host_memory_rate(host_cpu()["cores"])
    if not args.no_config1:
        log("config 1 ...")
        result["config1"] = config1(dev, args)
    if not args.no_config3:
        log("config 3 ...")
        result["config3"] = config3(dev, args.warmup, cpu_points)
    if not args.no_config4:
        log("config 4 ...")
        result["config4"] = config4(dev, args.warmup, cpu_points)
    if not args.no_heads:
        log("heads ...")
        result["heads"] = heads(dev, args.warmup, cpu_points)
    if not args.no_decode:
        log("decode at the 1.7B shape ...")
        result["decode_1p7b"] = decode_1p7b(dev, args.decode_steps, args.cpu_seconds, not args.no_cpu,
                                            graph=not args.decode_eager)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
