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

value = algorithmic bytes per step (weights + f32 x + f32 y) / time per
step, in GB/s; the roofline object prices the launch against 8 TB/s.
The CPU baseline times the oracle's restatement of tensomite's CPU path
(Quant.matmul, all host cores) on the same bytes, and checks the GPU's
output bits against it.

A second object, decode_1p7b, reports config 5: greedy decode tokens/s of a
SmolLM2-1.7B-shaped Q4_0 Llama at batch 1 and 8 through the device-resident
decoder (every op on the GPU with the host's bits), and the CPU oracle's
time per token beside it.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-decode]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "tensomite.cr_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20

# config 2: (name, n, k) per layer, then the head
LAYER = [("qkv", 960, 576), ("o", 576, 576), ("gate_up", 3072, 576), ("down", 576, 1536)]
LAYERS = 30
HEAD = ("head", 49152, 576)


def products_135m():
    out = []
    for layer in range(LAYERS):
        for name, n, k in LAYER:
            out.append((f"{name}.{layer}", n, k))
    out.append(HEAD)
    return out


def q4_0_bytes(n, k):
    return n * (k // 32) * 18


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def traffic_from_profiles():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by a copy kernel's reading), if the committed summary has them."""
    path = os.path.join(ROOT, "profiles", "traffic_q4_0_set_135m.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(weights, xs, prods, gpu_out, seconds):
    """The oracle's Quant.matmul restatement on the host's cores, timed over
    whole tokens for about `seconds`; also checks the GPU's bits."""
    from oracle import oracle

    variant = oracle.best_variant()
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    oracle.set_threads(cores, variant)
    # parity: every product's output bits
    mismatched = 0
    for i, (name, n, k) in enumerate(prods):
        want = oracle.matmul("Q4_0", xs[i], weights[i], 1, n, k, variant)[0]
        if not np.array_equal(want.view(np.uint32), gpu_out[i].view(np.uint32)):
            mismatched += 1
    tokens = 0
    start = time.perf_counter()
    while True:
        for i, (name, n, k) in enumerate(prods):
            oracle.matmul("Q4_0", xs[i], weights[i], 1, n, k, variant)
        tokens += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds:
            break
    algorithmic = sum(q4_0_bytes(n, k) + 4 * k + 4 * n for _, n, k in prods)
    return {
        "value": algorithmic * tokens / elapsed / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{tokens} tokens of the config-2 set (121 products each) in {elapsed:.1f} s; "
                  f"oracle Quant.matmul restatement, {variant} build, spin pool of {cores} threads",
        "ms_per_token": elapsed / tokens * 1e3,
        "parity_mismatched_products": mismatched,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decode measurement")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--batched", action="store_true",
                    help="config 3 instead (Q4_1 batched-decode products, B = 1..16); its own JSON line")
    ap.add_argument("--gemm", action="store_true",
                    help="config 4 instead (Q8_0 prefill GEMM on the matrix cores); its own JSON line")
    ap.add_argument("--decode-eager", action="store_true",
                    help="launch decode steps one kernel at a time, not from a captured graph (for kernel tracers)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path runs on one GPU's share only (asked for --gpus {args.gpus}); "
              "a product shards by output rows across GPUs, each GPU running this kernel on its share",
              file=sys.stderr)
        sys.exit(1)

    import quant_host
    import tensomite_hip as th

    dev = th.HIPDevice(0)
    log(f"device {dev.name or '?'} {dev.arch} CUs={dev.compute_units}")
    if args.gemm:
        print(json.dumps(gemm_config4(dev, args.steps, args.warmup)), flush=True)
        return
    if args.batched:
        print(json.dumps(batched_config3(dev, args.steps, args.warmup)), flush=True)
        return
    prods = products_135m()
    weight_bytes = sum(q4_0_bytes(n, k) for _, n, k in prods)
    algorithmic = sum(q4_0_bytes(n, k) + 4 * k + 4 * n for _, n, k in prods)
    copies = max(2, math.ceil(2 * MALL_BYTES / weight_bytes))

    # Host weights (one copy), quantised by the package's host quantiser.
    t0 = time.perf_counter()
    rng = np.random.default_rng(0x5EED0002)
    weights, xs = [], []
    for i, (name, n, k) in enumerate(prods):
        weights.append(quant_host.synthetic_weights("Q4_0", n, k, seed=0x5EED0002 + i))
        xs.append(rng.normal(0.0, 1.0, k).astype(np.float32))
    log(f"weights quantised in {time.perf_counter() - t0:.1f} s; {weight_bytes / 1e6:.1f} MB per token, "
        f"{copies} copies = {copies * weight_bytes / 1e6:.0f} MB")

    # Device: one packed weight buffer per copy, activations, outputs.
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
        items = []
        for i, (name, n, k) in enumerate(prods):
            items.append((wbufs[c], 0, xbufs[i], ybufs[i], None, n, k))
        # w_row is in rows; the packed offset is in bytes: pass it through a view
        plan_items = []
        for i, (w, _, x, y, b, n, k) in enumerate(items):
            plan_items.append((_View(w, offsets[i]), 0, x, y, b, n, k))
        plans.append(dev.plan("Q4_0", plan_items))
    dev.sync()

    # Warm-up, then the timed region: K launches back to back. The warm-up is
    # W launches, continued until they have kept the GPU busy for at least
    # 50 ms: the set takes ~16 us, and after the host-side set-up the GPU's
    # clocks need that long to settle (20 launches leave the mean ~1 us high).
    warm = 0
    t_warm = time.perf_counter()
    while warm < args.warmup or time.perf_counter() - t_warm < 0.05:
        for _ in range(100 if warm >= args.warmup else 1):
            plans[warm % copies].run()
            warm += 1
        if warm >= args.warmup:
            dev.sync()
    dev.sync()
    # HIP events on the library's stream bracket the K launches (one launch
    # per step, back to back): their mean is the kernel's launch duration.
    ev0, ev1 = dev.event(), dev.event()
    t_start = time.perf_counter()
    dev.record(ev0)
    for s in range(args.steps):
        plans[s % copies].run()
    dev.record(ev1)
    dev.sync()
    t_end = time.perf_counter()
    ms_per_step = (t_end - t_start) * 1e3 / args.steps
    launch_ms = dev.elapsed_ms(ev0, ev1) / args.steps
    value = algorithmic / (ms_per_step * 1e-3) / 1e9
    achieved = algorithmic / (launch_ms * 1e-3) / 1e9

    # Outputs of the last step, for the CPU parity check.
    gpu_out = [dev.to_array(y, np.float32, n) for y, (_, n, _) in zip(ybufs, prods)]

    # Per-product launches (the reference's one launch per product), for comparison.
    for s in range(3):
        for i, (name, n, k) in enumerate(prods):
            dev.lib.tmh_block_matmul(th.Q4_0, wbufs[s % copies].pointer, offsets[i], xbufs[i].pointer, k,
                                     ybufs[i].pointer, 0, 1, n, k, 0)
    dev.sync()
    reps = 20
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for s in range(reps):
        for i, (name, n, k) in enumerate(prods):
            dev.lib.tmh_block_matmul(th.Q4_0, wbufs[s % copies].pointer, offsets[i], xbufs[i].pointer, k,
                                     ybufs[i].pointer, 0, 1, n, k, 0)
    dev.record(e1)
    dev.sync()
    per_product_ms = dev.elapsed_ms(e0, e1) / reps

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
            "copy_bytes": int(packed.nbytes),
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 1),
        "roofline": {
            "kernel": plans[0].describe() + " (Q4_0; one launch = the 121 products of a token)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(),
            "launch_us_mean": round(launch_ms * 1e3, 2),
            "warmup_launches": warm,
        },
        "per_product_launches": {
            "ms_per_token": round(per_product_ms, 4),
            "GB_per_s": round(algorithmic / (per_product_ms * 1e-3) / 1e9, 1),
            "note": "the same 121 products as 121 tmh_block_matmul calls",
        },
    }
    if not args.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(weights, xs, prods, gpu_out, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    for buf in wbufs:
        buf.release()
    dev.sync()
    if not args.no_decode:
        log("decode at the 1.7B shape ...")
        result["decode_1p7b"] = decode_1p7b(dev, args.decode_steps, args.cpu_seconds, not args.no_cpu,
                                            graph=not args.decode_eager)
    print(json.dumps(result), flush=True)


def decode_1p7b(dev, steps, cpu_seconds, with_cpu, graph=True):
    """Config 5: greedy decode of a SmolLM2-1.7B-shaped Q4_0 Llama (random
    block weights, tied head) through the device-resident decoder, after a
    128-token prompt, at batch 1 and batch 8 (f32 KV capacity 2048). A step is
    one token per row, replayed from a captured HIP graph; timed with HIP
    events on the library's stream. The CPU figure is the oracle's forward
    (the restatement of tensomite's host path) per decoded token after a
    short prompt, on a bounded sample."""
    import quant_host
    import tensomite_hip as th

    config = dict(quant_host.SMOLLM2_1P7B)
    t0 = time.perf_counter()
    weights = quant_host.random_block_llama(config, seed=0x5EED0005)
    log(f"1.7B weights in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(0x5EED0005)
    out = {"model": "SmolLM2-1.7B shape, Q4_0, tied head (random block weights)", "prompt": 128,
           "capacity": 2048}
    weight_bytes = sum(w.nbytes for key in ("qkv", "o", "gate_up", "down") for w in weights[key]) + \
        weights["embed"].nbytes
    out["weight_bytes_per_token"] = weight_bytes
    for rows in (1, 8):
        model = th.HIPLlama(dev, config, weights, rows=rows, capacity=2048, max_tokens=128)
        prefill = []
        for r in range(rows):
            prompt = list(rng.integers(0, config["vocab"], 128))
            t = time.perf_counter()
            model.forward(prompt, row=r, last_only=True)
            prefill.append(time.perf_counter() - t)
        model.generate(4, graph=graph)  # graph captured, state on the device
        for _ in range(4):
            model.step(graph=graph)
        dev.sync()
        e0, e1 = dev.event(), dev.event()
        dev.record(e0)
        for _ in range(steps):
            model.step(graph=graph)
        dev.record(e1)
        ms = dev.elapsed_ms(e0, e1) / steps
        dev.sync()
        out[f"batch{rows}"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(rows * 1e3 / ms, 1), "graph": graph,
                               "steps": steps, "prefill_128_ms": round(1e3 * float(np.median(prefill)), 2),
                               "weight_GB_per_s": round(weight_bytes / (ms * 1e-3) / 1e9, 1)}
        model.destroy()
        log(f"decode batch {rows}: {ms * 1e3:.0f} us/step")
    if with_cpu:
        from oracle import oracle
        try:
            cores = len(os.sched_getaffinity(0))
        except AttributeError:
            cores = os.cpu_count() or 1
        cores = max(1, min(cores, 16))
        variant = oracle.best_variant()
        oracle.set_threads(cores, variant)
        cpu = oracle.Llama(config, weights, variant)
        cpu.forward(list(rng.integers(0, config["vocab"], 8)), last_only=True)
        tokens, start = 0, time.perf_counter()
        token = 0
        while time.perf_counter() - start < cpu_seconds and tokens < 64:
            token = oracle.argmax(cpu.forward([token], last_only=True)[0])
            tokens += 1
        elapsed = time.perf_counter() - start
        out["cpu_baseline"] = {"ms_per_token": round(elapsed / tokens * 1e3, 1), "cores": cores, "kind": "port",
                               "sample": f"{tokens} greedy tokens after an 8-token prompt, batch 1; the oracle's "
                                         f"Llama forward ({variant} build, {cores} threads)"}
    return out


def batched_config3(dev, steps, warmup):
    """Config 3: Q4_1 batched-decode products, W [8192, 2048] and [2048, 8192]
    against B = 1, 2, 4, 8, 16 activation rows. One call is tmh_block_matmul
    over f32 x (the activation quantiser, then the lanes product); calls
    rotate through enough weight copies (>= 512 MB) that the 256 MB Infinity
    Cache cannot serve them; HIP events over `steps` calls. Bytes a call:
    weights + 4·B·K of x + 4·B·N of y."""
    import quant_host
    out = {"metric": "Q4_1 batched-decode product GB/s (config 3)", "unit": "GB/s", "n_gpus": 1, "steps": steps,
           "warmup": warmup, "higher_is_better": True, "dtype": "int8 dot + f32 fold",
           "data": "synthetic: W ~ N(0,0.02) quantised to Q4_1, x ~ N(0,1)", "shapes": {}}
    rng = np.random.default_rng(0x5EED0003)
    for n, k in ((8192, 2048), (2048, 8192)):
        host = quant_host.synthetic_weights("Q4_1", n, k, seed=0x5EED0003 + n)
        copies = max(2, math.ceil(2 * MALL_BYTES / host.nbytes))
        first = dev.from_array(host)
        ws = [first] + [dev.alloc(host.nbytes) for _ in range(copies - 1)]
        for w in ws[1:]:
            dev.copy(w, first, host.nbytes)
        for b in (1, 2, 4, 8, 16):
            x = dev.from_array(rng.normal(0.0, 1.0, (b, k)).astype(np.float32))
            dst = dev.alloc(4 * b * n)
            for i in range(warmup):
                dev.block_matmul("Q4_1", ws[i % copies], x, b, n, k, dst=dst)
            dev.sync()
            e0, e1 = dev.event(), dev.event()
            dev.record(e0)
            for i in range(steps):
                dev.block_matmul("Q4_1", ws[i % copies], x, b, n, k, dst=dst)
            dev.record(e1)
            dev.sync()
            ms = dev.elapsed_ms(e0, e1) / steps
            nbytes = host.nbytes + 4 * b * k + 4 * b * n
            out["shapes"][f"{n}x{k} B={b}"] = {"us_per_call": round(ms * 1e3, 2),
                                               "GB_per_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                               "hbm_peak_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
            x.release()
            dst.release()
        for w in ws:
            w.release()
    out["value"] = out["shapes"]["8192x2048 B=1"]["GB_per_s"]
    return out


def gemm_config4(dev, steps, warmup):
    """Config 4: the Q8_0 prefill GEMM at the Llama-1.7B shape, 512 tokens x
    K = 2048 against N = 2048 (attention projections) and N = 8192 (MLP
    up/gate). One call is tmh_block_matmul over f32 x (the activation
    quantiser, then the matrix-core kernel, k_matmul_mfma); timed with HIP
    events over `steps` calls. int8 work: 2 · 512 · 2048 · N ops a call."""
    import quant_host
    rows, k = 512, 2048
    rng = np.random.default_rng(0x5EED0004)
    x = dev.from_array(rng.normal(0.0, 1.0, (rows, k)).astype(np.float32))
    out = {"metric": "Q8_0 prefill GEMM int8 TOP/s (config 4, 512 tokens x K=2048)", "unit": "TOP/s",
           "n_gpus": 1, "steps": steps, "warmup": warmup, "higher_is_better": True, "dtype": "int8 dot + f32 fold",
           "data": "synthetic: W ~ N(0,0.02) quantised to Q8_0, x ~ N(0,1)", "shapes": {}}
    for n in (2048, 8192):
        w = dev.from_array(quant_host.synthetic_weights("Q8_0", n, k, seed=0x5EED0004 + n))
        dst = dev.alloc(4 * rows * n)
        for _ in range(warmup):
            dev.block_matmul("Q8_0", w, x, rows, n, k, dst=dst)
        dev.sync()
        e0, e1 = dev.event(), dev.event()
        dev.record(e0)
        for _ in range(steps):
            dev.block_matmul("Q8_0", w, x, rows, n, k, dst=dst)
        dev.record(e1)
        dev.sync()
        ms = dev.elapsed_ms(e0, e1) / steps
        ops = 2.0 * rows * k * n
        out["shapes"][f"N={n}"] = {"ms_per_call": round(ms, 4), "TOP_per_s": round(ops / (ms * 1e-3) / 1e12, 1),
                                   "int8_mfma_peak_frac": round(ops / (ms * 1e-3) / 5.0e15, 4)}
        w.release()
        dst.release()
    out["value"] = out["shapes"]["N=8192"]["TOP_per_s"]
    return out


class _View:
    """A buffer seen from a byte offset (a product's weights inside the packed buffer)."""

    def __init__(self, buf, offset):
        self.pointer = buf.pointer + offset
        self.bytesize = buf.bytesize - offset


if __name__ == "__main__":
    main()
