"""Several host threads on one device at once, through the library's C ABI,
whose contract is that any thread may call (include/tensomite_hip.h): each
thread allocates, uploads, multiplies (one row, a few rows, many rows: the
one-row, lanes, few-rows and matrix-core kernels), downloads and gives
buffers back, some of them allocated by another thread, and syncs, which
drains the retired list into the pool, in a loop. Every product bit for bit
against the oracle's Quant.matmul (quant.cr:155-182). The library serialises
launches on its one stream; buffers one thread gives back are taken again by
the others through the pool (CUDA#alloc / #retire / #sync, cuda.cr:339-353,
439-454). And a decoder capturing its step graph while another thread's
products run on the same device: neither's work lands in the other's.
"""
import queue
import sys
import threading

import numpy as np
import pytest

from llama_fixtures import random_llama
from oracle import oracle
import tensomite_hip as th

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 30
# (format, rows, n, k) per thread
SHAPES = [("Q4_0", 1, 384, 1024), ("Q8_0", 3, 200, 512), ("Q4_1", 12, 256, 1024), ("Q4_0", 40, 192, 512)]


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_threads_share_one_device():
    dev = th.HIPDevice(0)
    rng = np.random.default_rng(1300)
    cases = []
    for fmt, rows, n, k in SHAPES:
        wq = oracle.quantize(fmt, rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02))
        x = rng.standard_normal(rows * k, dtype=np.float32)
        cases.append((fmt, rows, n, k, wq, x, oracle.matmul(fmt, x, wq, rows, n, k)))
    handed = queue.Queue()  # output buffers, released by whichever thread takes them
    failures = []
    before = dev.counters()

    def work(t):
        fmt, rows, n, k, wq, x, want = cases[t]
        try:
            for r in range(ROUNDS):
                wbuf, xbuf = dev.from_array(wq), dev.from_array(x)
                out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k)
                got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
                if not np.array_equal(bits(got), bits(want)):
                    failures.append((t, r, "bits"))
                wbuf.release()
                xbuf.release()
                handed.put(out)
                try:
                    handed.get_nowait().release()
                except queue.Empty:
                    pass
                if r % 5 == 4:
                    dev.sync()
        except Exception as e:  # reported below, on the test's thread
            failures.append((t, "raised", repr(e)))

    say("threads", THREADS, "rounds", ROUNDS, SHAPES)
    threads = [threading.Thread(target=work, args=(t,)) for t in range(THREADS)]
    for th_ in threads:
        th_.start()
    for th_ in threads:
        th_.join(timeout=240)
    assert not any(th_.is_alive() for th_ in threads), "a thread did not finish"
    while not handed.empty():
        handed.get_nowait().release()
    dev.sync()
    after = dev.counters()
    assert not failures, failures[:5]
    assert after["pool_hits"] > before["pool_hits"]  # memory given back by one thread taken by another call


def test_products_beside_a_decoder_capturing_its_step():
    # The decoder captures its step graph on a stream of the model's own, so
    # another thread's products on the device's stream meanwhile run at once
    # and are not recorded into the graph: every product and every decoded
    # token the CPU's (llama.cr:256-303, generative.cr:155-190).
    dev = th.HIPDevice(0)
    config = dict(layers=2, width=256, heads=4, kv_heads=2, head_width=64, hidden=512, vocab=300, context=128,
                  eps=1e-5, theta=10000.0, kind="Q4_0")
    weights = random_llama(config, seed=1400, norm_jitter=0.1)
    prompt = [int(v) for v in np.random.default_rng(1401).integers(0, 300, 20)]
    steps = 12
    want_tokens = oracle.Llama(config, weights).generate(prompt, steps)
    rng = np.random.default_rng(1402)
    fmt, rows, n, k = "Q4_1", 3, 320, 512
    wq = oracle.quantize(fmt, rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(rows * k, dtype=np.float32)
    want = oracle.matmul(fmt, x, wq, rows, n, k)
    stop = threading.Event()
    failures, done = [], [0]

    def products():
        try:
            while not stop.is_set():
                wbuf, xbuf = dev.from_array(wq), dev.from_array(x)
                out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k)
                got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
                if not np.array_equal(bits(got), bits(want)):
                    failures.append(("product", done[0]))
                for b in (wbuf, xbuf, out):
                    b.release()
                done[0] += 1
        except Exception as e:
            failures.append(("product raised", repr(e)))

    say("decoder captures beside products")
    worker = threading.Thread(target=products)
    worker.start()
    try:
        for i in range(6):
            model = th.HIPLlama(dev, config, weights, rows=1, capacity=64, max_tokens=32)
            model.forward(prompt, row=0, last_only=True)
            tokens = model.generate(steps, graph=True)[0]  # the first step captures the graph
            if list(tokens) != want_tokens:
                failures.append(("tokens", i, list(tokens)))
            model.destroy()
    finally:
        stop.set()
        worker.join(timeout=120)
    dev.sync()
    assert not worker.is_alive()
    assert not failures, failures[:5]
    assert done[0] > 0

