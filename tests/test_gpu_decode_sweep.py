"""A seeded sweep of small Llama shapes through the device decoder: head
widths, grouped kv heads, widths and hidden sizes (rows of block counts the
kernels handle differently), formats, rows decoded together and prompt
lengths. Every row's greedy tokens, from a captured graph, against the CPU
oracle's Llama (llama.cr:256-303, generative.cr:155-190), and each row's
last prefill logits bit for bit.

The fixed decoder tests name the shapes the fused kernels were built
around; this sweep reaches the ones in between.
"""
import sys

import numpy as np
import pytest

from llama_fixtures import random_llama
from oracle import oracle
import tensomite_hip as th

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return th.HIPDevice(0)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


CASES = 30


def configs():
    rng = np.random.default_rng(333)
    out = []
    for i in range(CASES):
        hw = int(rng.choice([16, 32, 64, 64, 128]))
        heads = int(rng.choice([2, 4, 8]))
        kv = int(rng.choice([d for d in (1, 2, 4, 8) if heads % d == 0]))
        width = int(rng.choice([128, 192, 256, 512, 1024]))
        hidden = int(rng.choice([256, 352, 512, 768, 1536]))
        kind = ["Q8_0", "Q4_0", "Q4_1"][i % 3]
        rows = int(rng.choice([1, 1, 2, 3, 5, 8]))
        c = dict(layers=int(rng.choice([1, 2])), width=width, heads=heads, kv_heads=kv, head_width=hw,
                 hidden=hidden, vocab=int(rng.choice([300, 512])), context=128, eps=1e-5, theta=10000.0, kind=kind)
        prompts = [list(rng.integers(0, c["vocab"], int(rng.integers(1, 40)))) for _ in range(rows)]
        out.append((c, prompts))
    return out


@pytest.mark.parametrize("case", range(CASES))
def test_random_decoder_shapes(dev, case):
    config, prompts = configs()[case]
    steps = 10
    say("decoder sweep", case, config, "rows", len(prompts), "prompts", [len(p) for p in prompts])
    weights = random_llama(config, seed=400 + case, norm_jitter=0.1)
    cpu = oracle.Llama(config, weights)
    capacity = max(len(p) for p in prompts) + steps + 8
    gpu = th.HIPLlama(dev, config, weights, rows=len(prompts), capacity=capacity, max_tokens=48)
    for r, p in enumerate(prompts):
        got = gpu.forward(p, row=r, last_only=True)
        want = oracle.Llama(config, weights).forward(p, last_only=True)
        assert np.array_equal(bits(got), bits(want)), ("prefill logits", r)
    tokens = gpu.generate(steps, graph=True)
    for r, p in enumerate(prompts):
        assert list(tokens[r]) == cpu.generate(p, steps), ("tokens", r)
