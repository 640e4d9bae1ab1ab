"""Writes tests/golden/config5/expected.json: BASELINE config 5's greedy
tokens from the CPU oracle (oracle/tmq_llama.c, the restatement of the
reference's host forward and Generative#generate with Sampler.greedy,
generative.cr:177-190, sampler.cr:35-36).

The model: SmolLM2-1.7B's shape (24 layers, width 2048, 32 heads of 64,
hidden 8192, vocab 49152, RoPE theta 10000, RMSNorm eps 1e-5, tied head),
every matrix W ~ N(0, 0.02) quantised to Q4_0 by quant_host.synthetic_llama
(seed 0x5EED0005), norms 1. Eight prompts of 128 ids from
default_rng(0x5EED0005 + 1); for each, 256 greedy tokens and the bits of
the last prefill logits (as a sha256 and the 16 largest, with indices).
Batch 1 runs prompt 0; batch 8 runs prompts 0..7 as one batch of rows, each
with the tokens of its prompt alone (the reference's row alone == in batch).

The weights' sha256 (every matrix's bytes in the decoder's order) is
recorded so a GPU test can show it made the same bytes before comparing.

    python tests/golden/config5/make_config5.py   # ~10 minutes on 8 cores
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(os.path.dirname(HERE)))
for p in (ROOT, os.path.join(ROOT, "tensomite.cr_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import quant_host  # noqa: E402
from oracle import oracle  # noqa: E402

SEED = 0x5EED0005
PROMPT = 128
STEPS = 256
ROWS = 8


def config():
    return dict(quant_host.SMOLLM2_1P7B)


def weights():
    return quant_host.synthetic_llama(config(), SEED)


def weights_sha256(w) -> str:
    h = hashlib.sha256()
    h.update(w["embed"].tobytes())
    for key in ("qkv", "o", "gate_up", "down"):
        for m in w[key]:
            h.update(m.tobytes())
    return h.hexdigest()


def prompts():
    rng = np.random.default_rng(SEED + 1)
    return [[int(t) for t in rng.integers(0, config()["vocab"], PROMPT)] for _ in range(ROWS)]


def logits_summary(logits: np.ndarray) -> dict:
    v = np.ascontiguousarray(logits, dtype=np.float32)
    top = np.argsort(-v, kind="stable")[:16]
    return {"sha256": hashlib.sha256(v.view(np.uint32).tobytes()).hexdigest(),
            "top_ids": [int(i) for i in top], "top_bits": [int(b) for b in v[top].view(np.uint32)]}


def main():
    variant = oracle.best_variant()
    cores = len(os.sched_getaffinity(0))
    oracle.set_threads(cores, variant)
    t0 = time.perf_counter()
    w = weights()
    print(f"weights in {time.perf_counter() - t0:.1f} s", flush=True)
    out = {"seed": SEED, "prompt_length": PROMPT, "steps": STEPS, "config": config(),
           "weights_sha256": weights_sha256(w), "prompts": prompts(), "rows": []}
    cpu = oracle.Llama(config(), w, variant)
    for r, prompt in enumerate(out["prompts"]):
        t = time.perf_counter()
        cpu.reset()
        logits = cpu.forward(prompt, last_only=True)[0]
        summary = logits_summary(logits)
        tokens = []
        for i in range(STEPS):
            token = oracle.argmax(logits)
            tokens.append(token)
            if i < STEPS - 1:
                logits = cpu.forward([token], last_only=True)[0]
        out["rows"].append({"prefill_logits": summary, "tokens": tokens})
        print(f"row {r}: {time.perf_counter() - t:.1f} s, first tokens {tokens[:8]}", flush=True)
    with open(os.path.join(HERE, "expected.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
