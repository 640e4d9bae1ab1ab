"""BASELINE config 5 exactly as stated, on the GPU against the CPU oracle.

A random-init SmolLM2-1.7B-shaped Llama (24 layers, width 2048, 32 heads of
64, hidden 8192, vocab 49152, RoPE theta 10000, RMSNorm eps 1e-5, tied head),
every matrix W ~ N(0, 0.02) quantised to Q4_0 (quant_host.synthetic_llama,
seed 0x5EED0005); prompts of 128 random ids; 256 greedy steps
(Generative#generate with Sampler.greedy, generative.cr:177-190,
sampler.cr:35-36) from a captured HIP graph with an f32 KV cache of 2048
positions, at batch 1 and at batch 8 with every row checked. The CPU's
tokens and last prefill logits come from tests/golden/config5/expected.json,
written by the oracle (make_config5.py beside it); the weights' sha256 shows
the GPU got the same bytes, and one row is re-run live through the oracle on
this host to tie the fixture to it.
"""
import json
import os
import sys

import pytest

import tensomite_hip as th
from oracle import oracle

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden", "config5"))
import make_config5 as fixture  # noqa: E402


def say(*args):
    print(*args, flush=True)


@pytest.fixture(scope="module")
def expected():
    with open(os.path.join(HERE, "golden", "config5", "expected.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def model_weights(expected):
    say("config 5 weights ...")
    w = fixture.weights()
    assert fixture.weights_sha256(w) == expected["weights_sha256"]
    return w


@pytest.fixture(scope="module")
def dev():
    return th.HIPDevice(0)


def test_fixture_matches_its_recipe(expected):
    assert expected["config"] == fixture.config()
    assert expected["prompts"] == fixture.prompts()
    assert expected["prompt_length"] == 128 and expected["steps"] == 256
    assert len(expected["rows"]) == 8 and all(len(r["tokens"]) == 256 for r in expected["rows"])


def run_rows(dev, weights, prompts, steps, graph=True):
    config = fixture.config()
    model = th.HIPLlama(dev, config, weights, rows=len(prompts), capacity=2048, max_tokens=128)
    summaries = []
    for r, p in enumerate(prompts):
        summaries.append(fixture.logits_summary(model.forward(p, row=r, last_only=True)[0]))
    tokens = model.generate(steps, graph=graph)
    lengths = [model.length(r) for r in range(len(prompts))]
    model.destroy()
    return summaries, tokens, lengths


@pytest.mark.parametrize("graph", [True, False])
def test_batch1_greedy_tokens_equal_cpu(dev, model_weights, expected, graph):
    say("config 5 batch 1, graph", graph)
    summaries, tokens, lengths = run_rows(dev, model_weights, expected["prompts"][:1], 256, graph)
    row = expected["rows"][0]
    assert summaries[0] == row["prefill_logits"]
    assert list(tokens[0]) == row["tokens"]
    assert lengths == [128 + 255]


def test_batch8_greedy_tokens_equal_cpu_every_row(dev, model_weights, expected):
    say("config 5 batch 8")
    summaries, tokens, lengths = run_rows(dev, model_weights, expected["prompts"], 256)
    for r, row in enumerate(expected["rows"]):
        assert summaries[r] == row["prefill_logits"], r
        assert list(tokens[r]) == row["tokens"], r
    assert lengths == [128 + 255] * 8


def test_fixture_row_equals_live_oracle(model_weights, expected):
    # The last row's prefill logits and first 24 tokens, recomputed by the
    # oracle on this host's cores.
    say("config 5 live oracle row 7")
    variant = oracle.best_variant()
    oracle.set_threads(len(os.sched_getaffinity(0)), variant)
    cpu = oracle.Llama(fixture.config(), model_weights, variant)
    prompt = expected["prompts"][7]
    logits = cpu.forward(prompt, last_only=True)[0]
    assert fixture.logits_summary(logits) == expected["rows"][7]["prefill_logits"]
    tokens = []
    for i in range(24):
        tokens.append(oracle.argmax(logits))
        logits = cpu.forward([tokens[-1]], last_only=True)[0]
    assert tokens == expected["rows"][7]["tokens"][:24]


def test_exported_gguf_loads_to_the_same_tokens(dev, model_weights, expected, tmp_path):
    # The config-5 weights written as a llama.cpp GGUF (what bench.py
    # --write-gguf gives the reference), loaded back by Llama.load's path
    # (tmh_llama_load_gguf: q/k unpermuted and projections merged while
    # staging): prompt 0's tokens equal the CPU's.
    import gguf_export
    say("config 5 through GGUF")
    path = str(tmp_path / "config5.gguf")
    gguf_export.write_llama(path, fixture.config(), model_weights)
    model = th.HIPLlama.load_gguf(dev, path, rows=1, capacity=2048, max_tokens=128)
    assert model.config["layers"] == 24 and model.config["kind"] == "Q4_0"
    logits = model.forward(expected["prompts"][0], last_only=True)[0]
    assert fixture.logits_summary(logits) == expected["rows"][0]["prefill_logits"]
    assert list(model.generate(256)[0]) == expected["rows"][0]["tokens"]
    model.destroy()
