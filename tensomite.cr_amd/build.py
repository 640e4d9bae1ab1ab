"""Builds libtensomite_hip.so in-tree for gfx950 with hipcc.

Flags that the results depend on:
  -ffp-contract=off       no fused multiply-add: each product and sum rounds
                          once, as the reference's host code does
  (no -ffast-math)        IEEE f32 division, no reassociation of the
                          ordered fold
  -Xclang -target-feature -Xclang -packed-fp32-ops
                          no packed f32 arithmetic in generated code
  -mllvm -amdgpu-mfma-vgpr-form=1
                          MFMA results in VGPRs, not AGPRs: the matrix-core
                          kernels read every result with VALU operations,
                          and an AGPR would cost a v_accvgpr_read each
  -mllvm -amdgpu-kernarg-preload-count=16
                          the first kernel arguments arrive in SGPRs when a
                          wave starts (gfx950 kernarg preloading) instead of
                          through a scalar load: the decode kernels are chains
                          of latencies from their first instruction (measured,
                          one box, alternating builds: 1.7B decode batch 1
                          831 -> 806 us/step, config 2 15.56 -> 15.33 us)
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libtensomite_hip.so")
SOURCES = [os.path.join(HERE, "csrc", name) for name in ("tmh_runtime.hip", "tmh_kernels.hip", "tmh_decode.hip", "tmh_llama.hip", "tmh_gguf.hip", "tmh_quant_host.hip")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"),
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Compiles every source to an object in parallel (the same flags), then
    links the shared library; always recompiles."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objects = [os.path.join(objdir, os.path.basename(src) + ".o") for src in SOURCES]
    jobs = [[HIPCC, *compile_flags, "-c", src, "-o", obj] for src, obj in zip(SOURCES, objects)]
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd in jobs]:
            f.result()
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-fno-gpu-rdc", *objects, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
