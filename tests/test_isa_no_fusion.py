"""The built library's gfx950 code keeps every multiply and add of the
reference's expressions separately rounded: the analogue of the reference's
check that CUDA compiles `a * b + c` to a multiply and an add, never one
fused multiply-add (spec/cuda_spec.cr:34-40). Runs on the CPU over this
build's own code object (the AMD assembly of code built here):

* no packed f32 operations and no fused or mixed-precision multiply-add
  forms (v_fmac/v_mac/v_mad_f32, v_fma_mix, v_pk_fma/mul/add_f32) at all;
* every fused f32 multiply-add (v_fma_f32, v_fmac_f32, v_fmamk_f32,
  v_fmaak_f32) inside a division expansion: the correctly rounded f32
  division (v_div_scale / v_rcp / v_div_fmas / v_div_fixup) or the integer
  division of index arithmetic (a float reciprocal, v_trunc, v_cvt, then the
  remainder by v_fma) -- the divisions' own algorithms, not a fusion of the
  reference's operations.

The one exception is the matrix-core kernel's unordered form
(k_matmul_mx<KIND, true>, TMH_MODE_UNORDERED), which folds each block with
one fused multiply-add on purpose and makes no bit-exact claim.
"""
import bisect
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tensomite.cr_amd", "libtensomite_hip.so")
TOOLS = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

# objdump names the encoding after the operation (v_fmac_f32_e32, v_rcp_f32_e64)
ENCODING = r"(_e32|_e64|_e64_dpp|_dpp|_sdwa)?$"
FORBIDDEN = re.compile(r"^v_(pk_fma_f32|pk_mul_f32|pk_add_f32|mac_f32|mad_f32|fma_mix\w*|mad_mix\w*|"
                       r"fma_legacy_f32|fmac_legacy_f32|mad_legacy_f32|mac_legacy_f32)" + ENCODING)
FMA = re.compile(r"^v_(fma_f32|fmac_f32|fmamk_f32|fmaak_f32)" + ENCODING)
DIVISION = re.compile(r"^v_(div_scale_f32|div_fmas_f32|div_fixup_f32|rcp_f32|rcp_iflag_f32)" + ENCODING)
INT_DIVISION = re.compile(r"^v_(cvt_u32_f32|cvt_i32_f32|trunc_f32)" + ENCODING)
# k_matmul_mx<KIND, true>: the unordered fold
UNORDERED = re.compile(r"^_ZN3tmh11k_matmul_mxILi\dELb1EE")


def code_ops(lib, tmp_path):
    """(function, mnemonic) of every gfx950 instruction in `lib`'s offload bundles."""
    for tool in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(TOOLS, tool)):
            pytest.skip(f"{tool} is not installed")
    fat = tmp_path / "lib.fat"
    subprocess.run([os.path.join(TOOLS, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", lib], check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundles in the library"
    ops = []
    for n, s in enumerate(starts):
        bundle = tmp_path / f"b{n}.fat"
        bundle.write_bytes(data[s:starts[n + 1] if n + 1 < len(starts) else len(data)])
        code = tmp_path / f"b{n}.co"
        r = subprocess.run([os.path.join(TOOLS, "clang-offload-bundler"), "--unbundle", "--type=o",
                            f"--input={bundle}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={code}"],
                           capture_output=True)
        if r.returncode != 0 or not code.exists() or code.stat().st_size == 0:
            continue
        text = subprocess.run([os.path.join(TOOLS, "llvm-objdump"), "-d", "--mcpu=gfx950", str(code)],
                              capture_output=True, text=True, check=True).stdout
        function = None
        for line in text.splitlines():
            head = re.match(r"^[0-9a-f]+ <(.+)>:", line)
            if head:
                function = head.group(1)
            elif re.match(r"^\s+[sv]_", line):
                ops.append((function, line.split()[0]))
    return ops


def violations(ops):
    """Forbidden forms present; each fused multiply-add outside a division
    expansion, as (function, neighbouring instructions); the fused
    multiply-adds counted."""
    names = [o for _, o in ops]
    bad = sorted({o for o in names if FORBIDDEN.match(o)})
    fma = [i for i, o in enumerate(names) if FMA.match(o)]
    div = [i for i, o in enumerate(names) if DIVISION.match(o)]
    idiv = [i for i, o in enumerate(names) if INT_DIVISION.match(o)]

    def near(marks, i, before, after):
        j = bisect.bisect_left(marks, i - before)
        return j < len(marks) and marks[j] <= i + after

    outside = [(ops[i][0], names[max(0, i - 4):i + 2]) for i in fma
               if not near(div, i, 24, 24) and not near(idiv, i, 4, 0)]
    return bad, outside, len(fma)


def test_no_fused_or_packed_float_arithmetic(tmp_path):
    if not os.path.exists(LIB):
        pytest.skip("the library is not built")
    ops = code_ops(LIB, tmp_path)
    assert len(ops) > 100000, "the gfx950 code object was not found"
    bad, outside, fmas = violations(ops)
    assert not bad, bad
    assert fmas, "no division expansions found"
    unordered = {f for f, _ in outside if UNORDERED.match(f)}
    # the unordered kernels fuse (so the exemption names live code), nothing else does
    assert len(unordered) == 3, unordered
    assert not [o for o in outside if not UNORDERED.match(o[0])], outside[:3]


def test_the_check_finds_a_fused_multiply_add(tmp_path):
    # a * b + c compiled with contraction on: the check must report it
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc is not installed")
    src = tmp_path / "madd.hip"
    src.write_text("#include <hip/hip_runtime.h>\n"
                   "__global__ void madd(const float* a, const float* b, const float* c, float* d) {\n"
                   "    const int i = threadIdx.x;\n"
                   "    d[i] = a[i] * b[i] + c[i];\n"
                   "}\n")
    lib = tmp_path / "libmadd.so"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-ffp-contract=fast", "-fPIC", "-shared", str(src), "-o",
                    str(lib)], check=True, capture_output=True)
    bad, outside, fmas = violations(code_ops(str(lib), tmp_path))
    assert not bad and outside and outside[0][1][-2].startswith("v_fmac_f32"), (bad, outside)
