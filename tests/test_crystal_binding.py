"""The committed Crystal binding (tensomite.cr_amd/crystal/src/tensomite/hip/lib.cr)
against the C header: one `fun` per declared entry point, with the same
number of arguments and Crystal types that match the C types (UInt64 for
device addresses and byte sizes, UInt32/Int32 as declared). There is no
Crystal compiler in this image; this keeps the binding honest by reading."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tensomite_hip.h")
LIB = os.path.join(ROOT, "tensomite.cr_amd", "crystal", "src", "tensomite", "hip", "lib.cr")
DEVICE = os.path.join(ROOT, "tensomite.cr_amd", "crystal", "src", "tensomite", "hip.cr")

C_TO_CRYSTAL = {
    "uint64_t": "UInt64", "int64_t": "Int64", "uint32_t": "UInt32", "int32_t": "Int32", "int": "Int32",
    "float": "Float32", "double": "Float64", "char": "UInt8", "uint8_t": "UInt8", "void": "Void",
    "tmh_device_info": "DeviceInfo", "tmh_counters": "Counters", "tmh_product": "Product",
    "tmh_llama_config": "LlamaConfig", "tmh_llama_weights": "LlamaWeights",
}


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|const char\*)\s+(tmh_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        types = []
        for a in args:
            a = re.sub(r"\bconst\b", "", a).strip()
            a = re.sub(r"\s+\w+(\[\d+\])?$", lambda mm: "*" if mm.group(1) else "", a).strip()
            stars = a.count("*")
            base = a.replace("*", "").strip()
            types.append(C_TO_CRYSTAL[base] + "*" * stars)
        out[m.group(1)] = types
    return out


def crystal_functions():
    text = open(LIB).read()
    out = {}
    for m in re.finditer(r"fun\s+\w+\s*=\s*(tmh_[a-z0-9_]+)\s*(\(([^)]*)\))?\s*:", text, flags=re.S):
        args = [a.strip() for a in (m.group(3) or "").split(",") if a.strip()]
        types = []
        for a in args:
            name, typ = [s.strip() for s in a.split(":", 1)]
            typ = typ.replace("DevicePtr", "UInt64")
            types.append(typ)
        out[m.group(1)] = types
    return out


def test_every_entry_point_is_bound_once_with_matching_types():
    c = header_functions()
    cr = crystal_functions()
    import tensomite_hip as th
    assert sorted(c) == sorted(th.SIGNATURES)  # the regex saw every declaration
    assert sorted(cr) == sorted(c)
    for name, types in c.items():
        assert len(cr[name]) == len(types), name
        for want, got in zip(types, cr[name]):
            # a device address is uint64_t in C and DevicePtr (UInt64) in Crystal
            assert got == want, (name, want, got)


def test_constants_match_header():
    text = open(HEADER).read()
    consts = dict((m.group(1), int(m.group(2))) for m in re.finditer(r"#define TMH_(\w+) (\d+)\b", text))
    lib = open(LIB).read()
    for name in ("SUCCESS", "ERROR_SHAPE", "ERROR_DTYPE", "ERROR_NO_KERNELS", "ERROR_EXECUTION", "ERROR_NOT_READY",
                 "ERROR_SCRATCH_LIMIT"):
        m = re.search(rf"\b{name}\s*=\s*(\d+)", lib)
        assert m and int(m.group(1)) == consts[name], name


def test_device_calls_only_bound_functions():
    used = set(re.findall(r"LibTensomiteHIP\.(\w+)\(", open(DEVICE).read()))
    bound = set(re.findall(r"fun\s+(\w+)\s*=", open(LIB).read()))
    assert used and used <= bound, used - bound
