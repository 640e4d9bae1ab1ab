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


C_FIELD = {"uint64_t": "UInt64", "int64_t": "Int64", "uint32_t": "UInt32", "int32_t": "Int32", "float": "Float32",
           "double": "Float64", "char": "UInt8"}


def header_structs():
    """typedef struct tmh_x { fields } tmh_x; -> {x: [(name, Crystal type)]}"""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef struct tmh_(\w+)\s*\{(.*?)\}\s*tmh_\1;", text, flags=re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = decl.strip()
            if not decl:
                continue
            f = re.match(r"(?:const\s+)?(\w+)\s*(\*?)\s*(.+)$", decl)
            assert f, decl
            base, star, names = f.groups()
            for item in names.split(","):  # uint64_t a, b, c;
                g = re.match(r"\s*(\w+)(?:\[(\d+)\])?\s*$", item)
                assert g, decl
                typ = C_FIELD.get(base, base) + star
                if g.group(2):
                    typ = f"{typ}[{g.group(2)}]"
                fields.append((g.group(1), typ))
        out[m.group(1)] = fields
    return out


def crystal_structs():
    text = open(LIB).read()
    out = {}
    for m in re.finditer(r"struct (\w+)\n(.*?)\n\s*end", text, flags=re.S):
        fields = []
        for line in m.group(2).splitlines():
            f = re.match(r"\s*(\w+)\s*:\s*(.+?)\s*$", line)
            if f:
                fields.append((f.group(1), f.group(2).replace("DevicePtr", "UInt64")))
        out[m.group(1)] = fields
    return out


def test_structs_match_header_field_by_field():
    # The library writes these structs (tmh_counters_get, tmh_device_info_get)
    # or reads them (plans, the decoder): Crystal's and Python's layouts must
    # be the header's, field for field.
    import tensomite_hip as th

    crystal = crystal_structs()
    names = {"device_info": "DeviceInfo", "counters": "Counters", "product": "Product"}
    structs = header_structs()
    for c_name, cr_name in names.items():
        want = structs[c_name]
        assert [f for f, _ in crystal[cr_name]] == [f for f, _ in want], c_name
        for (field, wt), (_, gt) in zip(want, crystal[cr_name]):
            assert gt == wt, (c_name, field, wt, gt)
        py = getattr(th, cr_name)
        assert [f for f, _ in py._fields_] == [f for f, _ in want], c_name
    assert [f for f, _ in structs["counters"]][-1] == "launches"


# CUDA::Profile's members (src/tensomite/cuda.cr:256-303), which the
# reference's profiling benches and ProfileReport read.
PROFILE_MEMBERS = ["per_kernel", "kernels", "host_ops", "launch", "alloc", "transfer", "wait", "launches", "uploads",
                   "downloads", "allocations", "pool_misses", "frees", "shapes"]


def test_device_has_the_profile_and_counter_surface():
    # HIP::Profile with every member of CUDA::Profile and its report; HIP
    # with #profile, #device_bytes, #buffer_pool (limit, held, hits, misses)
    # and .available? (cuda.cr:208-222, 305-306, 986-988; cuda/report.cr).
    text = open(DEVICE).read()
    profile = re.search(r"class Profile\n(.*?)\n    end\n", text, flags=re.S)
    assert profile, "no HIP::Profile"
    body = profile.group(1)
    for member in PROFILE_MEMBERS:
        assert re.search(rf"(getter\??|property)\s+{member}\b", body), member
    assert "def self.report(" in body and "ProfileReport.new(" in body
    assert re.search(r"property profile : Profile\? = nil", text)
    for method in ("def device_bytes : Int64", "def buffer_pool : Pool", "def self.available? : Bool",
                   "def limit : Int64", "def held : Int64", "def hits : Int64", "def misses : Int64"):
        assert method in text, method
    # every profiled path updates its counters
    for counter in ("profile.alloc +=", "profile.allocations += 1", "profile.pool_misses += 1",
                    "profile.uploads += 1", "profile.downloads += 1", "profile.transfer +=", "profile.wait +=",
                    "profile.frees +=", "profile.launch +=", "profile.launches +=", "add_host_op(", "add_kernel("):
        assert counter in text, counter
