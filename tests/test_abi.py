"""The C ABI without a GPU: the library loads, exports every entry point
include/tensomite_hip.h declares, the binding's signatures cover them all,
and error codes have names. No compute call is made here."""
import ctypes
import os
import re

import pytest

import tensomite_hip as th

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "tensomite_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = th.library()
    names = declared()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_binding_covers_the_header_exactly():
    assert sorted(th.SIGNATURES) == declared()


def test_error_names():
    lib = th.library()
    for code, name in ((0, "TMH_SUCCESS"), (1001, "TMH_ERROR_SHAPE"), (1002, "TMH_ERROR_DTYPE"),
                       (1003, "TMH_ERROR_NO_KERNELS"), (1005, "TMH_ERROR_EXECUTION")):
        assert lib.tmh_error_name(code).decode() == name
        assert lib.tmh_error_string(code)
    assert lib.tmh_error_name(2).decode().startswith("hip")  # a HIP code passes through


def test_row_bytes_and_kinds():
    # DType#bytes_for (dtype.cr:221-244), quant_spec.cr:100-107
    assert th.row_bytes("Q8_0", 64) == 68
    assert th.row_bytes("Q4_0", 64) == 36
    assert th.row_bytes("Q4_1", 32) == 20
    with pytest.raises(th.ShapeError):
        th.row_bytes("Q4_0", 48)
    with pytest.raises(th.DTypeError):
        th.kind_of("F32")


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict((m.group(1), int(m.group(2))) for m in re.finditer(r"#define (TMH_\w+) (\d+)", text))
    assert consts["TMH_Q8_0"] == th.Q8_0 and consts["TMH_Q4_0"] == th.Q4_0 and consts["TMH_Q4_1"] == th.Q4_1
    assert consts["TMH_ERROR_EXECUTION"] == th.ERROR_EXECUTION
    assert consts["TMH_ERROR_SHAPE"] == th.ERROR_SHAPE
    for name, value in th.MODES.items():
        assert consts["TMH_MODE_" + name.upper()] == value
