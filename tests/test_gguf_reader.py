"""The library's GGUF reader (tmh_gguf_open/tmh_gguf_tensor) without a GPU:
the directory of every fixture equals the test reader's (both follow
gguf.cr:289-329), and damaged files are errors, not faults."""
import glob
import os

import numpy as np
import pytest

import tensomite_hip as th
from gguf_io import BLOCK_BYTES, GGUF, write


def fixtures(golden):
    return sorted(glob.glob(os.path.join(golden, "*", "*.gguf")))


def test_directory_matches_the_test_reader(golden):
    files = fixtures(golden)
    assert len(files) >= 4
    for path in files:
        ref = GGUF(path)
        lib = th.GGUFFile(path)
        for name, (kind, shape, _) in ref.entries.items():
            got_kind, got_shape, got_bytes = lib.entry(name)
            count = int(np.prod(shape))
            want_bytes = count // 32 * BLOCK_BYTES[kind] if kind in BLOCK_BYTES else count * (4 if kind == "F32" else 2)
            assert (got_kind, got_shape, got_bytes) == (kind, shape, want_bytes), (path, name)
        with pytest.raises(th.DeviceError):
            lib.entry("no.such.tensor")
        lib.close()


def test_damaged_files_are_errors(tmp_path, golden):
    good = open(os.path.join(golden, "tiny_llama", "model-q8_0.gguf"), "rb").read()
    cases = {"magic": b"XXXX" + good[4:], "truncated": good[:200], "short": good[:10],
             "version": good[:4] + (9).to_bytes(4, "little") + good[8:], "data": good[:len(good) - 100]}
    for name, data in cases.items():
        path = tmp_path / f"{name}.gguf"
        path.write_bytes(data)
        with pytest.raises(th.DeviceError):
            th.GGUFFile(str(path))
    with pytest.raises(th.DeviceError):
        th.GGUFFile(str(tmp_path / "missing.gguf"))


def test_unknown_kind_is_a_dtype_error(tmp_path):
    path = str(tmp_path / "q4_k.gguf")
    write(path, [("general.architecture", "llama")], [("w", 12, [4, 256], bytes(4 * 144))])  # Q4_K
    with pytest.raises(th.DTypeError):
        th.GGUFFile(path)


def test_rows_not_whole_blocks_are_a_shape_error(tmp_path):
    path = str(tmp_path / "odd.gguf")
    write(path, [], [("w", "Q8_0", [2, 48], bytes(2 * 51))])
    with pytest.raises(th.ShapeError):
        th.GGUFFile(path)


def _one_tensor_file(tmp_path, name, alignment=32, metadata=()):
    path = str(tmp_path / name)
    write(path, list(metadata), [("w", "Q8_0", [2, 64], bytes(2 * 68))], alignment=alignment)
    return path


def test_offsets_that_wrap_are_errors(tmp_path):
    # A tensor offset near 2^64 that is a multiple of the alignment would
    # wrap to an in-file address when added to the data start; it must be
    # refused as a damaged file, never read (gguf.cr:320 refuses offsets
    # past the file).
    import struct
    path = _one_tensor_file(tmp_path, "ok.gguf")
    th.GGUFFile(path).close()
    data = bytearray(open(path, "rb").read())
    at = data.index(b"w", 24) + 1 + 4 + 2 * 8 + 4  # name, dims, shape, kind -> offset
    assert struct.unpack_from("<Q", data, at)[0] == 0
    for bad in (2 ** 64 - 32, 2 ** 64 - 4096, 2 ** 63, len(data)):
        struct.pack_into("<Q", data, at, bad)
        damaged = tmp_path / "wrapped.gguf"
        damaged.write_bytes(bytes(data))
        with pytest.raises(th.DeviceError):
            th.GGUFFile(str(damaged))


@pytest.mark.parametrize("alignment", [0, 3, 48, 1 << 21])
def test_unreasonable_alignment_is_an_error(tmp_path, alignment):
    path = _one_tensor_file(tmp_path, "align.gguf", metadata=[("general.alignment", alignment)])
    with pytest.raises(th.DeviceError):
        th.GGUFFile(path)


def test_larger_power_of_two_alignment_reads(tmp_path):
    path = _one_tensor_file(tmp_path, "align64.gguf", alignment=64, metadata=[("general.alignment", 64)])
    f = th.GGUFFile(path)
    assert f.entry("w") == ("Q8_0", [2, 64], 2 * 68)
    f.close()


def test_exported_llama_reads_back_in_hugging_face_order(tmp_path):
    # gguf_export.write_llama stores q/k rows in llama.cpp's rotary pairing;
    # taking them back in Llama.unpermute's order (llama.cr:226-235) gives the
    # decoder's rows, and every other tensor is stored as given.
    import gguf_export
    from llama_fixtures import random_llama, take_rows, unpermute_order
    config = dict(layers=2, width=128, heads=4, kv_heads=2, head_width=32, hidden=256, vocab=300, context=64,
                  eps=1e-5, theta=10000.0, kind="Q4_0")
    w = random_llama(config, seed=3, norm_jitter=0.1)
    path = str(tmp_path / "llama.gguf")
    gguf_export.write_llama(path, config, w)
    g = GGUF(path)
    rb = 128 // 32 * 18
    assert g.metadata["llama.block_count"] == 2 and g.metadata["llama.attention.head_count_kv"] == 2
    assert np.array_equal(g.raw("token_embd.weight"), w["embed"])
    for l in range(2):
        q = take_rows(g.raw(f"blk.{l}.attn_q.weight"), rb, unpermute_order(128, 4))
        k = take_rows(g.raw(f"blk.{l}.attn_k.weight"), rb, unpermute_order(64, 2))
        v = g.raw(f"blk.{l}.attn_v.weight")
        assert np.array_equal(np.concatenate([q, k, v]), w["qkv"][l])
        gu = np.concatenate([g.raw(f"blk.{l}.ffn_gate.weight"), g.raw(f"blk.{l}.ffn_up.weight")])
        assert np.array_equal(gu, w["gate_up"][l])
        assert np.array_equal(g.f32(f"blk.{l}.ffn_norm.weight"), w["ffn_norm"][l])
    lib = th.GGUFFile(path)
    assert lib.entry("blk.1.attn_q.weight") == ("Q4_0", [128, 128], 128 * rb)
    lib.close()


def test_exported_config1_is_bench_bytes(tmp_path):
    import gguf_export
    import quant_host
    [path] = gguf_export.export_configs(str(tmp_path), configs=(1,))
    g = GGUF(path)
    assert g.entries["c_attn.weight"][:2] == ("Q8_0", [2304, 768])
    assert np.array_equal(g.raw("c_attn.weight"), quant_host.synthetic_weights("Q8_0", 2304, 768, seed=0x5EED0001))
