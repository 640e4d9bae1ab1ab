"""ctypes binding of the CPU oracle (oracle/tmq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product (tensomite.cr_amd/).

Functions mirror the reference's `Quant` module (src/tensomite/quant.cr) and
`F16` (src/tensomite/f16.cr); numpy arrays in and out.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

Q8_0, Q4_0, Q4_1 = 0, 1, 2
KINDS = {"Q8_0": Q8_0, "Q4_0": Q4_0, "Q4_1": Q4_1}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20}


def build() -> None:
    """Compiles the four oracle builds (portable, x86-64-v3, x86-64-v4, x86-64-v4 with VNNI)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def _cpu_flags() -> set:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def variant_runs(variant: str) -> bool:
    """Whether the host CPU can run an oracle build."""
    flags = _cpu_flags()
    v4 = {"avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd"} <= flags
    return {"portable": True, "v3": {"avx2", "fma", "bmi2", "f16c", "movbe"} <= flags, "v4": v4,
            "vnni": v4 and "avx512_vnni" in flags}[variant]


def best_variant() -> str:
    """The widest oracle build the host CPU can run: vnni (AVX-512 with VNNI), v4 (AVX-512), v3 (AVX2) or
    portable."""
    flags = _cpu_flags()
    if {"avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd"} <= flags:
        return "vnni" if "avx512_vnni" in flags else "v4"
    if {"avx2", "fma", "bmi2", "f16c", "movbe"} <= flags:
        return "v3"
    return "portable"


_LIBS: dict = {}


def lib(variant: str = "portable") -> ctypes.CDLL:
    if variant in _LIBS:
        return _LIBS[variant]
    name = {"portable": "libtmq_oracle.so", "v3": "libtmq_oracle_v3.so", "v4": "libtmq_oracle_v4.so",
            "vnni": "libtmq_oracle_vnni.so"}[variant]
    path = os.path.join(HERE, name)
    if not os.path.exists(path):
        build()
    so = ctypes.CDLL(path)
    P = ctypes.c_void_p
    so.tmo_f16_bits.restype = ctypes.c_uint16
    so.tmo_f16_bits.argtypes = [ctypes.c_float]
    so.tmo_f16_value.restype = ctypes.c_float
    so.tmo_f16_value.argtypes = [ctypes.c_uint16]
    so.tmo_quantize.argtypes = [ctypes.c_int, P, ctypes.c_int64, P]
    so.tmo_dequantize.argtypes = [ctypes.c_int, P, ctypes.c_int64, P]
    so.tmo_quantize_activations.argtypes = [P, ctypes.c_int32, P, P, P, ctypes.c_int]
    so.tmo_quantize_activations.restype = None
    so.tmo_matmul_reference.argtypes = [ctypes.c_int, P, P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, P]
    so.tmo_matmul.argtypes = [ctypes.c_int, P, P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, P]
    so.tmo_gather.restype = ctypes.c_int64
    so.tmo_gather.argtypes = [ctypes.c_int, P, ctypes.c_int32, ctypes.c_int32, P, ctypes.c_int64, P]
    so.tmo_add_bias.argtypes = [P, P, ctypes.c_int64, ctypes.c_int32]
    so.tmo_add_bias.restype = None
    so.tmo_set_threads.argtypes = [ctypes.c_int]
    so.tmo_set_threads.restype = None
    so.tmo_threads.restype = ctypes.c_int
    so.tmo_f16_bits_many.argtypes = [P, ctypes.c_int64, P]
    so.tmo_f16_bits_many.restype = ctypes.c_int64
    so.tmo_f16_values_many.argtypes = [P, ctypes.c_int64, P]
    so.tmo_f16_values_many.restype = ctypes.c_int64
    _LIBS[variant] = so
    return so


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def kind_of(kind) -> int:
    return KINDS[kind] if isinstance(kind, str) else int(kind)


def row_bytes(kind, k: int) -> int:
    return k // 32 * BLOCK_BYTES[kind_of(kind)]


def f16_bits(value: float) -> int:
    """F16.new(value).bits, f16.cr:29-41."""
    return lib().tmo_f16_bits(float(value))


def f16_value(bits: int) -> float:
    """F16.from_bits(bits).to_f32, f16.cr:44-57."""
    return lib().tmo_f16_value(int(bits))


def f16_bits_many(values: np.ndarray) -> np.ndarray:
    words = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    out = np.empty(words.shape, dtype=np.uint16)
    lib().tmo_f16_bits_many(_ptr(words), words.size, _ptr(out))
    return out


def f16_values_many(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().tmo_f16_values_many(_ptr(b), b.size, _ptr(out))
    return out


def quantize(kind, values: np.ndarray) -> np.ndarray:
    """Quant.quantize, quant.cr:77-90: f32 values (a whole number of blocks) -> block bytes."""
    k = kind_of(kind)
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(v.size // 32 * BLOCK_BYTES[k], dtype=np.uint8)
    if lib().tmo_quantize(k, _ptr(v), v.size, _ptr(out)) != 0:
        raise ValueError("bad kind or count")
    return out


def dequantize(kind, data: np.ndarray, count: int) -> np.ndarray:
    """Quant.dequantize, quant.cr:93-105."""
    k = kind_of(kind)
    b = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    if b.size != count // 32 * BLOCK_BYTES[k]:
        raise ValueError(f"{b.size} bytes do not hold {count} values")
    out = np.empty(count, dtype=np.float32)
    lib().tmo_dequantize(k, _ptr(b), count, _ptr(out))
    return out


def quantize_activations(x: np.ndarray, with_sums: bool):
    """quantize_activations, quant.cr:424-442, one row: (scales, sums, qs)."""
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    nb = v.size // 32
    scales = np.zeros(nb, np.float32)
    sums = np.zeros(nb, np.float32)
    qs = np.zeros(v.size, np.int8)
    lib().tmo_quantize_activations(_ptr(v), v.size, _ptr(scales), _ptr(sums), _ptr(qs), int(with_sums))
    return scales, sums, qs


def matmul_reference(kind, x: np.ndarray, w: np.ndarray, rows: int, n: int, k: int) -> np.ndarray:
    """Quant.matmul_reference, quant.cr:122-142: the oracle, [rows, n] f32."""
    kk = kind_of(kind)
    xs = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    ws = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    if ws.size != n * row_bytes(kk, k) or xs.size != rows * k:
        raise ValueError("shape mismatch")
    out = np.empty(rows * n, dtype=np.float32)
    if lib().tmo_matmul_reference(kk, _ptr(xs), _ptr(ws), rows, n, k, _ptr(out)) != 0:
        raise ValueError("bad kind or k")
    return out.reshape(rows, n)


def matmul(kind, x: np.ndarray, w: np.ndarray, rows: int, n: int, k: int, variant: str = "portable") -> np.ndarray:
    """Quant.matmul, quant.cr:155-182: the fast CPU path on set_threads() threads."""
    kk = kind_of(kind)
    xs = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    ws = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    if ws.size != n * row_bytes(kk, k) or xs.size != rows * k:
        raise ValueError("shape mismatch")
    out = np.empty(rows * n, dtype=np.float32)
    if lib(variant).tmo_matmul(kk, _ptr(xs), _ptr(ws), rows, n, k, _ptr(out)) != 0:
        raise ValueError("bad kind or k")
    return out.reshape(rows, n)


def add_bias(dst: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """HostDevice#add_bias, devices/host.cr:725-734."""
    out = np.ascontiguousarray(dst, dtype=np.float32).copy()
    b = np.ascontiguousarray(bias, dtype=np.float32)
    lib().tmo_add_bias(_ptr(out), _ptr(b), out.size // b.size, b.size)
    return out


def gather(kind, table: np.ndarray, rows: int, width: int, ids) -> np.ndarray:
    """Quant.gather with HostDevice#block_gather's id check (quant.cr:417-422; host.cr:648-658)."""
    kk = kind_of(kind)
    t = np.ascontiguousarray(table, dtype=np.uint8).reshape(-1)
    idx = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    out = np.empty(idx.size * width, dtype=np.float32)
    bad = lib().tmo_gather(kk, _ptr(t), rows, width, _ptr(idx), idx.size, _ptr(out))
    if bad:
        raise IndexError(f"index {idx[bad - 1]} out of range for {rows} rows")
    return out.reshape(idx.size, width)


def set_threads(threads: int, variant: str = "portable") -> None:
    """Quant.threads=, quant.cr:188."""
    lib(variant).tmo_set_threads(int(threads))


def threads(variant: str = "portable") -> int:
    return lib(variant).tmo_threads()


# ---------------------------------------------------------------- Llama (tmq_llama.c)

class LlamaConfig(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int32), ("width", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("kv_heads", ctypes.c_int32), ("head_width", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("vocab", ctypes.c_int32), ("context", ctypes.c_int32), ("eps", ctypes.c_float),
                ("theta", ctypes.c_double), ("kind", ctypes.c_int32)]


class LlamaWeights(ctypes.Structure):
    _fields_ = [("embed", ctypes.c_void_p), ("head", ctypes.c_void_p), ("norm", ctypes.c_void_p),
                ("attn_norm", ctypes.POINTER(ctypes.c_void_p)), ("ffn_norm", ctypes.POINTER(ctypes.c_void_p)),
                ("qkv", ctypes.POINTER(ctypes.c_void_p)), ("o", ctypes.POINTER(ctypes.c_void_p)),
                ("gate_up", ctypes.POINTER(ctypes.c_void_p)), ("down", ctypes.POINTER(ctypes.c_void_p))]


def _llama_lib(variant="portable"):
    so = lib(variant)
    if not getattr(so, "_llama_ready", False):
        P = ctypes.c_void_p
        so.tmo_exp.restype = ctypes.c_float
        so.tmo_exp.argtypes = [ctypes.c_float]
        so.tmo_exp_many.argtypes = [P, ctypes.c_int64, P]
        so.tmo_exp_many.restype = None
        so.tmo_rmsnorm.argtypes = [P, P, ctypes.c_int32, ctypes.c_int32, ctypes.c_float, P]
        so.tmo_rmsnorm.restype = None
        so.tmo_rope_tables.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_double, P, P]
        so.tmo_rope_tables.restype = None
        so.tmo_swiglu_many.argtypes = [P, P, ctypes.c_int64, P]
        so.tmo_swiglu_many.restype = None
        so.tmo_llama_new.restype = P
        so.tmo_llama_new.argtypes = [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights)]
        so.tmo_llama_free.argtypes = [P]
        so.tmo_llama_free.restype = None
        so.tmo_llama_reset.argtypes = [P]
        so.tmo_llama_reset.restype = None
        so.tmo_llama_length.argtypes = [P]
        so.tmo_llama_length.restype = ctypes.c_int32
        so.tmo_llama_forward.argtypes = [P, P, ctypes.c_int32, ctypes.c_int32, P]
        so.tmo_llama_forward.restype = ctypes.c_int
        so.tmo_argmax.argtypes = [P, ctypes.c_int32]
        so.tmo_argmax.restype = ctypes.c_int32
        I = ctypes.c_int32
        so.tmo_attention.argtypes = [P, I, I, P, P, I, I, I, P, ctypes.c_float, P]
        so.tmo_attention.restype = None
        so.tmo_rope.argtypes = [P, I, I, I, I, P, P, P, P]
        so.tmo_rope.restype = None
        so._llama_ready = True
    return so


def exp_many(x: np.ndarray) -> np.ndarray:
    """Maths.exp, maths.cr:36-54, elementwise."""
    v = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(v)
    _llama_lib().tmo_exp_many(_ptr(v), v.size, _ptr(out))
    return out


def rmsnorm(x: np.ndarray, w, eps: float) -> np.ndarray:
    """rmsnorm_row, host.cr:374-386, over the rows of x."""
    v = np.ascontiguousarray(x, dtype=np.float32)
    n = v.shape[-1]
    out = np.empty_like(v)
    wp = _ptr(np.ascontiguousarray(w, dtype=np.float32)) if w is not None else None
    _llama_lib().tmo_rmsnorm(_ptr(v), wp, v.size // n, n, float(eps), _ptr(out))
    return out


def rope_tables(width: int, context: int, theta: float):
    """RotaryEmbedding's cos/sin tables, modules.cr:344-351: [context, width] each."""
    cos = np.empty((context, width), np.float32)
    sin = np.empty((context, width), np.float32)
    _llama_lib().tmo_rope_tables(width, context, float(theta), _ptr(cos), _ptr(sin))
    return cos, sin


def swiglu(gate: np.ndarray, value: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32)
    v = np.ascontiguousarray(value, dtype=np.float32)
    out = np.empty_like(g)
    _llama_lib().tmo_swiglu_many(_ptr(g), _ptr(v), g.size, _ptr(out))
    return out


def argmax(logits: np.ndarray) -> int:
    v = np.ascontiguousarray(logits, dtype=np.float32)
    return int(_llama_lib().tmo_argmax(_ptr(v), v.size))


def attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, table, scale: float) -> np.ndarray:
    """The Attention op on a host device (host.cr:408-440): q [tokens, heads,
    width]; keys/values [rows, kv_heads, capacity, width]; table [tokens, 3] of
    (cache row, last position seen, positions held)."""
    qv = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.float32)
    v = np.ascontiguousarray(values, dtype=np.float32)
    t = np.ascontiguousarray(table, dtype=np.int32).reshape(-1, 3)
    tokens, heads, width = qv.shape
    rows, kv_heads, capacity, _ = k.shape
    assert t.shape[0] == tokens and np.all((t[:, 0] >= 0) & (t[:, 0] < rows))
    assert np.all((t[:, 2] > 0) & (t[:, 2] <= capacity) & (t[:, 1] >= 0) & (t[:, 1] < t[:, 2]))
    out = np.empty_like(qv)
    _llama_lib().tmo_attention(_ptr(qv), tokens, heads, _ptr(k), _ptr(v), kv_heads, capacity, width, _ptr(t),
                               float(scale), _ptr(out))
    return out


def rope(x: np.ndarray, heads: int, width: int, cos: np.ndarray, sin: np.ndarray, positions) -> np.ndarray:
    """The Rope op (host.cr:448-466) on the first `heads` heads of each row of
    x [tokens, ≥ heads·width], row t at table row positions[t]: [tokens, heads, width]."""
    xv = np.ascontiguousarray(x, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    c = np.ascontiguousarray(cos, dtype=np.float32)
    s_ = np.ascontiguousarray(sin, dtype=np.float32)
    assert np.all((pos >= 0) & (pos < c.shape[0]))
    out = np.empty((xv.shape[0], heads, width), np.float32)
    _llama_lib().tmo_rope(_ptr(xv), xv.shape[1], xv.shape[0], heads, width, _ptr(c), _ptr(s_), _ptr(pos), _ptr(out))
    return out


class Llama:
    """The oracle's Llama forward on a host device (tmq_llama.c). Weights: a
    dict of numpy arrays -- embed [vocab·row bytes] blocks, head (or None when
    tied), norm [width], and per-layer lists attn_norm, ffn_norm, qkv, o,
    gate_up, down (block bytes, q/k rows in Hugging Face order)."""

    def __init__(self, config: dict, weights: dict, variant: str = "portable"):
        self.so = _llama_lib(variant)
        self.config = dict(config)
        self._keep = []

        def keep(a, dtype):
            arr = np.ascontiguousarray(a, dtype=dtype)
            self._keep.append(arr)
            return arr.ctypes.data

        def plist(arrays, dtype):
            ptrs = (ctypes.c_void_p * len(arrays))(*[keep(a, dtype) for a in arrays])
            self._keep.append(ptrs)
            return ptrs

        c = LlamaConfig(config["layers"], config["width"], config["heads"], config["kv_heads"],
                        config["head_width"], config["hidden"], config["vocab"], config["context"],
                        config["eps"], config["theta"], kind_of(config["kind"]))
        embed = keep(weights["embed"], np.uint8)
        head = keep(weights["head"], np.uint8) if weights.get("head") is not None else embed
        w = LlamaWeights(embed, head, keep(weights["norm"], np.float32),
                         plist(weights["attn_norm"], np.float32), plist(weights["ffn_norm"], np.float32),
                         plist(weights["qkv"], np.uint8), plist(weights["o"], np.uint8),
                         plist(weights["gate_up"], np.uint8), plist(weights["down"], np.uint8))
        self._keep += [c, w]
        self.handle = self.so.tmo_llama_new(ctypes.byref(c), ctypes.byref(w))

    def forward(self, ids, last_only: bool = False) -> np.ndarray:
        idx = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        rows = 1 if last_only else idx.size
        out = np.empty((rows, self.config["vocab"]), np.float32)
        code = self.so.tmo_llama_forward(self.handle, _ptr(idx), idx.size, int(last_only), _ptr(out))
        if code != 0:
            raise ValueError(f"tmo_llama_forward failed ({code})")
        return out

    def reset(self) -> None:
        self.so.tmo_llama_reset(self.handle)

    @property
    def length(self) -> int:
        return self.so.tmo_llama_length(self.handle)

    def generate(self, prompt, count: int):
        """Generative#generate with the greedy sampler (generative.cr:177-190)."""
        self.reset()
        logits = self.forward(prompt, last_only=True)[0]
        tokens = []
        for i in range(count):
            token = argmax(logits)
            tokens.append(token)
            if i < count - 1:
                logits = self.forward([token], last_only=True)[0]
        return tokens

    def __del__(self):
        try:
            if self.handle:
                self.so.tmo_llama_free(self.handle)
                self.handle = None
        except Exception:
            pass
