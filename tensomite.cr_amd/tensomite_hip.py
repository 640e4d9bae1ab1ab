"""Host binding of libtensomite_hip.so: a `HIP` device with the reference's
device API (src/tensomite/device.cr:6-68) for the quantised-product path.

The reference's host language is Crystal, whose toolchain is absent here; this
module is the same binding a Crystal `lib LibTensomiteHIP` would be (the same
functions and argument types as include/tensomite_hip.h), written with ctypes
so tests and bench.py drive the C ABI directly. It loads only the in-tree library and raises when
it is missing: there is no CPU fallback.

    dev = HIPDevice()
    w = dev.alloc(nbytes); dev.upload(w, weight_bytes)       # Device#alloc/#upload
    y = dev.block_matmul(Q4_0, w, x, rows=1, n=N, k=K)       # Op::BlockMatMul
    dev.sync()                                                # Device#sync
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libtensomite_hip.so")

Q8_0, Q4_0, Q4_1 = 0, 1, 2
KINDS = {"Q8_0": Q8_0, "Q4_0": Q4_0, "Q4_1": Q4_1}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20}

# BlockMatMulMode, quant.cr:5-28 (MATRIX is this device's own).
MODES = {"auto": 0, "thread": 1, "lanes": 2, "unordered": 3, "loads": 4, "stream": 5,
         "stream_activations": 6, "matrix": 7}

SUCCESS = 0
ERROR_INVALID_VALUE = 1000
ERROR_SHAPE = 1001
ERROR_DTYPE = 1002
ERROR_NO_KERNELS = 1003
ERROR_OUT_OF_MEMORY = 1004
ERROR_EXECUTION = 1005
ERROR_NO_DEVICE = 1006
ERROR_NOT_READY = 1008
ERROR_SCRATCH_LIMIT = 1009


class Error(Exception):
    """Base of the errors below (errors.cr:1-16)."""


class DeviceError(Error):
    """A failed runtime call: "call: NAME (text)", as CUDA.check raises (cuda.cr:1069-1075)."""


class ShapeError(Error):
    pass


class DTypeError(Error):
    pass


class ExecutionError(Error):
    """A kernel found an index out of range, reported at sync (cuda.cr:972-983)."""


class NoKernels(DeviceError):
    """The library's kernels are unavailable: the caller's host kernel must run."""


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("memory", ctypes.c_uint64),
                ("compute_units", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
                ("memory_clock_khz", ctypes.c_int32), ("memory_bus_width", ctypes.c_int32),
                ("l2_bytes", ctypes.c_int32), ("lds_bytes_per_block", ctypes.c_int32)]


class Product(ctypes.Structure):
    """tmh_product: one one-row product of a plan."""
    _fields_ = [("w", ctypes.c_uint64), ("w_byte_offset", ctypes.c_uint64), ("x", ctypes.c_uint64),
                ("dst", ctypes.c_uint64), ("bias", ctypes.c_uint64), ("n", ctypes.c_uint32), ("k", ctypes.c_uint32),
                ("x_mode", ctypes.c_uint32), ("eps", ctypes.c_float), ("norm", ctypes.c_uint64),
                ("scales", ctypes.c_uint64), ("sums", ctypes.c_uint64), ("totals", ctypes.c_uint64)]


X_F32, X_RMSNORM, X_QUANTISED = 0, 1, 2


class RMSNormInput:
    """A plan product's x taken through Op::RMSNorm (weights `norm`, `eps`) before the product."""

    def __init__(self, norm: "Buffer", eps: float):
        self.norm, self.eps = norm, eps


class QuantisedInput:
    """A plan product's x already quantised by HIPDevice.quantize_rows (x is its int8 values, qs)."""

    def __init__(self, scales: "Buffer", sums: "Buffer", totals: "Buffer"):
        self.scales, self.sums, self.totals = scales, sums, totals


class Counters(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int64) for name in
                ("uploads", "downloads", "gpu_ops", "device_bytes", "pool_held", "pool_limit", "pool_hits",
                 "pool_misses", "frees", "launches")]


class LlamaConfig(ctypes.Structure):
    """tmh_llama_config."""
    _fields_ = [("layers", ctypes.c_int32), ("width", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("kv_heads", ctypes.c_int32), ("head_width", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("vocab", ctypes.c_int32), ("context", ctypes.c_int32), ("eps", ctypes.c_float),
                ("theta", ctypes.c_double), ("kind", ctypes.c_uint32)]


class LlamaWeights(ctypes.Structure):
    """tmh_llama_weights: device addresses."""
    _fields_ = [("embed", ctypes.c_uint64), ("head", ctypes.c_uint64), ("norm", ctypes.c_uint64)] + [
        (name, ctypes.POINTER(ctypes.c_uint64)) for name in ("attn_norm", "ffn_norm", "qkv", "o", "gate_up", "down")]


# Every symbol include/tensomite_hip.h declares, with (restype, argtypes).
U32, I32, U64, I64 = ctypes.c_uint32, ctypes.c_int32, ctypes.c_uint64, ctypes.c_int64
VP, INT, F32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
SIGNATURES = {
    "tmh_init": (INT, [ctypes.POINTER(I32)]),
    "tmh_device_info_get": (INT, [I32, ctypes.POINTER(DeviceInfo)]),
    "tmh_set_device": (INT, [I32]),
    "tmh_get_device": (INT, [ctypes.POINTER(I32)]),
    "tmh_malloc": (INT, [ctypes.POINTER(U64), U64]),
    "tmh_free": (INT, [U64]),
    "tmh_free_any_thread": (INT, [U64]),
    "tmh_upload": (INT, [U64, VP, U64]),
    "tmh_upload_async": (INT, [U64, VP, U64]),
    "tmh_download": (INT, [VP, U64, U64]),
    "tmh_copy": (INT, [U64, U64, U64]),
    "tmh_synchronize": (INT, []),
    "tmh_alloc": (INT, [ctypes.POINTER(U64), U64]),
    "tmh_retire": (INT, [U64, U64]),
    "tmh_sync": (INT, []),
    "tmh_pool_set_limit": (INT, [I64]),
    "tmh_counters_get": (INT, [ctypes.POINTER(Counters)]),
    "tmh_error_name": (ctypes.c_char_p, [INT]),
    "tmh_error_string": (ctypes.c_char_p, [INT]),
    "tmh_error_report": (INT, [ctypes.POINTER(I32)]),
    "tmh_debug_fail_allocations": (INT, [I32]),
    "tmh_debug_disable_kernels": (INT, [I32]),
    "tmh_event_create": (INT, [ctypes.POINTER(U64)]),
    "tmh_event_record": (INT, [U64]),
    "tmh_event_elapsed_ms": (INT, [U64, U64, ctypes.POINTER(ctypes.c_float)]),
    "tmh_event_destroy": (INT, [U64]),
    "tmh_quantize_rows_q8": (INT, [U64, U32, U32, U32, U64, U64, U64, U64]),
    "tmh_block_matmul": (INT, [U32, U64, U64, U64, U32, U64, U64, U32, U32, U32, U32]),
    "tmh_block_matmul_quantised": (INT, [U32, U64, U64, U64, U64, U64, U64, U64, U64, U32, U32, U32, U32]),
    "tmh_block_matmul_fixed": (INT, [U32, U64, U64, U64, U32, U64, U64, U32, U32, U32, U32]),
    "tmh_gather_blocks": (INT, [U32, U64, U64, I32, U32, U64, U32, U64]),
    "tmh_quantize_weights": (INT, [U32, VP, U64, VP, I32]),
    "tmh_debug_f16_words": (INT, [U32, U32, U64]),
    "tmh_debug_read": (INT, [U64, U64, U32, U64]),
    "tmh_plan_create": (INT, [U32, ctypes.POINTER(Product), U32, ctypes.POINTER(U64)]),
    "tmh_plan_run": (INT, [U64]),
    "tmh_plan_destroy": (INT, [U64]),
    "tmh_plan_describe": (INT, [U64, ctypes.c_char_p, U32]),
    "tmh_plan_set_mode": (INT, [U64, U32]),
    "tmh_rmsnorm": (INT, [U64, U32, U64, U32, U32, F32, U64]),
    "tmh_rope_write": (INT, [U64, U32, U32, U32, U32, U32, U64, U64, U32, U64, U32, U32, U64, U64, U64]),
    "tmh_attention": (INT, [U64, U32, U32, U32, U64, U64, U32, U32, U32, U32, U64, F32, U64, U32]),
    "tmh_swiglu": (INT, [U64, U64, U32, U32, U32, U64]),
    "tmh_add": (INT, [U64, U64, U64, U64]),
    "tmh_argmax": (INT, [U64, U32, U32, U32, U64]),
    "tmh_llama_create": (INT, [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights), U32, U32, U32,
                               ctypes.POINTER(U64)]),
    "tmh_llama_forward": (INT, [U64, U32, VP, U32, U32, VP]),
    "tmh_llama_generate": (INT, [U64, U32, VP, U32]),
    "tmh_llama_length": (INT, [U64, U32, ctypes.POINTER(I32)]),
    "tmh_llama_reset": (INT, [U64, U32]),
    "tmh_llama_step": (INT, [U64, U32]),
    "tmh_llama_set_mode": (INT, [U64, U32]),
    "tmh_llama_destroy": (INT, [U64]),
    "tmh_gguf_open": (INT, [ctypes.c_char_p, ctypes.POINTER(U64)]),
    "tmh_gguf_close": (INT, [U64]),
    "tmh_gguf_tensor": (INT, [U64, ctypes.c_char_p, ctypes.POINTER(U32), ctypes.POINTER(I64), ctypes.POINTER(U32),
                              ctypes.POINTER(U64)]),
    "tmh_gguf_upload": (INT, [U64, ctypes.c_char_p, VP, U32, U64]),
    "tmh_llama_load_gguf": (INT, [ctypes.c_char_p, U32, U32, U32, ctypes.POINTER(LlamaConfig), ctypes.POINTER(U64)]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def library() -> ctypes.CDLL:
    """Loads the in-tree libtensomite_hip.so; raises when it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIBRARY):
                raise DeviceError(f"{LIBRARY} is missing: run __graft_entry__.build() (hipcc, gfx950)")
            so = ctypes.CDLL(LIBRARY)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(so, name)
                fn.restype, fn.argtypes = restype, argtypes
            _lib = so
    return _lib


def error_text(code: int) -> str:
    lib = library()
    return f"{lib.tmh_error_name(code).decode()} ({lib.tmh_error_string(code).decode()})"


def check(call: str, code: int) -> None:
    """Raises the reference's error for a failed call (CUDA.check, cuda.cr:1069-1075)."""
    if code == SUCCESS:
        return
    text = f"{call}: {error_text(code)}"
    if code == ERROR_SHAPE:
        raise ShapeError(text)
    if code == ERROR_DTYPE:
        raise DTypeError(text)
    if code == ERROR_NO_KERNELS:
        raise NoKernels(text)
    raise DeviceError(text)


def kind_of(kind) -> int:
    if isinstance(kind, str):
        if kind not in KINDS:
            raise DTypeError(f"{kind} is not a block format")
        return KINDS[kind]
    return int(kind)


def row_bytes(kind, k: int) -> int:
    """DType#bytes_for of one row (dtype.cr:221-244)."""
    if k % 32:
        raise ShapeError(f"rows of {k} do not split into blocks of 32")
    return k // 32 * BLOCK_BYTES[kind_of(kind)]


def device_count() -> int:
    n = I32(0)
    check("tmh_init", library().tmh_init(ctypes.byref(n)))
    return n.value


class Buffer:
    """Device memory owned by a device (device.cr:6-33): given back to the
    device's pool when released or collected."""

    def __init__(self, device: "HIPDevice", pointer: int, bytesize: int):
        self.device = device
        self.pointer = pointer
        self.bytesize = bytesize
        self._released = False

    @property
    def released(self) -> bool:
        return self._released

    def release(self) -> None:
        if self._released:
            return
        self._released = True
        self.device._retire(self)

    def __del__(self):
        if not getattr(self, "_released", True):
            try:
                self.device._retire(self)
            except Exception:
                pass


class Plan:
    """A recorded list of one-row products run as one launch (tmh_plan_*)."""

    def __init__(self, device: "HIPDevice", handle: int, keep):
        self.device, self.handle, self._keep = device, handle, keep

    def run(self) -> None:
        check("tmh_plan_run", self.device.lib.tmh_plan_run(self.handle))

    def set_mode(self, mode: str) -> None:
        """BlockMatMulMode of the plan's launch: "auto" (the host's bits) or "unordered" (measurement only)."""
        check("tmh_plan_set_mode", self.device.lib.tmh_plan_set_mode(self.handle, MODES[mode]))

    def describe(self) -> str:
        """The plan's launch: kernel, grid, LDS."""
        text = ctypes.create_string_buffer(256)
        check("tmh_plan_describe", self.device.lib.tmh_plan_describe(self.handle, text, len(text)))
        return text.value.decode()

    def destroy(self) -> None:
        if self.handle:
            self.device.lib.tmh_plan_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class HIPDevice:
    """An MI355X through libtensomite_hip.so: `#map` returns None, data moves
    through `#upload`/`#download`, and BlockMatMul and block Gather run on the
    GPU, queued in order on one stream (the pattern of `CUDA < HostDevice`,
    cuda.cr:92-415)."""

    def __init__(self, index: int = 0, block_mode: str = "auto"):
        self.lib = library()
        count = device_count()
        if index >= count:
            raise DeviceError(f"tmh_init: no GPU {index} ({count} found)")
        self.index = index
        self.block_mode = block_mode
        self.bind()
        info = DeviceInfo()
        check("tmh_device_info_get", self.lib.tmh_device_info_get(index, ctypes.byref(info)))
        self.name = info.name.decode()
        self.arch = info.arch.decode()
        self.memory = int(info.memory)
        self.compute_units = int(info.compute_units)

    def bind(self) -> None:
        """Makes this device current on the calling thread (Context#bind, cuda.cr:1118-1125)."""
        check("tmh_set_device", self.lib.tmh_set_device(self.index))

    # -- the Device contract (device.cr:39-68)
    def alloc(self, bytesize: int) -> Buffer:
        ptr = U64(0)
        check("tmh_alloc", self.lib.tmh_alloc(ctypes.byref(ptr), int(bytesize)))
        return Buffer(self, ptr.value, int(bytesize))

    def upload(self, buffer: Buffer, data, asynchronous: bool = False) -> None:
        arr = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                                   else data)
        nbytes = arr.nbytes
        if nbytes > buffer.bytesize:
            raise DeviceError(f"upload: {nbytes} bytes into a buffer of {buffer.bytesize}")
        fn = self.lib.tmh_upload_async if asynchronous else self.lib.tmh_upload
        check("tmh_upload_async" if asynchronous else "tmh_upload", fn(buffer.pointer, arr.ctypes.data, nbytes))

    def download(self, buffer: Buffer, out: np.ndarray) -> np.ndarray:
        if not out.flags["C_CONTIGUOUS"]:
            raise DeviceError("download needs contiguous host memory")
        if out.nbytes > buffer.bytesize:
            raise DeviceError(f"download: {out.nbytes} bytes from a buffer of {buffer.bytesize}")
        check("tmh_download", self.lib.tmh_download(out.ctypes.data, buffer.pointer, out.nbytes))
        return out

    def map(self, buffer: Buffer):
        """Device memory is not host-visible (cuda.cr:355-358)."""
        return None

    def sync(self) -> None:
        """Waits, recycles retired memory, and raises ExecutionError for an index
        a kernel reported out of range (CUDA#sync, cuda.cr:419-428)."""
        self.check_synced("tmh_sync", self.lib.tmh_sync())

    def check_synced(self, call: str, code: int) -> None:
        """check() for calls that end in tmh_sync: an index error is an ExecutionError."""
        if code == ERROR_EXECUTION:
            report = (I32 * 3)()
            check("tmh_error_report", self.lib.tmh_error_report(report))
            raise ExecutionError(f"index {report[1]} out of range for {report[2]} rows")
        check(call, code)

    def shape_invariant(self) -> bool:
        """Each output depends only on its own row and column (quant.cr:120-121)."""
        return True

    def fuses_attention(self) -> bool:
        return False

    # -- helpers
    def from_array(self, values: np.ndarray, asynchronous: bool = False) -> Buffer:
        arr = np.ascontiguousarray(values)
        buf = self.alloc(max(arr.nbytes, 1))
        if arr.nbytes:
            self.upload(buf, arr, asynchronous)
        return buf

    def to_array(self, buffer: Buffer, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        return self.download(buffer, out)

    def copy(self, dst: Buffer, src: Buffer, bytesize: int, dst_offset: int = 0, src_offset: int = 0) -> None:
        check("tmh_copy", self.lib.tmh_copy(dst.pointer + dst_offset, src.pointer + src_offset, bytesize))

    def counters(self) -> dict:
        c = Counters()
        check("tmh_counters_get", self.lib.tmh_counters_get(ctypes.byref(c)))
        return {name: getattr(c, name) for name, _ in Counters._fields_}

    def set_pool_limit(self, bytes_: int) -> None:
        check("tmh_pool_set_limit", self.lib.tmh_pool_set_limit(int(bytes_)))

    def _retire(self, buffer: Buffer) -> None:
        self.lib.tmh_retire(buffer.pointer, buffer.bytesize)

    # -- the quantised path
    def quantize_rows(self, x: Buffer, rows: int, k: int, ldx: Optional[int] = None):
        """quantize_rows_q8 into new buffers: (scales, sums, totals, qs)."""
        nb = k // 32
        stride = k if ldx is None else ldx
        if k % 32 or stride < k or (rows and ((rows - 1) * stride + k) * 4 > x.bytesize):
            raise ShapeError(f"{x.bytesize} bytes do not hold {rows} rows of {k} values {stride} apart")
        scales, sums, totals = (self.alloc(max(4 * rows * nb, 4)) for _ in range(3))
        qs = self.alloc(max(rows * k, 4))
        check("tmh_quantize_rows_q8", self.lib.tmh_quantize_rows_q8(
            x.pointer, rows, k, k if ldx is None else ldx, scales.pointer, sums.pointer, totals.pointer,
            qs.pointer))
        return scales, sums, totals, qs

    def block_matmul(self, kind, w: Buffer, x: Buffer, rows: int, n: int, k: int, dst: Optional[Buffer] = None,
                     bias: Optional[Buffer] = None, w_row: int = 0, ldx: Optional[int] = None,
                     mode: Optional[str] = None) -> Buffer:
        """Op::BlockMatMul: dst[rows, n] = x[rows, k] · w[w_row:w_row+n]ᵀ (+ bias), queued."""
        kk = kind_of(kind)
        rb = row_bytes(kk, k)
        if (w_row + n) * rb > w.bytesize:
            raise ShapeError(f"{w.bytesize} bytes do not hold rows {w_row}...{w_row + n} of {k} values")
        stride = k if ldx is None else ldx
        if stride < k or (rows and ((rows - 1) * stride + k) * 4 > x.bytesize):
            raise ShapeError(f"{x.bytesize} bytes do not hold {rows} rows of {k} values {stride} apart")
        if dst is None:
            dst = self.alloc(max(4 * rows * n, 4))
        if rows * n * 4 > dst.bytesize or (bias is not None and n * 4 > bias.bytesize):
            raise ShapeError(f"output or bias too small for [{rows}, {n}]")
        m = MODES[mode or self.block_mode]
        check("tmh_block_matmul", self.lib.tmh_block_matmul(
            kk, w.pointer, w_row * rb, x.pointer, k if ldx is None else ldx, dst.pointer,
            bias.pointer if bias is not None else 0, rows, n, k, m))
        return dst

    def block_matmul_quantised(self, kind, w: Buffer, act, rows: int, n: int, k: int, dst: Optional[Buffer] = None,
                               bias: Optional[Buffer] = None, w_row: int = 0, mode: Optional[str] = None) -> Buffer:
        """The product kernel alone on activations quantize_rows gave: act = (scales, sums, totals, qs)."""
        kk = kind_of(kind)
        rb = row_bytes(kk, k)
        scales, sums, totals, qs = act
        if (w_row + n) * rb > w.bytesize:
            raise ShapeError(f"{w.bytesize} bytes do not hold rows {w_row}...{w_row + n} of {k} values")
        nb = k // 32
        if k % 32 or qs.bytesize < rows * k or min(scales.bytesize, sums.bytesize, totals.bytesize) < 4 * rows * nb:
            raise ShapeError(f"quantised activations too small for [{rows}, {k}]")
        if dst is None:
            dst = self.alloc(max(4 * rows * n, 4))
        if rows * n * 4 > dst.bytesize or (bias is not None and n * 4 > bias.bytesize):
            raise ShapeError(f"output or bias too small for [{rows}, {n}]")
        m = MODES[mode or self.block_mode]
        check("tmh_block_matmul_quantised", self.lib.tmh_block_matmul_quantised(
            kk, w.pointer, w_row * rb, scales.pointer, sums.pointer, totals.pointer, qs.pointer, dst.pointer,
            bias.pointer if bias is not None else 0, rows, n, k, m))
        return dst

    def gather(self, kind, table: Buffer, table_rows: int, width: int, ids: Buffer, count: int,
               dst: Optional[Buffer] = None, first_row: int = 0) -> Buffer:
        """Op::Gather on a block table: rows ids of table[first_row:], dequantised to F32."""
        kk = kind_of(kind)
        rb = row_bytes(kk, width)
        if (first_row + table_rows) * rb > table.bytesize or count * 4 > ids.bytesize:
            raise ShapeError(f"table of {table.bytesize} bytes or ids of {ids.bytesize} too small")
        if dst is None:
            dst = self.alloc(max(4 * count * width, 4))
        if count * width * 4 > dst.bytesize:
            raise ShapeError("output too small")
        check("tmh_gather_blocks", self.lib.tmh_gather_blocks(
            kk, table.pointer, first_row * rb, table_rows, width, ids.pointer, count, dst.pointer))
        return dst

    # -- plans: many independent one-row products in one launch
    def plan(self, kind, products) -> "Plan":
        """products: iterable of (w Buffer, w_row, x Buffer, dst Buffer, bias Buffer|None, n, k[, xin]);
        xin None (x is f32), RMSNormInput or QuantisedInput (x is the int8 values)."""
        kk = kind_of(kind)
        items = list(products)
        arr = (Product * max(len(items), 1))()
        for i, item in enumerate(items):
            w, w_row, x, dst, bias, n, k = item[:7]
            xin = item[7] if len(item) > 7 else None
            rb = row_bytes(kk, k)
            x_bytes = k if isinstance(xin, QuantisedInput) else 4 * k
            if (w_row + n) * rb > w.bytesize or x_bytes > x.bytesize or n * 4 > dst.bytesize:
                raise ShapeError(f"product {i}: buffers too small for [{n}, {k}]")
            arr[i] = Product(w.pointer, w_row * rb, x.pointer, dst.pointer, bias.pointer if bias else 0, n, k)
            if isinstance(xin, RMSNormInput):
                if k * 4 > xin.norm.bytesize:
                    raise ShapeError(f"product {i}: norm weights too small for {k}")
                arr[i].x_mode, arr[i].eps, arr[i].norm = X_RMSNORM, xin.eps, xin.norm.pointer
            elif isinstance(xin, QuantisedInput):
                nb = k // 32
                if min(xin.scales.bytesize, xin.sums.bytesize, xin.totals.bytesize) < 4 * nb:
                    raise ShapeError(f"product {i}: quantised row's arrays too small for {k}")
                arr[i].x_mode = X_QUANTISED
                arr[i].scales, arr[i].sums, arr[i].totals = xin.scales.pointer, xin.sums.pointer, xin.totals.pointer
            elif xin is not None:
                raise TypeError(f"product {i}: input {xin!r} is neither RMSNormInput nor QuantisedInput")
        handle = U64(0)
        check("tmh_plan_create", self.lib.tmh_plan_create(kk, arr, len(items), ctypes.byref(handle)))
        return Plan(self, handle.value, items)

    # -- the rest of the decode graph (F32 buffers)
    def rmsnorm(self, x: Buffer, weight: Optional[Buffer], rows: int, n: int, eps: float,
                dst: Optional[Buffer] = None, ldx: Optional[int] = None) -> Buffer:
        """Op::RMSNorm (host.cr:374-386), queued."""
        stride = n if ldx is None else ldx
        if rows and ((rows - 1) * stride + n) * 4 > x.bytesize or (weight is not None and n * 4 > weight.bytesize):
            raise ShapeError(f"rmsnorm of {rows} rows of {n}: buffers too small")
        dst = dst or self.alloc(max(4 * rows * n, 4))
        check("tmh_rmsnorm", self.lib.tmh_rmsnorm(x.pointer, stride, weight.pointer if weight is not None else 0,
                                                  rows, n, eps, dst.pointer))
        return dst

    def rope_write(self, x: Buffer, ldx: int, tokens: int, heads: int, kv_heads: int, width: int, cos: Buffer,
                   sin: Buffer, table_rows: int, slots: Buffer, cache_rows: int, capacity: int, q_dst: Buffer,
                   keys: Buffer, values: Buffer) -> None:
        """Op::Rope of q and k and Op::WriteRows of k and v into the caches, queued."""
        cache = cache_rows * kv_heads * capacity * width * 4
        if (tokens and ((tokens - 1) * ldx + (heads + 2 * kv_heads) * width) * 4 > x.bytesize
                or table_rows * width * 4 > min(cos.bytesize, sin.bytesize) or tokens * 4 > slots.bytesize
                or tokens * heads * width * 4 > q_dst.bytesize or cache > min(keys.bytesize, values.bytesize)):
            raise ShapeError("rope_write: buffers too small")
        check("tmh_rope_write", self.lib.tmh_rope_write(
            x.pointer, ldx, tokens, heads, kv_heads, width, cos.pointer, sin.pointer, table_rows, slots.pointer,
            cache_rows, capacity, q_dst.pointer, keys.pointer, values.pointer))

    def attention(self, q: Buffer, tokens: int, heads: int, keys: Buffer, values: Buffer, cache_rows: int,
                  kv_heads: int, capacity: int, width: int, table: Buffer, scale: float,
                  dst: Optional[Buffer] = None) -> Buffer:
        """Attention of packed queries [tokens, heads, width] against the caches (host.cr:408-440), queued."""
        cache = cache_rows * kv_heads * capacity * width * 4
        if tokens * heads * width * 4 > q.bytesize or cache > min(keys.bytesize, values.bytesize) \
                or tokens * 12 > table.bytesize:
            raise ShapeError("attention: buffers too small")
        dst = dst or self.alloc(max(4 * tokens * heads * width, 4))
        check("tmh_attention", self.lib.tmh_attention(
            q.pointer, heads * width, tokens, heads, keys.pointer, values.pointer, cache_rows, kv_heads, capacity,
            width, table.pointer, scale, dst.pointer, heads * width))
        return dst

    def swiglu(self, gate: Buffer, value: Buffer, ld: int, rows: int, n: int, dst: Optional[Buffer] = None,
               gate_offset: int = 0, value_offset: int = 0) -> Buffer:
        """SwiGLU (kernels.cr:18) of row-strided gate and value, queued; offsets in elements."""
        if rows and ((rows - 1) * ld + n + gate_offset) * 4 > gate.bytesize or \
                rows and ((rows - 1) * ld + n + value_offset) * 4 > value.bytesize:
            raise ShapeError("swiglu: buffers too small")
        dst = dst or self.alloc(max(4 * rows * n, 4))
        check("tmh_swiglu", self.lib.tmh_swiglu(gate.pointer + 4 * gate_offset, value.pointer + 4 * value_offset,
                                                ld, rows, n, dst.pointer))
        return dst

    def add(self, a: Buffer, b: Buffer, count: int, dst: Optional[Buffer] = None) -> Buffer:
        if count * 4 > min(a.bytesize, b.bytesize):
            raise ShapeError("add: buffers too small")
        dst = dst or self.alloc(max(4 * count, 4))
        check("tmh_add", self.lib.tmh_add(a.pointer, b.pointer, dst.pointer, count))
        return dst

    def argmax(self, x: Buffer, rows: int, n: int, ids: Optional[Buffer] = None) -> Buffer:
        """Sampler.greedy per row (sampler.cr:35-36), queued: int32 ids."""
        if rows * n * 4 > x.bytesize:
            raise ShapeError("argmax: buffer too small")
        ids = ids or self.alloc(max(4 * rows, 4))
        check("tmh_argmax", self.lib.tmh_argmax(x.pointer, n, rows, n, ids.pointer))
        return ids

    # -- timing on the library's stream
    def event(self) -> int:
        ev = U64(0)
        check("tmh_event_create", self.lib.tmh_event_create(ctypes.byref(ev)))
        return ev.value

    def record(self, event: int) -> None:
        check("tmh_event_record", self.lib.tmh_event_record(event))

    def elapsed_ms(self, start: int, stop: int) -> float:
        ms = ctypes.c_float(0)
        check("tmh_event_elapsed_ms", self.lib.tmh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        return ms.value

    def destroy_event(self, event: int) -> None:
        check("tmh_event_destroy", self.lib.tmh_event_destroy(event))


class GGUFFile:
    """A GGUF file mapped by the library (tmh_gguf_*): tensor entries and
    uploads, whole or as rows in a given order (GGUF#[] then take_rows,
    gguf.cr:112-136, tensor/quantised.cr:32-43). Needs no GPU to open."""

    KINDS = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 8: "Q8_0", 30: "BF16"}

    def __init__(self, path: str):
        self.lib = library()
        self.path = path
        h = U64(0)
        check("tmh_gguf_open", self.lib.tmh_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h.value

    def entry(self, name: str):
        """(kind name, shape, bytes) of tensor `name`."""
        kind, dims, nbytes = U32(0), U32(0), U64(0)
        shape = (I64 * 4)()
        check("tmh_gguf_tensor", self.lib.tmh_gguf_tensor(self.handle, name.encode(), ctypes.byref(kind), shape,
                                                          ctypes.byref(dims), ctypes.byref(nbytes)))
        return self.KINDS[kind.value], [shape[i] for i in range(dims.value)], nbytes.value

    def upload(self, device: "HIPDevice", name: str, rows=None) -> Buffer:
        """Tensor `name` (or its rows in the order given) in a new device buffer."""
        _, shape, nbytes = self.entry(name)
        order = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
        size = nbytes if order is None else nbytes // shape[0] * order.size
        buf = device.alloc(max(size, 4))
        device.bind()
        check("tmh_gguf_upload", self.lib.tmh_gguf_upload(self.handle, name.encode(),
                                                          None if order is None else order.ctypes.data,
                                                          0 if order is None else order.size, buf.pointer))
        return buf

    def close(self) -> None:
        if getattr(self, "handle", 0):
            self.lib.tmh_gguf_close(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


LLAMA_LAYER_KEYS = ("attn_norm", "ffn_norm", "qkv", "o", "gate_up", "down")


class HIPLlama:
    """A Llama decoded on the device (tmh_llama_*): Llama#forward /
    #forward_last and Generative#generate with the greedy sampler
    (llama.cr:256-303, generative.cr:155-190), over `rows` sequences.

    `weights` is a dict as the oracle's Llama takes it: embed and head (None
    when tied) block bytes, norm, and per-layer lists attn_norm, ffn_norm (F32),
    qkv, o, gate_up, down (block bytes; q/k rows in Hugging Face order). They
    are uploaded once to device buffers this object owns."""

    def __init__(self, device: HIPDevice, config: dict, weights: dict, rows: int = 1,
                 capacity: Optional[int] = None, max_tokens: int = 128, asynchronous: bool = True):
        self.device = device
        self.config = dict(config)
        c = self.config
        self.rows = rows
        self.capacity = capacity or c["context"]
        up = lambda a, dt: device.from_array(np.ascontiguousarray(a, dtype=dt), asynchronous)
        self.buffers = {"embed": up(weights["embed"], np.uint8), "norm": up(weights["norm"], np.float32)}
        if weights.get("head") is not None:
            self.buffers["head"] = up(weights["head"], np.uint8)
        for key in LLAMA_LAYER_KEYS:
            dt = np.float32 if key.endswith("norm") else np.uint8
            self.buffers[key] = [up(a, dt) for a in weights[key]]
        ptrs = lambda key: (U64 * c["layers"])(*[b.pointer for b in self.buffers[key]])
        self._arrays = {key: ptrs(key) for key in LLAMA_LAYER_KEYS}
        cfg = LlamaConfig(c["layers"], c["width"], c["heads"], c["kv_heads"], c["head_width"], c["hidden"],
                          c["vocab"], c["context"], c["eps"], c["theta"], kind_of(c["kind"]))
        head = self.buffers["head"].pointer if "head" in self.buffers else 0
        w = LlamaWeights(self.buffers["embed"].pointer, head, self.buffers["norm"].pointer,
                         *[self._arrays[k] for k in LLAMA_LAYER_KEYS])
        handle = U64(0)
        device.bind()
        check("tmh_llama_create", device.lib.tmh_llama_create(ctypes.byref(cfg), ctypes.byref(w), rows,
                                                              self.capacity, max_tokens, ctypes.byref(handle)))
        self.handle = handle.value

    @classmethod
    def load_gguf(cls, device: HIPDevice, path: str, rows: int = 1, capacity: int = 0,
                  max_tokens: int = 128) -> "HIPLlama":
        """Llama.load of a GGUF file straight onto the device (tmh_llama_load_gguf):
        the decoder owns the weights it uploads."""
        self = cls.__new__(cls)
        self.device = device
        self.rows = rows
        self.buffers = {}
        cfg, handle = LlamaConfig(), U64(0)
        device.bind()
        check("tmh_llama_load_gguf", device.lib.tmh_llama_load_gguf(os.fsencode(path), rows, capacity, max_tokens,
                                                                    ctypes.byref(cfg), ctypes.byref(handle)))
        self.handle = handle.value
        kinds = {Q8_0: "Q8_0", Q4_0: "Q4_0", Q4_1: "Q4_1"}
        self.config = {name: getattr(cfg, name) for name, _ in LlamaConfig._fields_}
        self.config["kind"] = kinds[self.config["kind"]]
        self.capacity = capacity or self.config["context"]
        return self

    def forward(self, ids, row: int = 0, last_only: bool = False) -> np.ndarray:
        """Logits [len(ids) or 1, vocab] of ids run after the row's cached positions."""
        idx = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        out = np.empty((1 if last_only else idx.size, self.config["vocab"]), np.float32)
        self.device.bind()
        self.device.check_synced("tmh_llama_forward", self.device.lib.tmh_llama_forward(
            self.handle, row, idx.ctypes.data, idx.size, 1 if last_only else 0, out.ctypes.data))
        return out

    def generate(self, steps: int, graph: bool = True) -> np.ndarray:
        """[rows, steps] greedy tokens from every row's last forward."""
        out = np.empty((self.rows, steps), np.int32)
        self.device.bind()
        self.device.check_synced("tmh_llama_generate", self.device.lib.tmh_llama_generate(
            self.handle, steps, out.ctypes.data, 1 if graph else 0))
        return out

    def set_mode(self, mode: str) -> None:
        """BlockMatMulMode of the decoder's products: "auto" (the host's bits) or "unordered" (measurement only)."""
        check("tmh_llama_set_mode", self.device.lib.tmh_llama_set_mode(self.handle, MODES[mode]))

    def step(self, graph: bool = True) -> None:
        check("tmh_llama_step", self.device.lib.tmh_llama_step(self.handle, 1 if graph else 0))

    def length(self, row: int = 0) -> int:
        n = I32(0)
        check("tmh_llama_length", self.device.lib.tmh_llama_length(self.handle, row, ctypes.byref(n)))
        return n.value

    def reset(self, row: Optional[int] = None) -> None:
        for r in (range(self.rows) if row is None else [row]):
            check("tmh_llama_reset", self.device.lib.tmh_llama_reset(self.handle, r))

    def destroy(self) -> None:
        if getattr(self, "handle", 0):
            self.device.lib.tmh_llama_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
