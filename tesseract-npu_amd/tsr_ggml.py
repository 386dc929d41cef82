"""Python binding of libtsr_ggml (ctypes over include/tsr_ggml.h): the ggml-backend adapter that
decides placement (supports_op), holds the device's buffers (weights, KV planes, activations) and
lowers ggml graphs onto libtsr_hip (graph_compute, with the per-graph plan cache and HIP graph replay).

A ggml graph is described by ``Tensor`` records that mirror the ggml_tensor fields the adapter reads
(type, op, ne, nb, op_params, flags, sources, view source, data address, buffer, name). The library
must be built (``make -C tesseract-npu_amd``); there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtsr_ggml.so")

# include/tsr_ggml.h
OK, E_ARG, E_UNSUPPORTED, E_DEVICE, E_NOMEM, E_FLAG, E_NODEV = 0, -1, -2, -3, -4, -5, -6
F32, F16, BF16, Q8_0, Q4_K, I32, I64, FOREIGN = 0, 1, 2, 3, 4, 5, 6, 64
(OP_NONE, OP_RESHAPE, OP_VIEW, OP_PERMUTE, OP_TRANSPOSE, OP_MUL_MAT, OP_FLASH_ATTN_EXT, OP_SET_ROWS, OP_RMS_NORM,
 OP_MUL, OP_ADD, OP_ROPE, OP_GLU, OP_GET_ROWS, OP_ARGMAX, OP_SCALE, OP_UNARY) = range(17)
OP_OTHER = 255
GLU_SWIGLU, UNARY_TANH = 2, 1
FLAG_INPUT, FLAG_OUTPUT, FLAG_PARAM, FLAG_COMPUTE = 1, 2, 4, 16
USAGE_ANY, USAGE_WEIGHTS, USAGE_COMPUTE = 0, 1, 2
MODE_UNDECIDED, MODE_LINEAR, MODE_WEIGHTS, MODE_KV = 0, 1, 2, 3
(CALL_MUL_MAT, CALL_FLASH_ATTN, CALL_SET_ROWS, CALL_RMS_NORM, CALL_ADD, CALL_ROPE, CALL_SWIGLU, CALL_GET_ROWS,
 CALL_ARGMAX, CALL_ROPE_TABLE, CALL_ROPE_KV) = range(1, 12)
CALL_NAMES = {CALL_MUL_MAT: "MUL_MAT", CALL_FLASH_ATTN: "FLASH_ATTN_EXT", CALL_SET_ROWS: "SET_ROWS",
              CALL_RMS_NORM: "RMS_NORM", CALL_ADD: "ADD", CALL_ROPE: "ROPE", CALL_SWIGLU: "SWIGLU",
              CALL_GET_ROWS: "GET_ROWS", CALL_ARGMAX: "ARGMAX", CALL_ROPE_TABLE: "ROPE_TABLE", CALL_ROPE_KV: "ROPE_KV"}
CALL_IN_NEXT = 0x80000000    # flags: the call's work runs inside its group's FLASH_ATTN_EXT call

EXPORTS = (
    "tsr_gg_open", "tsr_gg_close", "tsr_gg_last_error", "tsr_gg_hip_ctx", "tsr_gg_register_type",
    "tsr_gg_alignment", "tsr_gg_alloc_size", "tsr_gg_buffer_alloc", "tsr_gg_buffer_set_usage", "tsr_gg_buffer_base",
    "tsr_gg_buffer_size", "tsr_gg_buffer_init_tensor", "tsr_gg_buffer_set_tensor", "tsr_gg_buffer_get_tensor",
    "tsr_gg_buffer_memset_tensor", "tsr_gg_buffer_clear", "tsr_gg_buffer_free", "tsr_gg_buffer_mode",
    "tsr_gg_supports_op", "tsr_gg_graph_compute", "tsr_gg_synchronize", "tsr_gg_get_stats", "tsr_gg_lower",
    "tsr_gg_kv_parse_name", "tsr_gg_graph_key", "tsr_gg_quantize_q8_0", "tsr_gg_set_options",
    "tsr_gg_buffer_cpy_tensor", "tsr_gg_buffer_reset", "tsr_gg_get_memory",
)
OPT_NO_FUSION = 1


class Tensor(C.Structure):
    pass


Tensor._fields_ = [
    ("type", C.c_int32), ("op", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4),
    ("op_params", C.c_int32 * 16), ("flags", C.c_int32), ("src", C.POINTER(Tensor) * 10),
    ("view_src", C.POINTER(Tensor)), ("view_offs", C.c_uint64), ("data", C.c_uint64), ("buffer", C.c_void_p),
    ("name", C.c_char * 64),
]


class Call(C.Structure):
    _fields_ = [
        ("kind", C.c_int32), ("node", C.c_int32), ("node2", C.c_int32), ("node3", C.c_int32),
        ("N", C.c_uint32), ("K", C.c_uint32), ("T", C.c_uint32), ("flags", C.c_uint32),
        ("x", C.c_uint64), ("y", C.c_uint64), ("add", C.c_uint64), ("w", C.c_uint64),
        ("x_stride", C.c_uint64), ("y_stride", C.c_uint64), ("add_stride", C.c_uint64),
        ("scale", C.c_float), ("scale2", C.c_float),
        ("D", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32), ("n_kv", C.c_uint32),
        ("kv_size", C.c_uint32), ("which", C.c_uint32), ("mode", C.c_uint32), ("n_dims", C.c_uint32),
    ]

    def as_dict(self) -> dict:
        d = {f: getattr(self, f) for f, _ in self._fields_}
        d["name"] = CALL_NAMES.get(self.kind, str(self.kind))
        return d


class Stats(C.Structure):
    _fields_ = [(f, C.c_uint64) for f in ("graphs", "plan_hits", "plan_misses", "captures", "replays", "eager_runs",
                                          "calls", "fused", "weights_converted", "masks_summarized")]


TO_FLOAT = C.CFUNCTYPE(None, C.c_void_p, C.POINTER(C.c_float), C.c_int64)


class GGError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what} ({code})")
        self.code = code


_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run `make -C {HERE}`")
    L = C.CDLL(path)
    vp, u32, u64, i32, sz = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_size_t
    TP = C.POINTER(Tensor)
    sig = {
        "tsr_gg_open": ([C.c_int, C.POINTER(vp)], C.c_int),
        "tsr_gg_close": ([vp], C.c_int),
        "tsr_gg_last_error": ([vp], C.c_char_p),
        "tsr_gg_hip_ctx": ([vp], vp),
        "tsr_gg_register_type": ([vp, C.c_char_p, u32, u32, TO_FLOAT, C.POINTER(i32)], C.c_int),
        "tsr_gg_alignment": ([], sz),
        "tsr_gg_alloc_size": ([vp, TP], sz),
        "tsr_gg_buffer_alloc": ([vp, sz, C.c_int, C.POINTER(vp)], C.c_int),
        "tsr_gg_buffer_set_usage": ([vp, C.c_int], C.c_int),
        "tsr_gg_buffer_base": ([vp], u64),
        "tsr_gg_buffer_size": ([vp], sz),
        "tsr_gg_buffer_init_tensor": ([vp, TP], C.c_int),
        "tsr_gg_buffer_set_tensor": ([vp, TP, vp, sz, sz], C.c_int),
        "tsr_gg_buffer_get_tensor": ([vp, TP, vp, sz, sz], C.c_int),
        "tsr_gg_buffer_memset_tensor": ([vp, TP, C.c_uint8, sz, sz], C.c_int),
        "tsr_gg_buffer_clear": ([vp, C.c_uint8], C.c_int),
        "tsr_gg_buffer_reset": ([vp], C.c_int),
        "tsr_gg_get_memory": ([vp, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)], C.c_int),
        "tsr_gg_buffer_free": ([vp], C.c_int),
        "tsr_gg_buffer_mode": ([vp], C.c_int),
        "tsr_gg_supports_op": ([vp, TP, C.c_char_p, sz], C.c_int),
        "tsr_gg_graph_compute": ([vp, C.POINTER(TP), C.c_int], C.c_int),
        "tsr_gg_synchronize": ([vp], C.c_int),
        "tsr_gg_get_stats": ([vp, C.POINTER(Stats)], C.c_int),
        "tsr_gg_lower": ([vp, C.POINTER(TP), C.c_int, C.POINTER(Call), C.c_int, C.POINTER(C.c_int)], C.c_int),
        "tsr_gg_kv_parse_name": ([C.c_char_p, C.POINTER(u32), C.POINTER(C.c_int)], C.c_int),
        "tsr_gg_graph_key": ([C.POINTER(TP), C.c_int, u64], u64),
        "tsr_gg_quantize_q8_0": ([vp, C.c_int64, vp], C.c_int),
        "tsr_gg_set_options": ([vp, u32], C.c_int),
        "tsr_gg_buffer_cpy_tensor": ([vp, TP, TP], C.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def _node_array(nodes):
    arr = (C.POINTER(Tensor) * max(1, len(nodes)))()
    for i, t in enumerate(nodes):
        arr[i] = C.pointer(t)
    return arr


def kv_parse_name(name: str):
    which, layer = C.c_uint32(), C.c_int()
    ok = load().tsr_gg_kv_parse_name(name.encode(), C.byref(which), C.byref(layer))
    return (int(which.value), int(layer.value)) if ok else None


def graph_key(nodes, salt: int = 0) -> int:
    return int(load().tsr_gg_graph_key(_node_array(nodes), len(nodes), salt))


def quantize_q8_0(x) -> np.ndarray:
    """f32 rows -> ggml block_q8_0 bytes (ggml's quantize_row_q8_0_ref)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * 34, np.uint8)
    rc = load().tsr_gg_quantize_q8_0(x.ctypes.data, x.size, out.ctypes.data)
    if rc:
        raise GGError(rc, "quantize_q8_0")
    return out


class Buffer:
    def __init__(self, dev: "Device", h: int):
        self.dev, self.h = dev, h

    @property
    def base(self) -> int:
        return int(self.dev.L.tsr_gg_buffer_base(self.h))

    @property
    def size(self) -> int:
        return int(self.dev.L.tsr_gg_buffer_size(self.h))

    @property
    def mode(self) -> int:
        return int(self.dev.L.tsr_gg_buffer_mode(self.h))

    def set_usage(self, usage: int) -> None:
        self.dev.check(self.dev.L.tsr_gg_buffer_set_usage(self.h, usage), "set_usage")

    def init_tensor(self, t: Tensor) -> None:
        self.dev.check(self.dev.L.tsr_gg_buffer_init_tensor(self.h, C.byref(t)), "init_tensor")

    def set_tensor(self, t: Tensor, data, offset: int = 0) -> None:
        a = np.ascontiguousarray(data)
        self.dev.check(self.dev.L.tsr_gg_buffer_set_tensor(self.h, C.byref(t), a.ctypes.data, offset, a.nbytes),
                       f"set_tensor {t.name.decode()}")

    def get_tensor(self, t: Tensor, nbytes: int, offset: int = 0) -> np.ndarray:
        out = np.empty(nbytes, np.uint8)
        self.dev.check(self.dev.L.tsr_gg_buffer_get_tensor(self.h, C.byref(t), out.ctypes.data, offset, nbytes),
                       f"get_tensor {t.name.decode()}")
        return out

    def memset_tensor(self, t: Tensor, value: int, offset: int, size: int) -> None:
        self.dev.check(self.dev.L.tsr_gg_buffer_memset_tensor(self.h, C.byref(t), value, offset, size), "memset_tensor")

    def cpy_tensor(self, src: Tensor, dst: Tensor) -> bool:
        rc = self.dev.L.tsr_gg_buffer_cpy_tensor(self.h, C.byref(src), C.byref(dst))
        if rc < 0:
            self.dev.check(rc, "cpy_tensor")
        return rc == 1

    def clear(self, value: int = 0) -> None:
        self.dev.check(self.dev.L.tsr_gg_buffer_clear(self.h, value), "clear")

    def reset(self) -> None:
        """ggml-alloc lays the buffer out anew (buffer_i.reset)."""
        self.dev.check(self.dev.L.tsr_gg_buffer_reset(self.h), "reset")

    def free(self) -> None:
        if self.h:
            self.dev.L.tsr_gg_buffer_free(self.h)
            self.h = None


class Device:
    """An adapter device: device >= 0 a GPU, -1 a probe device (placement questions only)."""

    def __init__(self, device: int = 0):
        self.L = load()
        h = C.c_void_p()
        rc = self.L.tsr_gg_open(device, C.byref(h))
        if rc:
            raise GGError(rc, f"tsr_gg_open({device})")
        self.h = h.value
        self._keep = []                      # ctypes callbacks registered with the device

    def error(self) -> str:
        return self.L.tsr_gg_last_error(self.h).decode()

    def check(self, rc: int, what: str) -> None:
        if rc:
            raise GGError(rc, f"{what}: {self.error()}")

    def close(self) -> None:
        if self.h:
            self.L.tsr_gg_close(self.h)
            self.h = None

    def buffer(self, size: int, usage: int = USAGE_ANY) -> Buffer:
        h = C.c_void_p()
        self.check(self.L.tsr_gg_buffer_alloc(self.h, size, usage, C.byref(h)), "buffer_alloc")
        return Buffer(self, h.value)

    def alloc_size(self, t: Tensor) -> int:
        return int(self.L.tsr_gg_alloc_size(self.h, C.byref(t)))

    def memory(self) -> tuple:
        """(free, total) bytes of the device's memory (device_i.get_memory)."""
        f, t = C.c_size_t(), C.c_size_t()
        self.check(self.L.tsr_gg_get_memory(self.h, C.byref(f), C.byref(t)), "get_memory")
        return int(f.value), int(t.value)

    def register_type(self, name: str, blck: int, tsize: int, to_float) -> int:
        cb = TO_FLOAT(to_float)
        self._keep.append(cb)
        tid = C.c_int32()
        self.check(self.L.tsr_gg_register_type(self.h, name.encode(), blck, tsize, cb, C.byref(tid)), "register_type")
        return int(tid.value)

    def supports_op(self, t: Tensor):
        why = C.create_string_buffer(512)
        rc = self.L.tsr_gg_supports_op(self.h, C.byref(t), why, 512)
        if rc < 0:
            raise GGError(rc, "supports_op")
        return bool(rc), why.value.decode()

    def graph_compute(self, nodes) -> None:
        """nodes: Tensor records, or an array from prepare() (built once, for a graph run many times)."""
        arr = nodes if isinstance(nodes, tuple) else (_node_array(nodes), len(nodes))
        self.check(self.L.tsr_gg_graph_compute(self.h, arr[0], arr[1]), "graph_compute")

    @staticmethod
    def prepare(nodes) -> tuple:
        return (_node_array(nodes), len(nodes))

    def set_options(self, options: int) -> None:
        self.check(self.L.tsr_gg_set_options(self.h, options), "set_options")

    def synchronize(self) -> None:
        self.check(self.L.tsr_gg_synchronize(self.h), "synchronize")

    def lower(self, nodes, cap: int = 4096) -> list:
        out = (Call * cap)()
        n = C.c_int()
        self.check(self.L.tsr_gg_lower(self.h, _node_array(nodes), len(nodes), out, cap, C.byref(n)), "lower")
        return [out[i].as_dict() for i in range(min(n.value, cap))]

    def stats(self) -> dict:
        s = Stats()
        self.check(self.L.tsr_gg_get_stats(self.h, C.byref(s)), "stats")
        return {f: int(getattr(s, f)) for f, _ in Stats._fields_}
