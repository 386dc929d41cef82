"""Python binding of libtsr_hip (ctypes over the C ABI of include/tsr_hip.h).

This is the host-side mirror of the reference's device interface for the hot path: a context
(the ggml backend's device), raw device buffers (set/get_tensor of activations), weights uploaded
from ggml blocks (set_tensor of a Q8_0 / Q4_K weight), MUL_MAT, QACT, the q8_0 KV cache
(SET_ROWS, get/set bytes) and FLASH_ATTN_EXT. Errors raise ``TsrHipError`` with the library's code.

The library must be built (``make -C tesseract-npu_amd``); there is no fallback: a missing library
raises at import of a context.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtsr_hip.so")

FMT_Q8_0, FMT_Q4_K = 0, 1
QA_A32, QA_A256 = 0, 1
KV_K, KV_V = 0, 1
MM_ACC_DST, MM_GLU, MM_SCALE, MM_SOFTCAP = 1, 2, 4, 8
ROPE_NORMAL, ROPE_NEOX, ROPE_IMROPE = 0, 2, 40

# the exported symbols of include/tsr_hip.h
EXPORTS = (
    "tsr_hip_open", "tsr_hip_close", "tsr_hip_strerror", "tsr_hip_stream", "tsr_hip_sync", "tsr_hip_device_info",
    "tsr_hip_alloc", "tsr_hip_free", "tsr_hip_write", "tsr_hip_read", "tsr_hip_memset",
    "tsr_hip_weight_upload", "tsr_hip_weight_read", "tsr_hip_weight_free", "tsr_hip_weight_info",
    "tsr_hip_qa_bytes", "tsr_hip_qact", "tsr_hip_mul_mat", "tsr_hip_mul_mat_isums",
    "tsr_hip_kv_create", "tsr_hip_kv_free", "tsr_hip_kv_set_bytes", "tsr_hip_kv_get_bytes", "tsr_hip_kv_set_rows",
    "tsr_hip_msum_build_f16", "tsr_hip_flash_attn", "tsr_hip_get_counters",
    "tsr_hip_rms_norm", "tsr_hip_rope", "tsr_hip_swiglu", "tsr_hip_add", "tsr_hip_get_rows", "tsr_hip_argmax",
    "tsr_hip_write_async", "tsr_hip_copy_async", "tsr_hip_fa_plan_create", "tsr_hip_fa_plan_set", "tsr_hip_flash_attn_plan",
    "tsr_hip_fa_plan_free", "tsr_hip_graph_begin", "tsr_hip_graph_end", "tsr_hip_graph_launch", "tsr_hip_graph_free",
    "tsr_hip_mul_mat_norm", "tsr_hip_rope_kv", "tsr_hip_flash_attn_plan_rope", "tsr_hip_rope_table",
    "tsr_hip_flash_attn_plan_rope_tab", "tsr_hip_mul_mat_epi", "tsr_hip_set_fa_wait_limit",
    "tsr_hip_flash_attn_noalloc", "tsr_hip_get_flags", "tsr_hip_msum_mask_f32", "tsr_hip_attn_qkv_plan_rope_tab",
    "tsr_hip_fa_plan_set_epoch",
)


class TsrHipError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {strerror(code)} ({code})")
        self.code = code


_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libtsr_hip.so (once)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run `make -C {HERE}`")
    L = C.CDLL(path)
    vp, u32, u64, i32, sz = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_size_t
    sig = {
        "tsr_hip_open": ([C.c_int, C.POINTER(vp)], C.c_int),
        "tsr_hip_close": ([vp], C.c_int),
        "tsr_hip_strerror": ([C.c_int], C.c_char_p),
        "tsr_hip_stream": ([vp], vp),
        "tsr_hip_sync": ([vp, vp], C.c_int),
        "tsr_hip_device_info": ([vp, C.POINTER(C.c_int), C.c_char_p, sz, C.POINTER(sz), C.POINTER(sz)], C.c_int),
        "tsr_hip_alloc": ([vp, sz, C.POINTER(vp)], C.c_int),
        "tsr_hip_free": ([vp, vp], C.c_int),
        "tsr_hip_write": ([vp, vp, vp, sz], C.c_int),
        "tsr_hip_read": ([vp, vp, vp, sz], C.c_int),
        "tsr_hip_memset": ([vp, vp, C.c_int, sz], C.c_int),
        "tsr_hip_weight_upload": ([vp, u32, vp, u32, u32, C.POINTER(vp)], C.c_int),
        "tsr_hip_weight_read": ([vp, vp, vp], C.c_int),
        "tsr_hip_weight_free": ([vp, vp], C.c_int),
        "tsr_hip_weight_info": ([vp, C.POINTER(u32), C.POINTER(u32), C.POINTER(u32), C.POINTER(sz)], C.c_int),
        "tsr_hip_qa_bytes": ([u32, u32], sz),
        "tsr_hip_qact": ([vp, u32, vp, u32, u32, u64, vp, vp], C.c_int),
        "tsr_hip_mul_mat": ([vp, vp, vp, u32, u64, vp, u64, vp, u64, u32, vp], C.c_int),
        "tsr_hip_mul_mat_isums": ([vp, vp, vp, vp, vp], C.c_int),
        "tsr_hip_kv_create": ([vp, u32, u32, C.POINTER(vp)], C.c_int),
        "tsr_hip_kv_free": ([vp, vp], C.c_int),
        "tsr_hip_kv_set_bytes": ([vp, vp, u32, sz, vp, sz], C.c_int),
        "tsr_hip_kv_get_bytes": ([vp, vp, u32, sz, vp, sz], C.c_int),
        "tsr_hip_kv_set_rows": ([vp, vp, u32, vp, u32, u64, vp, vp, vp], C.c_int),
        "tsr_hip_msum_build_f16": ([vp, sz, u32, u32, vp], C.c_int),
        "tsr_hip_msum_mask_f32": ([vp, sz, u32, u32, C.c_float, vp], C.c_int),
        "tsr_hip_get_flags": ([vp, C.POINTER(C.c_int32), C.c_int], C.c_int),
        "tsr_hip_flash_attn": ([vp, vp, u32, u64, vp, vp, u32, u32, u32, C.c_float, vp, vp, vp, u32, vp, u64, vp],
                               C.c_int),
        "tsr_hip_flash_attn_noalloc": ([vp, vp, u32, u64, vp, vp, u32, u32, u32, C.c_float, vp, vp, vp, u32, vp, u64,
                                        vp], C.c_int),
        "tsr_hip_get_counters": ([vp, vp], C.c_int),
        "tsr_hip_rms_norm": ([vp, vp, u32, u32, u64, C.c_float, vp, u64, u32, vp, u64, vp], C.c_int),
        "tsr_hip_rope": ([vp, vp, u32, u64, u32, u32, u32, C.c_int, vp, C.c_float, C.c_float, C.c_float, vp, vp, u64,
                          vp], C.c_int),
        "tsr_hip_swiglu": ([vp, vp, u64, vp, u64, u32, u32, vp, u64, vp], C.c_int),
        "tsr_hip_add": ([vp, vp, u64, vp, u64, u32, u32, u32, vp, u64, vp], C.c_int),
        "tsr_hip_get_rows": ([vp, vp, u64, u32, u32, vp, u32, vp, u64, vp, vp], C.c_int),
        "tsr_hip_argmax": ([vp, vp, u32, u32, u64, vp, vp], C.c_int),
        "tsr_hip_write_async": ([vp, vp, vp, sz, vp], C.c_int),
        "tsr_hip_copy_async": ([vp, vp, vp, sz, vp], C.c_int),
        "tsr_hip_fa_plan_create": ([vp, u32, u32, u32, u32, u32, C.POINTER(vp)], C.c_int),
        "tsr_hip_fa_plan_set": ([vp, vp, vp, C.c_int, vp, u32, C.POINTER(C.c_int), vp], C.c_int),
        "tsr_hip_flash_attn_plan": ([vp, vp, vp, u64, vp, vp, C.c_float, vp, vp, u64, vp], C.c_int),
        "tsr_hip_fa_plan_free": ([vp, vp], C.c_int),
        "tsr_hip_graph_begin": ([vp, vp], C.c_int),
        "tsr_hip_graph_end": ([vp, vp, C.POINTER(vp)], C.c_int),
        "tsr_hip_graph_launch": ([vp, vp, vp], C.c_int),
        "tsr_hip_graph_free": ([vp, vp], C.c_int),
        "tsr_hip_mul_mat_norm": ([vp, vp, vp, u32, u64, C.c_float, vp, vp, u64, vp, u64, u32, vp], C.c_int),
        "tsr_hip_rope_kv": ([vp, vp, u32, u64, u32, u32, u32, u32, C.c_int, vp, C.c_float, C.c_float, vp, vp, vp, vp,
                             vp], C.c_int),
        "tsr_hip_flash_attn_plan_rope": ([vp, vp, vp, vp, vp, C.c_float, u32, C.c_int, vp, C.c_float, C.c_float, vp, vp,
                                          vp, vp, u64, vp], C.c_int),
        "tsr_hip_rope_table": ([vp, vp, u32, C.c_float, C.c_float, vp, vp], C.c_int),
        "tsr_hip_mul_mat_epi": ([vp, vp, vp, u32, u64, vp, u64, vp, u64, u32, C.c_float, C.c_float, vp], C.c_int),
        "tsr_hip_set_fa_wait_limit": ([vp, u32], C.c_int),
        "tsr_hip_fa_plan_set_epoch": ([vp, vp, u32], C.c_int),
        "tsr_hip_flash_attn_plan_rope_tab": ([vp, vp, vp, vp, vp, C.c_float, u32, C.c_int, vp, vp, vp, vp, vp, u64, vp],
                                             C.c_int),
        "tsr_hip_attn_qkv_plan_rope_tab": ([vp, vp, vp, vp, C.c_float, vp, vp, vp, vp, C.c_float, u32, C.c_int, vp, vp,
                                            vp, vp, vp, u64, vp], C.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def strerror(code: int) -> str:
    return load().tsr_hip_strerror(code).decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise TsrHipError(rc, what)


def qa_bytes(kind: int, K: int) -> int:
    return int(load().tsr_hip_qa_bytes(kind, K))


def msum_build_f16(mask_f16) -> np.ndarray:
    """MSUM words of an f16 mask [n_q][n_kv] (host)."""
    m = np.ascontiguousarray(np.atleast_2d(mask_f16).view(np.uint16))
    n_q, n_kv = m.shape
    words = np.zeros(8 + 4 * n_q, np.uint32)
    rc = load().tsr_hip_msum_build_f16(m.ctypes.data, n_kv, n_kv, n_q, words.ctypes.data)
    if rc < 0:
        raise TsrHipError(rc, "msum_build_f16")
    return words


def msum_mask_f32(mask_f16, scale: float) -> np.ndarray:
    """The f32 mask copy of a GENERAL summary (host): [n_q, 16 ceil(n_kv / 16)] f32."""
    m = np.ascontiguousarray(mask_f16, np.float16)
    n_q, n_kv = m.shape
    out = np.empty((n_q, 16 * ((n_kv + 15) // 16)), np.float32)
    rc = load().tsr_hip_msum_mask_f32(m.ctypes.data, n_kv, n_kv, n_q, float(scale), out.ctypes.data)
    if rc < 0:
        raise TsrHipError(rc, "msum_mask_f32")
    return out


class Buffer:
    """A device allocation of the context (raw bytes)."""

    def __init__(self, dev: "Device", nbytes: int):
        self.dev, self.nbytes = dev, int(nbytes)
        p = C.c_void_p()
        _check(dev.L.tsr_hip_alloc(dev.ctx, self.nbytes, C.byref(p)), "alloc")
        self.ptr = p.value

    def write(self, arr, offset: int = 0) -> "Buffer":
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("write beyond the buffer")
        _check(self.dev.L.tsr_hip_write(self.dev.ctx, self.ptr + offset, a.ctypes.data, a.nbytes), "write")
        return self

    def read(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("read beyond the buffer")
        _check(self.dev.L.tsr_hip_read(self.dev.ctx, out.ctypes.data, self.ptr + offset, out.nbytes), "read")
        return out

    def fill(self, value: int = 0) -> "Buffer":
        _check(self.dev.L.tsr_hip_memset(self.dev.ctx, self.ptr, value, self.nbytes), "memset")
        return self

    def free(self) -> None:
        if self.ptr:
            self.dev.L.tsr_hip_free(self.dev.ctx, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    def __init__(self, dev: "Device", fmt: int, blocks, N: int, K: int):
        self.dev, self.fmt, self.N, self.K = dev, fmt, N, K
        b = np.ascontiguousarray(blocks, np.uint8)
        h = C.c_void_p()
        _check(dev.L.tsr_hip_weight_upload(dev.ctx, fmt, b.ctypes.data, N, K, C.byref(h)), "weight_upload")
        self.h = h.value

    def read(self) -> np.ndarray:
        rb = self.K // 32 * 34 if self.fmt == FMT_Q8_0 else self.K // 256 * 144
        out = np.empty((self.N, rb), np.uint8)
        _check(self.dev.L.tsr_hip_weight_read(self.dev.ctx, self.h, out.ctypes.data), "weight_read")
        return out

    def dev_bytes(self) -> int:
        n = C.c_size_t()
        _check(self.dev.L.tsr_hip_weight_info(self.h, None, None, None, C.byref(n)), "weight_info")
        return n.value

    def free(self) -> None:
        if self.h:
            self.dev.L.tsr_hip_weight_free(self.dev.ctx, self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class KvCache:
    def __init__(self, dev: "Device", E: int, kv_size: int):
        self.dev, self.E, self.kv_size = dev, E, kv_size
        h = C.c_void_p()
        _check(dev.L.tsr_hip_kv_create(dev.ctx, E, kv_size, C.byref(h)), "kv_create")
        self.h = h.value

    @property
    def row_bytes(self) -> int:
        return self.E // 32 * 34

    def set_bytes(self, which: int, data, off: int = 0) -> None:
        a = np.ascontiguousarray(data, np.uint8)
        _check(self.dev.L.tsr_hip_kv_set_bytes(self.dev.ctx, self.h, which, off, a.ctypes.data, a.nbytes), "kv_set_bytes")

    def get_bytes(self, which: int, off: int = 0, nbytes: int | None = None) -> np.ndarray:
        n = self.kv_size * self.row_bytes - off if nbytes is None else nbytes
        out = np.empty(n, np.uint8)
        _check(self.dev.L.tsr_hip_kv_get_bytes(self.dev.ctx, self.h, which, off, out.ctypes.data, n), "kv_get_bytes")
        return out

    def free(self) -> None:
        if self.h:
            self.dev.L.tsr_hip_kv_free(self.dev.ctx, self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class FaPlan:
    """A FLASH_ATTN_EXT work list in device memory (tsr_hip_fa_plan_*)."""

    def __init__(self, dev: "Device", D: int, n_head: int, n_head_kv: int, T: int, kv_size: int):
        self.dev = dev
        h = C.c_void_p()
        _check(dev.L.tsr_hip_fa_plan_create(dev.ctx, D, n_head, n_head_kv, T, kv_size, C.byref(h)), "fa_plan_create")
        self.h = h.value

    def set(self, msum, new_runs=None, mask_f32: bool = False, stream=None) -> bool:
        """Plans the MSUM words; True when the list's shape changed (captured launches are stale)."""
        words = np.ascontiguousarray(msum, np.uint32)
        nr = None if new_runs is None else np.ascontiguousarray(new_runs, np.uint32).reshape(-1, 2)
        ch = C.c_int()
        _check(self.dev.L.tsr_hip_fa_plan_set(self.dev.ctx, self.h, words.ctypes.data, int(mask_f32),
                                              None if nr is None else nr.ctypes.data, 0 if nr is None else nr.shape[0],
                                              C.byref(ch), stream), "fa_plan_set")
        return bool(ch.value)

    def set_epoch(self, epoch: int) -> None:
        """Test hook: every KV head's epoch word of the one-launch decode form (the next launch's tag
        follows it)."""
        _check(self.dev.L.tsr_hip_fa_plan_set_epoch(self.dev.ctx, self.h, epoch), "fa_plan_set_epoch")

    def free(self) -> None:
        if self.h:
            self.dev.L.tsr_hip_fa_plan_free(self.dev.ctx, self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Graph:
    """Launches recorded between Device.graph_begin and graph_end, replayed by launch()."""

    def __init__(self, dev: "Device", h: int):
        self.dev, self.h = dev, h

    def launch(self, stream=None) -> None:
        _check(self.dev.L.tsr_hip_graph_launch(self.dev.ctx, self.h, stream), "graph_launch")

    def free(self) -> None:
        if self.h:
            self.dev.L.tsr_hip_graph_free(self.dev.ctx, self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Device:
    """A libtsr_hip context on one GPU."""

    def __init__(self, device: int = 0):
        self.L = load()
        h = C.c_void_p()
        _check(self.L.tsr_hip_open(device, C.byref(h)), "open")
        self.ctx = h.value

    def close(self) -> None:
        if self.ctx:
            self.L.tsr_hip_close(self.ctx)
            self.ctx = None

    @property
    def stream(self) -> int:
        return self.L.tsr_hip_stream(self.ctx)

    def sync(self, stream=None) -> None:
        _check(self.L.tsr_hip_sync(self.ctx, stream), "sync")

    def get_flags(self, clear: bool = True) -> int:
        """The context's device flag word (kernels given no flag word of their own raise it)."""
        v = C.c_int32()
        _check(self.L.tsr_hip_get_flags(self.ctx, C.byref(v), int(clear)), "get_flags")
        return int(v.value)

    def info(self) -> dict:
        n = C.c_int()
        name = C.create_string_buffer(128)
        f, t = C.c_size_t(), C.c_size_t()
        _check(self.L.tsr_hip_device_info(self.ctx, C.byref(n), name, 128, C.byref(f), C.byref(t)), "device_info")
        return {"n_cu": n.value, "arch": name.value.decode(), "mem_free": f.value, "mem_total": t.value}

    def counters(self) -> dict:
        keys = ("mul_mat_calls", "mul_mat_rows", "mul_mat_weight_bytes", "flash_attn_calls", "flash_attn_kv_bytes",
                "set_rows_calls", "qact_calls", "fa_dec_launches", "fa_dec_qkv_launches")
        buf = (C.c_uint64 * len(keys))()
        _check(self.L.tsr_hip_get_counters(self.ctx, buf), "get_counters")
        return dict(zip(keys, list(buf)))

    # -- buffers ---------------------------------------------------------------------------------
    def alloc(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def upload(self, arr) -> Buffer:
        a = np.ascontiguousarray(arr)
        return Buffer(self, max(a.nbytes, 1)).write(a)

    def weight(self, fmt: int, blocks, N: int, K: int) -> Weight:
        return Weight(self, fmt, blocks, N, K)

    def kv(self, E: int, kv_size: int) -> KvCache:
        return KvCache(self, E, kv_size)

    # -- ops (device pointers are ints or Buffers) -----------------------------------------------
    @staticmethod
    def _p(x) -> int | None:
        if x is None:
            return None
        return x.ptr if isinstance(x, Buffer) else int(x)

    def qact(self, kind: int, x, K: int, T: int, x_stride: int, qa, stream=None) -> None:
        _check(self.L.tsr_hip_qact(self.ctx, kind, self._p(x), K, T, x_stride, self._p(qa), stream), "qact")

    def mul_mat(self, w: Weight, x, T: int, x_stride: int, y, y_stride: int, add=None, add_stride: int = 0,
                flags: int = 0, stream=None) -> None:
        _check(self.L.tsr_hip_mul_mat(self.ctx, w.h, self._p(x), T, x_stride, self._p(y), y_stride, self._p(add),
                                      add_stride, flags, stream), "mul_mat")

    def mul_mat_epi(self, w: "Weight", x, T: int, x_stride: int, y, y_stride: int, flags: int, first_scale: float,
                    scale: float, add=None, add_stride: int = 0, stream=None) -> None:
        """mul_mat with the SCALE / SOFTCAP epilogue of flags (MM_SCALE, MM_SOFTCAP) after the addend / ACC."""
        _check(self.L.tsr_hip_mul_mat_epi(self.ctx, w.h, self._p(x), T, x_stride, self._p(y), y_stride, self._p(add),
                                          add_stride, flags, float(first_scale), float(scale), stream), "mul_mat_epi")

    def mul_mat_norm(self, w: Weight, x, T: int, x_stride: int, eps: float, norm_w, y, y_stride: int, add=None,
                     add_stride: int = 0, flags: int = 0, stream=None) -> None:
        """MUL_MAT of RMS_NORM(x) * norm_w (norm_w None: no MUL) in one launch; flags as mul_mat (MM_GLU:
        rows 2j, 2j+1 of w are gate / up of output j, y[j] = SWIGLU(gate, up))."""
        _check(self.L.tsr_hip_mul_mat_norm(self.ctx, w.h, self._p(x), T, x_stride, float(eps), self._p(norm_w),
                                           self._p(y), y_stride, self._p(add), add_stride, flags, stream),
               "mul_mat_norm")

    def rope_kv(self, qkv, T: int, stride: int, head_dim: int, n_head: int, n_head_kv: int, n_dims: int, mode: int,
                pos, freq_base: float, kc: KvCache, vc: KvCache, cell, bad=None, attn_factor: float = 1.0,
                stream=None) -> None:
        """ROPE of the q and k heads of fused Q|K|V rows in place, then SET_ROWS_KV of k and v, in one launch."""
        _check(self.L.tsr_hip_rope_kv(self.ctx, self._p(qkv), T, stride, head_dim, n_head, n_head_kv, n_dims, mode,
                                      self._p(pos), float(freq_base), float(attn_factor), kc.h, vc.h, self._p(cell),
                                      self._p(bad), stream), "rope_kv")

    def mul_mat_isums(self, w: Weight, x, isums, stream=None) -> None:
        _check(self.L.tsr_hip_mul_mat_isums(self.ctx, w.h, self._p(x), self._p(isums), stream), "mul_mat_isums")

    def kv_set_rows(self, kv: KvCache, which: int, src, n_rows: int, src_stride: int, idx, bad=None,
                    stream=None) -> None:
        _check(self.L.tsr_hip_kv_set_rows(self.ctx, kv.h, which, self._p(src), n_rows, src_stride, self._p(idx),
                                          self._p(bad), stream), "kv_set_rows")

    def flash_attn(self, q, T: int, q_stride: int, kc: KvCache, vc: KvCache, D: int, n_head: int, n_head_kv: int,
                   scale: float, msum, out, out_stride: int, mask_f32=None, new_runs=None, stream=None) -> None:
        words = np.ascontiguousarray(msum, np.uint32)
        nr = None if new_runs is None else np.ascontiguousarray(new_runs, np.uint32).reshape(-1, 2)
        _check(self.L.tsr_hip_flash_attn(self.ctx, self._p(q), T, q_stride, kc.h, vc.h, D, n_head, n_head_kv,
                                         float(scale), words.ctypes.data, self._p(mask_f32),
                                         None if nr is None else nr.ctypes.data, 0 if nr is None else nr.shape[0],
                                         self._p(out), out_stride, stream), "flash_attn")

    def flash_attn_noalloc(self, q, T: int, q_stride: int, kc: KvCache, vc: KvCache, D: int, n_head: int,
                           n_head_kv: int, scale: float, msum, out, out_stride: int, mask_f32=None, new_runs=None,
                           stream=None) -> None:
        """flash_attn through the entry point that allocates nothing (its partials in the library's fixed
        device array: T <= 8, <= 48 chunks, <= 16 MiB of partials)."""
        words = np.ascontiguousarray(msum, np.uint32)
        nr = None if new_runs is None else np.ascontiguousarray(new_runs, np.uint32).reshape(-1, 2)
        _check(self.L.tsr_hip_flash_attn_noalloc(self.ctx, self._p(q), T, q_stride, kc.h, vc.h, D, n_head, n_head_kv,
                                                 float(scale), words.ctypes.data, self._p(mask_f32),
                                                 None if nr is None else nr.ctypes.data,
                                                 0 if nr is None else nr.shape[0], self._p(out), out_stride, stream),
               "flash_attn_noalloc")

    def write_async(self, dst, arr, stream=None) -> None:
        """Stream-ordered host-to-device copy of arr (<= 16 KiB); arr may be reused at once."""
        a = np.ascontiguousarray(arr)
        _check(self.L.tsr_hip_write_async(self.ctx, self._p(dst), a.ctypes.data, a.nbytes, stream), "write_async")

    def copy_async(self, dst, src, nbytes: int, stream=None) -> None:
        _check(self.L.tsr_hip_copy_async(self.ctx, self._p(dst), self._p(src), nbytes, stream), "copy_async")

    def fa_plan(self, D: int, n_head: int, n_head_kv: int, T: int, kv_size: int) -> "FaPlan":
        return FaPlan(self, D, n_head, n_head_kv, T, kv_size)

    def flash_attn_plan(self, plan: "FaPlan", q, q_stride: int, kc: KvCache, vc: KvCache, scale: float, out,
                        out_stride: int, mask_f32=None, stream=None) -> None:
        _check(self.L.tsr_hip_flash_attn_plan(self.ctx, plan.h, self._p(q), q_stride, kc.h, vc.h, float(scale),
                                              self._p(mask_f32), self._p(out), out_stride, stream), "flash_attn_plan")

    def flash_attn_plan_rope(self, plan: "FaPlan", qkv, kc: KvCache, vc: KvCache, scale: float, n_dims: int, mode: int,
                             pos, freq_base: float, cell, out, out_stride: int, bad=None, attn_factor: float = 1.0,
                             mask_f32=None, stream=None) -> None:
        """One decode token's ROPE + SET_ROWS_KV + planned FLASH_ATTN_EXT (qkv: the unrotated Q|K|V row)."""
        _check(self.L.tsr_hip_flash_attn_plan_rope(self.ctx, plan.h, self._p(qkv), kc.h, vc.h, float(scale), n_dims, mode,
                                                   self._p(pos), float(freq_base), float(attn_factor), self._p(cell),
                                                   self._p(bad), self._p(mask_f32), self._p(out), out_stride, stream),
               "flash_attn_plan_rope")

    def set_fa_wait_limit(self, polls: int) -> None:
        """Polls of the fused decode FA's bounded wait (0: the default)."""
        _check(self.L.tsr_hip_set_fa_wait_limit(self.ctx, polls), "set_fa_wait_limit")

    def rope_table(self, pos, n_dims: int, freq_base: float, tab, attn_factor: float = 1.0, stream=None) -> None:
        """The ROPE angles of position *pos: tab[2 i], tab[2 i + 1] = M cos, M sin of theta_i, i < n_dims / 2."""
        _check(self.L.tsr_hip_rope_table(self.ctx, self._p(pos), n_dims, float(freq_base), float(attn_factor),
                                         self._p(tab), stream), "rope_table")

    def flash_attn_plan_rope_tab(self, plan: "FaPlan", qkv, kc: KvCache, vc: KvCache, scale: float, n_dims: int,
                                 mode: int, tab, cell, out, out_stride: int, bad=None, mask_f32=None, stream=None) -> None:
        """flash_attn_plan_rope with the angles from a rope_table of the token's position."""
        _check(self.L.tsr_hip_flash_attn_plan_rope_tab(self.ctx, plan.h, self._p(qkv), kc.h, vc.h, float(scale), n_dims,
                                                       mode, self._p(tab), self._p(cell), self._p(bad),
                                                       self._p(mask_f32), self._p(out), out_stride, stream),
               "flash_attn_plan_rope_tab")

    def attn_qkv_plan_rope_tab(self, plan: "FaPlan", w_qkv: Weight, x, eps: float, norm_w, qkv, kc: KvCache,
                               vc: KvCache, scale: float, n_dims: int, mode: int, tab, cell, out, out_stride: int,
                               bad=None, mask_f32=None, stream=None) -> None:
        """mul_mat_norm(w_qkv, x, 1, ..., eps, norm_w -> qkv) then flash_attn_plan_rope_tab(plan, qkv, ...), in
        one launch where the decode form allows it (same bits either way)."""
        _check(self.L.tsr_hip_attn_qkv_plan_rope_tab(self.ctx, plan.h, w_qkv.h, self._p(x), float(eps), self._p(norm_w),
                                                     self._p(qkv), kc.h, vc.h, float(scale), n_dims, mode,
                                                     self._p(tab), self._p(cell), self._p(bad), self._p(mask_f32),
                                                     self._p(out), out_stride, stream),
               "attn_qkv_plan_rope_tab")

    def graph_begin(self, stream=None) -> None:
        _check(self.L.tsr_hip_graph_begin(self.ctx, stream), "graph_begin")

    def graph_end(self, stream=None) -> "Graph":
        h = C.c_void_p()
        _check(self.L.tsr_hip_graph_end(self.ctx, stream, C.byref(h)), "graph_end")
        return Graph(self, h.value)

    # -- decode-layer glue ops (rows of n f32; strides in floats) -------------------------------------
    def rms_norm(self, x, n: int, rows: int, x_stride: int, eps: float, y, y_stride: int, w=None, w_stride: int = 0,
                 w_period: int = 1, stream=None) -> None:
        _check(self.L.tsr_hip_rms_norm(self.ctx, self._p(x), n, rows, x_stride, float(eps), self._p(w), w_stride,
                                       w_period, self._p(y), y_stride, stream), "rms_norm")

    def rope(self, x, T: int, x_stride: int, head_dim: int, n_heads: int, n_dims: int, mode: int, pos,
             freq_base: float, y, y_stride: int, freq_scale: float = 1.0, attn_factor: float = 1.0,
             freq_factors=None, stream=None) -> None:
        _check(self.L.tsr_hip_rope(self.ctx, self._p(x), T, x_stride, head_dim, n_heads, n_dims, mode, self._p(pos),
                                   float(freq_base), float(freq_scale), float(attn_factor), self._p(freq_factors),
                                   self._p(y), y_stride, stream), "rope")

    def swiglu(self, g, g_stride: int, u, u_stride: int, n: int, rows: int, y, y_stride: int, stream=None) -> None:
        _check(self.L.tsr_hip_swiglu(self.ctx, self._p(g), g_stride, self._p(u), u_stride, n, rows, self._p(y),
                                     y_stride, stream), "swiglu")

    def add(self, a, a_stride: int, b, b_stride: int, n: int, rows: int, y, y_stride: int, b_period: int = 1,
            stream=None) -> None:
        _check(self.L.tsr_hip_add(self.ctx, self._p(a), a_stride, self._p(b), b_stride, b_period, n, rows,
                                  self._p(y), y_stride, stream), "add")

    def get_rows(self, src, src_stride: int, n: int, n_src: int, ids, count: int, y, y_stride: int, bad=None,
                 stream=None) -> None:
        _check(self.L.tsr_hip_get_rows(self.ctx, self._p(src), src_stride, n, n_src, self._p(ids), count, self._p(y),
                                       y_stride, self._p(bad), stream), "get_rows")

    def argmax(self, x, n: int, rows: int, x_stride: int, out, stream=None) -> None:
        _check(self.L.tsr_hip_argmax(self.ctx, self._p(x), n, rows, x_stride, self._p(out), stream), "argmax")

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
