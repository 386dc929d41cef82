"""ctypes access to the CPU checkers. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module. It loads

* ``liboracle.so`` -- this repository's C restatement of the reference numerics (oc_num.c, oc_attn.c),
* ``_ref/libtsr_ref.so`` -- the reference's own numerics library (sw/sim/tsr_ref.c, tsr_ref_at.c,
  tsr_ref_math.c) compiled in place by ``make ref``; used to pin the restatement.

Both take and return numpy arrays. Weight rows are ggml blocks (block_q8_0 34 B, block_q4_K 144 B);
KV caches are llama.cpp q8_0 images [kv_size][E/32 blocks].
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
FMT_Q8_0, FMT_Q4_K = 0, 1
QA_A32, QA_A256 = 0, 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref/libtsr_ref.so where /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if ref and os.path.isdir(os.environ.get("TSR_REFERENCE", "/root/reference")):
        subprocess.run(["make", "-s", "-C", HERE, "ref",
                        "REF=" + os.environ.get("TSR_REFERENCE", "/root/reference")], check=True)


def row_bytes(fmt: int, K: int) -> int:
    return K // 32 * 34 if fmt == FMT_Q8_0 else K // 256 * 144


def qa_bytes(kind: int, K: int) -> int:
    bs = 32 if kind == QA_A32 else 256
    n = -(-K // 64) * 64 + -(-(4 * (K // bs)) // 64) * 64
    if kind == QA_A256:
        n += -(-(2 * (K // 16)) // 64) * 64
    return n


def qa_d_off(K: int) -> int:
    return -(-K // 64) * 64


def qa_bs_off(kind: int, K: int) -> int:
    bs = 32 if kind == QA_A32 else 256
    return qa_d_off(K) + -(-(4 * (K // bs)) // 64) * 64


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path: str | None = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build(ref=False)
        L = self.lib = C.CDLL(path)
        L.oc_fop_n.argtypes = [C.c_int, _f32p, _f32p, _f32p, C.c_size_t]
        L.oc_f2h_n.argtypes = [_f32p, _u16p, C.c_size_t]
        L.oc_h2f_n.argtypes = [_u16p, _f32p, C.c_size_t]
        L.oc_i2f_n.argtypes = [_i32p, _f32p, C.c_size_t]
        L.oc_round8_n.argtypes = [C.c_int, _f32p, _i32p, C.c_size_t]
        L.oc_qact_n.argtypes = [C.c_uint32, _f32p, C.c_uint32, C.c_uint32, C.c_uint64, _u8p]
        L.oc_isums_n.argtypes = [C.c_uint32, _u8p, C.c_uint32, C.c_uint32, _u8p, _i32p]
        L.oc_mul_mat.argtypes = [C.c_uint32, _u8p, C.c_uint32, C.c_uint32, _f32p, C.c_uint32, C.c_uint64,
                                 C.c_void_p, C.c_uint64, _f32p, C.c_uint64, C.c_uint32]
        L.oc_expk_n.argtypes = [_f32p, _f32p, C.c_size_t]
        L.oc_maxt_n.argtypes = [_f32p, _f32p, _f32p, C.c_size_t]
        L.oc_bf_f_n.argtypes = [_i64p, _i32p, _f32p, C.c_size_t]
        L.oc_bf_int_n.argtypes = [_f32p, _i32p, _i32p, C.c_size_t]
        L.oc_tree16.argtypes = [_f32p]
        L.oc_tree16.restype = C.c_float
        L.oc_msum_build.argtypes = [_u16p, C.c_size_t, C.c_uint32, C.c_uint32, _u32p]
        L.oc_msum_build.restype = C.c_uint32
        L.oc_mask_f32.argtypes = [_u16p, C.c_size_t, C.c_uint32, C.c_uint32, C.c_float, _f32p]
        L.oc_kv_set_rows.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint64, _i64p, _u8p]
        L.oc_flash_attn.argtypes = [_f32p, C.c_uint32, C.c_uint64, _u8p, _u8p, C.c_uint32, C.c_uint32,
                                    C.c_uint32, C.c_uint32, C.c_float, _u32p, C.c_void_p, C.c_void_p,
                                    C.c_uint32, _f32p, C.c_uint64]
        L.oc_flash_attn.restype = C.c_int
        L.oc_fa_plan_row.argtypes = [C.c_uint32, C.c_uint32, _u32p, C.c_uint32, C.c_void_p, C.c_uint32,
                                     C.c_void_p, C.c_size_t]
        L.oc_fa_plan_row.restype = C.c_long
        L.oc_rms_norm_rows.argtypes = [C.c_uint32, C.c_uint32, _f32p, C.c_uint64, C.c_float, C.c_float, C.c_void_p,
                                       C.c_uint64, C.c_uint32, _f32p, C.c_uint64]
        L.oc_sincos.argtypes = [C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.oc_rope.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _f32p, C.c_uint64, _f32p,
                              C.c_uint64, _i32p, C.c_float, C.c_float, C.c_float, C.c_void_p]
        L.oc_silu.argtypes = [C.c_float]
        L.oc_silu.restype = C.c_float
        L.oc_tanh.argtypes = [C.c_float]
        L.oc_tanh.restype = C.c_float
        L.oc_mm_epilogue.argtypes = [_f32p, C.c_uint64, C.c_uint32, C.c_float, C.c_float]
        L.oc_swiglu_rows.argtypes = [C.c_uint32, C.c_uint32, _f32p, C.c_uint64, _f32p, C.c_uint64, _f32p, C.c_uint64]
        L.oc_add_rows.argtypes = [C.c_uint32, C.c_uint32, _f32p, C.c_uint64, _f32p, C.c_uint64, _f32p, C.c_uint64]
        L.oc_get_rows.argtypes = [C.c_uint32, _f32p, C.c_uint64, _i32p, C.c_uint32, _f32p, C.c_uint64]
        L.oc_argmax_rows.argtypes = [C.c_uint32, C.c_uint32, _f32p, C.c_uint64, _i32p]

    # -- scalar rules, vectorised ---------------------------------------------------------------
    def fop(self, op: str, a, b=None) -> np.ndarray:
        code = {"add": 0, "sub": 1, "mul": 2, "div": 3, "recip": 4}[op]
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(a if b is None else b, np.float32)
        out = np.empty_like(a)
        self.lib.oc_fop_n(code, a, b, out, a.size)
        return out

    def f2h(self, x) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.oc_f2h_n(x, out, x.size)
        return out

    def h2f(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.oc_h2f_n(h, out, h.size)
        return out

    def i2f(self, v) -> np.ndarray:
        v = np.ascontiguousarray(v, np.int32)
        out = np.empty(v.shape, np.float32)
        self.lib.oc_i2f_n(v, out, v.size)
        return out

    def round8(self, x, even: bool) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.int32)
        self.lib.oc_round8_n(1 if even else 0, x, out, x.size)
        return out

    def tree16(self, p) -> float:
        return self.lib.oc_tree16(np.ascontiguousarray(p, np.float32))

    def expk(self, v) -> np.ndarray:
        v = np.ascontiguousarray(v, np.float32)
        out = np.empty_like(v)
        self.lib.oc_expk_n(v, out, v.size)
        return out

    def maxt(self, a, b) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty_like(a)
        self.lib.oc_maxt_n(a, b, out, a.size)
        return out

    def bf_f(self, A, k) -> np.ndarray:
        A = np.ascontiguousarray(A, np.int64)
        k = np.ascontiguousarray(np.broadcast_to(k, A.shape), np.int32)
        out = np.empty(A.shape, np.float32)
        self.lib.oc_bf_f_n(A, k, out, A.size)
        return out

    def bf_int(self, w, es) -> np.ndarray:
        w = np.ascontiguousarray(w, np.float32)
        es = np.ascontiguousarray(np.broadcast_to(es, w.shape), np.int32)
        out = np.empty(w.shape, np.int32)
        self.lib.oc_bf_int_n(w, es, out, w.size)
        return out

    # -- QACT / MVM ------------------------------------------------------------------------------
    def qact(self, kind: int, x) -> np.ndarray:
        """QA images of the rows of x ([T][K] f32): uint8 [T][qa_bytes]."""
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        T, K = x.shape
        out = np.zeros((T, qa_bytes(kind, K)), np.uint8)
        self.lib.oc_qact_n(kind, x, K, T, K, out)
        return out

    def isums(self, fmt: int, w, K: int, qa) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        N = w.shape[0]
        per = K // 32 if fmt == FMT_Q8_0 else 2 * (K // 256)
        out = np.empty((N, per), np.int32)
        self.lib.oc_isums_n(fmt, w, N, K, np.ascontiguousarray(qa, np.uint8).ravel(), out)
        return out

    def mul_mat(self, fmt: int, w, K: int, x, add=None, threads: int = 1, epi=None) -> np.ndarray:
        """y[T][N] = MUL_MAT(w [N][row_bytes], x [T][K]); add: [T][N] addend (or [1][N]); epi:
        (1, _, scale) SCALE or (2, first_scale, scale) SOFTCAP after the addend."""
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        N, T = w.shape[0], x.shape[0]
        y = np.empty((T, N), np.float32)
        add_p, add_s = None, 0
        if add is not None:
            add = np.ascontiguousarray(np.atleast_2d(add), np.float32)
            add_p, add_s = add.ctypes.data, (N if add.shape[0] > 1 else 0)
        self.lib.oc_mul_mat(fmt, w, N, K, x, T, K, add_p, add_s, y, N, threads)
        if epi is not None:
            self.lib.oc_mm_epilogue(y, y.size, int(epi[0]), float(epi[1]), float(epi[2]))
        return y

    # -- attention -------------------------------------------------------------------------------
    def msum(self, mask_f16) -> np.ndarray:
        m = np.ascontiguousarray(np.atleast_2d(mask_f16).view(np.uint16))
        n_q, n_kv = m.shape
        words = np.zeros(8 + 4 * n_q, np.uint32)
        self.lib.oc_msum_build(m, n_kv, n_kv, n_q, words)
        return words

    def mask_f32(self, mask_f16, scale: float) -> np.ndarray:
        m = np.ascontiguousarray(np.atleast_2d(mask_f16).view(np.uint16))
        n_q, n_kv = m.shape
        out = np.empty((n_q, 16 * (-(-n_kv // 16))), np.float32)
        self.lib.oc_mask_f32(m, n_kv, n_kv, n_q, scale, out)
        return out

    def kv_set_rows(self, cache, src, idx) -> None:
        src = np.ascontiguousarray(np.atleast_2d(src), np.float32)
        idx = np.ascontiguousarray(idx, np.int64)
        E = src.shape[1]
        self.lib.oc_kv_set_rows(src, E, src.shape[0], E, idx, cache)

    def plan_row(self, E: int, D: int, msum, q: int, new_runs=None) -> list[tuple]:
        nr = None if new_runs is None else np.ascontiguousarray(new_runs, np.uint32).reshape(-1, 2)
        nrp, nn = (None, 0) if nr is None else (nr.ctypes.data, nr.shape[0])
        n = self.lib.oc_fa_plan_row(E, D, msum, q, nrp, nn, None, 0)
        if n < 0:
            raise ValueError(f"plan error {n}")
        buf = np.zeros((n, 5), np.uint32)
        self.lib.oc_fa_plan_row(E, D, msum, q, nrp, nn, buf.ctypes.data, n)
        return [tuple(int(v) for v in r) for r in buf]

    def flash_attn(self, q, kc, vc, D: int, n_head: int, n_head_kv: int, scale: float, msum,
                   mask_f32=None, new_runs=None) -> np.ndarray:
        q = np.ascontiguousarray(np.atleast_2d(q), np.float32).reshape(-1, n_head * D)
        T = q.shape[0]
        kv_size = kc.shape[0]
        out = np.empty((T, n_head * D), np.float32)
        mf = None if mask_f32 is None else np.ascontiguousarray(mask_f32, np.float32)
        nr = None if new_runs is None else np.ascontiguousarray(new_runs, np.uint32).reshape(-1, 2)
        rc = self.lib.oc_flash_attn(q, T, n_head * D, np.ascontiguousarray(kc), np.ascontiguousarray(vc), kv_size,
                                    D, n_head, n_head_kv, scale, np.ascontiguousarray(msum, np.uint32),
                                    None if mf is None else mf.ctypes.data,
                                    None if nr is None else nr.ctypes.data, 0 if nr is None else nr.shape[0],
                                    out, n_head * D)
        if rc != 0:
            raise ValueError(f"oc_flash_attn failed: {rc}")
        return out


# ----------------------------------------------------------------------------------------------
# The reference library (pinning only)
# ----------------------------------------------------------------------------------------------
class _KvGeom(C.Structure):
    _fields_ = [("E", C.c_uint32), ("C", C.c_uint32), ("LG", C.c_uint32)]


class _AttCfg(C.Structure):
    _fields_ = [("C", C.c_uint32), ("t_max", C.c_uint32), ("pcap", C.c_uint32), ("k_max", C.c_uint32)]


class _Msum(C.Structure):
    _fields_ = [("n_q", C.c_uint32), ("n_kv", C.c_uint32), ("flags", C.c_uint32), ("rows", C.c_void_p)]


class _FaArgs(C.Structure):
    _fields_ = [("T", C.c_uint32), ("D", C.c_uint32), ("G", C.c_uint32), ("scale", C.c_float),
                ("q", C.c_void_p), ("E", C.c_uint32), ("LG", C.c_uint32), ("kplane", C.c_void_p),
                ("vplane", C.c_void_p), ("msum", C.POINTER(_Msum)), ("mask_f32", C.c_void_p),
                ("new_runs", C.c_void_p), ("n_new", C.c_uint32), ("out", C.c_void_p), ("stats", C.c_void_p)]



# -- decode-layer glue ops (oc_glue.c), bound onto Oracle ---------------------------------------
def _o_rms_norm(self, x, eps: float, w=None, w_period: int = 1) -> np.ndarray:
    """RMS_NORM (+ MUL by weight row r % w_period) of the rows of x [rows, n]."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    rows, n = x.shape
    y = np.empty_like(x)
    inv_n = np.float32(1.0) / np.float32(n)
    wp = None
    if w is not None:
        w = np.ascontiguousarray(np.atleast_2d(w), np.float32)
        wp = w.ctypes.data
    self.lib.oc_rms_norm_rows(n, rows, x, n, float(np.float32(eps)), float(inv_n), wp, n, w_period, y, n)
    return y


def _o_sincos(self, t):
    t = np.ascontiguousarray(t, np.float32).ravel()
    s = np.empty_like(t)
    c = np.empty_like(t)
    sv, cv = C.c_float(), C.c_float()
    for i in range(t.size):
        self.lib.oc_sincos(float(t[i]), C.byref(sv), C.byref(cv))
        s[i], c[i] = sv.value, cv.value
    return s, c


def _o_rope(self, x, pos, head_dim: int, n_dims: int, neox: bool, ts, m=1.0, freq_scale=1.0, ff=None):
    """ROPE of x [T, n_heads * head_dim] at positions pos [T] (int32)."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    T, width = x.shape
    pos = np.ascontiguousarray(pos, np.int32)
    y = np.empty_like(x)
    ffp = None
    if ff is not None:
        ff = np.ascontiguousarray(ff, np.float32)
        ffp = ff.ctypes.data
    self.lib.oc_rope(1 if neox else 0, head_dim, n_dims, width // head_dim, T, x, width, y, width, pos,
                     float(np.float32(ts)), float(np.float32(m)), float(np.float32(freq_scale)), ffp)
    return y


def _o_silu(self, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    return np.array([self.lib.oc_silu(float(v)) for v in x], np.float32)


def _o_tanh(self, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    return np.array([self.lib.oc_tanh(float(v)) for v in x], np.float32)


def _o_swiglu(self, g, u) -> np.ndarray:
    g = np.ascontiguousarray(np.atleast_2d(g), np.float32)
    u = np.ascontiguousarray(np.atleast_2d(u), np.float32)
    rows, n = g.shape
    y = np.empty_like(g)
    self.lib.oc_swiglu_rows(n, rows, g, n, u, n, y, n)
    return y


def _o_add(self, a, b) -> np.ndarray:
    a = np.ascontiguousarray(np.atleast_2d(a), np.float32)
    b = np.ascontiguousarray(np.atleast_2d(b), np.float32)
    rows, n = a.shape
    y = np.empty_like(a)
    self.lib.oc_add_rows(n, rows, a, n, b, n, y, n)
    return y


def _o_get_rows(self, src, ids) -> np.ndarray:
    src = np.ascontiguousarray(np.atleast_2d(src), np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    if ids.size and (ids.min() < 0 or ids.max() >= src.shape[0]):
        raise IndexError(f"get_rows: id outside [0, {src.shape[0]})")
    out = np.empty((ids.size, src.shape[1]), np.float32)
    self.lib.oc_get_rows(src.shape[1], src, src.shape[1], ids, ids.size, out, src.shape[1])
    return out


def _o_argmax(self, x) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    out = np.empty(x.shape[0], np.int32)
    self.lib.oc_argmax_rows(x.shape[1], x.shape[0], x, x.shape[1], out)
    return out


Oracle.rms_norm = _o_rms_norm
Oracle.sincos = _o_sincos
Oracle.rope = _o_rope
Oracle.silu = _o_silu
Oracle.tanh = _o_tanh
Oracle.swiglu = _o_swiglu
Oracle.add = _o_add
Oracle.get_rows = _o_get_rows
Oracle.argmax = _o_argmax


class _RopeCfg(C.Structure):   # tsr_ref_rope_cfg (sw/sim/include/tsr_ref_vu.h:111-123)
    _fields_ = [("mode", C.c_uint32), ("ff", C.c_uint32), ("fs", C.c_uint32), ("atab", C.c_uint32), ("m", C.c_uint32),
                ("ts", C.c_uint32), ("freq_scale", C.c_uint32), ("head_dim", C.c_uint32), ("n_dims", C.c_uint32),
                ("n_heads", C.c_uint32), ("T", C.c_uint32)]


REF_PATH = os.path.join(HERE, "_ref", "libtsr_ref.so")


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


class Ref:
    """The reference's numerics library compiled from /root/reference (oracle/_ref)."""

    def __init__(self, path: str = REF_PATH):
        L = self.lib = C.CDLL(path)
        for fn in ("tsr_fadd", "tsr_fsub", "tsr_fmul", "tsr_fdiv"):
            getattr(L, fn).argtypes = [C.c_float, C.c_float]
            getattr(L, fn).restype = C.c_float
        L.tsr_frecip.argtypes = [C.c_float]
        L.tsr_frecip.restype = C.c_float
        L.tsr_f32_to_fp16.argtypes = [C.c_float]
        L.tsr_f32_to_fp16.restype = C.c_uint16
        L.tsr_fp16_to_f32.argtypes = [C.c_uint16]
        L.tsr_fp16_to_f32.restype = C.c_float
        L.tsr_i32_to_f32.argtypes = [C.c_int32]
        L.tsr_i32_to_f32.restype = C.c_float
        L.tsr_q8_round_away.argtypes = [C.c_float]
        L.tsr_q8_round_away.restype = C.c_int8
        L.tsr_q8_round_even.argtypes = [C.c_float]
        L.tsr_q8_round_even.restype = C.c_int8
        L.tsr_m_exp.argtypes = [C.c_float]
        L.tsr_m_exp.restype = C.c_float
        L.tsr_att_bf_f.argtypes = [C.c_int64, C.c_int32]
        L.tsr_att_bf_f.restype = C.c_float
        L.tsr_att_bf_int.argtypes = [C.c_float, C.c_int32]
        L.tsr_att_bf_int.restype = C.c_int32
        L.tsr_att_maxt.argtypes = [C.c_float, C.c_float]
        L.tsr_att_maxt.restype = C.c_float
        L.tsr_qa_lines.argtypes = [C.c_uint32, C.c_uint32]
        L.tsr_qa_lines.restype = C.c_uint32
        L.tsr_row_beats.argtypes = [C.c_uint32, C.c_uint32]
        L.tsr_row_beats.restype = C.c_uint32
        L.tsr_qact.argtypes = [C.c_uint32, _f32p, C.c_uint32, _u8p]
        L.tsr_repack_row.argtypes = [C.c_uint32, _u8p, C.c_uint32, _u8p]
        L.tsr_unrepack_row.argtypes = [C.c_uint32, _u8p, C.c_uint32, _u8p]
        L.tsr_dot_row.argtypes = [C.c_uint32, _u8p, C.c_uint32, _u8p]
        L.tsr_dot_row.restype = C.c_float
        L.tsr_tree16.argtypes = [_f32p]
        L.tsr_tree16.restype = C.c_float
        L.tsr_kv_lg_min.argtypes = [C.c_uint32, C.c_uint32]
        L.tsr_kv_lg_min.restype = C.c_uint32
        L.tsr_kv_plane_beats.argtypes = [C.POINTER(_KvGeom)]
        L.tsr_kv_plane_beats.restype = C.c_uint64
        L.tsr_kv_set_bytes.argtypes = [C.c_uint32, C.POINTER(_KvGeom), C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]
        L.tsr_kv_get_bytes.argtypes = [C.c_uint32, C.POINTER(_KvGeom), C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]
        L.tsr_msum_build_f16.argtypes = [_u16p, C.c_size_t, C.c_uint32, C.c_uint32, C.c_uint32, _u32p]
        L.tsr_msum_build_f16.restype = C.c_uint32
        L.tsr_msum_view.argtypes = [_u32p, C.c_size_t, C.POINTER(_Msum)]
        L.tsr_msum_view.restype = C.c_int
        L.tsr_msum_mask_f32.argtypes = [_u16p, C.c_size_t, C.c_uint32, C.c_uint32, C.c_float, _f32p]
        L.tsr_ref_fa.argtypes = [C.POINTER(_AttCfg), C.POINTER(_FaArgs)]
        L.tsr_ref_fa.restype = C.c_int
        L.tsr_fsqrt.argtypes = [C.c_float]
        L.tsr_fsqrt.restype = C.c_float
        L.tsr_ref_red_row.argtypes = [C.c_uint32, C.c_uint32, _u32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.tsr_ref_red_row.restype = C.c_uint32
        L.tsr_ref_vop_elem.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
        L.tsr_ref_vop_elem.restype = C.c_uint32
        L.tsr_m_sincos.argtypes = [C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.tsr_m_silu.argtypes = [C.c_float]
        L.tsr_m_silu.restype = C.c_float
        L.tsr_m_tanh.argtypes = [C.c_float]
        L.tsr_m_tanh.restype = C.c_float
        L.tsr_ref_rope.argtypes = [C.POINTER(_RopeCfg), _u32p, C.c_uint32, _u32p, C.c_uint32, _u32p, C.c_void_p]

    def scalar(self, fn: str, *args):
        return getattr(self.lib, fn)(*args)

    def vec(self, fn: str, *arrays, out_dtype=np.float32) -> np.ndarray:
        f = getattr(self.lib, fn)
        flat = [np.asarray(a).ravel() for a in arrays]
        out = np.empty(flat[0].shape, out_dtype)
        for i in range(out.size):
            out[i] = f(*(a[i].item() for a in flat))
        return out

    def qact(self, kind: int, x) -> np.ndarray:
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        T, K = x.shape
        out = np.zeros((T, self.lib.tsr_qa_lines(kind, K) * 64), np.uint8)
        for t in range(T):
            row = np.ascontiguousarray(x[t])
            buf = np.zeros(out.shape[1], np.uint8)
            self.lib.tsr_qact(kind, row, K, buf)
            out[t] = buf
        return out

    def dot_rows(self, fmt: int, w, K: int, qa) -> np.ndarray:
        """tsr_dot_row of every ggml row of w against one QA image (repacked as the device does)."""
        w = np.ascontiguousarray(w, np.uint8)
        rb = self.lib.tsr_row_beats(fmt, K) * 64
        qa = np.ascontiguousarray(qa, np.uint8).ravel()
        y = np.empty(w.shape[0], np.float32)
        dev = np.zeros(rb, np.uint8)
        for n in range(w.shape[0]):
            self.lib.tsr_repack_row(fmt, np.ascontiguousarray(w[n]), K, dev)
            y[n] = self.lib.tsr_dot_row(fmt, dev, K, qa)
        return y

    def msum(self, mask_f16) -> np.ndarray:
        m = np.ascontiguousarray(np.atleast_2d(mask_f16).view(np.uint16))
        n_q, n_kv = m.shape
        words = np.zeros(8 + 4 * n_q, np.uint32)
        self.lib.tsr_msum_build_f16(m, n_kv, n_kv, n_q, 0, words)
        return words

    def mask_f32(self, mask_f16, scale: float) -> np.ndarray:
        m = np.ascontiguousarray(np.atleast_2d(mask_f16).view(np.uint16))
        n_q, n_kv = m.shape
        out = np.empty((n_q, 16 * (-(-n_kv // 16))), np.float32)
        self.lib.tsr_msum_mask_f32(m, n_kv, n_kv, n_q, scale, out)
        return out

    def flash_attn(self, q, kc, vc, D: int, n_head: int, n_head_kv: int, scale: float, msum_words,
                   mask_f32=None, new_runs=None) -> np.ndarray:
        """tsr_ref_fa with C = 4, T_MAX = 1, PCAP = 9344 on planes built from the q8_0 cache images."""
        E = n_head_kv * D
        kv_size = kc.shape[0]
        geom = _KvGeom(E, 4, self.lib.tsr_kv_lg_min(kv_size, 4))
        pbytes = self.lib.tsr_kv_plane_beats(C.byref(geom)) * 64
        planes = []
        ptrs = []
        for which, img in ((0, kc), (1, vc)):
            chans = [np.zeros(pbytes, np.uint8) for _ in range(4)]
            arr = (C.c_void_p * 4)(*[c.ctypes.data for c in chans])
            img = np.ascontiguousarray(img, np.uint8)
            self.lib.tsr_kv_set_bytes(which, C.byref(geom), arr, img.ctypes.data, 0, img.size)
            planes.append(chans)
            ptrs.append(arr)
        q = np.ascontiguousarray(np.atleast_2d(q), np.float32).reshape(-1, n_head * D)
        T = q.shape[0]
        words = np.ascontiguousarray(msum_words, np.uint32)
        ms = _Msum()
        assert self.lib.tsr_msum_view(words, words.size, C.byref(ms)) == 0
        out = np.empty((T, n_head * D), np.float32)
        nr = None if new_runs is None else np.ascontiguousarray(new_runs, np.uint32).reshape(-1, 2)
        mf = None if mask_f32 is None else np.ascontiguousarray(mask_f32, np.float32)
        args = _FaArgs(T, D, n_head // n_head_kv, scale, q.ctypes.data, E, geom.LG,
                       C.cast(ptrs[0], C.c_void_p), C.cast(ptrs[1], C.c_void_p), C.pointer(ms),
                       None if mf is None else mf.ctypes.data, None if nr is None else nr.ctypes.data,
                       0 if nr is None else nr.shape[0], out.ctypes.data, None)
        cfg = _AttCfg(4, 1, 9344, 32768)
        rc = self.lib.tsr_ref_fa(C.byref(cfg), C.byref(args))
        if rc != 0:
            raise ValueError(f"tsr_ref_fa failed: {rc}")
        return out


# -- the reference's vector-unit functions (tsr_ref_vu.c, tsr_ref_math.c), bound onto Ref ----------
_F32_BITS = lambda v: int(np.float32(v).view(np.uint32))  # noqa: E731
VOP_ADD, VOP_SWIGLU, VOP_MULCB = 0, 7, 12       # sw/sim/include/tsr_tables.h:2163-2175
RED_SUMSQ, RED_POST_RMS = 1, 2                  # sw/sim/include/tsr_tables.h:2254-2258


def _r_rms_norm(self, x, eps: float, w=None, w_period: int = 1) -> np.ndarray:
    """RED.SUMSQ post RMS, then VOP.MULCB (or MULC, as FM(x, s)) per row: the reference's RMS_NORM."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    rows, n = x.shape
    inv_n = _F32_BITS(np.float32(1.0) / np.float32(n))
    y = np.empty((rows, n), np.uint32)
    xb = x.view(np.uint32)
    wb = None if w is None else np.ascontiguousarray(np.atleast_2d(w), np.float32).view(np.uint32)
    for r in range(rows):
        row = np.ascontiguousarray(xb[r])
        s = self.lib.tsr_ref_red_row(RED_SUMSQ, RED_POST_RMS, row, n, inv_n, _F32_BITS(eps))
        for j in range(n):
            if wb is None:
                y[r, j] = self.lib.tsr_ref_vop_elem(2, int(row[j]), int(s), 0)       # MUL: FM(x, s)
            else:
                y[r, j] = self.lib.tsr_ref_vop_elem(VOP_MULCB, int(row[j]), int(wb[r % w_period, j]), int(s))
    return y.view(np.float32)


def _r_sincos(self, t):
    t = np.ascontiguousarray(t, np.float32).ravel()
    s = np.empty_like(t)
    c = np.empty_like(t)
    sv, cv = C.c_float(), C.c_float()
    for i in range(t.size):
        self.lib.tsr_m_sincos(float(t[i]), C.byref(sv), C.byref(cv))
        s[i], c[i] = sv.value, cv.value
    return s, c


def _r_rope(self, x, pos, head_dim: int, n_dims: int, neox: bool, ts, m=1.0, freq_scale=1.0, ff=None):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    T, width = x.shape
    cfg = _RopeCfg(1 if neox else 0, 0 if ff is None else 1, 1 if _F32_BITS(freq_scale) != 0x3F800000 else 0, 0,
                   _F32_BITS(m), _F32_BITS(ts), _F32_BITS(freq_scale), head_dim, n_dims, width // head_dim, T)
    src = x.view(np.uint32).copy()
    dst = np.zeros_like(src)
    posb = np.ascontiguousarray(pos, np.int32).view(np.uint32)
    table = None if ff is None else np.ascontiguousarray(ff, np.float32)
    self.lib.tsr_ref_rope(C.byref(cfg), dst, width // 16, src, width // 16, posb,
                          None if table is None else table.ctypes.data)
    return dst.view(np.float32)


def _r_vop(self, func: int, a, b=None, c=0.0) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32).ravel().view(np.uint32)
    b = np.zeros_like(a) if b is None else np.ascontiguousarray(b, np.float32).ravel().view(np.uint32)
    cb = _F32_BITS(c)
    out = np.empty(a.size, np.uint32)
    for i in range(a.size):
        out[i] = self.lib.tsr_ref_vop_elem(func, int(a[i]), int(b[i]), cb)
    return out.view(np.float32)


def _r_tanh(self, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    return np.array([self.lib.tsr_m_tanh(float(v)) for v in x], np.float32)


Ref.tanh = _r_tanh
Ref.rms_norm = _r_rms_norm
Ref.sincos = _r_sincos
Ref.rope = _r_rope
Ref.vop = _r_vop
