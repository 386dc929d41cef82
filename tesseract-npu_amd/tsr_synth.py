"""Seeded synthetic inputs and ggml-block quantizers for the benchmark and the tests.

The reference quantizes weights with ggml's ``quantize_row_q8_0_ref`` (used by the backend at load
time, sw/ggml-tesseract/tsr-weights.cpp:33-49) and its test models with a Q4_K encoder
(sw/ggml-tesseract/tests/gen_tiny_models.py:91-122). Neither is importable here, so this module
carries its own:

* ``normal(seed, n, std)``: counter-based SplitMix64 -> two uniforms -> Box-Muller in float64, rounded
  to float32 (C helper synth/tsr_synth.c). Every value depends only on (seed, index).
* ``quantize_q8_0``: d = amax / 127 in f32, q = round-half-away(x / d ... as x * (1/d)), fp16(d) -- the
  rule of quantize_row_q8_0_ref, which is also QACT A32's (sw/sim/tsr_ref.c:472-487).
* ``quantize_q4_k``: per 32-value sub-block an affine step/min, 6-bit scales and mins packed as ggml's
  get_scale_min_k4 reads them (sw/sim/tsr_ref.c:359-367), 4-bit quants low nibble = sub-block 2g,
  high = 2g+1. Only the resulting blocks matter for parity; any valid Q4_K encoder would do.
"""
from __future__ import annotations

import numpy as np

import ctypes as _C
import os as _os

_M64 = (1 << 64) - 1
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = _os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "libtsr_synth.so")
        if not _os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built: run `make -C {_os.path.dirname(path)}`")
        _LIB = _C.CDLL(path)
        _LIB.tsr_synth_normal.argtypes = [_C.c_uint64, _C.c_uint64, _C.c_uint64, _C.c_float, _C.c_void_p]
        _LIB.tsr_synth_quant.argtypes = [_C.c_int, _C.c_uint64, _C.c_uint64, _C.c_uint64, _C.c_uint64, _C.c_float,
                                         _C.c_void_p]
    return _LIB


def normal(seed: int, n: int, std: float = 1.0, start: int = 0) -> np.ndarray:
    """n float32 values ~ N(0, std^2): value i uses uniforms 2i and 2i+1 of the seed's SplitMix64
    stream (synth/tsr_synth.c). Values depend only on (seed, index)."""
    out = np.empty(n, np.float32)
    _lib().tsr_synth_normal(seed & _M64, start, n, std, out.ctypes.data)
    return out


def quant_rows(fmt: int, seed: int, N: int, K: int, std: float = 0.02, r0: int = 0) -> np.ndarray:
    """Rows r0 .. r0+N-1 of normal(seed, *, std) as [*, K], quantized to Q8_0 (fmt 0) or Q4_K (fmt 1):
    bit for bit quantize_q8_0 / quantize_q4_k of normal(seed, ...) rows, computed in C on 16 threads."""
    bs, bb = (256, 144) if fmt else (32, 34)
    out = np.empty((N, K // bs * bb), np.uint8)
    if _lib().tsr_synth_quant(fmt, seed & _M64, K, r0, N, std, out.ctypes.data) != 0:
        raise ValueError(f"quant_rows: K={K} is not a multiple of {bs} (or > 32768)")
    return out


def seed_of(config: str, tensor: str) -> int:
    """A documented 64-bit seed per (config, tensor): FNV-1a over 'config/tensor'."""
    h = 0xCBF29CE484222325
    for b in f"{config}/{tensor}".encode():
        h = ((h ^ b) * 0x100000001B3) & _M64
    return h


# ---------------------------------------------------------------------------------------------
# Q8_0: blocks of 32, {fp16 d, int8 qs[32]} = 34 bytes
# ---------------------------------------------------------------------------------------------
def _round_half_away(v: np.ndarray) -> np.ndarray:
    t = np.trunc(v)
    frac = v - t                                   # exact for |v| < 2^23
    return t + np.where(np.abs(frac) >= 0.5, np.sign(v), 0.0).astype(v.dtype)


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """f32 [N, K] (K % 32 == 0) -> uint8 [N, K/32 * 34]."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    b = w.reshape(N, K // 32, 32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    q = np.clip(_round_half_away((b * idv[:, :, None]).astype(np.float32)), -128, 127).astype(np.int8)
    out = np.empty((N, K // 32, 34), np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(N, K // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(N, K // 32 * 34)


def dequantize_q8_0(blocks: np.ndarray, K: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1, K // 32, 34)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = b[:, :, 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(-1, K)


# ---------------------------------------------------------------------------------------------
# Q4_K: super-blocks of 256 = 8 sub-blocks of 32; {fp16 d, fp16 dmin, u8 scales[12], u8 qs[128]}
# ---------------------------------------------------------------------------------------------
def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """f32 [N, K] (K % 256 == 0) -> uint8 [N, K/256 * 144].

    Sub-block j: x ~ d*sc_j*q - dmin*m_j with q in 0..15, sc_j and m_j 6-bit unsigned."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    nb = N * (K // 256)
    x = w.reshape(nb, 8, 32)
    lo = np.minimum(x.min(axis=2), 0.0)
    hi = np.maximum(x.max(axis=2), lo)
    step = (hi - lo) / 15.0
    mins = -lo
    d = (step.max(axis=1) / 63.0).astype(np.float16)
    dmin = (mins.max(axis=1) / 63.0).astype(np.float16)
    d32, m32 = d.astype(np.float32), dmin.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d32[:, None] > 0, np.rint(step / d32[:, None]), 0).clip(0, 63).astype(np.uint8)
        mn = np.where(m32[:, None] > 0, np.rint(mins / m32[:, None]), 0).clip(0, 63).astype(np.uint8)
        eff = d32[:, None] * sc.astype(np.float32)
        off = m32[:, None] * mn.astype(np.float32)
        q = np.where(eff[:, :, None] > 0, np.rint((x + off[:, :, None]) / eff[:, :, None]), 0).clip(0, 15).astype(np.uint8)
    scales = np.empty((nb, 12), np.uint8)
    scales[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    scales[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    scales[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    q = q.reshape(nb, 4, 2, 32)
    qs = (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(nb, 128)
    out = np.concatenate([d.view(np.uint8).reshape(nb, 2), dmin.view(np.uint8).reshape(nb, 2), scales, qs], axis=1)
    return out.reshape(N, K // 256 * 144)


def q4k_scale_min(scales: np.ndarray):
    """The 8 (sc, m) pairs of each 12-byte scales row (get_scale_min_k4)."""
    s = scales.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    mn = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, mn


def dequantize_q4_k(blocks: np.ndarray, K: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = q4k_scale_min(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)
    y = (d[:, None] * sc)[:, :, None] * q - (dmin[:, None] * mn)[:, :, None]
    return y.reshape(-1, K)
