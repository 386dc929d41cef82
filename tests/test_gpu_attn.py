"""GPU parity of FLASH_ATTN_EXT over the q8_0 KV cache against the CPU oracle (bit-exact; the
contract's tolerance is 2e-3 absolute, asserted as well against the float64 model of the test suite)."""
import math

import numpy as np
import pytest

import tsr_hip
import tsr_synth as S
from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


def _cache(oc, kv_size, E, seed):
    kf = S.normal(seed, kv_size * E).reshape(kv_size, E)
    vf = S.normal(seed + 1, kv_size * E).reshape(kv_size, E)
    kc = np.zeros((kv_size, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    oc.kv_set_rows(kc, kf, np.arange(kv_size))
    oc.kv_set_rows(vc, vf, np.arange(kv_size))
    return kc, vc


def _fa(dev, oc, n_kv, kv_size, n_head, n_head_kv, D, T=1, mask=None, new_runs=None, seed=3, q=None):
    E = n_head_kv * D
    kc, vc = _cache(oc, kv_size, E, seed)
    if q is None:   # Q drawn as f16 N(0, 1) and widened exactly
        q = S.normal(seed + 2, T * n_head * D).reshape(T, n_head * D).astype(np.float16).astype(np.float32)
    mask = np.zeros((T, n_kv), np.float16) if mask is None else mask
    scale = np.float32(1.0 / math.sqrt(D))
    msum = oc.msum(mask)
    mf = oc.mask_f32(mask, scale) if msum[3] else None
    want = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, msum, mf, new_runs)
    K_, V_ = dev.kv(E, kv_size), dev.kv(E, kv_size)
    K_.set_bytes(0, kc)
    V_.set_bytes(1, vc)
    out = dev.alloc(4 * T * n_head * D)
    dev.flash_attn(dev.upload(q), T, n_head * D, K_, V_, D, n_head, n_head_kv, scale, msum, out, n_head * D,
                   mask_f32=None if mf is None else dev.upload(mf), new_runs=new_runs)
    got = out.read(np.float32, (T, n_head * D))
    return got, want


def test_fa_decode_baseline_shape(dev, oc):
    """32 q heads, 8 KV heads, D 128, n_kv 8192, batch 1."""
    got, want = _fa(dev, oc, 8192, 8192, 32, 8, 128)
    assert np.abs(got - want).max() <= 2e-3
    assert_bits_equal(got, want, "fa decode 8192")


@pytest.mark.parametrize("n_kv,kv_size,n_head,n_head_kv,D", [
    (512, 512, 32, 8, 128), (300, 512, 8, 2, 64), (1000, 1024, 4, 4, 256), (77, 96, 4, 1, 512),
    (4096, 4096, 8, 8, 128), (1, 16, 32, 8, 128), (17, 33, 12, 4, 64), (2500, 2560, 64, 1, 64)])
def test_fa_decode_shapes(dev, oc, n_kv, kv_size, n_head, n_head_kv, D):
    got, want = _fa(dev, oc, n_kv, kv_size, n_head, n_head_kv, D, seed=n_kv)
    assert_bits_equal(got, want, f"fa {n_kv} {n_head}/{n_head_kv} D{D}")


def test_fa_new_runs_order(dev, oc):
    got, want = _fa(dev, oc, 5000, 5120, 8, 2, 128, new_runs=[[17, 18]])
    assert_bits_equal(got, want, "newest last")


def test_fa_causal_prefill(dev, oc):
    T = 96
    mask = np.full((T, T), -np.inf, np.float16)
    for i in range(T):
        mask[i, :i + 1] = 0
    got, want = _fa(dev, oc, T, T, 32, 8, 128, T=T, mask=mask, new_runs=[[0, T]])
    assert_bits_equal(got, want, "causal prefill")


def test_fa_causal_prefill_baseline_512(dev, oc):
    """causal flash attention over a 512-token ubatch at cells 0 .. 511, 32 q / 8 KV
    heads, D 128, q8_0 K / V, Q drawn f16 N(0, 1): row t sees cells [0, t], the ubatch's cells newest
    last. Every output of every row bit-exact (the contract allows 2e-3 absolute, asserted too)."""
    T = 512
    mask = np.full((T, T), -np.inf, np.float16)
    mask[np.tril_indices(T)] = 0
    got, want = _fa(dev, oc, T, T, 32, 8, 128, T=T, mask=mask, new_runs=[[0, T]], seed=512)
    assert np.abs(got - want).max() <= 2e-3
    assert_bits_equal(got, want, "causal prefill 512")


def test_fa_general_and_two_run_masks(dev, oc):
    m2 = np.zeros((3, 100), np.float16); m2[:, 10:20] = -2.5; m2[1, 50:] = -np.inf
    got, want = _fa(dev, oc, 100, 112, 8, 2, 64, T=3, mask=m2)
    assert_bits_equal(got, want, "general mask")
    m3 = np.full((2, 200), -np.inf, np.float16); m3[:, 0:20] = 0; m3[:, 150:180] = 0
    got, want = _fa(dev, oc, 200, 208, 4, 1, 256, T=2, mask=m3)
    assert_bits_equal(got, want, "two runs")
    m4 = np.full((2, 64), -np.inf, np.float16); m4[1, 3] = 0
    got, want = _fa(dev, oc, 64, 64, 4, 1, 128, T=2, mask=m4)
    assert_bits_equal(got, want, "empty row")


def test_fa_special_q(dev, oc):
    q = S.normal(9, 2 * 8 * 128).reshape(2, 8 * 128)
    q[0, 5] = np.inf
    q[1, 130] = np.nan
    q[1, 300:332] = 0
    got, want = _fa(dev, oc, 600, 600, 8, 2, 128, T=2, q=q, mask=np.zeros((2, 600), np.float16))
    assert_bits_equal(got, want, "special q")


class _Hip:
    """The few HIP runtime calls these tests need (libamdhip64 via ctypes)."""

    def __init__(self):
        import ctypes as C
        self.C = C
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipStreamCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        self.h.hipStreamDestroy.argtypes = [C.c_void_p]
        self.h.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.h.hipGraphDestroy.argtypes = [C.c_void_p]

    def stream(self):
        s = self.C.c_void_p()
        assert self.h.hipStreamCreateWithFlags(self.C.byref(s), 1) == 0      # non-blocking, default priority
        return s.value


def _decode_case(oc, dev, n_kv, seed):
    E, n_head, n_head_kv, D = 256, 8, 2, 128
    kc, vc = _cache(oc, n_kv, E, seed)
    q = S.normal(seed + 2, n_head * D).reshape(1, n_head * D).astype(np.float16).astype(np.float32)
    msum = oc.msum(np.zeros((1, n_kv), np.float16))
    scale = np.float32(1.0 / math.sqrt(D))
    want = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, msum)
    K_, V_ = dev.kv(E, n_kv), dev.kv(E, n_kv)
    K_.set_bytes(0, kc)
    V_.set_bytes(1, vc)
    return dict(q=dev.upload(q), K=K_, V=V_, msum=msum, scale=scale, out=dev.alloc(4 * n_head * D), want=want,
                args=(D, n_head, n_head_kv))


def _run(dev, c, stream=None):
    D, n_head, n_head_kv = c["args"]
    dev.flash_attn(c["q"], 1, n_head * D, c["K"], c["V"], D, n_head, n_head_kv, c["scale"], c["msum"], c["out"],
                   n_head * D, stream=stream)


def test_fa_scratch_shared_by_two_streams(dev, oc):
    """Two calls on different streams share the context's scratch: the second waits for the first."""
    hip = _Hip()
    s1 = hip.stream()
    try:
        a, b = _decode_case(oc, dev, 4096, 21), _decode_case(oc, dev, 3000, 22)
        for _ in range(3):
            _run(dev, a, stream=s1)
            _run(dev, b)
            assert hip.h.hipStreamSynchronize(s1) == 0
            dev.sync()
            assert_bits_equal(a["out"].read(np.float32, a["want"].shape), a["want"], "stream 1")
            assert_bits_equal(b["out"].read(np.float32, b["want"].shape), b["want"], "context stream")
    finally:
        hip.h.hipStreamDestroy(s1)


def test_fa_decode_graph_replays(dev, oc):
    """A decode call captured into a HIP graph replays exactly, with eager calls between replays;
    a call whose work list needs a host copy is refused during capture."""
    hip = _Hip()
    C = hip.C
    a, b = _decode_case(oc, dev, 2048, 31), _decode_case(oc, dev, 1000, 32)
    _run(dev, a)                                        # warm: the scratch is large enough
    _run(dev, b)
    dev.sync()
    T, D, n_head, n_head_kv = 40, 128, 8, 2             # 40 query rows: a host-built work list
    qq, oo = dev.alloc(4 * T * n_head * D), dev.alloc(4 * T * n_head * D)
    ms40 = oc.msum(np.zeros((T, 2048), np.float16))
    s = dev.stream
    assert hip.h.hipStreamBeginCapture(s, 2) == 0
    _run(dev, a)
    with pytest.raises(tsr_hip.TsrHipError):
        dev.flash_attn(qq, T, n_head * D, a["K"], a["V"], D, n_head, n_head_kv, a["scale"], ms40, oo, n_head * D)
    g, ge = C.c_void_p(), C.c_void_p()
    assert hip.h.hipStreamEndCapture(s, C.byref(g)) == 0
    assert hip.h.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
    try:
        for i in range(4):
            a["out"].fill(0)
            assert hip.h.hipGraphLaunch(ge, s) == 0
            dev.sync()
            assert_bits_equal(a["out"].read(np.float32, a["want"].shape), a["want"], f"replay {i}")
            _run(dev, b)                               # eager work between the replays
            dev.sync()
            assert_bits_equal(b["out"].read(np.float32, b["want"].shape), b["want"], f"eager {i}")
    finally:
        hip.h.hipGraphExecDestroy(ge)
        hip.h.hipGraphDestroy(g)


def test_graph_refused_after_scratch_growth(oc):
    """A graph whose capture used the context's scratch (the unplanned FLASH_ATTN_EXT's partials) replays
    while the scratch block stays; after a larger call has grown (reallocated) it, the launch is refused
    and the stale graph never runs; a new capture replays exactly. A fresh context, so that the scratch
    starts empty."""
    d2 = tsr_hip.Device(0)
    try:
        a = _decode_case(oc, d2, 1024, 41)
        _run(d2, a)                                     # warm: the scratch holds a's partials
        d2.sync()
        d2.graph_begin()
        _run(d2, a)
        g = d2.graph_end()
        a["out"].fill(0)
        g.launch()
        d2.sync()
        assert_bits_equal(a["out"].read(np.float32, a["want"].shape), a["want"], "replay before growth")
        big = _decode_case(oc, d2, 8192, 42)            # its byte upload and partials grow the scratch
        _run(d2, big)
        d2.sync()
        assert_bits_equal(big["out"].read(np.float32, big["want"].shape), big["want"], "the growing call")
        with pytest.raises(tsr_hip.TsrHipError):
            g.launch()
        g.free()
        d2.graph_begin()
        _run(d2, a)
        g2 = d2.graph_end()
        a["out"].fill(0)
        g2.launch()
        d2.sync()
        assert_bits_equal(a["out"].read(np.float32, a["want"].shape), a["want"], "replay of the new capture")
        g2.free()
    finally:
        d2.close()
