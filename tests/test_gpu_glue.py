"""GPU decode-layer glue ops (RMS_NORM + MUL, ROPE, SWIGLU, ADD, GET_ROWS, ARGMAX) through the C ABI,
bit for bit against the oracle (oracle/oc_glue.c, itself pinned against the reference's vector-unit
library in test_oracle_glue.py) on the same seeded inputs, special values included."""
import ctypes as C

import numpy as np
import pytest

from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

SPECIALS = np.array([0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x00800000, 0x7F800000, 0xFF800000,
                     0x7FC00000, 0xFFC00001, 0x3F800000, 0xBF800000, 0x7F7FFFFF, 0x39800000, 0x4B000000],
                    np.uint32).view(np.float32)

_libm = C.CDLL("libm.so.6")
_libm.powf.argtypes = [C.c_float, C.c_float]
_libm.powf.restype = C.c_float


def theta_scale(freq_base, n_dims):
    """TS = powf(freq_base, -2 / n_dims) with the C library's powf, as the host side computes it."""
    return np.float32(_libm.powf(float(np.float32(freq_base)), float(np.float32(-2.0) / np.float32(n_dims))))


@pytest.mark.parametrize("n,rows", [(4096, 64), (896, 7), (14336, 2), (100, 5), (130, 3), (1, 4), (5120, 1)])
def test_rms_norm(dev, oc, n, rows):
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.01, 50, (rows, 1))).astype(np.float32)
    w = rng.standard_normal((2, n)).astype(np.float32)
    xb, wb, yb = dev.upload(x), dev.upload(w), dev.alloc(x.nbytes)
    for eps, wt, period in ((1e-5, w[:1], 1), (1e-6, w, 2), (1e-5, None, 1)):
        dev.rms_norm(xb, n, rows, n, eps, yb, n, w=None if wt is None else wb, w_stride=n, w_period=period)
        got = yb.read(np.float32, (rows, n))
        assert_bits_equal(got, oc.rms_norm(x, eps, wt, w_period=period), f"rms n={n} eps={eps} period={period}")


def test_rms_norm_specials_and_in_place(dev, oc):
    rng = np.random.default_rng(21)
    n = 300
    x = rng.standard_normal((8, n)).astype(np.float32)
    x[0, :SPECIALS.size] = SPECIALS
    x[1] = 0.0
    x[2, 7] = np.inf
    x[3, 11] = np.nan
    x[4] *= np.float32(1e-30)
    x[5, :] = np.float32(3e-39)                     # a subnormal row: zero after DAZ
    x[6] *= np.float32(1e19)                        # sum of squares overflows
    w = rng.standard_normal((1, n)).astype(np.float32)
    w[0, 3] = np.float32(1e-40)
    want = oc.rms_norm(x, 1e-6, w)
    xb = dev.upload(x)
    dev.rms_norm(xb, n, 8, n, 1e-6, xb, n, w=dev.upload(w), w_stride=n)          # in place
    assert_bits_equal(xb.read(np.float32, (8, n)), want, "rms specials in place")


def test_rms_norm_strided_rows(dev, oc):
    rng = np.random.default_rng(22)
    n, rows, xs, ys = 256, 9, 320, 272
    x = rng.standard_normal((rows, xs)).astype(np.float32)
    w = rng.standard_normal((1, n)).astype(np.float32)
    yb = dev.upload(np.full((rows, ys), 7.0, np.float32))
    dev.rms_norm(dev.upload(x), n, rows, xs, 1e-5, yb, ys, w=dev.upload(w), w_stride=n)
    got = yb.read(np.float32, (rows, ys))
    assert_bits_equal(got[:, :n], oc.rms_norm(np.ascontiguousarray(x[:, :n]), 1e-5, w), "rms strided")
    assert (got[:, n:] == 7.0).all()


@pytest.mark.parametrize("mode", [0, 2, 40])
@pytest.mark.parametrize("hd,n_dims,nh", [(128, 128, 32), (128, 64, 8), (64, 64, 3), (256, 192, 4)])
def test_rope(dev, oc, mode, hd, n_dims, nh):
    rng = np.random.default_rng(hd + n_dims + nh + mode)
    pos = np.array([0, 1, 2, 17, 511, 4095, 8191, 70000, 131071], np.int32)
    T = pos.size
    x = rng.standard_normal((T, nh * hd)).astype(np.float32)
    neox = mode != 0
    xb, pb, yb = dev.upload(x), dev.upload(pos), dev.alloc(x.nbytes)
    for base, fs, m, ff in ((500000.0, 1.0, 1.0, None), (10000.0, 0.25, 0.9, None),
                            (1000000.0, 1.0, 1.0, rng.uniform(1, 8, n_dims // 2).astype(np.float32))):
        ts = theta_scale(base, n_dims)
        dev.rope(xb, T, nh * hd, hd, nh, n_dims, mode, pb, base, yb, nh * hd, freq_scale=fs, attn_factor=m,
                 freq_factors=None if ff is None else dev.upload(ff))
        want = oc.rope(x, pos, hd, n_dims, neox, ts, m, fs, ff)
        assert_bits_equal(yb.read(np.float32, (T, nh * hd)), want, f"rope mode={mode} base={base} fs={fs}")


def test_rope_specials_in_place_and_strided(dev, oc):
    rng = np.random.default_rng(23)
    hd, nh, T, xs = 128, 4, 3, 640
    x = rng.standard_normal((T, xs)).astype(np.float32)
    x[0, :SPECIALS.size] = SPECIALS
    x[1, 200:200 + SPECIALS.size] = SPECIALS
    pos = np.array([3, -5, 2000000000], np.int32)
    want = oc.rope(np.ascontiguousarray(x[:, :nh * hd]), pos, hd, hd, False, theta_scale(10000.0, hd))
    xb = dev.upload(x)
    dev.rope(xb, T, xs, hd, nh, hd, 0, dev.upload(pos), 10000.0, xb, xs)
    got = xb.read(np.float32, (T, xs))
    assert_bits_equal(got[:, :nh * hd], want, "rope in place")
    assert_bits_equal(got[:, nh * hd:], x[:, nh * hd:], "rope leaves the row tail")


def _g_u(rng, rows, n):
    g = (rng.standard_normal((rows, n)) * 6).astype(np.float32)
    u = rng.standard_normal((rows, n)).astype(np.float32)
    k = min(SPECIALS.size, n)
    g[0, :k] = SPECIALS[:k]
    u[0, :k] = SPECIALS[::-1][:k]
    k = min(500, n)
    g[1 % rows, :k] = rng.integers(0, 2**32, k, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return g, u


@pytest.mark.parametrize("n,rows", [(14336, 1), (14336, 5), (4864, 3), (77, 2)])
def test_swiglu(dev, oc, n, rows):
    g, u = _g_u(np.random.default_rng(n + rows), rows, n)
    yb = dev.alloc(g.nbytes)
    dev.swiglu(dev.upload(g), n, dev.upload(u), n, n, rows, yb, n)
    assert_bits_equal(yb.read(np.float32, (rows, n)), oc.swiglu(g, u), f"swiglu n={n}")


@pytest.mark.parametrize("n,rows,period", [(4096, 1, 1), (4096, 6, 6), (896, 9, 3), (77, 4, 1)])
def test_add(dev, oc, n, rows, period):
    a, b = _g_u(np.random.default_rng(n + rows + 100), rows, n)
    bp = np.ascontiguousarray(b[:period])
    yb = dev.alloc(a.nbytes)
    dev.add(dev.upload(a), n, dev.upload(bp), n, n, rows, yb, n, b_period=period)
    want = oc.add(a, np.ascontiguousarray(bp[np.arange(rows) % period]))
    assert_bits_equal(yb.read(np.float32, (rows, n)), want, f"add n={n} period={period}")
    ab = dev.upload(a)                                                   # in place: y = a
    dev.add(ab, n, dev.upload(bp), n, n, rows, ab, n, b_period=period)
    assert_bits_equal(ab.read(np.float32, (rows, n)), want, "add in place")


def test_get_rows(dev, oc):
    rng = np.random.default_rng(31)
    n_src, n = 1000, 4096
    src = rng.standard_normal((n_src, n)).astype(np.float32)
    src[5, :SPECIALS.size] = SPECIALS
    ids = np.array([5, 0, 999, 5, 123], np.int32)
    yb, bad = dev.alloc(ids.size * n * 4), dev.upload(np.zeros(1, np.int32))
    dev.get_rows(dev.upload(src), n, n, n_src, dev.upload(ids), ids.size, yb, n, bad=bad)
    assert_bits_equal(yb.read(np.float32, (ids.size, n)), oc.get_rows(src, ids), "get_rows")
    assert bad.read(np.int32, (1,))[0] == 0


def test_get_rows_bad_id_flag(dev):
    src = np.arange(4 * 64, dtype=np.float32).reshape(4, 64)
    y0 = np.full((3, 64), -1.0, np.float32)
    yb, bad = dev.upload(y0), dev.upload(np.zeros(1, np.int32))
    dev.get_rows(dev.upload(src), 64, 64, 4, dev.upload(np.array([1, 4, -1], np.int32)), 3, yb, 64, bad=bad)
    got = yb.read(np.float32, (3, 64))
    assert (got[0] == src[1]).all() and (got[1:] == -1.0).all()
    assert bad.read(np.int32, (1,))[0] == 1


def test_argmax(dev, oc):
    rng = np.random.default_rng(41)
    n = 128256
    x = rng.standard_normal((8, n)).astype(np.float32)
    x[1, 10] = x[1, 100000] = x[1, 5000] = 9.0                 # ties: the first index
    x[2, 3] = np.nan
    x[2, 64000] = 11.0
    x[3, :] = -np.inf                                           # nothing above -inf: 0
    x[4, :] = np.nan
    x[5, 7] = np.inf
    x[6, 1023] = x[6, 1024] = 50.0                              # ties across threads and waves
    x[7, :] = 0.0
    x[7, 9] = -0.0
    out = dev.alloc(8 * 4)
    dev.argmax(dev.upload(x), n, 8, n, out)
    got = out.read(np.int32, (8,))
    assert (got == oc.argmax(x)).all(), (got, oc.argmax(x))
    assert got[1] == 10 and got[3] == 0 and got[4] == 0 and got[5] == 7 and got[6] == 1023


@pytest.mark.parametrize("n", [1, 63, 1025, 151936])
def test_argmax_sizes(dev, oc, n):
    x = np.random.default_rng(n).standard_normal((3, n)).astype(np.float32)
    out = dev.alloc(12)
    dev.argmax(dev.upload(x), n, 3, n, out)
    assert (out.read(np.int32, (3,)) == oc.argmax(x)).all()


def test_glue_argument_checks(dev):
    import tsr_hip
    b = dev.alloc(4096)
    with pytest.raises(tsr_hip.TsrHipError):
        dev.rms_norm(b, 0, 1, 0, 1e-5, b, 0)
    with pytest.raises(tsr_hip.TsrHipError):
        dev.rope(b, 1, 128, 128, 1, 130, 0, b, 10000.0, b, 128)           # n_dims > head_dim
    with pytest.raises(tsr_hip.TsrHipError):
        dev.rope(b, 1, 128, 128, 1, 128, 8, b, 10000.0, b, 128)           # MROPE is not supported
    with pytest.raises(tsr_hip.TsrHipError):
        dev.add(b, 16, b, 16, 16, 2, b, 16, b_period=0)
    with pytest.raises(tsr_hip.TsrHipError):
        dev.swiglu(b, 8, b, 16, 16, 2, b, 16)                              # overlapping rows


def test_swiglu_expk_sweep(dev, oc):
    """SWIGLU (so SILU and the device EXPK under it) over 2^24 gate values: every exponent field of both
    signs, 32768 seeded mantissas each (specials and subnormals included), u = 1, against the oracle."""
    rng = np.random.default_rng(2024)
    sign = np.repeat(np.arange(2, dtype=np.uint32), 256 * 32768) << 31
    expo = np.tile(np.repeat(np.arange(256, dtype=np.uint32), 32768), 2) << 23
    mant = rng.integers(0, 1 << 23, 2 * 256 * 32768, dtype=np.uint32)
    mant[::32768] = 0                                             # each field's power of two (and 0, Inf)
    g = (sign | expo | mant).view(np.float32).reshape(1024, 16384)
    u = np.ones_like(g)
    yb = dev.alloc(g.nbytes)
    dev.swiglu(dev.upload(g), 16384, dev.upload(u), 16384, 16384, 1024, yb, 16384)
    assert_bits_equal(yb.read(np.float32, (1024, 16384)), oc.swiglu(g, u), "swiglu sweep")
