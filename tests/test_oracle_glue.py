"""The CPU restatement of the decode-layer glue ops (oracle/oc_glue.c), pinned:

* bit for bit against the reference's own vector-unit library compiled in place (oracle/_ref:
  sw/sim/tsr_ref_vu.c, tsr_ref_math.c): RED.SUMSQ post RMS + VOP.MULCB, tsr_m_sincos, tsr_ref_rope,
  VOP.SWIGLU and VOP.ADD, on random values, random bit patterns and special values;
* against what the mathematics fixes: float64 sin / cos / RMS norm / rotation / SiLU within a
  stated tolerance, the symmetries sin(-t) = -sin(t) and cos(-t) = cos(t) (exact in the algorithm),
  and ROPE at position 0 being the identity times the attention factor;
* GET_ROWS and ARGMAX against numpy.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")


@pytest.fixture(scope="module")
def o():
    return O.Oracle()


@pytest.fixture(scope="module")
def r():
    return O.Ref()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


SPECIALS = np.array([0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x00800000, 0x7F800000, 0xFF800000,
                     0x7FC00000, 0xFFC00001, 0x3F800000, 0xBF800000, 0x7F7FFFFF, 0x39800000, 0x397FFFFF,
                     0x40490FDB, 0x3FC90FDB, 0x4B000000, 0x5F000000, 0x42C80000], np.uint32).view(np.float32)


def test_sincos_bitwise_vs_ref(o, r):
    rng = np.random.default_rng(7)
    t = np.concatenate([SPECIALS, rng.uniform(-10, 10, 20000).astype(np.float32),
                        rng.uniform(-5000, 5000, 10000).astype(np.float32),
                        rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        (np.arange(-3000, 3000) * np.float32(np.pi / 4)).astype(np.float32)])
    so, co = o.sincos(t)
    sr, cr = r.sincos(t)
    assert np.array_equal(bits(so), bits(sr))
    assert np.array_equal(bits(co), bits(cr))


def test_sincos_accuracy_and_symmetry(o):
    rng = np.random.default_rng(8)
    t = np.concatenate([rng.uniform(-8, 8, 20000), rng.uniform(-4000, 4000, 5000)]).astype(np.float32)
    s, c = o.sincos(t)
    td = t.astype(np.float64)
    assert np.max(np.abs(s - np.sin(td))) < 3e-7
    assert np.max(np.abs(c - np.cos(td))) < 3e-7
    sn, cn = o.sincos(-t)
    assert np.array_equal(bits(sn), bits(s) ^ np.uint32(0x80000000))
    assert np.array_equal(bits(cn), bits(c))
    small = np.array([1e-5, -3e-6, 2.0**-13], np.float32)               # |t| < 2^-12: sin = t, cos = 1
    ss, cs = o.sincos(small)
    assert np.array_equal(bits(ss), bits(small)) and np.all(cs == 1.0)


def test_rms_norm_bitwise_vs_ref(o, r):
    rng = np.random.default_rng(9)
    for n, rows in ((4096, 2), (896, 3), (100, 4), (16, 2), (1, 1)):
        x = rng.standard_normal((rows, n)).astype(np.float32)
        w = rng.standard_normal((1, n)).astype(np.float32)
        for eps in (1e-5, 1e-6):
            assert np.array_equal(bits(o.rms_norm(x, eps, w)), bits(r.rms_norm(x, eps, w)))
        assert np.array_equal(bits(o.rms_norm(x, 1e-5)), bits(r.rms_norm(x, 1e-5)))
    x = rng.standard_normal((6, 300)).astype(np.float32)
    x[0, :5] = SPECIALS[:5]
    x[1] = 0.0
    x[2, 7] = np.inf
    x[3, 11] = np.nan
    x[4] *= np.float32(1e-30)
    x[5, :] = np.float32(3e-39)                                          # subnormal row: DAZ -> zero
    w = rng.standard_normal((2, 300)).astype(np.float32)
    assert np.array_equal(bits(o.rms_norm(x, 1e-6, w, w_period=2)), bits(r.rms_norm(x, 1e-6, w, w_period=2)))


def test_rms_norm_closed_form(o):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    w = rng.standard_normal((1, 4096)).astype(np.float32)
    y = o.rms_norm(x, 1e-5, w).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(y - want) / (np.abs(want) + 1e-6)) < 1e-5


@pytest.mark.parametrize("neox", [False, True])
def test_rope_bitwise_vs_ref(o, r, neox):
    rng = np.random.default_rng(11 + neox)
    T, nh, hd = 5, 4, 128
    x = rng.standard_normal((T, nh * hd)).astype(np.float32)
    pos = np.array([0, 1, 17, 4095, 70000], np.int32)
    ts = np.float32(np.power(np.float32(500000.0), np.float32(-2.0 / 128)))
    for n_dims, m, fs, ff in ((128, 1.0, 1.0, None), (64, 1.0, 1.0, None), (128, 0.9, 0.25, None),
                              (128, 1.0, 1.0, rng.uniform(1, 8, 64).astype(np.float32))):
        got = o.rope(x, pos, hd, n_dims, neox, ts, m, fs, ff)
        want = r.rope(x, pos, hd, n_dims, neox, ts, m, fs, ff)
        assert np.array_equal(bits(got), bits(want)), (n_dims, m, fs, ff is None)


def test_rope_closed_form(o):
    rng = np.random.default_rng(13)
    T, nh, hd = 3, 2, 128
    x = rng.standard_normal((T, nh * hd)).astype(np.float32)
    pos = np.array([0, 5, 300], np.int32)
    base = 10000.0
    ts = np.float32(np.power(np.float32(base), np.float32(-2.0 / hd)))
    y = o.rope(x, pos, hd, hd, True, ts).astype(np.float64)
    theta = pos[:, None].astype(np.float64) * np.power(np.float64(ts), np.arange(hd // 2))[None, :]
    xd = x.reshape(T, nh, hd).astype(np.float64)
    x0, x1 = xd[..., : hd // 2], xd[..., hd // 2:]
    c, s = np.cos(theta)[:, None, :], np.sin(theta)[:, None, :]
    want = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1).reshape(T, nh * hd)
    assert np.max(np.abs(y - want)) < 2e-4        # the f32 angle recurrence drifts over 64 steps
    y0 = o.rope(x, np.zeros(T, np.int32), hd, hd, False, ts, m=1.0)     # position 0: identity
    assert np.array_equal(bits(y0), bits(x))


def test_swiglu_add_bitwise_vs_ref(o, r):
    rng = np.random.default_rng(14)
    g = np.concatenate([SPECIALS, rng.standard_normal(3000).astype(np.float32) * 6,
                        rng.integers(0, 2**32, 3000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    u = np.concatenate([SPECIALS[::-1], rng.standard_normal(g.size - SPECIALS.size).astype(np.float32)])
    assert np.array_equal(bits(o.swiglu(g[None], u[None])[0]), bits(r.vop(O.VOP_SWIGLU, g, u)))
    assert np.array_equal(bits(o.add(g[None], u[None])[0]), bits(r.vop(O.VOP_ADD, g, u)))
    x = rng.standard_normal(2000).astype(np.float32) * 4
    assert np.array_equal(bits(o.silu(x)), bits(np.array([r.lib.tsr_m_silu(float(v)) for v in x], np.float32)))
    xd = x.astype(np.float64)
    assert np.max(np.abs(o.silu(x) - xd / (1.0 + np.exp(-xd)))) < 1e-5


def test_get_rows_argmax(o):
    rng = np.random.default_rng(15)
    src = rng.standard_normal((50, 64)).astype(np.float32)
    ids = np.array([3, 0, 49, 3], np.int32)
    assert np.array_equal(o.get_rows(src, ids), src[ids])
    x = rng.standard_normal((4, 1000)).astype(np.float32)
    x[1, 10] = x[1, 500] = 9.0                                         # first maximum wins
    x[2, 3] = np.nan
    assert np.array_equal(o.argmax(x), np.array([np.argmax(x[0]), 10, np.nanargmax(x[2]), np.argmax(x[3])]))


def test_tanh_bitwise_vs_ref(o, r):
    """oc_tanh (the MUL_MAT softcap's TANH) bit for bit against tsr_m_tanh: random values across both
    branches (|x| < 2^-6 and above), the branch boundary, subnormals, specials and random bit patterns."""
    rng = np.random.default_rng(11)
    edge = np.array([0x3C800000, 0x3C7FFFFF, 0xBC800000, 0xBC7FFFFF, 0x41200000, 0x42000000, 0x00400000,
                     0x80400000, 0x7F000000, 0x7E800000], np.uint32).view(np.float32)
    x = np.concatenate([SPECIALS, edge, rng.uniform(-12, 12, 20000).astype(np.float32),
                        (rng.standard_normal(10000) * 0.01).astype(np.float32),
                        rng.integers(0, 2 ** 32, 40000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    assert (bits(o.tanh(x)) == bits(r.tanh(x))).all()


def test_tanh_closed_form(o):
    """Against float64 tanh (the EXPK error, < 4 ulp, grows by the 1 - e cancellation below |x| ~ 0.1),
    odd symmetry bit for bit, the limits, zeros, DAZ and the canonical NaN."""
    x = np.linspace(-9, 9, 20001, dtype=np.float32)
    got = o.tanh(x).astype(np.float64)
    want = np.tanh(x.astype(np.float64))
    assert (np.abs(got - want) <= 2e-5 * np.abs(want) + 1e-7).all()
    assert (bits(o.tanh(-x)) == (bits(o.tanh(x)) ^ 0x80000000)).all()
    sp = np.array([0x7F800000, 0xFF800000, 0x00000000, 0x80000000, 0x00000001, 0x80000001, 0x7FC00000, 0xFFC00001],
                  np.uint32).view(np.float32)
    assert bits(o.tanh(sp)).tolist() == [0x3F800000, 0xBF800000, 0, 0x80000000, 0, 0x80000000, 0x7FC00000, 0x7FC00000]


def test_mul_mat_epilogue_wiring(o):
    """oc_mul_mat's SCALE / SOFTCAP epilogue is applied after the addend, with the scales in their
    places: SCALE y = (dot + add) * sc, SOFTCAP y = TANH((dot + add) * fs) * sc (float32 products of
    normal values: the rule's FM)."""
    import tsr_synth as S
    N, K = 64, 256
    w = S.quant_rows(0, 5, N, K)
    x = S.normal(6, 2 * K).reshape(2, K)
    add = S.normal(7, 2 * N).reshape(2, N)
    y = o.mul_mat(0, w, K, x, add=add)
    fs, sc = np.float32(0.0333), np.float32(30.0)
    assert (bits(o.mul_mat(0, w, K, x, add=add, epi=(1, 0.0, sc))) == bits(y * sc)).all()
    soft = o.mul_mat(0, w, K, x, add=add, epi=(2, fs, sc))
    assert (bits(soft) == bits(o.tanh(y * fs).reshape(y.shape) * sc)).all()
    assert np.abs(soft).max() <= sc
