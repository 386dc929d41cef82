"""Pins of the CPU oracle (oracle/oc_*.c), CPU only.

Each check is chosen so that a plausible slip in the restatement fails it:
  * known-answer vectors held by the reference's own tests (tests/golden/known_answers.json),
  * closed forms and brute force (numpy float64, exact integer arithmetic, IEEE float16),
  * the reference library itself, compiled from /root/reference by `make -C oracle ref` (skipped
    where that library is not built),
  * planted mistakes: a perturbed input must change the answer.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O
import tsr_synth as S
from helpers import bits

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))


def u(h):
    return np.array([int(h, 16)], np.uint32).view(np.float32)


# ---- spec f32 rules -------------------------------------------------------------------------
def test_fop_known_answers(oc):
    for op, a, b, want in KA["fop"]:
        got = oc.fop(op, u(a), None if b is None else u(b))
        assert bits(got)[0] == int(want, 16), (op, a, b, hex(bits(got)[0]), want)


def test_ftz_window_closed_form(oc):
    """FTZ iff |exact| < 2^-126 - 2^-150 (docs/spec.md:1405-1418), on products exact in float64."""
    lo = 2.0 ** -126 - 2.0 ** -150
    rng = np.random.default_rng(5)
    b = (((1 + rng.integers(0, 2, 20000)) << 23) | rng.integers(0, 1 << 23, 20000)).astype(np.uint32).view(np.float32)
    a0 = (lo / b.astype(np.float64)).astype(np.float32).view(np.uint32)
    a = (a0.astype(np.int64) + rng.integers(-2, 3, 20000)).astype(np.uint32).view(np.float32)
    ex = a.astype(np.float64) * b.astype(np.float64)
    want = np.where(np.abs(ex) < lo, np.where(ex < 0, np.float32(-0.0), np.float32(0.0)), ex.astype(np.float32))
    got = oc.fop("mul", a, b)
    assert (bits(got) == bits(want)).all()
    window = ((np.abs(ex) >= lo) & (np.abs(ex) < 2.0 ** -126 - 2.0 ** -151)).sum()
    assert window > 100                              # the window x86 FTZ would flush is exercised


def test_fop_random_vs_float64(oc):
    """Normal-range operands: one IEEE operation == float64 result rounded once (innocuous double rounding)."""
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(50000) * 10.0 ** rng.integers(-10, 10, 50000)).astype(np.float32)
    b = (rng.standard_normal(50000) * 10.0 ** rng.integers(-10, 10, 50000)).astype(np.float32)
    A, B = a.astype(np.float64), b.astype(np.float64)
    for op, ex in (("add", A + B), ("sub", A - B), ("mul", A * B), ("div", A / B)):
        want = ex.astype(np.float32)
        ok = np.abs(want) >= np.float32(2.0 ** -126)
        assert (bits(oc.fop(op, a, b))[ok] == bits(want)[ok]).all(), op


def test_tree16_known_answers(oc):
    for p, want in KA["tree16"]:
        v = np.array([int(x, 16) for x in p], np.uint32).view(np.float32)
        assert bits(np.float32(oc.tree16(v)))[()] == int(want, 16)


def test_tree16_is_pairwise_not_sequential(oc):
    p = np.zeros(16, np.float32)
    p[0], p[2], p[3] = 1.0, 2.0 ** -24, 2.0 ** -24
    # pairwise: 1 + (2^-24 + 2^-24) = 1 + 2^-23 exact; left to right would give 1.0
    assert oc.tree16(p) == np.float32(1.0 + 2.0 ** -23)


def test_i2f(oc):
    for v, want in KA["i2f"]:
        assert bits(oc.i2f(np.array([v], np.int32)))[0] == int(want, 16)
    v = np.random.default_rng(2).integers(-2 ** 31, 2 ** 31, 200000).astype(np.int32)
    assert (bits(oc.i2f(v)) == bits(v.astype(np.float64).astype(np.float32))).all()


def test_fp16_known_answers_and_exhaustive(oc):
    for h, want in KA["h2f"]:
        assert bits(oc.h2f(np.array([int(h, 16)], np.uint16)))[0] == int(want, 16)
    for f, want in KA["f2h"]:
        assert oc.f2h(u(f))[0] == int(want, 16), f
    h = np.arange(65536, dtype=np.uint16)
    f = oc.h2f(h)
    nan = (h & 0x7C00) == 0x7C00
    nan &= (h & 0x3FF) != 0
    # IEEE half -> single is exact: numpy's conversion agrees on every non-NaN half
    assert (bits(f)[~nan] == bits(h.view(np.float16).astype(np.float32))[~nan]).all()
    assert (oc.f2h(f)[~nan] == h[~nan]).all()                       # round trip is the identity
    # f32 -> f16 RNE against numpy (IEEE RNE) on random non-NaN bit patterns
    x = np.random.default_rng(3).integers(0, 2 ** 32, 300000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        assert (oc.f2h(x) == x.astype(np.float16).view(np.uint16)).all()


def test_round8_closed_form(oc):
    x = np.concatenate([np.arange(-300, 300, 0.25, dtype=np.float32),
                        np.array([0.49999997, -0.49999997, 127.5, -128.5, np.inf, -np.inf, np.nan, 1e-40], np.float32)])
    fin = np.where(np.isnan(x), 0.0, x).astype(np.float64)
    away = np.clip(np.sign(fin) * np.floor(np.abs(fin) + 0.5), -128, 127)
    even = np.clip(np.round(fin), -128, 127)
    assert (oc.round8(x, False) == away).all()
    assert (oc.round8(x, True) == even).all()


# ---- QACT -----------------------------------------------------------------------------------
def _qs(qa, K):
    return qa[:, :K].view(np.int8)


def _d(qa, kind, K):
    nb = K // (32 if kind == 0 else 256)
    off = O.qa_d_off(K)
    return qa[:, off:off + 4 * nb].copy().view(np.float32)


def _bs(qa, K):
    off = O.qa_bs_off(1, K)
    return qa[:, off:off + 2 * (K // 16)].copy().view(np.int16)


def test_qact_a32_closed_form(oc):
    """A32 == quantize_row_q8_0_ref on normal inputs (docs/spec.md:1431-1437): the numpy quantizer."""
    x = S.normal(9, 8 * 4096).reshape(8, 4096)
    qa = oc.qact(0, x)
    blocks = S.quantize_q8_0(x).reshape(8, 128, 34)
    assert (_qs(qa, 4096).reshape(8, 128, 32) == blocks[:, :, 2:].view(np.int8)).all()
    d16 = blocks[:, :, 0:2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    assert (bits(_d(qa, 0, 4096)) == bits(d16)).all()


def test_qact_a256_closed_form(oc):
    x = S.normal(10, 4 * 4096).reshape(4, 4096)
    qa = oc.qact(1, x)
    b = x.reshape(4, 16, 256)
    i = np.argmax(np.abs(b), axis=2)                       # numpy argmax: first maximal index
    mx = np.take_along_axis(b, i[:, :, None], 2)[:, :, 0]
    iscale = (np.float32(-127.0) / mx).astype(np.float32)
    q = np.clip(np.round((iscale[:, :, None] * b).astype(np.float32)), -128, 127).astype(np.int8)
    assert (_qs(qa, 4096).reshape(4, 16, 256) == q).all()
    assert (bits(_d(qa, 1, 4096)) == bits((np.float32(1.0) / iscale).astype(np.float32))).all()
    assert (_bs(qa, 4096) == q.reshape(4, 256, 16).sum(axis=2, dtype=np.int32).astype(np.int16)).all()


def test_qact_specials(oc):
    """The special-value answers of sw/sim/tests/test_ref_ggml.c:245-340."""
    def q1(kind, x):
        x = np.asarray(x, np.float32)
        qa = oc.qact(kind, x[None, :])
        return _qs(qa, x.size)[0], _d(qa, kind, x.size)[0], (_bs(qa, x.size)[0] if kind else None)

    x = np.ones(256, np.float32); x[10] = -4; x[20] = 4
    q, d, _ = q1(1, x)
    assert q[10] == -127 and q[20] == 127 and d[0] == np.float32(1) / (np.float32(-127) / np.float32(-4))
    x[10], x[20] = 4, -4
    assert q1(1, x)[1][0] < 0                                           # first max +4 -> d < 0
    x = np.zeros(32, np.float32); x[:] = np.arange(32).astype(np.uint32) + np.uint32(0x00400000)
    x = x.astype(np.uint32).view(np.float32)                              # all subnormal
    q, d, _ = q1(0, x)
    assert bits(d)[0] == 0 and (q == 0).all()
    x = np.zeros(32, np.float32); x[0] = u(hex(0x04000000))[0]; x[1] = u(hex(0x007FFFFF))[0]; x[2] = u(hex(0x807FFFFF))[0]
    q, d, _ = q1(0, x)
    assert list(q[:3]) == [127, 0, 0]
    x = np.zeros(256, np.float32); x[0] = -2.0 ** -119; x[1] = u(hex(0x007FFFFF))[0]; x[17] = u(hex(0x807FFFFF))[0]
    q, d, bs = q1(1, x)
    assert list(q[[0, 1, 17]]) == [-127, 0, 0] and list(bs[:2]) == [-127, 0]
    x = np.zeros(256, np.float32); x[5] = u(hex(0x00400000))[0]; x[9] = u(hex(0x80300000))[0]
    q, d, bs = q1(1, x)
    assert bits(d)[0] == 0 and (q == 0).all() and (bs == 0).all()
    x = np.zeros(32, np.float32); x[3] = 2.0 ** -122; x[4] = -2.0 ** -123
    q, d, _ = q1(0, x)
    assert bits(d)[0] == 0 and q[3] == 0
    x = np.arange(32, dtype=np.float32) - 16; x[5] = np.nan
    q, d, _ = q1(0, x)
    assert d[0] == np.float16(np.float32(16.0) / np.float32(127.0)).astype(np.float32) and q[5] == 0 and q[0] == -127
    x[5] = np.inf
    q, d, _ = q1(0, x)
    assert bits(d)[0] == 0x7F800000 and (q == 0).all()
    x = np.full(256, np.nan, np.float32)
    q, d, bs = q1(1, x)
    assert bits(d)[0] == 0 and (bs == 0).all()
    x = np.ones(256, np.float32); x[7] = np.inf
    q, d, _ = q1(1, x)
    assert bits(d)[0] == 0xFF800000 and (q == 0).all()
    x = np.zeros(256, np.float32); x[0] = 2.0 ** -125; x[1] = -2.0 ** -126
    q, d, bs = q1(1, x)
    assert bits(d)[0] == 0x80000000 and q[0] == -128 and q[1] == 127 and q[2] == 0 and bs[0] == -1


def test_qact_tie_example(oc):
    ex = KA["a32_tie_example"]
    x = np.zeros(32, np.float32); x[:3] = ex["x"]
    assert list(_qs(oc.qact(0, x[None, :]), 32)[0, :3]) == ex["q"]


# ---- MVM ------------------------------------------------------------------------------------
def test_isums_brute_force(oc):
    """Integer block sums by direct numpy arithmetic on the ggml blocks."""
    K = 1024
    x = S.normal(21, K)[None, :]
    w8 = S.quantize_q8_0(S.normal(22, 8 * K, 0.02).reshape(8, K))
    qa8 = oc.qact(0, x)
    qx = _qs(qa8, K)[0].astype(np.int64)
    qw = w8.reshape(8, K // 32, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    assert (oc.isums(0, w8, K, qa8) == (qw * qx.reshape(K // 32, 32)).sum(axis=2)).all()
    w4 = S.quantize_q4_k(S.normal(23, 8 * K, 0.02).reshape(8, K))
    qa4 = oc.qact(1, x)
    qx = _qs(qa4, K)[0].astype(np.int64).reshape(K // 256, 8, 32)
    b = w4.reshape(8, K // 256, 144)
    sc, mn = S.q4k_scale_min(b[:, :, 4:16])
    qs = b[:, :, 16:].reshape(8, K // 256, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=3).reshape(8, K // 256, 8, 32).astype(np.int64)
    isum = (sc * (q * qx).sum(axis=3)).sum(axis=2)
    bsp = _bs(qa4, K)[0].astype(np.int64).reshape(K // 256, 8, 2).sum(axis=2)
    msum = (mn * bsp).sum(axis=2)
    got = oc.isums(1, w4, K, qa4).reshape(8, K // 256, 2)
    assert (got[:, :, 0] == isum).all() and (got[:, :, 1] == msum).all()


def _dot_model(oc, fmt, w, K, qa):
    """Independent model of the row rule in float32 numpy: terms, 16 partials, pairwise tree."""
    N = w.shape[0]
    is_ = oc.isums(fmt, w, K, qa).astype(np.float32)
    if fmt == 0:
        d = w.reshape(N, K // 32, 34)[:, :, 0:2].copy().view(np.float16).astype(np.float32)[:, :, 0]
        t = (d * _d(qa, 0, K)[0]) * is_
    else:
        b = w.reshape(N, K // 256, 144)
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[:, :, 0]
        dm = b[:, :, 2:4].copy().view(np.float16).astype(np.float32)[:, :, 0]
        dx = _d(qa, 1, K)[0]
        t = (d * dx) * is_[:, 0::2] - (dm * dx) * is_[:, 1::2]
    nb = t.shape[1]
    p = np.zeros((N, 16), np.float32)
    for i in range(nb):
        p[:, i % 16] = p[:, i % 16] + t[:, i]
    while p.shape[1] > 1:
        p = p[:, 0::2] + p[:, 1::2]
    return p[:, 0]


@pytest.mark.parametrize("fmt,K", [(0, 896), (0, 4096), (1, 4096), (1, 14336)])
def test_dot_row_model(oc, fmt, K):
    w = S.quantize_q8_0(S.normal(31, 64 * K, 0.02).reshape(64, K)) if fmt == 0 else \
        S.quantize_q4_k(S.normal(31, 64 * K, 0.02).reshape(64, K))
    x = S.normal(32, K)[None, :]
    qa = oc.qact(0 if fmt == 0 else 1, x)
    y = oc.mul_mat(fmt, w, K, x)[0]
    assert (bits(y) == bits(_dot_model(oc, fmt, w, K, qa))).all()
    # and close to the float64 product of the dequantized operands (1e-5 relative to sum |terms|)
    deq = S.dequantize_q8_0(w, K) if fmt == 0 else S.dequantize_q4_k(w, K)
    xq = _qs(qa, K)[0].astype(np.float64) * np.repeat(_d(qa, 0 if fmt == 0 else 1, K)[0], 32 if fmt == 0 else 256)
    ex = deq.astype(np.float64) @ xq
    scale = np.abs(deq.astype(np.float64)) @ np.abs(xq)
    assert (np.abs(y - ex) <= 1e-5 * scale + 1e-30).all()


def test_mul_mat_add_and_tokens(oc):
    K, N = 512, 40
    w = S.quantize_q4_k(S.normal(41, N * K, 0.02).reshape(N, K))
    x = S.normal(42, 3 * K).reshape(3, K)
    add = S.normal(43, 3 * N).reshape(3, N)
    y = oc.mul_mat(1, w, K, x)
    ya = oc.mul_mat(1, w, K, x, add=add)
    assert (bits(ya) == bits(oc.fop("add", add, y))).all()
    assert (bits(oc.mul_mat(1, w, K, x[1:2])[0]) == bits(y[1])).all()       # tokens independent


# ---- EXP and block floating point -----------------------------------------------------------
def test_expk_accuracy(oc):
    v = np.concatenate([np.linspace(-87, 88, 200001, dtype=np.float32), -np.abs(S.normal(4, 100000) * 20)])
    e = oc.expk(v).astype(np.float64)
    ex = np.exp(v.astype(np.float64))
    ok = (ex > 2.0 ** -126) & (ex < 3e38)
    rel = np.abs(e[ok] - ex[ok]) / ex[ok]
    assert rel.max() < 4 * 2.0 ** -24                     # a few ulps: the table / Horner approximation
    sp = oc.expk(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, 89.0, -104.0], np.float32))
    assert list(bits(sp)) == [0x3F800000, 0x3F800000, 0x7F800000, 0, 0x7FC00000, 0x3F800000, 0x7F800000, 0]


def test_bf_int_and_bf_f_exact(oc):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    e = (np.frexp(w.astype(np.float64))[1] - 1).astype(np.int32)
    es = e + rng.integers(0, 30, w.size).astype(np.int32)
    got = oc.bf_int(w, es)
    for i in range(0, w.size, 97):
        v = float(w[i]) * 2.0 ** (23 - int(es[i]))        # exact in float64
        want = int(np.round(v))                           # numpy round: half to even
        assert got[i] == want, (w[i], es[i])
    A = rng.integers(-2 ** 45, 2 ** 45, 20000).astype(np.int64)
    k = rng.integers(-60, 10, 20000).astype(np.int32)
    f = oc.bf_f(A, k)
    for i in range(0, A.size, 97):
        a = int(A[i])
        if a == 0:
            continue
        m = abs(a)
        sh = max(0, m.bit_length() - 24)
        r = m >> sh
        rem = m - (r << sh)
        half = (1 << (sh - 1)) if sh else 0
        if sh and (rem > half or (rem == half and r & 1)):
            r += 1
        want = math.copysign(math.ldexp(r, sh + int(k[i])), a)
        assert f[i] == np.float32(want), (a, k[i])


def test_maxt(oc):
    a = np.array([-0.0, 0.0, 1.0, -np.inf, np.nan, 1e-40], np.float32)
    b = np.array([0.0, -0.0, 2.0, -1.0, 1.0, -1e-40], np.float32)
    got = oc.maxt(a, b)
    assert list(bits(got)) == [0x00000000, 0x00000000, 0x40000000, 0xBF800000, 0x7FC00000, 0x00000000]


# ---- attention ------------------------------------------------------------------------------
def _kv(oc, kv_size, E, seed):
    kf = S.normal(seed, kv_size * E).reshape(kv_size, E)
    vf = S.normal(seed + 1, kv_size * E).reshape(kv_size, E)
    kc = np.zeros((kv_size, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    oc.kv_set_rows(kc, kf, np.arange(kv_size))
    oc.kv_set_rows(vc, vf, np.arange(kv_size))
    return kc, vc


def _fa_f64(oc, q, kc, vc, D, n_head, n_head_kv, scale, vis):
    """float64 softmax attention over the dequantized q8 cache and the dequantized QA(A32) of q
    (the algorithm quantizes Q before the scores, sw/sim/tsr_ref_at.c:809-810)."""
    E = n_head_kv * D
    qa = oc.qact(0, q)
    Kq = n_head * D
    q = _qs(qa, Kq).astype(np.float64) * np.repeat(_d(qa, 0, Kq), 32, axis=1)
    K = S.dequantize_q8_0(kc, E).astype(np.float64)
    V = S.dequantize_q8_0(vc, E).astype(np.float64)
    G = n_head // n_head_kv
    out = np.zeros((q.shape[0], n_head * D))
    for t in range(q.shape[0]):
        for h in range(n_head):
            g = h // G
            s = K[:, g * D:(g + 1) * D] @ q[t, h * D:(h + 1) * D].astype(np.float64) * scale
            s = np.where(vis[t], s, -np.inf)
            p = np.exp(s - s.max())
            out[t, h * D:(h + 1) * D] = (p @ V[:, g * D:(g + 1) * D]) / p.sum()
    return out


@pytest.mark.parametrize("n_kv,n_head,n_head_kv,D", [(512, 32, 8, 128), (300, 8, 2, 64), (1000, 4, 4, 256)])
def test_fa_decode_vs_float64(oc, n_kv, n_head, n_head_kv, D):
    kc, vc = _kv(oc, n_kv, n_head_kv * D, 50)
    q = S.normal(52, n_head * D).astype(np.float16).astype(np.float32)[None, :]
    scale = np.float32(1.0 / math.sqrt(D))
    msum = oc.msum(np.zeros((1, n_kv), np.float16))
    y = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, msum)
    want = _fa_f64(oc, q, kc, vc, D, n_head, n_head_kv, float(scale), np.ones((1, n_kv), bool))
    assert np.abs(y - want).max() < 2e-3


def test_fa_causal_prefill_vs_float64(oc):
    T, D, n_head, n_head_kv = 48, 128, 8, 2
    kc, vc = _kv(oc, T, n_head_kv * D, 60)
    q = S.normal(62, T * n_head * D).reshape(T, n_head * D)
    mask = np.full((T, T), -np.inf, np.float16)
    for i in range(T):
        mask[i, :i + 1] = 0
    scale = np.float32(1.0 / math.sqrt(D))
    y = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, oc.msum(mask), new_runs=[[0, T]])
    want = _fa_f64(oc, q, kc, vc, D, n_head, n_head_kv, float(scale), np.isfinite(mask.astype(np.float32)))
    assert np.abs(y - want).max() < 2e-3


def test_fa_plan_rules(oc):
    E, D = 1024, 128
    msum = oc.msum(np.zeros((1, 8192), np.float16))
    ch = oc.plan_row(E, D, msum, 0)
    assert [(c[0], c[1]) for c in ch] == [(0, 128), (128, 128), (256, 128), (384, 128)]   # NCG = 128
    ch = oc.plan_row(E, D, msum, 0, new_runs=[[8191, 8192]])
    assert [c[0] for c in ch] == [0, 128, 256, 384][:3] + [384]                        # newest last (already last)
    ch = oc.plan_row(E, D, msum, 0, new_runs=[[5, 6]])
    assert [c[0] for c in ch] == [128, 256, 384, 0]
    m = np.full((1, 300), -np.inf, np.float16); m[0, 10:40] = 0; m[0, 200:260] = 0
    ch = oc.plan_row(E, D, oc.msum(m), 0)
    assert [(c[0], c[1], c[2], c[3], c[4]) for c in ch] == [(0, 3, 10, 40, 0), (12, 5, 8, 68, 0)]
    assert oc.plan_row(E, D, oc.msum(np.full((1, 64), -np.inf, np.float16)), 0) == [(0, 1, 0, 0, 0)]


def test_fa_new_runs_change_order_and_bits(oc):
    """A planted difference: merging chunks in another order changes the result bits."""
    kc, vc = _kv(oc, 8192, 256, 70)                   # 4 chunks: with 2 the merge is symmetric
    q = S.normal(72, 256)[None, :]
    msum = oc.msum(np.zeros((1, 8192), np.float16))
    a = oc.flash_attn(q, kc, vc, 128, 2, 2, np.float32(0.088), msum)
    b = oc.flash_attn(q, kc, vc, 128, 2, 2, np.float32(0.088), msum, new_runs=[[0, 1]])
    assert np.abs(a - b).max() < 1e-5 and (bits(a) != bits(b)).any()


# ---- against the reference library -----------------------------------------------------------
def test_vs_ref_scalar_rules(oc, ref):
    rng = np.random.default_rng(11)
    a = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    b = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for op, fn in (("add", "tsr_fadd"), ("sub", "tsr_fsub"), ("mul", "tsr_fmul"), ("div", "tsr_fdiv")):
        assert (bits(oc.fop(op, a, b)) == bits(ref.vec(fn, a, b))).all(), op
    assert (bits(oc.fop("recip", a)) == bits(ref.vec("tsr_frecip", a))).all()
    h = np.arange(65536, dtype=np.uint16)
    assert (bits(oc.h2f(h)) == bits(ref.vec("tsr_fp16_to_f32", h))).all()
    assert (oc.f2h(a) == ref.vec("tsr_f32_to_fp16", a, out_dtype=np.uint16)).all()
    x = (rng.standard_normal(30000) * 100).astype(np.float32)
    assert (oc.round8(x, False) == ref.vec("tsr_q8_round_away", x, out_dtype=np.int32)).all()
    assert (oc.round8(x, True) == ref.vec("tsr_q8_round_even", x, out_dtype=np.int32)).all()


def test_vs_ref_expk(oc, ref):
    rng = np.random.default_rng(12)
    v = np.concatenate([(rng.standard_normal(30000) * 30).astype(np.float32),
                        rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        -np.arange(0, 100, 0.001, dtype=np.float32)])
    assert (bits(oc.expk(v)) == bits(ref.vec("tsr_m_exp", v))).all()


def test_vs_ref_block_float(oc, ref):
    rng = np.random.default_rng(13)
    A = rng.integers(-2 ** 44, 2 ** 44, 5000).astype(np.int64)
    k = rng.integers(-200, 120, 5000).astype(np.int32)
    assert (bits(oc.bf_f(A, k)) == bits(ref.vec("tsr_att_bf_f", A, k))).all()


@pytest.mark.parametrize("kind,K", [(0, 896), (1, 4096), (0, 4096), (1, 14336)])
def test_vs_ref_qact(oc, ref, kind, K):
    from helpers import special_row
    x = np.stack([S.normal(14, K), special_row(K, 15), S.normal(16, K, 1e-30)])
    assert (oc.qact(kind, x) == ref.qact(kind, x)).all()


@pytest.mark.parametrize("fmt,N,K", [(0, 64, 896), (1, 32, 4096), (1, 16, 14336), (0, 16, 32), (1, 16, 256)])
def test_vs_ref_dot_rows(oc, ref, fmt, N, K):
    w = S.quantize_q8_0(S.normal(17, N * K, 0.02).reshape(N, K)) if fmt == 0 else \
        S.quantize_q4_k(S.normal(17, N * K, 0.02).reshape(N, K))
    x = S.normal(18, K)[None, :]
    qa = oc.qact(0 if fmt == 0 else 1, x)
    assert (bits(oc.mul_mat(fmt, w, K, x)[0]) == bits(ref.dot_rows(fmt, w, K, qa[0]))).all()


def _fa_case(oc, ref, n_kv, kv_size, n_head, n_head_kv, D, T=1, mask=None, new_runs=None, seed=3):
    E = n_head_kv * D
    kc, vc = _kv(oc, kv_size, E, seed)
    q = S.normal(seed + 2, T * n_head * D).reshape(T, n_head * D).astype(np.float16).astype(np.float32)
    mask = np.zeros((T, n_kv), np.float16) if mask is None else mask
    scale = np.float32(1 / math.sqrt(D))
    mw = oc.msum(mask)
    assert (mw == ref.msum(mask)).all()
    mf = oc.mask_f32(mask, scale) if mw[3] else None
    if mf is not None:
        assert (bits(mf) == bits(ref.mask_f32(mask, scale))).all()
    yo = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, mw, mf, new_runs)
    yr = ref.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, mw, mf, new_runs)
    assert (bits(yo) == bits(yr)).all()


def test_vs_ref_fa_decode(oc, ref):
    _fa_case(oc, ref, 512, 512, 32, 8, 128)
    _fa_case(oc, ref, 300, 512, 8, 2, 64)
    _fa_case(oc, ref, 1000, 1024, 4, 4, 128, new_runs=[[999, 1000]])


@pytest.mark.parametrize("n_kv", [8192, 13000])
def test_vs_ref_fa_decode_chunks(oc, ref, n_kv):
    """BASELINE configs[2]'s shape (32 q / 8 KV heads, D 128) at 8192 cells (4 chunks of 2048: three
    online merges, tsr_ref_at.c:600-633) and at 13000 cells (7 chunks, a short last one), the newest
    cell last."""
    _fa_case(oc, ref, n_kv, n_kv, 32, 8, 128, new_runs=[[n_kv - 1, n_kv]], seed=n_kv)


def test_vs_ref_fa_masks(oc, ref):
    T = 40
    m = np.full((T, T), -np.inf, np.float16)
    for i in range(T):
        m[i, :i + 1] = 0
    _fa_case(oc, ref, T, 48, 8, 2, 128, T=T, mask=m, new_runs=[[0, T]])
    m2 = np.zeros((3, 100), np.float16); m2[:, 10:20] = -2.5; m2[1, 50:] = -np.inf
    _fa_case(oc, ref, 100, 112, 8, 2, 64, T=3, mask=m2)
    m3 = np.full((2, 200), -np.inf, np.float16); m3[:, 0:20] = 0; m3[:, 150:180] = 0
    _fa_case(oc, ref, 200, 208, 4, 1, 256, T=2, mask=m3)
    _fa_case(oc, ref, 64, 64, 4, 1, 512, T=1, mask=np.full((1, 64), -np.inf, np.float16))
