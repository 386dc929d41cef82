"""GPU parity of the planned FLASH_ATTN_EXT decode entry point (tsr_hip_flash_attn_plan: one launch of the
decode form, k_fa_dec) against the CPU oracle, at the BASELINE shape and beyond: every chunk count that
makes the reducers run one, two or three rounds of items, bit for bit. Also the tag wrap of the form's
exchanges and the counter that names the form that ran."""
import math

import numpy as np
import pytest

import tsr_hip as H
import tsr_synth as S
from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


def _case(dev, oc, n_kv, n_head=32, n_head_kv=8, D=128, kv_size=None, seed=None):
    """BASELINE configs[2]'s draws: K, V f32 N(0, 1) through SET_ROWS (QACT A32) into q8_0 caches, Q f16
    N(0, 1) widened exactly, scale 1/sqrt(D), a mask of zeros over n_kv cells (one FAST run)."""
    kv_size = kv_size or n_kv
    E = n_head_kv * D
    seed = n_kv if seed is None else seed
    kc = np.zeros((kv_size, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    oc.kv_set_rows(kc, S.normal(S.seed_of("fa-plan-k", str(seed)), n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    oc.kv_set_rows(vc, S.normal(S.seed_of("fa-plan-v", str(seed)), n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    q = S.normal(S.seed_of("fa-plan-q", str(seed)), n_head * D).reshape(1, n_head * D)
    q = q.astype(np.float16).astype(np.float32)
    scale = np.float32(1.0 / math.sqrt(D))
    msum = oc.msum(np.zeros((1, n_kv), np.float16))
    want = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, msum)
    K_, V_ = dev.kv(E, kv_size), dev.kv(E, kv_size)
    K_.set_bytes(0, kc)
    V_.set_bytes(1, vc)
    return dict(q=dev.upload(q), K=K_, V=V_, msum=msum, scale=scale, want=want, shape=(D, n_head, n_head_kv),
                kv_size=kv_size)


def _free(c):
    c["K"].free()
    c["V"].free()


# 2048-cell chunks at this shape (NCG 128 groups); the reducers load 3 items per round
@pytest.mark.parametrize("n_kv", [
    8192,    # 4 chunks, two reducer rounds (3 + 1)
    6200,    # 4 chunks, the last one short
    12288,   # 6 chunks: two full rounds
    13000,   # 7 chunks: two full rounds and a partial one
    4136,    # 3 chunks, one round (the e2e decode's context)
    100,     # one chunk of 7 groups
])
def test_flash_attn_plan_decode(dev, oc, n_kv):
    print(f"\nflash_attn_plan n_kv {n_kv}", flush=True)
    c = _case(dev, oc, n_kv)
    D, n_head, n_head_kv = c["shape"]
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, c["kv_size"])
    try:
        plan.set(c["msum"])
        out = dev.alloc(4 * n_head * D)
        before = dev.counters()
        for rep in range(3):                  # the second and third launch tag with the next epochs
            out.write(np.full(n_head * D, np.nan, np.float32))
            dev.flash_attn_plan(plan, c["q"], n_head * D, c["K"], c["V"], c["scale"], out, n_head * D)
            got = out.read(np.float32, (1, n_head * D))
            assert np.abs(got - c["want"]).max() <= 2e-3
            assert_bits_equal(got, c["want"], f"planned decode {n_kv} cells, launch {rep}")
        after = dev.counters()
        assert after["fa_dec_launches"] - before["fa_dec_launches"] == 3, "the one-launch decode form did not run"
        assert dev.get_flags() == 0
        # the unplanned entry point (QK, P.V and merge launches) on the same inputs: the same bits
        out2 = dev.alloc(4 * n_head * D)
        dev.flash_attn(c["q"], 1, n_head * D, c["K"], c["V"], D, n_head, n_head_kv, c["scale"], c["msum"], out2,
                       n_head * D)
        assert_bits_equal(out2.read(np.float32, (1, n_head * D)), c["want"], "unplanned")
    finally:
        plan.free()
        _free(c)


def test_flash_attn_plan_grows_and_shrinks(dev, oc):
    """One plan re-planned per token as the context moves across chunk counts (2 -> 4 -> 7 -> 3 chunks):
    slots of items that the previous launch did not use carry older tags and are never taken for this
    launch's."""
    kv_size = 13056
    D, n_head, n_head_kv = 128, 32, 8
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, kv_size)
    full = _case(dev, oc, kv_size, seed=77)
    try:
        out = dev.alloc(4 * n_head * D)
        kc, vc = full["K"].get_bytes(0).reshape(kv_size, -1), full["V"].get_bytes(1).reshape(kv_size, -1)
        for n_kv in (3000, 8192, 13000, 5000, 12288, 100):
            msum = oc.msum(np.zeros((1, n_kv), np.float16))
            want = oc.flash_attn(full["q"].read(np.float32, (1, n_head * D)), kc, vc, D, n_head, n_head_kv,
                                 full["scale"], msum)
            plan.set(msum)
            out.write(np.full(n_head * D, np.nan, np.float32))
            dev.flash_attn_plan(plan, full["q"], n_head * D, full["K"], full["V"], full["scale"], out, n_head * D)
            assert_bits_equal(out.read(np.float32, (1, n_head * D)), want, f"{n_kv} cells")
        assert dev.get_flags() == 0
    finally:
        plan.free()
        _free(full)


@pytest.mark.parametrize("epoch", [0x0FFFFFFE, 0x0FFFFFFF])
def test_flash_attn_plan_tag_wrap(dev, oc, epoch):
    """The launches around the tag wrap: with the epoch words at 2^28 - 2 the launches tag with 2^28 - 1,
    then 1, 2; at 2^28 - 1 with 1, 2, 3. Plan memory no launch has written holds tag 0, which no launch
    uses, so a fresh plan's slots never pass for results."""
    c = _case(dev, oc, 8192, seed=8)
    D, n_head, n_head_kv = c["shape"]
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, c["kv_size"])
    try:
        plan.set(c["msum"])
        plan.set_epoch(epoch)
        out = dev.alloc(4 * n_head * D)
        for rep in range(3):
            out.write(np.full(n_head * D, np.nan, np.float32))
            dev.flash_attn_plan(plan, c["q"], n_head * D, c["K"], c["V"], c["scale"], out, n_head * D)
            assert_bits_equal(out.read(np.float32, (1, n_head * D)), c["want"], f"epoch {epoch:#x} launch {rep}")
        assert dev.get_flags() == 0
    finally:
        plan.free()
        _free(c)


@pytest.mark.parametrize("a,flushed", [(7.16, True), (5.3, False)])
def test_flash_attn_plan_subnormal_merge(dev, oc, a, flushed):
    """The online merge's FTZ: the first 2048-cell chunk holds the only nonzero values (one cell, 127 2^-24
    in every dimension: O ~ 7.6e-6), the second a cell whose score is a 128 higher (q all ones, k all a), so
    the first chunk's merge factor is EXPK(-11.3 a) (scale 1/sqrt(128)). At a = 7.16 it is ~6.6e-36, a
    normal number, and O times it (~5e-41) is subnormal: the f32 rule flushes it and every output is +0.
    At a = 5.3 the product (~7e-32) is normal and survives to the output."""
    D, n_head, n_head_kv, n_kv = 128, 32, 8, 4096
    E = n_head_kv * D
    print(f"\nsubnormal merge a={a}", flush=True)
    kf = np.zeros((n_kv, E), np.float32)
    vf = np.zeros((n_kv, E), np.float32)
    kf[3000, :] = a
    vf[5, :] = 127 * 2.0 ** -24
    kc = np.zeros((n_kv, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    oc.kv_set_rows(kc, kf, np.arange(n_kv))
    oc.kv_set_rows(vc, vf, np.arange(n_kv))
    qh = np.ones((1, n_head * D), np.float32)
    scale = np.float32(1.0 / math.sqrt(D))
    msum = oc.msum(np.zeros((1, n_kv), np.float16))
    want = oc.flash_attn(qh, kc, vc, D, n_head, n_head_kv, scale, msum)
    assert (np.count_nonzero(want) == 0) == flushed
    K_, V_ = dev.kv(E, n_kv), dev.kv(E, n_kv)
    K_.set_bytes(0, kc)
    V_.set_bytes(1, vc)
    q = dev.upload(qh)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, n_kv)
    try:
        plan.set(msum)
        out = dev.alloc(4 * n_head * D)
        out.write(np.full(n_head * D, np.nan, np.float32))
        dev.flash_attn_plan(plan, q, n_head * D, K_, V_, scale, out, n_head * D)
        assert_bits_equal(out.read(np.float32, (1, n_head * D)), want, f"planned, a={a}")
        out.write(np.full(n_head * D, np.nan, np.float32))
        dev.flash_attn(q, 1, n_head * D, K_, V_, D, n_head, n_head_kv, scale, msum, out, n_head * D)
        assert_bits_equal(out.read(np.float32, (1, n_head * D)), want, f"unplanned, a={a}")
        assert dev.get_flags() == 0
    finally:
        plan.free()
        K_.free()
        V_.free()
