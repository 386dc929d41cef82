"""GPU parity of FLASH_ATTN_EXT over the q8_0 KV cache against the CPU oracle (bit-exact; the
contract's tolerance is 2e-3 absolute, asserted as well against the float64 model of the test suite)."""
import math

import numpy as np
import pytest

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
