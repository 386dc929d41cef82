"""The FLASH_ATTN_EXT entry point that allocates nothing (tsr_hip_flash_attn_noalloc, partials in the
library's fixed device array) against the entry point that uses the context's scratch
(tsr_hip_flash_attn): bit-identical outputs on two calls in a row through the C ABI, the second with a
smaller input (the array keeps the first call's contents), and the oracle's bits; sizes beyond the fixed
array are refused before anything runs."""
import math

import numpy as np
import pytest

import tsr_hip
import tsr_synth as S
from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


def _case(oc, dev, n_kv, T, n_head, n_head_kv, D, seed):
    """Causal rows over the newest T of n_kv cells. oc None: a refusal case (cache bytes are zeros, no
    expected output)."""
    E = n_head_kv * D
    kc = np.zeros((n_kv, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    if oc is not None:
        oc.kv_set_rows(kc, S.normal(seed, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
        oc.kv_set_rows(vc, S.normal(seed + 1, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    q = S.normal(seed + 2, T * n_head * D).reshape(T, n_head * D).astype(np.float16).astype(np.float32)
    mask = np.full((T, n_kv), -np.inf, np.float16)
    for t in range(T):
        mask[t, :n_kv - T + t + 1] = 0
    scale = np.float32(1.0 / math.sqrt(D))
    msum = tsr_hip.msum_build_f16(mask)
    runs = [[n_kv - T, n_kv]]
    K_, V_ = dev.kv(E, n_kv), dev.kv(E, n_kv)
    K_.set_bytes(0, kc)
    V_.set_bytes(1, vc)
    c = dict(q=dev.upload(q), K=K_, V=V_, msum=msum, scale=scale, runs=runs, T=T, args=(D, n_head, n_head_kv))
    c["want"] = oc.flash_attn(q, kc, vc, D, n_head, n_head_kv, scale, msum, None, runs) if oc is not None else None
    return c


def _call(dev, c, noalloc):
    D, n_head, n_head_kv = c["args"]
    T, K = c["T"], n_head * D
    out = dev.alloc(4 * T * K).fill(0xFF)
    fn = dev.flash_attn_noalloc if noalloc else dev.flash_attn
    fn(c["q"], T, K, c["K"], c["V"], D, n_head, n_head_kv, c["scale"], c["msum"], out, K, new_runs=c["runs"])
    dev.sync()
    return out.read(np.float32, (T, K))


def test_noalloc_matches_scratch_entry(dev, oc):
    big = _case(oc, dev, 8192, 4, 32, 8, 128, 71)       # 4 rows, 4 chunks each: 16 items
    small = _case(oc, dev, 700, 1, 8, 2, 64, 72)        # then a smaller call over the same array
    for name, c in (("first, 4 rows x 8192 cells", big), ("second, 1 row x 700 cells", small)):
        print(f"\nnoalloc FA: {name}", flush=True)
        got = _call(dev, c, True)
        want = _call(dev, c, False)
        assert_bits_equal(got, want, f"{name}: noalloc vs scratch entry")
        assert_bits_equal(got, c["want"], f"{name}: noalloc vs oracle")
    assert_bits_equal(_call(dev, big, True), big["want"], "the first shape again")


def test_noalloc_refusals(dev):
    """More than 8 rows, or partials beyond the 16 MiB array (8 rows x 12288 cells x 64 heads of scores,
    48 chunks): TSR_HIP_E_RANGE, nothing launched; the scratch entry point takes the same calls."""
    c9 = _case(None, dev, 64, 9, 8, 2, 64, 73)
    with pytest.raises(tsr_hip.TsrHipError) as e:
        _call(dev, c9, True)
    assert e.value.code == -5
    c8 = _case(None, dev, 12288, 8, 64, 8, 128, 74)
    with pytest.raises(tsr_hip.TsrHipError) as e:
        _call(dev, c8, True)
    assert e.value.code == -5
    assert _call(dev, c9, False).shape == (9, 8 * 64)   # the scratch entry takes both
    assert _call(dev, c8, False).shape == (8, 64 * 128)
