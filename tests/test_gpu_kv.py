"""GPU KV cache: the ggml q8_0 image round trip (exact) and SET_ROWS against the oracle."""
import numpy as np
import pytest

import tsr_synth as S

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,kv_size", [(1024, 256), (256, 100), (64, 33)])
def test_kv_bytes_round_trip(dev, E, kv_size):
    kv = dev.kv(E, kv_size)
    rng = np.random.default_rng(E + kv_size)
    for which in (0, 1):
        img = rng.integers(0, 256, kv_size * E // 32 * 34, dtype=np.uint8)
        kv.set_bytes(which, img)
        assert (kv.get_bytes(which) == img).all()
        # partial, unaligned ranges
        off, n = 37, 1000
        patch = rng.integers(0, 256, n, dtype=np.uint8)
        kv.set_bytes(which, patch, off)
        img[off:off + n] = patch
        assert (kv.get_bytes(which) == img).all()
        assert (kv.get_bytes(which, 5, 77) == img[5:82]).all()


def test_kv_set_rows_matches_oracle(dev, oc):
    E, kv_size, n = 1024, 64, 10
    kv = dev.kv(E, kv_size)
    src = S.normal(3, n * E).reshape(n, E)
    src[2, 5] = np.nan
    src[3, :32] = 0
    idx = np.array([0, 5, 63, 17, 16, 1, 2, 40, 41, 9], np.int64)
    want = np.zeros((kv_size, E // 32 * 34), np.uint8)
    oc.kv_set_rows(want, src, idx)
    for which in (0, 1):
        kv.set_bytes(which, np.zeros(kv_size * E // 32 * 34, np.uint8))
        bad = dev.upload(np.zeros(1, np.int32))
        dev.kv_set_rows(kv, which, dev.upload(src), n, E, dev.upload(idx), bad)
        got = kv.get_bytes(which).reshape(kv_size, -1)
        assert (got == want).all()
        assert bad.read(np.int32, (1,))[0] == 0


def test_kv_set_rows_bad_index_flag(dev):
    kv = dev.kv(64, 16)
    bad = dev.upload(np.zeros(1, np.int32))
    dev.kv_set_rows(kv, 0, dev.upload(np.ones((2, 64), np.float32)), 2, 64,
                    dev.upload(np.array([3, 16], np.int64)), bad)
    dev.sync()
    assert bad.read(np.int32, (1,))[0] == 1
