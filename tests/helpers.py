"""Input builders shared by the tests (numpy only)."""
import numpy as np

import tsr_synth as S


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    g, w = bits(got), bits(want)
    bad = np.flatnonzero(g.ravel() != w.ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ; first at {i}: "
                             f"got {g.ravel()[i]:#010x} ({got.ravel()[i]!r}) want {w.ravel()[i]:#010x} ({want.ravel()[i]!r})")


def weights(fmt, N, K, seed, std=0.02):
    w = S.normal(seed, N * K, std).reshape(N, K)
    return S.quantize_q8_0(w) if fmt == 0 else S.quantize_q4_k(w)


def special_row(K, seed):
    """A row mixing normals with the values QACT treats specially."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(K).astype(np.float32)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-42, 3.0e38, -3.0e38, 0.5, -0.5, 2.5, -127.0,
                   1e-30, 6e-39], np.float32)
    idx = rng.choice(K, size=min(K // 4, 64), replace=False)
    x[idx] = rng.choice(sp, size=idx.size)
    return x
