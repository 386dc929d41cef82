"""GPU parity of prefill MUL_MAT (T >= 16 tokens, Q8_0 weights, int8 matrix cores) through the C
ABI against the CPU oracle: bit-exact f32 outputs, as for the matvec path.

The prefill path quantizes every token row (QACT A32), takes the integer block sums from the i8
matrix core and the scale products from the f32 matrix core; these tests cover ragged tiles (T and
N not multiples of 64), every K class (one block, under 16 blocks, many rounds of the 16 partials),
the fused addend / accumulate flags, special activations and weight scales, and the BASELINE
prefill shape (512 tokens x 4096 x 4096) on a sample of tokens and rows."""
import numpy as np
import pytest

import tsr_hip
import tsr_synth as S
from helpers import assert_bits_equal, special_row, weights

pytestmark = pytest.mark.gpu


def _mm(dev, oc, N, K, T, seed=1, x=None, add=False, acc=False, wblocks=None, fmt=0):
    blocks = weights(fmt, N, K, seed) if wblocks is None else wblocks
    w = dev.weight(fmt, blocks, N, K)
    if x is None:
        x = S.normal(seed + 100, T * K).reshape(T, K)
    y0 = S.normal(seed + 200, T * N).reshape(T, N)
    yb = dev.upload(y0)
    a = S.normal(seed + 300, T * N).reshape(T, N) if add else None
    dev.mul_mat(w, dev.upload(x), T, K, yb, N, dev.upload(a) if add else None, N if add else 0,
                tsr_hip.MM_ACC_DST if acc else 0)
    got = yb.read(np.float32, (T, N))
    want = oc.mul_mat(fmt, blocks, K, x, add=(a if add else (y0 if acc else None)), threads=8)
    w.free()
    return got, want


@pytest.mark.parametrize("T,N,K", [(16, 64, 32), (17, 100, 896), (64, 4864, 896), (100, 33, 4096),
                                   (70, 128, 14336), (16, 1, 512), (130, 200, 1024)])
def test_mm_q8_0_shapes(dev, oc, T, N, K):
    got, want = _mm(dev, oc, N, K, T, seed=T + N)
    assert_bits_equal(got, want, f"T {T} {N}x{K}")


def test_mm_q8_0_add_acc(dev, oc):
    got, want = _mm(dev, oc, 96, 896, 40, seed=3, add=True)
    assert_bits_equal(got, want, "add")
    got, want = _mm(dev, oc, 96, 896, 40, seed=4, acc=True)
    assert_bits_equal(got, want, "acc")


def test_mm_q8_0_specials(dev, oc):
    N, K, T = 48, 1024, 32
    x = np.stack([special_row(K, t) if t % 3 == 0 else S.normal(50 + t, K, 1e-3 if t % 3 == 1 else 1.0)
                  for t in range(T)])
    blocks = weights(0, N, K, 9).copy()
    v = blocks.reshape(N, -1, 34)
    rng = np.random.default_rng(3)
    specials = np.array([0x0001, 0x03FF, 0x8005, 0x7C00, 0xFC00, 0x7E01, 0x0000], np.uint16).view(np.uint8).reshape(-1, 2)
    for r in range(0, N, 2):
        v[r, rng.integers(0, v.shape[1]), 0:2] = specials[r % len(specials)]
    got, want = _mm(dev, oc, N, K, T, x=x, wblocks=blocks)
    assert_bits_equal(got, want, "specials")


def test_mm_q8_0_baseline_prefill_shape(dev, oc):
    """BASELINE configs[3] (512 tokens x W[4096 x 4096] Q8_0): every output of a sample of tokens,
    and every token of a sample of rows."""
    T, N, K = 512, 4096, 4096
    blocks = S.quantize_q8_0(S.normal(S.seed_of("cfg4", "w_q"), N * K, 0.02).reshape(N, K))
    x = S.normal(S.seed_of("cfg4", "x"), T * K).reshape(T, K)
    w = dev.weight(0, blocks, N, K)
    yb = dev.alloc(4 * T * N)
    dev.mul_mat(w, dev.upload(x), T, K, yb, N)
    got = yb.read(np.float32, (T, N))
    toks = [0, 1, 31, 32, 63, 64, 255, 510, 511]
    assert_bits_equal(got[toks], oc.mul_mat(0, blocks, K, x[toks], threads=8), "token sample")
    rows = np.r_[0:40, 2040:2056, 4060:4096]
    assert_bits_equal(got[:, rows], oc.mul_mat(0, blocks[rows], K, x, threads=8), "row sample")


def test_mm_q8_0_baseline_prefill_ffn_shape(dev, oc):
    """BASELINE configs[3] (512 tokens x W[14336 x 4096] Q8_0, the FFN up shape): every output of a
    sample of tokens, and every token of a sample of rows (first, middle and last row blocks)."""
    T, N, K = 512, 14336, 4096
    blocks = S.quantize_q8_0(S.normal(S.seed_of("cfg4", "w_14336"), N * K, 0.02).reshape(N, K))
    x = S.normal(S.seed_of("cfg4", "x"), T * K).reshape(T, K)
    w = dev.weight(0, blocks, N, K)
    yb = dev.alloc(4 * T * N)
    dev.mul_mat(w, dev.upload(x), T, K, yb, N)
    got = yb.read(np.float32, (T, N))
    toks = [0, 1, 31, 32, 95, 96, 257, 510, 511]
    assert_bits_equal(got[toks], oc.mul_mat(0, blocks, K, x[toks], threads=8), "token sample")
    rows = np.r_[0:40, 7160:7176, 14300:14336]
    assert_bits_equal(got[:, rows], oc.mul_mat(0, blocks[rows], K, x, threads=8), "row sample")
    w.free()
    yb.free()


# ---- Q4_K (QACT A256, i8 matrix core per sub-block, exact f32 matrix-core msum) ----

@pytest.mark.parametrize("T,N,K", [(16, 64, 256), (17, 100, 4096), (64, 256, 14336), (100, 33, 4096),
                                   (16, 1, 512), (130, 200, 1024), (33, 47, 3840), (40, 96, 32768)])
def test_mm_q4_k_shapes(dev, oc, T, N, K):
    print(f"\nmm Q4_K T {T} {N}x{K}", flush=True)
    got, want = _mm(dev, oc, N, K, T, seed=T + N + 1, fmt=1)
    assert_bits_equal(got, want, f"Q4_K T {T} {N}x{K}")


def test_mm_q4_k_add_acc(dev, oc):
    got, want = _mm(dev, oc, 96, 2048, 40, seed=13, add=True, fmt=1)
    assert_bits_equal(got, want, "add")
    got, want = _mm(dev, oc, 96, 2048, 40, seed=14, acc=True, fmt=1)
    assert_bits_equal(got, want, "acc")


@pytest.mark.parametrize("tiny_rows", [False, True], ids=["specials", "tiny-scales"])
def test_mm_q4_k_specials(dev, oc, tiny_rows):
    """Special activations (NaN, Inf, subnormal, zero rows) and special weight scales; with tiny_rows,
    token rows whose A256 scale is below 2^-60 (the spec-operation path of their waves and trees)."""
    N, K, T = 48, 1024, 40
    rows = []
    for t in range(T):
        if t % 4 == 0:
            rows.append(special_row(K, t))
        elif tiny_rows and t % 4 == 1:
            rows.append(S.normal(60 + t, K, 1e-25))
        elif t % 4 == 2:
            rows.append(S.normal(60 + t, K, 3e-18))
        else:
            rows.append(S.normal(60 + t, K))
    x = np.stack(rows)
    blocks = weights(1, N, K, 19).copy()
    v = blocks.reshape(N, -1, 144)
    rng = np.random.default_rng(5)
    specials = np.array([0x0001, 0x03FF, 0x8005, 0x7C00, 0xFC00, 0x7E01, 0x0000], np.uint16).view(np.uint8).reshape(-1, 2)
    for r in range(0, N, 3):
        b = rng.integers(0, v.shape[1])
        v[r, b, 0:2] = specials[r % len(specials)]
        v[r, b, 2:4] = specials[(r + 3) % len(specials)]
    got, want = _mm(dev, oc, N, K, T, x=x, wblocks=blocks, fmt=1)
    assert_bits_equal(got, want, "Q4_K specials")


def test_mm_q4_k_llama_prefill_shape(dev, oc):
    """A Llama-3-8B ubatch: 512 tokens x W[4096 x 14336] Q4_K (the FFN down projection): every output
    of a sample of tokens, and every token of a sample of rows."""
    T, N, K = 512, 4096, 14336
    blocks = S.quant_rows(1, 91, N, K)
    x = S.normal(92, T * K).reshape(T, K)
    w = dev.weight(1, blocks, N, K)
    yb = dev.alloc(4 * T * N)
    dev.mul_mat(w, dev.upload(x), T, K, yb, N)
    got = yb.read(np.float32, (T, N))
    toks = [0, 1, 31, 32, 63, 64, 255, 510, 511]
    assert_bits_equal(got[toks], oc.mul_mat(1, blocks, K, x[toks], threads=8), "token sample")
    rows = np.r_[0:40, 2040:2056, 4060:4096]
    assert_bits_equal(got[:, rows], oc.mul_mat(1, blocks[rows], K, x, threads=8), "row sample")
    w.free()


@pytest.mark.parametrize("T,N,K", [(16, 64, 256), (40, 512, 4096), (100, 130, 1024)])
def test_mm_q4_k_glu(dev, oc, T, N, K):
    """The GLU epilogue of the Q4_K matrix-core path: rows 2j, 2j + 1 are gate / up of output j, y[j] =
    SWIGLU(gate, up), against the oracle's MUL_MAT of the gate and up rows then SWIGLU."""
    print(f"\nmm Q4_K GLU T {T} {N}x{K}", flush=True)
    blocks = weights(1, N, K, T + N + 7)
    x = S.normal(T + 8, T * K).reshape(T, K)
    x[T // 2] = special_row(K, 3)
    w = dev.weight(1, blocks, N, K)
    yb = dev.alloc(4 * T * (N // 2))
    dev.mul_mat(w, dev.upload(x), T, K, yb, N // 2, flags=tsr_hip.MM_GLU)
    got = yb.read(np.float32, (T, N // 2))
    g = oc.mul_mat(1, blocks[0::2], K, x, threads=8)
    u = oc.mul_mat(1, blocks[1::2], K, x, threads=8)
    assert_bits_equal(got, oc.swiglu(g, u), f"GLU T {T} {N}x{K}")
    w.free()


def test_mm_q4_k_glu_llama_gate_up(dev, oc):
    """The Llama-3-8B gate|up with the GLU epilogue (W[28672 x 4096] Q4_K, 66 MB: the XCD-grouped tile
    order), 40 tokens: every output against the oracle's gate and up MUL_MATs then SWIGLU."""
    T, N, K = 40, 28672, 4096
    print(f"\nmm Q4_K GLU T {T} {N}x{K}", flush=True)
    blocks = S.quant_rows(1, 93, N, K)
    x = S.normal(94, T * K).reshape(T, K)
    x[7] = special_row(K, 5)
    w = dev.weight(1, blocks, N, K)
    yb = dev.alloc(4 * T * (N // 2))
    dev.mul_mat(w, dev.upload(x), T, K, yb, N // 2, flags=tsr_hip.MM_GLU)
    got = yb.read(np.float32, (T, N // 2))
    g = oc.mul_mat(1, blocks[0::2], K, x, threads=8)
    u = oc.mul_mat(1, blocks[1::2], K, x, threads=8)
    assert_bits_equal(got, oc.swiglu(g, u), "GLU 8B gate|up")
    w.free()
    yb.free()
