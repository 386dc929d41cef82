"""GPU parity of QACT and MUL_MAT (Q8_0, Q4_K) through the C ABI against the CPU oracle.

Bar: bit-exact for the QA images, the integer block sums and the f32 outputs (the contract's
tolerance is 1e-5 relative; the kernels reproduce the reference's operation order exactly)."""
import numpy as np
import pytest

import tsr_hip
import tsr_synth as S
from helpers import assert_bits_equal, special_row, weights

pytestmark = pytest.mark.gpu


def test_device_is_gfx950(dev):
    info = dev.info()
    assert info["arch"].startswith("gfx950"), info
    assert info["n_cu"] >= 200


@pytest.mark.parametrize("fmt,N,K", [(0, 300, 896), (1, 70, 4096), (0, 5, 32), (1, 3, 256)])
def test_weight_round_trip(dev, fmt, N, K):
    blocks = weights(fmt, N, K, 1)
    w = dev.weight(fmt, blocks, N, K)
    assert (w.read() == blocks).all()


@pytest.mark.parametrize("kind,K,T", [(0, 896, 3), (1, 4096, 2), (0, 4096, 1), (1, 14336, 1), (0, 32, 5), (1, 256, 4)])
def test_qact_bytes(dev, oc, kind, K, T):
    x = np.stack([special_row(K, 7 + t) if t % 2 else S.normal(11 + t, K) for t in range(T)])
    xb = dev.upload(x)
    nq = tsr_hip.qa_bytes(kind, K)
    qa = dev.alloc(T * nq).fill(0xA5)
    dev.qact(kind, xb, K, T, K, qa)
    got = qa.read(np.uint8, (T, nq))
    want = oc.qact(kind, x)
    assert (got == want).all(), np.argwhere(got != want)[:5]


def test_qact_ftz_boundary_sweep(dev, oc):
    """A32 d = amax/127 swept across 2^-126: the kept window [2^-126 - 2^-150, 2^-126) and the flushed
    values below it must match the spec rule (native division with gradual underflow, then FTZ)."""
    center = np.float32(127.0 * 2.0 ** -126).view(np.uint32)
    amax = (center.astype(np.int64) + np.arange(-2048, 2048)).astype(np.uint32).view(np.float32)
    x = np.zeros((amax.size, 32), np.float32)
    x[:, 0] = amax
    x[:, 1] = -amax * np.float32(0.5)
    x[:, 2] = amax * np.float32(0.25)
    T, K = x.shape                                     # one 32-block per token row
    nq = tsr_hip.qa_bytes(0, K)
    qa = dev.alloc(T * nq)
    dev.qact(0, dev.upload(x), K, T, K, qa)
    assert (qa.read(np.uint8, (T, nq)) == oc.qact(0, x)).all()


def _mm_case(dev, oc, fmt, N, K, T=1, seed=1, x=None, add=False, acc=False, wblocks=None):
    blocks = weights(fmt, N, K, seed) if wblocks is None else wblocks
    w = dev.weight(fmt, blocks, N, K)
    if x is None:
        x = S.normal(seed + 100, T * K).reshape(T, K)
    xb = dev.upload(x)
    y0 = S.normal(seed + 200, T * N).reshape(T, N)
    yb = dev.upload(y0)
    a = S.normal(seed + 300, T * N).reshape(T, N) if add else None
    ab = dev.upload(a) if add else None
    dev.mul_mat(w, xb, T, K, yb, N, ab, N if add else 0, tsr_hip.MM_ACC_DST if acc else 0)
    got = yb.read(np.float32, (T, N))
    want = oc.mul_mat(fmt, blocks, K, x, add=(a if add else (y0 if acc else None)), threads=8)
    return got, want


@pytest.mark.parametrize("fmt,N,K", [
    (0, 4864, 896),        # Qwen2.5-0.5B FFN up, Q8_0
    (1, 14336, 4096),      # Llama-3-8B FFN up, Q4_K
    (1, 4096, 14336),      # Llama-3-8B FFN down, Q4_K
])
def test_mul_mat_baseline_shapes(dev, oc, fmt, N, K):
    got, want = _mm_case(dev, oc, fmt, N, K)
    assert_bits_equal(got, want, f"fmt {fmt} {N}x{K}")


@pytest.mark.parametrize("fmt,N,K", [(0, 1, 32), (0, 17, 64), (0, 33, 4096), (0, 7, 14336), (0, 3, 32768),
                                     (1, 1, 256), (1, 19, 512), (1, 16, 2048), (1, 5, 32768), (1, 9, 3840)])
def test_mul_mat_edge_shapes(dev, oc, fmt, N, K):
    got, want = _mm_case(dev, oc, fmt, N, K, seed=N + K)
    assert_bits_equal(got, want, f"fmt {fmt} {N}x{K}")


@pytest.mark.parametrize("fmt", [0, 1])
def test_mul_mat_tokens_add_acc(dev, oc, fmt):
    K = 512 if fmt else 896
    got, want = _mm_case(dev, oc, fmt, 100, K, T=3, add=True, seed=5)
    assert_bits_equal(got, want, "add")
    got, want = _mm_case(dev, oc, fmt, 100, K, T=3, acc=True, seed=6)
    assert_bits_equal(got, want, "acc")
    got, want = _mm_case(dev, oc, fmt, 64, K, T=9, seed=7)
    assert_bits_equal(got, want, "T=9")


@pytest.mark.parametrize("fmt", [0, 1])
def test_mul_mat_special_activations(dev, oc, fmt):
    K = 1024
    x = np.stack([special_row(K, 1), S.normal(2, K, 1e-25), S.normal(3, K, 3e-18), np.zeros(K, np.float32)])
    got, want = _mm_case(dev, oc, fmt, 48, K, T=4, x=x, seed=8)
    assert_bits_equal(got, want, "special x")


@pytest.mark.parametrize("fmt", [0, 1])
def test_mul_mat_special_weight_scales(dev, oc, fmt):
    N, K = 40, 1024
    blocks = weights(fmt, N, K, 9).copy()
    bb = 34 if fmt == 0 else 144
    v = blocks.reshape(N, -1, bb)
    rng = np.random.default_rng(3)
    specials = np.array([0x0001, 0x03FF, 0x8005, 0x7C00, 0xFC00, 0x7E01, 0x0000], np.uint16).view(np.uint8).reshape(-1, 2)
    for r in range(0, N, 3):
        b = rng.integers(0, v.shape[1])
        v[r, b, 0:2] = specials[r % len(specials)]
        if fmt == 1:
            v[r, b, 2:4] = specials[(r + 3) % len(specials)]
    got, want = _mm_case(dev, oc, fmt, N, K, seed=10, wblocks=blocks)
    assert_bits_equal(got, want, "special scales")


@pytest.mark.parametrize("fmt,N,K", [(0, 4864, 896), (1, 512, 4096), (1, 256, 14336)])
def test_mul_mat_isums(dev, oc, fmt, N, K):
    blocks = weights(fmt, N, K, 11)
    w = dev.weight(fmt, blocks, N, K)
    x = S.normal(12, K)[None, :]
    per = K // 32 if fmt == 0 else 2 * (K // 256)
    isb = dev.alloc(N * per * 4)
    dev.mul_mat_isums(w, dev.upload(x), isb)
    got = isb.read(np.int32, (N, per))
    want = oc.isums(fmt, blocks, K, oc.qact(0 if fmt == 0 else 1, x))
    assert (got == want).all()


def test_mul_mat_errors(dev):
    w = dev.weight(0, weights(0, 4, 64, 1), 4, 64)
    x, y, a = dev.alloc(64 * 4), dev.alloc(16), dev.alloc(16)
    with pytest.raises(tsr_hip.TsrHipError) as e:
        dev.mul_mat(w, x, 1, 64, y, 4, a, 4, tsr_hip.MM_ACC_DST)
    assert e.value.code == -1
    with pytest.raises(tsr_hip.TsrHipError) as e:
        dev.weight(1, np.zeros(144, np.uint8), 1, 100)
    assert e.value.code == -2
    with pytest.raises(tsr_hip.TsrHipError) as e:
        dev.weight(7, np.zeros(144, np.uint8), 1, 256)
    assert e.value.code == -7


@pytest.mark.parametrize("fmt", [0, 1])
def test_mul_mat_vocab_head(dev, oc, fmt):
    """The output head of a Llama-3-8B-shaped model: 128256 rows x 4096 (the most rows per block)."""
    N, K = 128256, 4096
    got, want = _mm_case(dev, oc, fmt, N, K, seed=9, wblocks=S.quant_rows(fmt, 77, N, K))
    assert_bits_equal(got, want, f"fmt {fmt} {N}x{K}")


@pytest.mark.parametrize("fmt,N,K,T,mode,extra", [
    (1, 4096, 4096, 1, 2, "add"),          # Q4_K matvec, SOFTCAP after the residual addend
    (0, 4864, 896, 1, 1, "acc"),           # Q8_0 matvec, SCALE after ACC
    (1, 512, 4096, 3, 2, None),            # Q4_K, several tokens (the matvec per token)
    (0, 300, 896, 40, 2, "add"),           # Q8_0 T >= 16: the matrix-core prefill path
    (0, 130, 1024, 33, 1, None),           # prefill, SCALE, ragged tiles
    (0, 48, 1024, 4, 2, "special"),        # special activations: NaN / Inf dots through TANH
])
def test_mul_mat_scale_softcap(dev, oc, fmt, N, K, T, mode, extra):
    """tsr_hip_mul_mat_epi (the MVM record's local SCALE / SOFTCAP after ACC, sw/sim/tsr_sim.c:1648-1667)
    against the oracle's MUL_MAT with the same epilogue, bit for bit."""
    print(f"\nmul_mat_epi fmt {fmt} {N}x{K} T {T} mode {mode} {extra}", flush=True)
    seed = N + K + T
    blocks = weights(fmt, N, K, seed)
    w = dev.weight(fmt, blocks, N, K)
    if extra == "special":
        x = np.stack([special_row(K, 1), S.normal(2, K, 1e-25), S.normal(3, K, 30.0), np.zeros(K, np.float32)])
    else:
        x = S.normal(seed + 100, T * K).reshape(T, K)
    y0 = S.normal(seed + 200, T * N).reshape(T, N)
    a = S.normal(seed + 300, T * N).reshape(T, N) if extra == "add" else None
    yb = dev.upload(y0)
    fs, sc = (np.float32(1.0 / 30.0), np.float32(30.0)) if mode == 2 else (np.float32(0.0), np.float32(0.125))
    flags = (tsr_hip.MM_SOFTCAP if mode == 2 else tsr_hip.MM_SCALE) | (tsr_hip.MM_ACC_DST if extra == "acc" else 0)
    dev.mul_mat_epi(w, dev.upload(x), T, K, yb, N, flags, fs, sc, add=None if a is None else dev.upload(a),
                    add_stride=N if a is not None else 0)
    got = yb.read(np.float32, (T, N))
    want = oc.mul_mat(fmt, blocks, K, x, add=(a if a is not None else (y0 if extra == "acc" else None)), threads=8,
                      epi=(mode, fs, sc))
    assert_bits_equal(got, want, f"epilogue {mode} fmt {fmt} {N}x{K} T {T}")
    w.free()


def test_mul_mat_scale_softcap_refusals(dev):
    w = dev.weight(0, weights(0, 64, 256, 1), 64, 256)
    b = dev.alloc(4 * 4096)
    for call, code in [
        (lambda: dev.mul_mat(w, b, 1, 256, b.ptr + 4096, 64, flags=tsr_hip.MM_SCALE), -1),     # no scales here
        (lambda: dev.mul_mat_epi(w, b, 1, 256, b.ptr + 4096, 64, tsr_hip.MM_SCALE | tsr_hip.MM_SOFTCAP, 1.0, 1.0), -1),
        (lambda: dev.mul_mat_epi(w, b, 1, 256, b.ptr + 4096, 32, tsr_hip.MM_GLU | tsr_hip.MM_SCALE, 1.0, 1.0), -1),
    ]:
        with pytest.raises(tsr_hip.TsrHipError) as e:
            call()
        assert e.value.code == code
    w.free()
