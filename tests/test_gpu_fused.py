"""GPU fused decode-layer entry points through the C ABI, bit for bit against the oracle's separate
ops on the same seeded inputs: MUL_MAT of RMS_NORM(x) * w (tsr_hip_mul_mat_norm), the gate / up
MUL_MAT with its SWIGLU epilogue (TSR_HIP_MM_GLU), ROPE + SET_ROWS_KV (tsr_hip_rope_kv) and the
attention half of a decode layer in one launch (tsr_hip_attn_qkv_plan_rope_tab)."""
import numpy as np
import pytest

import tsr_hip as H
import tsr_synth as S
from helpers import assert_bits_equal, special_row
from test_gpu_glue import SPECIALS, theta_scale

pytestmark = pytest.mark.gpu


def _x_rows(K, T, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, K)) * rng.uniform(0.05, 20, (T, 1))).astype(np.float32)
    x[0] = special_row(K, seed)
    return x


@pytest.mark.parametrize("fmt,N,K,T", [
    (H.FMT_Q4_K, 6144, 4096, 1),        # Llama-3-8B Q|K|V
    (H.FMT_Q4_K, 28672, 4096, 1),       # Llama-3-8B gate|up
    (H.FMT_Q4_K, 300, 2048, 3),         # waves without super-blocks
    (H.FMT_Q4_K, 257, 8192, 2),         # two super-blocks per wave
    (H.FMT_Q8_0, 4864, 896, 1),         # Qwen2.5-0.5B FFN-up
    (H.FMT_Q8_0, 1000, 8192, 2),        # sixteen blocks per wave
    (H.FMT_Q8_0, 70, 4096, 5),
], ids=lambda v: str(v))
def test_mul_mat_norm(dev, oc, fmt, N, K, T):
    print(f"\nmul_mat_norm fmt {fmt} {N}x{K} T {T}", flush=True)
    blocks = S.quant_rows(fmt, S.seed_of("fused-norm", f"{fmt}-{N}-{K}"), N, K)
    x = _x_rows(K, T, N + K + T)
    rng = np.random.default_rng(K)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    nw[:SPECIALS.size] = SPECIALS
    add = rng.standard_normal((T, N)).astype(np.float32)
    wt = dev.weight(fmt, blocks, N, K)
    xb, nb, yb, ab = dev.upload(x), dev.upload(nw), dev.alloc(4 * T * N), dev.upload(add)
    for eps, w in ((1e-5, nw), (1e-6, None)):
        xn = oc.rms_norm(x, eps, None if w is None else w[None])
        dev.mul_mat_norm(wt, xb, T, K, eps, None if w is None else nb, yb, N)
        assert_bits_equal(yb.read(np.float32, (T, N)), oc.mul_mat(fmt, blocks, K, xn, threads=8),
                          f"norm eps={eps} w={w is not None}")
        dev.mul_mat_norm(wt, xb, T, K, eps, None if w is None else nb, yb, N, add=ab, add_stride=N)
        assert_bits_equal(yb.read(np.float32, (T, N)), oc.mul_mat(fmt, blocks, K, xn, add=add, threads=8),
                          f"norm + addend eps={eps}")
    wt.free()


def test_mul_mat_norm_specials(dev, oc):
    """Rows whose squares or scale hit the rule's special cases: zeros, subnormals, an overflowing sum,
    NaN and Inf, tiny rows whose scaled values quantize with the spec operations."""
    K, N = 4096, 512
    blocks = S.quant_rows(H.FMT_Q4_K, S.seed_of("fused-norm", "specials"), N, K)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, K)).astype(np.float32)
    x[0] = 0.0
    x[1] = np.float32(3e-39)
    x[2] *= np.float32(1e19)
    x[3, 17] = np.nan
    x[4, 99] = np.inf
    x[5] *= np.float32(1e-30)
    x[6, :SPECIALS.size] = SPECIALS
    nw = rng.standard_normal(K).astype(np.float32)
    nw[5] = np.float32(1e-40)
    wt = dev.weight(H.FMT_Q4_K, blocks, N, K)
    yb = dev.alloc(4 * 7 * N)
    dev.mul_mat_norm(wt, dev.upload(x), 7, K, 1e-5, dev.upload(nw), yb, N)
    want = oc.mul_mat(H.FMT_Q4_K, blocks, K, oc.rms_norm(x, 1e-5, nw[None]), threads=8)
    assert_bits_equal(yb.read(np.float32, (7, N)), want, "norm specials")
    wt.free()


@pytest.mark.parametrize("fmt,K", [(H.FMT_Q4_K, 4096), (H.FMT_Q8_0, 896), (H.FMT_Q8_0, 8192)], ids=lambda v: str(v))
def test_norm_subnormal_squares(dev, oc, fmt, K):
    """RMS_NORM with eps = 0 over rows whose squares are partly subnormal: values ~1e-18 square to normal
    numbers, values ~3e-20 to subnormals (~1e-39) that the rule flushes to +0 before the sum. Kept, they
    would move the sum's low bits and with it the scale. The standalone RMS_NORM and the fused MUL_MAT
    (the norm in the matvec's leaders) against the oracle."""
    N, T = 256, 4
    print(f"\nnorm subnormal squares fmt {fmt} K {K}", flush=True)
    rng = np.random.default_rng(K + fmt)
    x = (rng.standard_normal((T, K)) * 1e-18).astype(np.float32)
    tiny = rng.random((T, K)) < 0.5
    x[tiny] = (rng.standard_normal(int(tiny.sum())) * 3e-20).astype(np.float32)
    x[3] = (rng.standard_normal(K) * 3e-20).astype(np.float32)         # every square subnormal: scale of +0
    sq = (x.astype(np.float64) ** 2)
    assert ((sq > 0) & (sq < 2.0 ** -126)).sum() > K                  # the case is there
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    want_n = oc.rms_norm(x, 0.0, nw[None])
    xb, nb = dev.upload(x), dev.upload(nw)
    yb = dev.alloc(x.nbytes)
    dev.rms_norm(xb, K, T, K, 0.0, yb, K, w=nb, w_stride=K)
    assert_bits_equal(yb.read(np.float32, (T, K)), want_n, "rms_norm eps 0")
    blocks = S.quant_rows(fmt, S.seed_of("fused-norm", f"sub-{fmt}-{K}"), N, K)
    wt = dev.weight(fmt, blocks, N, K)
    ym = dev.alloc(4 * T * N)
    dev.mul_mat_norm(wt, xb, T, K, 0.0, nb, ym, N)
    assert_bits_equal(ym.read(np.float32, (T, N)), oc.mul_mat(fmt, blocks, K, want_n, threads=8), "mul_mat_norm eps 0")
    wt.free()


@pytest.mark.parametrize("fmt,F,K,T,norm", [
    (H.FMT_Q4_K, 14336, 4096, 1, True),   # Llama-3-8B gate|up with the ffn norm
    (H.FMT_Q4_K, 14336, 4096, 1, False),
    (H.FMT_Q4_K, 300, 2048, 2, True),
    (H.FMT_Q4_K, 64, 24576, 1, False),    # later rounds of x loads
    (H.FMT_Q8_0, 4864, 896, 1, True),     # Qwen2.5-0.5B gate|up
    (H.FMT_Q8_0, 100, 8192, 3, True),
    (H.FMT_Q8_0, 77, 14336, 2, False),
], ids=lambda v: str(v))
def test_mul_mat_glu(dev, oc, fmt, F, K, T, norm):
    """TSR_HIP_MM_GLU over interleaved gate / up rows: y = SWIGLU(gate . x', up . x') with x' = x or
    RMS_NORM(x) * w, against the oracle's MUL_MATs of the two weights and its SWIGLU."""
    print(f"\nmul_mat glu fmt {fmt} F {F} K {K} T {T} norm {norm}", flush=True)
    gate = S.quant_rows(fmt, S.seed_of("fused-glu", f"g-{fmt}-{F}-{K}"), F, K)
    up = S.quant_rows(fmt, S.seed_of("fused-glu", f"u-{fmt}-{F}-{K}"), F, K)
    inter = np.stack([gate, up], axis=1).reshape(2 * F, -1)
    x = _x_rows(K, T, F + K)
    nw = (1.0 + 0.1 * np.random.default_rng(F).standard_normal(K)).astype(np.float32)
    xn = oc.rms_norm(x, 1e-5, nw[None]) if norm else x
    g = oc.mul_mat(fmt, gate, K, xn, threads=8)
    u = oc.mul_mat(fmt, up, K, xn, threads=8)
    want = oc.swiglu(g, u)
    wt = dev.weight(fmt, inter, 2 * F, K)
    xb, yb = dev.upload(x), dev.alloc(4 * T * F)
    if norm:
        dev.mul_mat_norm(wt, xb, T, K, 1e-5, dev.upload(nw), yb, F, flags=H.MM_GLU)
    else:
        dev.mul_mat(wt, xb, T, K, yb, F, flags=H.MM_GLU)
    assert_bits_equal(yb.read(np.float32, (T, F)), want, "glu")
    wt.free()


def test_fused_shape_refusals(dev):
    blocks = S.quant_rows(H.FMT_Q4_K, 1, 16, 16384)
    wt = dev.weight(H.FMT_Q4_K, blocks, 16, 16384)
    b = dev.alloc(4 * 16384 * 16)
    with pytest.raises(H.TsrHipError) as e:                              # norm over K > 8192
        dev.mul_mat_norm(wt, b, 1, 16384, 1e-5, None, b, 16)
    assert e.value.code == -2
    w8 = dev.weight(H.FMT_Q8_0, S.quant_rows(H.FMT_Q8_0, 2, 32, 256), 32, 256)
    with pytest.raises(H.TsrHipError):                                   # the matrix-core prefill shape
        dev.mul_mat_norm(w8, b, 16, 256, 1e-5, None, b, 32)
    with pytest.raises(H.TsrHipError):                                   # GLU with an addend
        dev.mul_mat(w8, b, 1, 256, b, 16, add=b, flags=H.MM_GLU)
    w7 = dev.weight(H.FMT_Q8_0, S.quant_rows(H.FMT_Q8_0, 3, 31, 256), 31, 256)
    with pytest.raises(H.TsrHipError) as e:                              # GLU over an odd row count
        dev.mul_mat(w7, b, 1, 256, b, 15, flags=H.MM_GLU)
    assert e.value.code == -2
    for w in (wt, w8, w7):
        w.free()


@pytest.mark.parametrize("mode,hd,nh,nkv,T", [
    (H.ROPE_NORMAL, 128, 32, 8, 1),     # Llama-3-8B
    (H.ROPE_NEOX, 128, 32, 8, 1),
    (H.ROPE_NEOX, 64, 14, 2, 3),        # Qwen2.5-0.5B
    (H.ROPE_NORMAL, 256, 8, 1, 2),
    (H.ROPE_IMROPE, 128, 16, 4, 2),
], ids=lambda v: str(v))
def test_rope_kv(dev, oc, mode, hd, nh, nkv, T):
    rng = np.random.default_rng(hd * nh + nkv + T + mode)
    E, nq = nkv * hd, nh * hd
    w3 = nq + 2 * E
    kv_size = 300
    x = rng.standard_normal((T, w3)).astype(np.float32)
    x[0, nq:nq + SPECIALS.size] = SPECIALS                              # specials in k
    x[-1, nq + E + 5:nq + E + 5 + SPECIALS.size] = SPECIALS             # and in v
    pos = rng.integers(0, 70000, T).astype(np.int32)
    cells = rng.choice(kv_size, T, replace=False).astype(np.int64)
    base = 500000.0 if mode == H.ROPE_NORMAL else 1000000.0
    ts = theta_scale(base, hd)
    kc, vc = dev.kv(E, kv_size), dev.kv(E, kv_size)
    k0 = rng.integers(0, 256, (kv_size, E // 32 * 34), dtype=np.uint8)
    v0 = rng.integers(0, 256, (kv_size, E // 32 * 34), dtype=np.uint8)
    kc.set_bytes(0, k0)
    vc.set_bytes(1, v0)
    xb, bad = dev.upload(x), dev.upload(np.zeros(1, np.int32))
    dev.rope_kv(xb, T, w3, hd, nh, nkv, hd, mode, dev.upload(pos), base, kc, vc, dev.upload(cells), bad)
    neox = mode != H.ROPE_NORMAL
    q = oc.rope(np.ascontiguousarray(x[:, :nq]), pos, hd, hd, neox, ts)
    k = oc.rope(np.ascontiguousarray(x[:, nq:nq + E]), pos, hd, hd, neox, ts)
    got = xb.read(np.float32, (T, w3))
    assert_bits_equal(got[:, :nq], q, "rotated q")
    assert_bits_equal(got[:, nq:nq + E], k, "rotated k")
    assert_bits_equal(got[:, nq + E:], x[:, nq + E:], "v untouched")
    kw, vw = k0.copy(), v0.copy()
    oc.kv_set_rows(kw, k, cells)
    oc.kv_set_rows(vw, np.ascontiguousarray(x[:, nq + E:]), cells)
    assert (kc.get_bytes(0).reshape(kv_size, -1) == kw).all()
    assert (vc.get_bytes(1).reshape(kv_size, -1) == vw).all()
    assert bad.read(np.int32, (1,))[0] == 0
    kc.free()
    vc.free()


def test_rope_kv_bad_cell(dev, oc):
    """A cell outside the caches stores nothing and raises the flag; q and k are still rotated."""
    hd, nh, nkv = 64, 4, 2
    E, nq = nkv * hd, nh * hd
    x = np.random.default_rng(3).standard_normal((1, nq + 2 * E)).astype(np.float32)
    kc, vc = dev.kv(E, 32), dev.kv(E, 32)
    k0 = np.zeros((32, E // 32 * 34), np.uint8)
    kc.set_bytes(0, k0)
    vc.set_bytes(1, k0)
    xb, bad = dev.upload(x), dev.upload(np.zeros(1, np.int32))
    pos = np.array([9], np.int32)
    dev.rope_kv(xb, 1, nq + 2 * E, hd, nh, nkv, hd, H.ROPE_NEOX, dev.upload(pos), 10000.0, kc, vc,
                dev.upload(np.array([32], np.int64)), bad)
    assert bad.read(np.int32, (1,))[0] == 1
    assert (kc.get_bytes(0) == 0).all() and (vc.get_bytes(1) == 0).all()
    q = oc.rope(np.ascontiguousarray(x[:, :nq]), pos, hd, hd, True, theta_scale(10000.0, hd))
    assert_bits_equal(xb.read(np.float32, (1, nq + 2 * E))[:, :nq], q, "q rotated despite the bad cell")
    kc.free()
    vc.free()


@pytest.mark.parametrize("n_kv,pos,cell,n_head,n_head_kv,D,mode,n_dims,general", [
    (4232, 4200, 4200, 32, 8, 128, H.ROPE_NORMAL, 128, False),    # Llama-3-8B decode (three chunks)
    (4232, 4231, 4231, 32, 8, 128, H.ROPE_NEOX, 128, False),
    (4232, 4215, 4215, 32, 8, 128, H.ROPE_NORMAL, 128, False),    # the new cell's group in channel 3
    (2100, 2090, 2068, 16, 8, 128, H.ROPE_NEOX, 64, False),       # G = 2, half the dims rotated, channel 1
    (1500, 1400, 1400, 12, 4, 64, H.ROPE_NORMAL, 32, True),       # G = 3, a GENERAL mask
    (4232, 4100, 4100, 32, 8, 128, H.ROPE_NEOX, 128, True),       # GENERAL mask at the decode shape
    (300, 257, 257, 14, 2, 64, H.ROPE_NEOX, 64, False),           # Qwen2.5-0.5B heads; a second chunk of one cell
    (700, 513, 100, 8, 2, 128, H.ROPE_IMROPE, 128, False),        # the new row lands in a cell other than its position
    (96, 0, 0, 4, 4, 64, H.ROPE_NORMAL, 64, False),               # position 0: the first cell of an empty cache
    (640, 600, 600, 64, 8, 64, H.ROPE_NORMAL, 64, False),         # G = 8: the three-launch form
    (4232, 5000, 100, 32, 8, 128, H.ROPE_NORMAL, 128, "swa"),     # wrapped sliding window over a full ring:
    (1500, 3000, 700, 12, 4, 64, H.ROPE_NEOX, 64, "swa"),         #   runs [0, cell] and [lo, n_kv), two FAST runs
    (8192, 8191, 8191, 32, 8, 128, H.ROPE_NORMAL, 128, False),    # 4 chunks: the reducers' two rounds
    (13000, 12999, 12999, 32, 8, 128, H.ROPE_NEOX, 128, False),   # 7 chunks: three rounds
    (8208, 8200, 8200, 32, 8, 128, H.ROPE_NORMAL, 128, True),     # GENERAL mask over 5 chunks
], ids=lambda v: str(v))
def test_flash_attn_plan_rope(dev, oc, n_kv, pos, cell, n_head, n_head_kv, D, mode, n_dims, general):
    """tsr_hip_flash_attn_plan_rope against the oracle's ROPE of q and k, SET_ROWS_KV of k and v and
    FLASH_ATTN_EXT (one decode token seeing cells [0, max(pos, cell)] of a mask n_kv wide; with
    `general`, some of those cells carry finite biases and some are masked out; with "swa", a full
    ring cache whose sliding window wraps: cells [0, cell] and [cell + 1000 or n_kv - 300, n_kv), the
    new cell in the first run)."""
    import math
    print(f"\nflash_attn_plan_rope n_kv {n_kv} pos {pos} cell {cell} heads {n_head}/{n_head_kv} D {D} mode {mode} "
          f"n_dims {n_dims} general {general}", flush=True)
    rng = np.random.default_rng(n_kv + pos + D)
    E, nq = n_head_kv * D, n_head * D
    swa = general == "swa"
    general = general is True
    kv_size = 16 * -(-n_kv // 16) if general else n_kv   # a GENERAL mask covers whole groups of the cache
    k0 = np.zeros((kv_size, E // 32 * 34), np.uint8)
    v0 = np.zeros_like(k0)
    hist = n_kv if swa else max(pos, cell)
    oc.kv_set_rows(k0, S.normal(11 + D, hist * E).reshape(hist, E), np.arange(hist))
    oc.kv_set_rows(v0, S.normal(12 + D, hist * E).reshape(hist, E), np.arange(hist))
    row = rng.standard_normal((1, nq + 2 * E)).astype(np.float32)
    row[0, :SPECIALS.size] = SPECIALS
    base = 500000.0
    ts = theta_scale(base, n_dims)
    neox = mode != H.ROPE_NORMAL
    q = oc.rope(np.ascontiguousarray(row[:, :nq]), np.array([pos], np.int32), D, n_dims, neox, ts)
    k = oc.rope(np.ascontiguousarray(row[:, nq:nq + E]), np.array([pos], np.int32), D, n_dims, neox, ts)
    kw, vw = k0.copy(), v0.copy()
    oc.kv_set_rows(kw, k, np.array([cell], np.int64))
    oc.kv_set_rows(vw, np.ascontiguousarray(row[:, nq + E:]), np.array([cell], np.int64))
    scale = np.float32(1.0 / math.sqrt(D))
    mf = None
    if general:
        mask = np.full((1, n_kv), -np.inf, np.float16)
        mask[0, :hist + 1] = 0
        mask[0, rng.integers(0, hist + 1, hist // 7)] = -1.75
        mask[0, rng.integers(0, hist + 1, hist // 11)] = -np.inf
        mask[0, cell] = 0.5
        msum = oc.msum(mask)
        assert msum[3], "the mask must plan as GENERAL"
        mf = oc.mask_f32(mask, scale)
    elif swa:
        msum = np.zeros(12, np.uint32)
        msum[0], msum[1], msum[2] = 0x4D55534D, 1, n_kv
        msum[8], msum[9], msum[10], msum[11] = 0, cell + 1, min(cell + 1000, n_kv - 300), n_kv
    else:
        msum = np.zeros(12, np.uint32)
        msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, n_kv, hist + 1
    runs = np.array([[cell, cell + 1]], np.uint32)
    want = oc.flash_attn(q, kw, vw, D, n_head, n_head_kv, scale, msum, mf, new_runs=runs)
    kc, vc = dev.kv(E, kv_size), dev.kv(E, kv_size)
    kc.set_bytes(0, k0)
    vc.set_bytes(1, v0)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, kv_size)
    plan.set(msum, runs, mask_f32=general)
    rb, out, bad = dev.upload(row), dev.alloc(4 * nq), dev.upload(np.zeros(1, np.int32))
    pb, cb = dev.upload(np.array([pos], np.int32)), dev.upload(np.array([cell], np.int64))
    mb = None if mf is None else dev.upload(mf)
    dev.flash_attn_plan_rope(plan, rb, kc, vc, scale, n_dims, mode, pb, base, cb, out, nq, bad=bad, mask_f32=mb)
    assert_bits_equal(out.read(np.float32, (1, nq)), want, "fa + rope")
    assert (kc.get_bytes(0).reshape(kv_size, -1) == kw).all()
    assert (vc.get_bytes(1).reshape(kv_size, -1) == vw).all()
    assert bad.read(np.int32, (1,))[0] == 0
    assert_bits_equal(rb.read(np.float32, (1, nq + 2 * E)), row, "the Q|K|V row is read, not rotated")
    # the same with the angles from a table of the position, over fresh caches
    kc.set_bytes(0, k0)
    vc.set_bytes(1, v0)
    tab, out2 = dev.alloc(4 * n_dims), dev.alloc(4 * nq)
    dev.rope_table(pb, n_dims, base, tab)
    dev.flash_attn_plan_rope_tab(plan, rb, kc, vc, scale, n_dims, mode, tab, cb, out2, nq, bad=bad, mask_f32=mb)
    assert_bits_equal(out2.read(np.float32, (1, nq)), want, "fa + rope (table)")
    assert (kc.get_bytes(0).reshape(kv_size, -1) == kw).all()
    assert (vc.get_bytes(1).reshape(kv_size, -1) == vw).all()
    assert bad.read(np.int32, (1,))[0] == 0
    plan.free()
    kc.free()
    vc.free()


@pytest.mark.parametrize("fmt,K,n_kv,pos,cell,n_head,n_head_kv,D,mode,n_dims,general,one", [
    (H.FMT_Q4_K, 4096, 4232, 4200, 4200, 32, 8, 128, H.ROPE_NORMAL, 128, False, True),   # Llama-3-8B decode layer
    (H.FMT_Q4_K, 4096, 4232, 5000, 100, 32, 8, 128, H.ROPE_NEOX, 128, "swa", True),      # wrapped window, new cell 100
    (H.FMT_Q4_K, 2048, 2100, 2090, 2068, 16, 8, 128, H.ROPE_NEOX, 64, False, True),      # G = 2
    (H.FMT_Q4_K, 1024, 1500, 1400, 1400, 8, 8, 64, H.ROPE_NORMAL, 64, True, True),       # G = 1, GENERAL mask, D 64
    (H.FMT_Q4_K, 768, 640, 600, 600, 24, 8, 64, H.ROPE_NEOX, 64, False, True),           # 3 super-blocks, G = 3
    (H.FMT_Q4_K, 1024, 1500, 1400, 1400, 12, 4, 64, H.ROPE_NORMAL, 32, False, False),    # 4 KV heads: two launches
    (H.FMT_Q4_K, 8192, 300, 257, 257, 32, 8, 128, H.ROPE_NORMAL, 128, False, False),     # K > 4096: two launches
    (H.FMT_Q8_0, 1024, 300, 257, 257, 16, 8, 64, H.ROPE_NEOX, 64, False, False),         # Q8_0: two launches
    (H.FMT_Q4_K, 4096, 8208, 8200, 8200, 32, 8, 128, H.ROPE_NORMAL, 128, False, False),  # beyond residency: two
    (H.FMT_Q4_K, 4096, 5300, 5299, 5299, 32, 8, 128, H.ROPE_NEOX, 128, False, True),     # near the residency bound
], ids=lambda v: str(v))
def test_attn_qkv_plan_rope_tab(dev, oc, fmt, K, n_kv, pos, cell, n_head, n_head_kv, D, mode, n_dims, general, one):
    """tsr_hip_attn_qkv_plan_rope_tab against the oracle's RMS_NORM + MUL, Q|K|V MUL_MAT, ROPE,
    SET_ROWS_KV and FLASH_ATTN_EXT of one decode token (the Q|K|V row, the output and both caches),
    twice on one plan (the second launch tags with the next epoch), and against the two calls it
    replaces. `one`: whether the one-launch form is expected to run (the counter of such launches says
    which ran; its two-call fallback gives the same bits)."""
    import math
    print(f"\nattn_qkv_plan_rope_tab fmt {fmt} K {K} n_kv {n_kv} pos {pos} cell {cell} heads {n_head}/{n_head_kv} "
          f"D {D} mode {mode} n_dims {n_dims} general {general}", flush=True)
    rng = np.random.default_rng(n_kv + pos + D + K)
    E, nq = n_head_kv * D, n_head * D
    N = nq + 2 * E
    swa = general == "swa"
    general = general is True
    kv_size = 16 * -(-n_kv // 16) if general else n_kv
    k0 = np.zeros((kv_size, E // 32 * 34), np.uint8)
    v0 = np.zeros_like(k0)
    hist = n_kv if swa else max(pos, cell)
    oc.kv_set_rows(k0, S.normal(21 + D, hist * E).reshape(hist, E), np.arange(hist))
    oc.kv_set_rows(v0, S.normal(22 + D, hist * E).reshape(hist, E), np.arange(hist))
    blocks = S.quant_rows(fmt, S.seed_of("attn-qkv", f"{fmt}-{N}-{K}"), N, K)
    x = _x_rows(K, 1, N + K)
    x[0, :SPECIALS.size] = rng.standard_normal(SPECIALS.size).astype(np.float32)   # a finite row: q feeds FA
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    eps = 1e-5
    row = oc.mul_mat(fmt, blocks, K, oc.rms_norm(x, eps, nw[None]), threads=8)
    base = 500000.0
    ts = theta_scale(base, n_dims)
    neox = mode != H.ROPE_NORMAL
    q = oc.rope(np.ascontiguousarray(row[:, :nq]), np.array([pos], np.int32), D, n_dims, neox, ts)
    k = oc.rope(np.ascontiguousarray(row[:, nq:nq + E]), np.array([pos], np.int32), D, n_dims, neox, ts)
    kw, vw = k0.copy(), v0.copy()
    oc.kv_set_rows(kw, k, np.array([cell], np.int64))
    oc.kv_set_rows(vw, np.ascontiguousarray(row[:, nq + E:]), np.array([cell], np.int64))
    scale = np.float32(1.0 / math.sqrt(D))
    mf = None
    if general:
        mask = np.full((1, n_kv), -np.inf, np.float16)
        mask[0, :hist + 1] = 0
        mask[0, rng.integers(0, hist + 1, hist // 7)] = -1.75
        mask[0, cell] = 0.5
        msum = oc.msum(mask)
        mf = oc.mask_f32(mask, scale)
    elif swa:
        msum = np.zeros(12, np.uint32)
        msum[0], msum[1], msum[2] = 0x4D55534D, 1, n_kv
        msum[8], msum[9], msum[10], msum[11] = 0, cell + 1, min(cell + 1000, n_kv - 300), n_kv
    else:
        msum = np.zeros(12, np.uint32)
        msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, n_kv, hist + 1
    runs = np.array([[cell, cell + 1]], np.uint32)
    want = oc.flash_attn(q, kw, vw, D, n_head, n_head_kv, scale, msum, mf, new_runs=runs)
    wt = dev.weight(fmt, blocks, N, K)
    kc, vc = dev.kv(E, kv_size), dev.kv(E, kv_size)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, kv_size)
    plan.set(msum, runs, mask_f32=general)
    xb, nb = dev.upload(x), dev.upload(nw)
    qkv, out, bad = dev.alloc(4 * N), dev.alloc(4 * nq), dev.upload(np.zeros(1, np.int32))
    pb, cb = dev.upload(np.array([pos], np.int32)), dev.upload(np.array([cell], np.int64))
    mb = None if mf is None else dev.upload(mf)
    tab = dev.alloc(4 * n_dims)
    dev.rope_table(pb, n_dims, base, tab)
    for rep in range(3):
        kc.set_bytes(0, k0)
        vc.set_bytes(1, v0)
        qkv.write(np.full(N, np.nan, np.float32))
        out.write(np.full(nq, np.nan, np.float32))
        if rep < 2:
            n0 = dev.counters()["fa_dec_qkv_launches"]
            dev.attn_qkv_plan_rope_tab(plan, wt, xb, eps, nb, qkv, kc, vc, scale, n_dims, mode, tab, cb, out, nq,
                                       bad=bad, mask_f32=mb)
            ran_one = dev.counters()["fa_dec_qkv_launches"] - n0
            assert ran_one == (1 if one else 0), f"one-launch form ran {ran_one} times, expected {int(one)}"
        else:                                                     # the two calls it replaces
            dev.mul_mat_norm(wt, xb, 1, K, eps, nb, qkv, N)
            dev.flash_attn_plan_rope_tab(plan, qkv, kc, vc, scale, n_dims, mode, tab, cb, out, nq, bad=bad, mask_f32=mb)
        what = f"call {rep}"
        assert_bits_equal(qkv.read(np.float32, (1, N)), row, f"Q|K|V row, {what}")
        assert_bits_equal(out.read(np.float32, (1, nq)), want, f"attention, {what}")
        assert (kc.get_bytes(0).reshape(kv_size, -1) == kw).all(), what
        assert (vc.get_bytes(1).reshape(kv_size, -1) == vw).all(), what
        assert bad.read(np.int32, (1,))[0] == 0, what
    half = dev.weight(fmt, blocks[:N // 2], N // 2, K)
    with pytest.raises(H.TsrHipError):                            # a weight of another row count
        dev.attn_qkv_plan_rope_tab(plan, half, xb, eps, nb, qkv, kc, vc, scale, n_dims, mode, tab, cb, out, nq, bad=bad)
    half.free()
    plan.free()
    kc.free()
    vc.free()
    wt.free()


@pytest.mark.parametrize("alias", ["out=x", "out=norm"])
def test_attn_qkv_overlapping_buffers_run_two_launches(dev, oc, alias):
    """The one-launch form reads x and the norm weight in its row workgroups while its reducers write
    the attention output: when the output overlaps either, the entry point runs the two launches
    instead (the launch counter says so), and the results are those of the ops in order (the Q|K|V
    row from x before the output overwrites it)."""
    import math
    n_kv, pos, n_head, n_head_kv, D, K = 4232, 4200, 32, 8, 128, 4096
    print(f"\nattn_qkv overlapping buffers {alias}", flush=True)
    E, nq = n_head_kv * D, n_head * D
    N = nq + 2 * E
    fmt = H.FMT_Q4_K
    k0 = np.zeros((n_kv, E // 32 * 34), np.uint8)
    v0 = np.zeros_like(k0)
    oc.kv_set_rows(k0, S.normal(41, pos * E).reshape(pos, E), np.arange(pos))
    oc.kv_set_rows(v0, S.normal(42, pos * E).reshape(pos, E), np.arange(pos))
    blocks = S.quant_rows(fmt, S.seed_of("attn-qkv-alias", "w"), N, K)
    x = S.normal(S.seed_of("attn-qkv-alias", "x"), K).reshape(1, K)
    nw = (1.0 + 0.1 * S.normal(S.seed_of("attn-qkv-alias", "nw"), K)).astype(np.float32)
    eps = 1e-5
    row = oc.mul_mat(fmt, blocks, K, oc.rms_norm(x, eps, nw[None]), threads=8)
    ts = theta_scale(500000.0, D)
    q = oc.rope(np.ascontiguousarray(row[:, :nq]), np.array([pos], np.int32), D, D, False, ts)
    k = oc.rope(np.ascontiguousarray(row[:, nq:nq + E]), np.array([pos], np.int32), D, D, False, ts)
    kw, vw = k0.copy(), v0.copy()
    oc.kv_set_rows(kw, k, np.array([pos], np.int64))
    oc.kv_set_rows(vw, np.ascontiguousarray(row[:, nq + E:]), np.array([pos], np.int64))
    scale = np.float32(1.0 / math.sqrt(D))
    msum = np.zeros(12, np.uint32)
    msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, n_kv, pos + 1
    runs = np.array([[pos, pos + 1]], np.uint32)
    want = oc.flash_attn(q, kw, vw, D, n_head, n_head_kv, scale, msum, None, new_runs=runs)
    wt = dev.weight(fmt, blocks, N, K)
    kc, vc = dev.kv(E, n_kv), dev.kv(E, n_kv)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, n_kv)
    plan.set(msum, runs)
    xb, nb = dev.upload(x), dev.upload(nw)
    qkv, bad = dev.alloc(4 * N), dev.upload(np.zeros(1, np.int32))
    pb, cb = dev.upload(np.array([pos], np.int32)), dev.upload(np.array([pos], np.int64))
    tab = dev.alloc(4 * D)
    dev.rope_table(pb, D, 500000.0, tab)
    out = xb if alias == "out=x" else nb                          # nq == K floats: the whole buffer
    for rep in range(2):
        xb.write(x)
        nb.write(nw)
        kc.set_bytes(0, k0)
        vc.set_bytes(1, v0)
        n0 = dev.counters()["fa_dec_qkv_launches"]
        dev.attn_qkv_plan_rope_tab(plan, wt, xb, eps, nb, qkv, kc, vc, scale, D, H.ROPE_NORMAL, tab, cb, out, nq, bad=bad)
        assert dev.counters()["fa_dec_qkv_launches"] == n0, "the one-launch form ran over overlapping buffers"
        assert_bits_equal(qkv.read(np.float32, (1, N)), row, f"Q|K|V row, call {rep}")
        assert_bits_equal(out.read(np.float32, (1, nq)), want, f"attention, call {rep}")
        assert (kc.get_bytes(0).reshape(n_kv, -1) == kw).all()
        assert (vc.get_bytes(1).reshape(n_kv, -1) == vw).all()
        assert bad.read(np.int32, (1,))[0] == 0
    plan.free()
    kc.free()
    vc.free()
    wt.free()


def test_attn_qkv_plan_rope_tab_wait_expires(dev, oc):
    """The attention launch with its Q|K|V rows, its bounded waits (the row workgroups' flags, the chunk
    maxima, the reducers' polls) forced to expire from the host (a poll limit of 1): the launch still
    ends and raises *bad = 2; the next launch with the default limit is bit-exact again (the flags carry
    the launch's tag: nothing needs clearing)."""
    import math
    n_kv, pos, n_head, n_head_kv, D, K = 4232, 4100, 32, 8, 128, 4096
    E, nq = n_head_kv * D, n_head * D
    N = nq + 2 * E
    k0 = np.zeros((n_kv, E // 32 * 34), np.uint8)
    v0 = np.zeros_like(k0)
    oc.kv_set_rows(k0, S.normal(31, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    oc.kv_set_rows(v0, S.normal(32, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    blocks = S.quant_rows(H.FMT_Q4_K, S.seed_of("attn-qkv-expire", "w"), N, K)
    x = S.normal(33, K).reshape(1, K)
    nw = (1.0 + 0.1 * S.normal(34, K)).astype(np.float32)
    eps = 1e-5
    row = oc.mul_mat(H.FMT_Q4_K, blocks, K, oc.rms_norm(x, eps, nw[None]), threads=8)
    base = 500000.0
    ts = theta_scale(base, D)
    q = oc.rope(np.ascontiguousarray(row[:, :nq]), np.array([pos], np.int32), D, D, False, ts)
    k = oc.rope(np.ascontiguousarray(row[:, nq:nq + E]), np.array([pos], np.int32), D, D, False, ts)
    kw, vw = k0.copy(), v0.copy()
    oc.kv_set_rows(kw, k, np.array([pos], np.int64))
    oc.kv_set_rows(vw, np.ascontiguousarray(row[:, nq + E:]), np.array([pos], np.int64))
    msum = np.zeros(12, np.uint32)
    msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, n_kv, pos + 1
    runs = np.array([[pos, pos + 1]], np.uint32)
    scale = np.float32(1.0 / math.sqrt(D))
    want = oc.flash_attn(q, kw, vw, D, n_head, n_head_kv, scale, msum, new_runs=runs)
    wt = dev.weight(H.FMT_Q4_K, blocks, N, K)
    kc, vc = dev.kv(E, n_kv), dev.kv(E, n_kv)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, n_kv)
    plan.set(msum, runs)
    xb, nb, qkv = dev.upload(x), dev.upload(nw), dev.alloc(4 * N)
    pb, cb = dev.upload(np.array([pos], np.int32)), dev.upload(np.array([pos], np.int64))
    tab = dev.alloc(4 * D)
    dev.rope_table(pb, D, base, tab)
    expired = 0
    try:
        for limit in (1, 0, 1, 0):
            kc.set_bytes(0, k0)
            vc.set_bytes(1, v0)
            bad, out = dev.upload(np.zeros(1, np.int32)), dev.alloc(4 * nq)
            dev.set_fa_wait_limit(limit)
            dev.attn_qkv_plan_rope_tab(plan, wt, xb, eps, nb, qkv, kc, vc, scale, D, H.ROPE_NORMAL, tab, cb, out, nq,
                                       bad=bad)
            dev.sync()
            got_bad = int(bad.read(np.int32, (1,))[0])
            assert got_bad in (0, 2), got_bad
            if limit:
                expired |= got_bad
            else:
                assert got_bad == 0
                assert_bits_equal(qkv.read(np.float32, (1, N)), row, "Q|K|V row after an expired wait")
                assert_bits_equal(out.read(np.float32, (1, nq)), want, "after an expired wait")
                assert (kc.get_bytes(0).reshape(n_kv, -1) == kw).all()
        assert expired == 2, "a poll limit of 1 never expired"
    finally:
        dev.set_fa_wait_limit(0)
        plan.free()
        kc.free()
        vc.free()
        wt.free()


@pytest.mark.parametrize("pos,n_dims,m", [(0, 128, 1.0), (7, 64, 1.0), (4231, 128, 1.0), (131071, 128, 0.75),
                                          (-5, 8, 1.0), (1000, 2, 1.25)])
def test_rope_table(dev, oc, pos, n_dims, m):
    """tsr_hip_rope_table against the oracle's ROPE of a row of (1, 0) pairs (NORMAL): y_2i =
    FS(FM(1, c), FM(0, s)) = c and y_2i+1 = FA(FM(1, s), FM(0, c)) = s, c = FM(M, cos theta_i) and
    s = FM(M, sin theta_i), for every i < n_dims / 2."""
    base = 500000.0
    x = np.zeros((1, n_dims), np.float32)
    x[0, 0::2] = 1.0
    want = oc.rope(x, np.array([pos], np.int32), n_dims, n_dims, False, theta_scale(base, n_dims), m)
    tab = dev.alloc(4 * n_dims)
    dev.rope_table(dev.upload(np.array([pos], np.int32)), n_dims, base, tab, attn_factor=m)
    assert_bits_equal(tab.read(np.float32, (1, n_dims)), want, f"rope table pos {pos}")


def test_rope_table_refusals(dev):
    b = dev.alloc(4096)
    for n_dims in (0, 3, 130):
        with pytest.raises(H.TsrHipError) as e:
            dev.rope_table(b, n_dims, 10000.0, b)
        assert e.value.code == -2
    with pytest.raises(H.TsrHipError) as e:
        dev.rope_table(b, 64, 10000.0, b.ptr + 4)                 # the table 8-byte aligned
    assert e.value.code == -1
    with pytest.raises(H.TsrHipError) as e:
        dev.rope_table(b, 64, -1.0, b)
    assert e.value.code == -1


def test_flash_attn_plan_rope_bad_cell(dev, oc):
    """A cell outside the caches: the flag is raised, the caches are left alone, and the attention
    runs over the cached cells with the rotated query."""
    import math
    n_kv, pos, n_head, n_head_kv, D = 600, 520, 32, 8, 128
    E, nq = n_head_kv * D, n_head * D
    k0 = np.zeros((n_kv, E // 32 * 34), np.uint8)
    v0 = np.zeros_like(k0)
    oc.kv_set_rows(k0, S.normal(5, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    oc.kv_set_rows(v0, S.normal(6, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    row = np.random.default_rng(4).standard_normal((1, nq + 2 * E)).astype(np.float32)
    base = 10000.0
    q = oc.rope(np.ascontiguousarray(row[:, :nq]), np.array([pos], np.int32), D, D, False, theta_scale(base, D))
    msum = np.zeros(12, np.uint32)
    msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, n_kv, pos + 1
    scale = np.float32(1.0 / math.sqrt(D))
    want = oc.flash_attn(q, k0, v0, D, n_head, n_head_kv, scale, msum)
    kc, vc = dev.kv(E, n_kv), dev.kv(E, n_kv)
    kc.set_bytes(0, k0)
    vc.set_bytes(1, v0)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, n_kv)
    plan.set(msum)
    out, bad = dev.alloc(4 * nq), dev.upload(np.zeros(1, np.int32))
    dev.flash_attn_plan_rope(plan, dev.upload(row), kc, vc, scale, D, H.ROPE_NORMAL, dev.upload(np.array([pos], np.int32)),
                             base, dev.upload(np.array([n_kv], np.int64)), out, nq, bad=bad)
    assert bad.read(np.int32, (1,))[0] == 1
    assert (kc.get_bytes(0).reshape(n_kv, -1) == k0).all() and (vc.get_bytes(1).reshape(n_kv, -1) == v0).all()
    assert_bits_equal(out.read(np.float32, (1, nq)), want, "fa + rope, bad cell")
    plan.free()
    kc.free()
    vc.free()


def test_flash_attn_plan_rope_refusals(dev):
    plan = dev.fa_plan(128, 64, 8, 1, 64)                 # G = 8: (8 + 2) 128 > 1024
    kc, vc = dev.kv(1024, 64), dev.kv(1024, 64)
    b = dev.alloc(4 * 16384)
    msum = np.zeros(12, np.uint32)
    msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, 64, 10
    plan.set(msum)
    with pytest.raises(H.TsrHipError) as e:
        dev.flash_attn_plan_rope(plan, b, kc, vc, 0.1, 128, H.ROPE_NORMAL, b, 10000.0, b, b, 8192)
    assert e.value.code == -2
    plan.free()
    kc.free()
    vc.free()


def test_flash_attn_plan_rope_wait_expires(dev, oc):
    """The one-launch decode form's bounded wait forced to expire from the host (a poll limit of 1): the
    launch still ends, raises *bad = 2, and leaves the plan's keys and counters clear, so that the next
    launch with the default limit is bit-exact again."""
    import math
    n_kv, pos, n_head, n_head_kv, D = 4232, 4100, 32, 8, 128
    E, nq = n_head_kv * D, n_head * D
    k0 = np.zeros((n_kv, E // 32 * 34), np.uint8)
    v0 = np.zeros_like(k0)
    oc.kv_set_rows(k0, S.normal(21, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    oc.kv_set_rows(v0, S.normal(22, n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    row = np.random.default_rng(5).standard_normal((1, nq + 2 * E)).astype(np.float32)
    base = 500000.0
    ts = theta_scale(base, D)
    q = oc.rope(np.ascontiguousarray(row[:, :nq]), np.array([pos], np.int32), D, D, False, ts)
    k = oc.rope(np.ascontiguousarray(row[:, nq:nq + E]), np.array([pos], np.int32), D, D, False, ts)
    kw, vw = k0.copy(), v0.copy()
    oc.kv_set_rows(kw, k, np.array([pos], np.int64))
    oc.kv_set_rows(vw, np.ascontiguousarray(row[:, nq + E:]), np.array([pos], np.int64))
    msum = np.zeros(12, np.uint32)
    msum[0], msum[1], msum[2], msum[9] = 0x4D55534D, 1, n_kv, pos + 1
    runs = np.array([[pos, pos + 1]], np.uint32)
    scale = np.float32(1.0 / math.sqrt(D))
    want = oc.flash_attn(q, kw, vw, D, n_head, n_head_kv, scale, msum, new_runs=runs)
    kc, vc = dev.kv(E, n_kv), dev.kv(E, n_kv)
    plan = dev.fa_plan(D, n_head, n_head_kv, 1, n_kv)
    plan.set(msum, runs)
    rb, pb, cb = dev.upload(row), dev.upload(np.array([pos], np.int32)), dev.upload(np.array([pos], np.int64))
    tab = dev.alloc(4 * D)
    dev.rope_table(pb, D, base, tab)
    expired = 0
    try:
        # a workgroup gives up when its first poll finds a tile of its chunk unpublished: the tiles of
        # a chunk publish microseconds apart, so with 16 chunks x KV heads per launch some always do
        for limit in (1, 0, 1, 0):
            kc.set_bytes(0, k0)
            vc.set_bytes(1, v0)
            bad, out = dev.upload(np.zeros(1, np.int32)), dev.alloc(4 * nq)
            dev.set_fa_wait_limit(limit)
            dev.flash_attn_plan_rope_tab(plan, rb, kc, vc, scale, D, H.ROPE_NORMAL, tab, cb, out, nq, bad=bad)
            dev.sync()
            got_bad = int(bad.read(np.int32, (1,))[0])
            assert got_bad in (0, 2), got_bad
            if limit:
                expired |= got_bad
            else:
                assert got_bad == 0
                assert_bits_equal(out.read(np.float32, (1, nq)), want, "after an expired wait")
        assert expired == 2, "a poll limit of 1 never expired"
    finally:
        dev.set_fa_wait_limit(0)
    plan.free()
    kc.free()
    vc.free()
