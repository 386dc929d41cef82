"""llama.cpp's Llama graph through the ggml-backend adapter (libtsr_ggml: buffers, supports_op,
graph_compute with the plan cache and HIP graph replay) on the GPU, against the oracle's composition
of the same ops (oracle/oracle_llama.py): logits bit for bit, greedy tokens, KV cache images; and the
adapter's other device paths (weight conversion, KV buffer images, GENERAL masks, epilogues, flags)."""
import ctypes as C

import numpy as np
import pytest

import tsr_ggml_graph as GL
import tsr_ggml as G
import tsr_hip as H
import tsr_llama as LL
from helpers import assert_bits_equal
from test_gpu_llama import oracle_model

pytestmark = pytest.mark.gpu

_libm = C.CDLL("libm.so.6")
_libm.powf.argtypes = [C.c_float, C.c_float]
_libm.powf.restype = C.c_float


@pytest.fixture(scope="module")
def gdev():
    d = G.Device(0)
    yield d
    d.close()


def ts_of(cfg):
    return np.float32(_libm.powf(float(np.float32(cfg.rope_base)), float(np.float32(-2.0) / np.float32(cfg.head_dim))))


def history_images(ref, cfg, hist):
    return {(il, w): (ref.kc[il] if w == 0 else ref.vc[il])[:hist].copy() for il in range(cfg.n_layer) for w in (0, 1)}


@pytest.mark.parametrize("cfg,kv_size,hist,n_steps", [
    (LL.tiny_config(), 512, 100, 5),
    (LL.tiny_config("tiny-qwen", wfmt=H.FMT_Q8_0, ofmt=H.FMT_Q8_0, rope_mode=H.ROPE_NEOX, eps=1e-6,
                    rope_base=1000000.0), 640, 300, 4),
    (LL.tiny_config("tiny-gqa8", n_head=8, n_head_kv=1, head_dim=128, n_embd=512, n_ff=768, n_vocab=1000), 300, 250, 4),
    (LL.tiny_config("tiny-kv8", n_head=16, n_head_kv=8, head_dim=64, n_embd=512, n_ff=768, n_vocab=1000), 300, 250, 4),
], ids=["q4k", "q80-neox", "gqa8-d128", "q4k-kv8"])
@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_llama_decode_through_adapter(gdev, oc, cfg, kv_size, hist, n_steps, fused):
    """One decode token per graph_compute of llama.cpp's graph: the first run lowers and runs the calls,
    the second captures them into a HIP graph, the rest replay it with only the FLASH_ATTN_EXT chunk
    lists re-planned from the written masks; logits, greedy tokens and the caches equal the oracle's.
    Fused: the decoder's launch list (Q|K|V with the norm, one ROPE + SET_ROWS_KV + FA launch, gate|up
    with the GLU epilogue); unfused: one call per node."""
    print(f"\nadapter decode {cfg.name} fused={fused}: kv {kv_size} history {hist} steps {n_steps}", flush=True)
    gdev.set_options(0 if fused else G.OPT_NO_FUSION)
    w = LL.SyntheticWeights(cfg, cache=True)
    ref = oracle_model(oc, cfg, w, kv_size, hist)
    _, W, caches, wbuf, kvbuf = GL.load_model(gdev, cfg, w, kv_size, history_images(ref, cfg, hist))
    assert kvbuf.mode == G.MODE_KV and wbuf.mode == G.MODE_WEIGHTS
    n_kv = min(kv_size, (hist + n_steps + 255) // 256 * 256)
    g = GL.LlamaGraph(gdev, cfg, W, caches, kv_size, 1, n_kv, argmax=True)
    s0 = gdev.stats()
    ts = ts_of(cfg)
    tok = 7
    for i in range(n_steps):
        pos = hist + i
        g.set_inputs([tok], pos)
        gdev.graph_compute(g.ctx.nodes)
        got = g.logits_host()
        want = ref.step(tok, pos, ts, n_kv)
        assert_bits_equal(got, want, f"{cfg.name} step {i} (pos {pos})")
        nxt = int(g.buf.get_tensor(g.next, 4).view(np.int32)[0])
        assert nxt == int(oc.argmax(want[None])[0])
        tok = nxt
    s = gdev.stats()
    assert s["plan_misses"] - s0["plan_misses"] == 1 and s["plan_hits"] - s0["plan_hits"] == n_steps - 1
    assert s["replays"] - s0["replays"] == n_steps - 1 and s["captures"] - s0["captures"] >= 1
    row = cfg.E // 32 * 34
    for il in range(cfg.n_layer):
        for tag, img in (("k", ref.kc[il]), ("v", ref.vc[il])):
            got = kvbuf.get_tensor(caches[f"cache_{tag}_l{il}"], kv_size * row)
            assert (got == img.reshape(-1)).all(), f"layer {il} {tag} cache"
    g.free()
    kvbuf.free()
    wbuf.free()
    gdev.set_options(0)


@pytest.mark.parametrize("cfg,T,hist", [
    (LL.tiny_config(), 32, 40),
    (LL.tiny_config("tiny-qwen", wfmt=H.FMT_Q8_0, ofmt=H.FMT_Q8_0, rope_mode=H.ROPE_NEOX, eps=1e-6,
                    rope_base=1000000.0), 20, 0),
], ids=["q4k-T32", "q80-T20-from0"])
@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_llama_prefill_then_decode_through_adapter(gdev, oc, cfg, T, hist, fused):
    """A ubatch of T tokens (the MUL_MATs on the matrix cores, the causal FLASH_ATTN_EXT with the ubatch's
    cells newest last), then a decode token, through the adapter: logits equal the oracle's forward and
    step, the caches its bytes."""
    print(f"\nadapter prefill {cfg.name} fused={fused}: T {T} after {hist}", flush=True)
    gdev.set_options(0 if fused else G.OPT_NO_FUSION)
    kv_size = 256
    w = LL.SyntheticWeights(cfg, cache=True)
    ref = oracle_model(oc, cfg, w, kv_size, hist)
    _, W, caches, wbuf, kvbuf = GL.load_model(gdev, cfg, w, kv_size, history_images(ref, cfg, hist) if hist else None)
    ts = ts_of(cfg)
    toks = np.random.default_rng(5).integers(0, cfg.n_vocab, T).astype(np.int32)
    gp = GL.LlamaGraph(gdev, cfg, W, caches, kv_size, T, kv_size)
    gp.set_inputs(toks, hist)
    gdev.graph_compute(gp.ctx.nodes)
    assert_bits_equal(gp.logits_host(), ref.forward(toks, hist, ts, kv_size), f"{cfg.name} prefill")
    gd = GL.LlamaGraph(gdev, cfg, W, caches, kv_size, 1, kv_size, argmax=True)
    pos = hist + T
    gd.set_inputs([3], pos)
    gdev.graph_compute(gd.ctx.nodes)
    assert_bits_equal(gd.logits_host(), ref.step(3, pos, ts, kv_size), f"{cfg.name} decode after prefill")
    row = cfg.E // 32 * 34
    for il in range(cfg.n_layer):
        got = kvbuf.get_tensor(caches[f"cache_k_l{il}"], kv_size * row)
        assert (got == ref.kc[il].reshape(-1)).all()
    gdev.synchronize()
    for x in (gp, gd, kvbuf, wbuf):
        x.free()
    gdev.set_options(0)


def test_weight_types_converted_to_q8_0(gdev, oc):
    """MUL_MAT weights of F32, F16, BF16 and a registered type are converted to Q8_0 at first use
    (ggml's to_float, then quantize_row_q8_0_ref: tsr-weights.cpp:33-49); the results equal the oracle's
    MUL_MAT of the converted blocks, and a rewrite of the weight is picked up."""
    rng = np.random.default_rng(11)
    N, K, T = 96, 256, 3
    x = rng.standard_normal((T, K)).astype(np.float32)
    w32 = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
    tid = gdev.register_type("f32x32", 32, 128, lambda src, dst, n: C.memmove(dst, src, 4 * n))
    c = GL.Ctx({tid: (32, 128)})
    cases = [(G.F32, w32, w32), (G.F16, w32.astype(np.float16), w32.astype(np.float16).astype(np.float32)),
             (G.BF16, (w32.view(np.uint32) >> 16).astype(np.uint16),
              ((w32.view(np.uint32) >> 16) << 16).astype(np.uint32).view(np.float32)),
             (tid, w32, w32)]
    wbuf = gdev.buffer(len(cases) * N * K * 4 + 4096, G.USAGE_WEIGHTS)
    cbuf = gdev.buffer(1 << 20, G.USAGE_COMPUTE)
    off = coff = 0
    for type_, raw, as_f32 in cases:
        wt = c.new(type_, [K, N], f"w{type_}")
        off = c.place(wt, wbuf, off)
        wbuf.set_tensor(wt, raw)
        xt = c.new(G.F32, [K, T], "x")
        coff = c.place(xt, cbuf, coff)
        cbuf.set_tensor(xt, x)
        y = c.mul_mat(wt, xt, "y")
        coff = c.place(y, cbuf, coff)
        gdev.graph_compute([y])
        got = cbuf.get_tensor(y, 4 * N * T).view(np.float32).reshape(T, N)
        blocks = G.quantize_q8_0(as_f32).reshape(N, -1)
        assert_bits_equal(got, oc.mul_mat(H.FMT_Q8_0, blocks, K, x), f"type {type_}")
    # rewriting a converted weight drops its device copy: the next graph converts again
    wt = c.new(G.F32, [K, N], "w_rewritten")
    off = c.place(wt, wbuf, off)
    wbuf.set_tensor(wt, w32)
    xt = c.new(G.F32, [K, T], "x2")
    coff = c.place(xt, cbuf, coff)
    cbuf.set_tensor(xt, x)
    y = c.mul_mat(wt, xt, "y2")
    coff = c.place(y, cbuf, coff)
    gdev.graph_compute([y])
    wbuf.set_tensor(wt, -w32)
    n0 = gdev.stats()["weights_converted"]
    gdev.graph_compute([y])
    assert gdev.stats()["weights_converted"] == n0 + 1
    got = cbuf.get_tensor(y, 4 * N * T).view(np.float32).reshape(T, N)
    assert_bits_equal(got, oc.mul_mat(H.FMT_Q8_0, G.quantize_q8_0(-w32).reshape(N, -1), K, x), "rewritten")
    cbuf.free()
    wbuf.free()


def test_kv_buffer_image_round_trip(gdev):
    """A KV buffer (cache tensors by name) holds the exact ggml q8_0 image: byte ranges that start and end
    inside rows and span two tensors, memset, clear."""
    c = GL.Ctx()
    E, kv_size = 128, 40
    row = E // 32 * 34
    buf = gdev.buffer(2 * kv_size * row + 128)
    ts, off = [], 0
    for name in ("cache_k_l0", "cache_v_l0"):
        t = c.new(G.Q8_0, [E, kv_size, 1], name)
        off = c.place(t, buf, off)
        ts.append(t)
    assert ts[1].data == ts[0].data + kv_size * row                 # adjacent: a range may span both
    buf.clear(0x5A)
    assert buf.mode == G.MODE_KV
    assert (buf.get_tensor(ts[0], kv_size * row) == 0x5A).all()
    rng = np.random.default_rng(2)
    img = rng.integers(0, 256, 2 * kv_size * row, dtype=np.uint8)
    buf.set_tensor(ts[0], img)                                     # both tensors in one write
    assert (buf.get_tensor(ts[0], 2 * kv_size * row) == img).all()
    part = rng.integers(0, 256, 3 * row + 17, dtype=np.uint8)
    buf.set_tensor(ts[0], part, offset=kv_size * row - row - 5)    # crosses into the V tensor
    img[kv_size * row - row - 5:kv_size * row - row - 5 + part.size] = part
    assert (buf.get_tensor(ts[0], 2 * kv_size * row) == img).all()
    buf.memset_tensor(ts[1], 0, 7, 2 * row)
    img[kv_size * row + 7:kv_size * row + 7 + 2 * row] = 0
    assert (buf.get_tensor(ts[1], kv_size * row) == img[kv_size * row:]).all()
    buf.free()


def test_general_mask_and_no_mask_flash_attn(gdev, oc):
    """FLASH_ATTN_EXT graphs whose mask summary is GENERAL (a finite mask value and a third run: the f32
    mask copy the library makes from the written mask) and with no mask (every cell visible), against
    the oracle."""
    rng = np.random.default_rng(4)
    D, H_, Hk, kv_size, T, n_kv = 128, 8, 2, 300, 3, 288
    E = Hk * D
    row = E // 32 * 34
    kimg = np.zeros((kv_size, row), np.uint8)
    vimg = np.zeros((kv_size, row), np.uint8)
    oc.kv_set_rows(kimg, rng.standard_normal((kv_size, E)).astype(np.float32), np.arange(kv_size))
    oc.kv_set_rows(vimg, rng.standard_normal((kv_size, E)).astype(np.float32), np.arange(kv_size))
    c = GL.Ctx()
    kvbuf = gdev.buffer(2 * kv_size * row + 128)
    kc, vc = c.new(G.Q8_0, [E, kv_size, 1], "cache_k_l0"), c.new(G.Q8_0, [E, kv_size, 1], "cache_v_l0")
    off = c.place(kc, kvbuf, 0)
    c.place(vc, kvbuf, off)
    kvbuf.set_tensor(kc, kimg)
    kvbuf.set_tensor(vc, vimg)
    cbuf = gdev.buffer(1 << 22, G.USAGE_COMPUTE)
    q = c.new(G.F32, [D, H_, T], "q")
    mask = c.new(G.F16, [n_kv, T], "attn_inp_kq_mask")
    coff = c.place(q, cbuf, 0)
    coff = c.place(mask, cbuf, coff)
    kv4 = [D // 32 * 34, row, row * kv_size]
    kp = c.permute(c.view(kc, [D, Hk, n_kv, 1], kv4, 0), 0, 2, 1, 3)
    vp = c.permute(c.view(vc, [D, Hk, n_kv, 1], kv4, 0), 0, 2, 1, 3)
    qp = c.permute(q, 0, 2, 1, 3)
    scale = float(np.float32(0.088388346))
    out_m = c.flash_attn_ext(qp, kp, vp, mask, scale, name="fa_mask")
    out_n = c.flash_attn_ext(qp, kp, vp, None, scale, name="fa_nomask")
    c.alloc_nodes(cbuf, coff)
    qv = rng.standard_normal((T, H_ * D)).astype(np.float32)
    cbuf.set_tensor(q, qv)
    m = np.full((T, n_kv), -np.inf, np.float16)
    m[:, :100] = 0
    m[:, 150:200] = 0
    m[:, 250:260] = 0                                              # a third run: GENERAL
    m[1, 10] = -2.5                                                # a finite value: GENERAL
    cbuf.set_tensor(mask, m)
    gdev.graph_compute(c.nodes)
    msum = oc.msum(m)
    assert msum[3] & 1
    want = oc.flash_attn(qv, kimg, vimg, D, H_, Hk, scale, msum, mask_f32=oc.mask_f32(m, scale))
    got = cbuf.get_tensor(out_m, 4 * T * H_ * D).view(np.float32).reshape(T, -1)
    assert_bits_equal(got, want, "GENERAL mask")
    allv = np.zeros((T, n_kv), np.float16)
    want_n = oc.flash_attn(qv, kimg, vimg, D, H_, Hk, scale, oc.msum(allv))
    got_n = cbuf.get_tensor(out_n, 4 * T * H_ * D).view(np.float32).reshape(T, -1)
    assert_bits_equal(got_n, want_n, "no mask")
    cbuf.free()
    kvbuf.free()


def test_mul_mat_epilogues_through_adapter(gdev, oc):
    """MUL_MAT + SCALE and the logit soft cap (SCALE, TANH, SCALE) lowered to the MUL_MAT epilogue."""
    rng = np.random.default_rng(6)
    N, K = 1000, 256
    c = GL.Ctx()
    wb = (rng.standard_normal((N, K)) * 0.2).astype(np.float32)
    blocks = G.quantize_q8_0(wb).reshape(N, -1)
    wbuf = gdev.buffer(blocks.nbytes + 64, G.USAGE_WEIGHTS)
    w = c.new(G.Q8_0, [K, N], "output.weight")
    c.place(w, wbuf, 0)
    wbuf.set_tensor(w, blocks)
    cbuf = gdev.buffer(1 << 20, G.USAGE_COMPUTE)
    x = c.new(G.F32, [K, 2], "x")
    coff = c.place(x, cbuf, 0)
    xv = rng.standard_normal((2, K)).astype(np.float32) * 4
    cbuf.set_tensor(x, xv)
    s2 = c.scale(c.tanh(c.scale(c.mul_mat(w, x), 1.0 / 30.0)), 30.0)
    sc = c.scale(c.mul_mat(w, x), 0.25)
    c.alloc_nodes(cbuf, coff)
    gdev.graph_compute(c.nodes)
    got = cbuf.get_tensor(s2, 4 * 2 * N).view(np.float32).reshape(2, N)
    assert_bits_equal(got, oc.mul_mat(H.FMT_Q8_0, blocks, K, xv, epi=(2, np.float32(1.0 / 30.0), 30.0)), "softcap")
    got = cbuf.get_tensor(sc, 4 * 2 * N).view(np.float32).reshape(2, N)
    assert_bits_equal(got, oc.mul_mat(H.FMT_Q8_0, blocks, K, xv, epi=(1, 0.0, 0.25)), "scale")
    cbuf.free()
    wbuf.free()


def test_device_flag_reported(gdev):
    """A SET_ROWS index outside the cache stores nothing and raises the library's device flag (the
    kernel's own bounds check); the adapter reports it at the next read (TSR_GG_E_FLAG) and clears it."""
    c = GL.Ctx()
    E, kv_size = 128, 16
    row = E // 32 * 34
    kvbuf = gdev.buffer(kv_size * row * 2 + 128)
    kc = c.new(G.Q8_0, [E, kv_size, 1], "cache_k_l0")
    vc = c.new(G.Q8_0, [E, kv_size, 1], "cache_v_l0")
    off = c.place(kc, kvbuf, 0)
    c.place(vc, kvbuf, off)
    kvbuf.clear(0)
    cbuf = gdev.buffer(1 << 16, G.USAGE_COMPUTE)
    rows = c.new(G.F32, [E, 2], "rows")
    idx = c.new(G.I64, [2], "k_idxs")
    coff = c.place(rows, cbuf, 0)
    c.place(idx, cbuf, coff)
    cbuf.set_tensor(rows, np.ones((2, E), np.float32))
    cbuf.set_tensor(idx, np.array([3, kv_size + 5], np.int64))
    c.set_rows(kc, rows, idx)
    c.alloc_nodes(cbuf, 1 << 15)
    gdev.graph_compute(c.nodes)
    with pytest.raises(G.GGError) as e:
        kvbuf.get_tensor(kc, kv_size * row)
    assert e.value.code == G.E_FLAG
    img = kvbuf.get_tensor(kc, kv_size * row).reshape(kv_size, row)   # flag cleared; cell 3 written
    assert (img[3] != 0).any() and (np.delete(img, 3, axis=0) == 0).all()
    cbuf.free()
    kvbuf.free()


def test_reset_compute_buffer_forgets_mask_summaries(gdev, oc):
    """buffer_i.reset of the compute buffer (ggml-tesseract.cpp:2015-2024): the mask summaries and cell
    index copies kept for its addresses are forgotten, so a graph_compute whose mask was not written
    again since fails (TSR_GG_E_UNSUPPORTED) instead of planning FLASH_ATTN_EXT from an earlier
    layout's summary; with the inputs written again the token is the oracle's, bit for bit. Also
    device_i.get_memory of the GPU."""
    free_b, total_b = gdev.memory()
    assert 0 < free_b <= total_b and total_b > 100 << 30
    cfg, kv_size, hist = LL.tiny_config(), 512, 100
    w = LL.SyntheticWeights(cfg, cache=True)
    ref = oracle_model(oc, cfg, w, kv_size, hist)
    _, W, caches, wbuf, kvbuf = GL.load_model(gdev, cfg, w, kv_size, history_images(ref, cfg, hist))
    g = GL.LlamaGraph(gdev, cfg, W, caches, kv_size, 1, 256, argmax=True)
    ts = ts_of(cfg)
    g.set_inputs([7], hist)
    gdev.graph_compute(g.ctx.nodes)
    assert_bits_equal(g.logits_host(), ref.step(7, hist, ts, 256), "before the reset")
    g.buf.reset()
    with pytest.raises(G.GGError) as e:
        gdev.graph_compute(g.ctx.nodes)
    assert e.value.code == G.E_UNSUPPORTED and "mask" in str(e.value)
    g.set_inputs([9], hist + 1)
    gdev.graph_compute(g.ctx.nodes)
    assert_bits_equal(g.logits_host(), ref.step(9, hist + 1, ts, 256), "after the reset, inputs written again")
    gdev.synchronize()
    for x in (g, kvbuf, wbuf):
        x.free()
