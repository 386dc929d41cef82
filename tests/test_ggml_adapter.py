"""libtsr_ggml on the CPU (a probe device: no GPU): the library exports include/tsr_ggml.h, and its
host logic -- KV-cache names, the Q8_0 load-time conversion, supports_op's rules with their reasons,
the lowering of llama.cpp's Llama graph (fusions, FLASH_ATTN_EXT arguments), the graph identity of the
plan cache -- follows the reference backend's rules (sw/ggml-tesseract). Also the library's f32 mask
copy against the oracle's."""
import os
import re

import numpy as np
import pytest

import tsr_ggml_graph as GL
import tsr_ggml as G
import tsr_hip
import tsr_llama as LL

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_header():
    txt = re.sub(r"/\*.*?\*/", "", open(os.path.join(REPO, "include", "tsr_ggml.h")).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(tsr_gg_\w+)\s*\(", txt)) - {"tsr_gg_to_float_fn"})
    L = G.load()
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/tsr_ggml.h but not exported"
    assert sorted(G.EXPORTS) == names


@pytest.mark.parametrize("name,want", [
    ("cache_k_l0", (0, 0)), ("cache_v_l31", (1, 31)), ("cache_xk_l3", (0, 3)), ("cache_shared_v_l12", (1, 12)),
    ("cache_k_l", None), ("cache_k_lx", None), ("cache_q_l0", None), ("kv_k_l0", None), ("cache_k_l0a", None),
    ("cache_l0", None),
])
def test_kv_parse_name(name, want):
    """tsr_kv_parse_name (sw/ggml-tesseract/tsr-kvbuf.h:56-60): cache_<tag>k_l<n> / cache_<tag>v_l<n>."""
    assert G.kv_parse_name(name) == want


def q8_0_closed_form(x):
    """ggml's quantize_row_q8_0_ref in numpy: d = amax / 127 (f32), id = 1 / d, q = roundf(x id) (half
    away from zero), d stored as fp16 (round to nearest even)."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    out = np.empty((x.shape[0], 34), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def test_quantize_q8_0_closed_form():
    """The load-time conversion of non-native weights (tsr-weights.cpp:33-49): ggml's
    quantize_row_q8_0_ref, against its closed form; blocks of zeros, exact .5 ties, fp16
    scales that round, and large values (a block whose d is subnormal divides by a subnormal: ggml's
    conversion is undefined there, and no such block is tested)."""
    rng = np.random.default_rng(1)
    rows = [rng.standard_normal(4096).astype(np.float32),
            np.zeros(64, np.float32),
            np.concatenate([[127.0], np.arange(31) - 15.5]).astype(np.float32),   # d = 1: x id = k + .5 ties
            (rng.standard_normal(96) * 1e4).astype(np.float32),
            (rng.random(32) * 3e-5).astype(np.float32)]
    for x in rows:
        got = G.quantize_q8_0(x)
        want = q8_0_closed_form(x)
        assert (got == want).all()
    # a planted mistake (round half to even instead of away) is caught by the tie row
    x = rows[2]
    d = np.float32(np.abs(x).max() / np.float32(127))
    v = (x * (np.float32(1) / d)).astype(np.float32)
    assert (np.abs(v - np.trunc(v)) == 0.5).any()
    assert (np.rint(v) != np.sign(v) * np.floor(np.abs(v) + 0.5)).any()


def test_alloc_size_and_alignment():
    dev = G.Device(-1)
    c = GL.Ctx()
    assert G.load().tsr_gg_alignment() == 64
    assert dev.alloc_size(c.new(G.F32, [5], "a")) == 64
    assert dev.alloc_size(c.new(G.Q4_K, [4096, 3], "w")) == 3 * 16 * 144
    assert dev.alloc_size(c.new(G.Q8_0, [96, 1], "q")) == 128
    dev.close()


class Probe:
    """A probe device with a weights buffer, a KV buffer and a compute buffer, for supports_op."""

    def __init__(self, E=256, kv_size=512):
        self.dev = G.Device(-1)
        self.c = GL.Ctx()
        self.wbuf = self.dev.buffer(1 << 26, G.USAGE_WEIGHTS)
        self.kvbuf = self.dev.buffer(1 << 24)
        self.cbuf = self.dev.buffer(1 << 26, G.USAGE_COMPUTE)
        self.woff = self.koff = self.coff = 0
        self.kc = self.kv(G.Q8_0, [E, kv_size, 1], "cache_k_l0")
        self.vc = self.kv(G.Q8_0, [E, kv_size, 1], "cache_v_l0")

    def w(self, type_, ne, name):
        t = self.c.new(type_, ne, name)
        self.woff = self.c.place(t, self.wbuf, self.woff)
        return t

    def kv(self, type_, ne, name):
        t = self.c.new(type_, ne, name)
        self.koff = self.c.place(t, self.kvbuf, self.koff)
        return t

    def a(self, type_, ne, name="act", flags=0):
        t = self.c.new(type_, ne, name, flags)
        self.coff = self.c.place(t, self.cbuf, self.coff)
        return t

    def node(self, t):
        """An op result: placed in the compute buffer (views take their base's address)."""
        if t.view_src:
            b = t.view_src.contents
            t.data, t.buffer = b.data + t.view_offs, b.buffer
        else:
            self.coff = self.c.place(t, self.cbuf, self.coff)
        return t

    def ok(self, t):
        ok, why = self.dev.supports_op(t)
        assert ok, why

    def no(self, t, reason):
        ok, why = self.dev.supports_op(t)
        assert not ok and re.search(reason, why), why


def test_supports_op_mul_mat():
    """supports_op for MUL_MAT (ggml-tesseract.cpp:4197-4298)."""
    p = Probe()
    c = p.c
    w = p.w(G.Q4_K, [4096, 256], "blk.0.attn_q.weight")
    x = p.a(G.F32, [4096, 7])
    p.ok(p.node(c.mul_mat(w, x)))
    p.ok(p.node(c.mul_mat(p.w(G.Q8_0, [896, 64], "w80"), p.a(G.F32, [896, 1]))))
    p.ok(p.node(c.mul_mat(p.w(G.F16, [128, 32], "w16"), p.a(G.F32, [128, 2]))))      # converted to Q8_0
    p.no(p.node(c.mul_mat(w, p.a(G.F16, [4096, 7]))), "MUL_MAT f32-io")
    p.no(p.node(c.mul_mat(p.w(G.F32, [96 + 16, 8], "odd"), p.a(G.F32, [112, 1]))), "MUL_MAT k-range")
    p.no(p.node(c.mul_mat(p.w(G.Q8_0, [32768 + 32, 2], "big"), p.a(G.F32, [32800, 1]))), "MUL_MAT k-range.*K_MAX")
    p.no(p.node(c.mul_mat(p.a(G.Q8_0, [4096, 16], "wact"), p.a(G.F32, [4096, 1]))), "MUL_MAT weight-home")
    p.no(p.node(c.mul_mat(p.w(G.Q8_0, [64, 8, 2], "batched"), p.a(G.F32, [64, 1, 2]))), "MUL_MAT matrix")
    p.no(p.node(c.mul_mat(p.w(G.I32, [64, 8], "ints"), p.a(G.F32, [64, 1]))), "MUL_MAT device-format")
    xt = p.node(c.permute(p.a(G.F32, [64, 4]), 1, 0, 2, 3))
    p.no(p.node(c.mul_mat(p.w(G.F32, [4, 64], "w4"), xt)), "MUL_MAT dense")
    # a src1 view that is not 64-byte aligned
    big = p.a(G.F32, [64 * 3 + 8])
    v = p.node(c.view(big, [64, 1], [256], 8 * 4))
    p.no(p.node(c.mul_mat(p.w(G.F32, [64, 8], "w64"), v)), "MUL_MAT x-aligned")
    p.dev.close()


def fa_graph(p, D=128, H=8, Hk=2, T=1, n_kv=256, mask_type=G.F16, q_type=G.F32, **kw):
    c = p.c
    q = p.a(q_type, [D, H, T], "q")
    qp = p.node(c.permute(q, 0, 2, 1, 3))
    E = Hk * D
    row = E // 32 * 34
    kv4 = [D // 32 * 34, row, row * 512]
    k = p.node(c.permute(p.node(c.view(p.kc, [D, Hk, n_kv, 1], kv4, 0)), 0, 2, 1, 3))
    v = p.node(c.permute(p.node(c.view(p.vc, [D, Hk, n_kv, 1], kv4, 0)), 0, 2, 1, 3))
    m = p.a(mask_type, [n_kv, T], "attn_inp_kq_mask", G.FLAG_INPUT) if mask_type is not None else None
    return p.node(c.flash_attn_ext(qp, k, v, m, 0.088, **kw))


def test_supports_op_flash_attn():
    """supports_op for FLASH_ATTN_EXT (tsr_lower_fa, sw/ggml-tesseract/tsr-build.cpp:673-773)."""
    p = Probe(E=256)
    p.ok(fa_graph(p))
    p.ok(fa_graph(p, T=64))
    p.ok(fa_graph(p, mask_type=None))
    p.no(fa_graph(p, q_type=G.F16), "FLASH_ATTN_EXT types: q F32")
    p.no(fa_graph(p, max_bias=8.0), "FLASH_ATTN_EXT plain-softmax.*max_bias=8")
    p.no(fa_graph(p, softcap=30.0), "FLASH_ATTN_EXT plain-softmax.*softcap=30")
    p.no(fa_graph(p, mask_type=G.F32), "FLASH_ATTN_EXT mask:")
    p.no(fa_graph(p, T=681), "FLASH_ATTN_EXT rows:.*T=681")
    p.no(fa_graph(p, H=9), "FLASH_ATTN_EXT gqa")
    t = fa_graph(p)
    t.src[4] = t.src[0]
    p.no(t, "FLASH_ATTN_EXT no-sinks")
    # K / V from a weights buffer, not a KV cache
    c = p.c
    q = p.node(c.permute(p.a(G.F32, [128, 8, 1]), 0, 2, 1, 3))
    kw = p.w(G.Q8_0, [128, 256, 2], "cache_k_l0")
    p.no(p.node(c.flash_attn_ext(q, kw, kw, None, 0.1)), "FLASH_ATTN_EXT kv-views")
    # V and K swapped
    t = fa_graph(p)
    t.src[1], t.src[2] = t.src[2], t.src[1]
    p.no(t, "FLASH_ATTN_EXT one-layer")
    p.dev.close()


def test_supports_op_glue():
    p = Probe()
    c = p.c
    x = p.a(G.F32, [256, 4])
    n = p.node(c.rms_norm(x, 1e-5))
    p.ok(n)
    p.ok(p.node(c.mul(n, p.w(G.F32, [256], "norm.weight"))))
    p.no(p.node(c.mul(x, p.a(G.F32, [256, 4]))), "MUL norm-weight")
    p.ok(p.node(c.add(x, p.a(G.F32, [256, 4]))))
    p.ok(p.node(c.add(x, p.a(G.F32, [256, 1]))))
    p.no(p.node(c.add(x, p.a(G.F32, [256, 3]))), "ADD row-broadcast")
    g, u = p.a(G.F32, [128, 2]), p.a(G.F32, [128, 2])
    p.ok(p.node(c.swiglu_split(g, u)))
    geglu = p.node(c.swiglu_split(g, u))
    geglu.op_params[0] = 1
    p.no(geglu, "GLU swiglu")
    pos = p.a(G.I32, [4], "inp_pos")
    h = p.a(G.F32, [64, 4, 4])
    p.ok(p.node(c.rope_ext(h, pos, 64, 0, 10000.0)))
    p.ok(p.node(c.rope_ext(h, pos, 32, 2, 10000.0)))
    p.no(p.node(c.rope_ext(h, pos, 64, 8, 10000.0)), "ROPE mode:.*mode=8")
    p.no(p.node(c.rope_ext(h, pos, 64, 0, 10000.0, ext_factor=1.0)), "ROPE no-yarn")
    emb = p.w(G.F32, [256, 1000], "token_embd.weight")
    ids = p.a(G.I32, [3], "inp_tokens")
    p.ok(p.node(c.get_rows(emb, ids)))
    p.no(p.node(c.get_rows(p.w(G.Q4_K, [256, 1000], "token_embd.q"), ids)), "table .* is not f32 rows")
    lg = p.a(G.F32, [1000, 2])
    p.ok(p.node(c.argmax(lg)))
    mm = p.node(c.mul_mat(p.w(G.Q8_0, [256, 64], "wo"), x))
    p.ok(p.node(c.scale(mm, 0.5)))
    p.no(p.node(c.scale(x, 0.5)), "SCALE/TANH epilogue")
    p.no(p.node(c.tanh(x)), "SCALE/TANH epilogue")
    rows = p.a(G.F32, [256, 4])
    idx = p.a(G.I64, [4], "k_idxs")
    p.ok(p.node(c.set_rows(p.kc, rows, idx)))
    p.no(p.node(c.set_rows(p.a(G.F32, [256, 16]), rows, idx)), "SET_ROWS kv-dest")
    p.no(p.node(c.set_rows(p.kc, rows, p.a(G.I32, [4]))), "SET_ROWS i64-cells")
    for op in (G.OP_VIEW, G.OP_RESHAPE, G.OP_PERMUTE, G.OP_TRANSPOSE, G.OP_NONE):
        t = p.a(G.F32, [4])
        t.op = op
        p.ok(t)
    t = p.a(G.F32, [4])
    t.op = G.OP_OTHER
    p.no(t, "not on the device")
    p.dev.close()


def declare_model(p, cfg, kv_size):
    """The weights and caches of a Llama model placed in a probe device's buffers (no data)."""
    fmt = {0: G.Q8_0, 1: G.Q4_K}
    W = {"token_embd.weight": p.w(G.F32, [cfg.n_embd, cfg.n_vocab], "token_embd.weight"),
         "output_norm.weight": p.w(G.F32, [cfg.n_embd], "output_norm.weight"),
         "output.weight": p.w(fmt[cfg.ofmt], [cfg.n_embd, cfg.n_vocab], "output.weight")}
    caches = {}
    for il in range(cfg.n_layer):
        for name, N, K in LL.layer_tensors(cfg, il):
            W[name] = p.w(fmt[cfg.wfmt], [K, N], name)
        for nm in ("attn_norm", "ffn_norm"):
            W[f"blk.{il}.{nm}.weight"] = p.w(G.F32, [cfg.n_embd], f"blk.{il}.{nm}.weight")
        for tag in "kv":
            caches[f"cache_{tag}_l{il}"] = p.kv(G.Q8_0, [cfg.E, kv_size, 1], f"cache_{tag}_l{il}")
    return W, caches


@pytest.mark.parametrize("T", [1, 24])
def test_lower_llama_graph_unfused(T):
    """With fusions off, llama.cpp's Llama graph lowers to the library calls of the reference's op list:
    per layer one RMS_NORM+MUL record, the Q / K / V MUL_MATs, two ROPEs, two SET_ROWS_KV, one
    FLASH_ATTN_EXT (scale from op_params[0], q's token stride, the new-cell indices of the K SET_ROWS),
    the o MUL_MAT with the residual ADD (tsr_fuse_mm_add, kept in every lowering), RMS_NORM+MUL, gate,
    up, SWIGLU, down+ADD."""
    cfg = LL.tiny_config()
    p = Probe()
    p.kvbuf = p.dev.buffer(1 << 24)
    p.koff = 0
    kv_size = 512
    W, caches = declare_model(p, cfg, kv_size)
    g = GL.LlamaGraph(p.dev, cfg, W, caches, kv_size, T, 256, argmax=True)
    p.dev.set_options(G.OPT_NO_FUSION)
    calls = p.dev.lower(g.ctx.nodes)
    names = [c["name"] for c in calls]
    L = cfg.n_layer
    per_layer = ["RMS_NORM", "MUL_MAT", "MUL_MAT", "MUL_MAT", "ROPE", "ROPE", "SET_ROWS", "SET_ROWS", "FLASH_ATTN_EXT",
                 "MUL_MAT", "ADD", "RMS_NORM", "MUL_MAT", "MUL_MAT", "SWIGLU", "MUL_MAT", "ADD"]
    last = per_layer[:10] + ["GET_ROWS", "GET_ROWS", "ADD"] + per_layer[11:]
    want = ["GET_ROWS"] + per_layer * (L - 1) + last + ["RMS_NORM", "MUL_MAT", "ARGMAX"]
    assert names == want
    nodes = g.ctx.nodes
    fas = [c for c in calls if c["name"] == "FLASH_ATTN_EXT"]
    assert len(fas) == L
    D, H = cfg.head_dim, cfg.n_head
    for f in fas:
        assert f["D"] == D and f["n_head"] == H and f["n_head_kv"] == cfg.n_head_kv
        assert f["n_kv"] == 256 and f["kv_size"] == kv_size and f["T"] == T
        assert np.float32(f["scale"]) == np.float32(1.0) / np.sqrt(np.float32(D))
        assert f["x_stride"] == H * D and f["y_stride"] == H * D
        assert f["w"] == g.k_idxs.data and f["K"] == T            # FA_NEW: the K SET_ROWS' indices
        assert f["add"] == g.kq_mask.data
    norms = [c for c in calls if c["name"] == "RMS_NORM"]
    assert all(c["node2"] >= 0 and nodes[c["node2"]].op == G.OP_MUL for c in norms)
    assert np.float32(norms[0]["scale"]) == np.float32(cfg.eps)
    assert all(c["node2"] == -1 for c in calls if c["name"] == "MUL_MAT")
    ropes = [c for c in calls if c["name"] == "ROPE"]
    assert all(r["n_dims"] == D and r["mode"] == cfg.rope_mode and r["add"] == g.inp_pos.data for r in ropes)
    assert np.float32(ropes[0]["scale"]) == np.float32(cfg.rope_base)
    sets = [c for c in calls if c["name"] == "SET_ROWS"]
    assert [s["which"] for s in sets] == [0, 1] * L and all(s["T"] == T and s["N"] == cfg.E for s in sets)
    p.dev.close()


@pytest.mark.parametrize("T", [1, 24])
def test_lower_llama_graph_fused(T):
    """The same graph lowered with its fusions: the decoder's launch list. One token, per layer: the
    Q|K|V matvec with the attention RMS_NORM folded in (its rows concatenated), one ROPE + SET_ROWS_KV +
    FLASH_ATTN_EXT launch (the angle table once per graph; the Q|K|V matvec runs inside it, its call
    marked CALL_IN_NEXT), o + residual, gate|up with the FFN norm and the SWIGLU epilogue, down +
    residual. A ubatch (T = 24): the norms stay calls (the matrix-core
    MUL_MATs take no norm), the Q|K|V MUL_MAT, ROPE_KV, the planned FLASH_ATTN_EXT."""
    cfg = LL.tiny_config()
    p = Probe()
    p.kvbuf = p.dev.buffer(1 << 24)
    p.koff = 0
    kv_size = 512
    W, caches = declare_model(p, cfg, kv_size)
    g = GL.LlamaGraph(p.dev, cfg, W, caches, kv_size, T, 256, argmax=True)
    calls = p.dev.lower(g.ctx.nodes)
    names = [c["name"] for c in calls]
    L, D, H, E = cfg.n_layer, cfg.head_dim, cfg.n_head, cfg.E
    nodes = g.ctx.nodes
    if T == 1:
        first = ["MUL_MAT", "ROPE_TABLE", "FLASH_ATTN_EXT", "MUL_MAT", "MUL_MAT", "MUL_MAT"]
        mid = ["MUL_MAT", "FLASH_ATTN_EXT", "MUL_MAT", "MUL_MAT", "MUL_MAT"]
        last = ["MUL_MAT", "FLASH_ATTN_EXT", "MUL_MAT", "GET_ROWS", "GET_ROWS", "ADD", "MUL_MAT", "MUL_MAT"]
        want = ["GET_ROWS"] + first + mid * (L - 2) + last + ["MUL_MAT", "ARGMAX"]
    else:
        per = ["RMS_NORM", "MUL_MAT", "ROPE_KV", "FLASH_ATTN_EXT", "MUL_MAT", "RMS_NORM", "MUL_MAT", "MUL_MAT"]
        last = per[:5] + ["GET_ROWS", "GET_ROWS", "ADD", "MUL_MAT", "MUL_MAT"]   # one row from here: folds again
        want = ["GET_ROWS"] + per * (L - 1) + last + ["MUL_MAT", "ARGMAX"]
    assert names == want
    mms = [c for c in calls if c["name"] == "MUL_MAT"]
    qkv = [c for c in mms if c["N"] == H * D + 2 * E]
    glu = [c for c in mms if c["flags"] == tsr_hip.MM_GLU]
    assert len(qkv) == L and len(glu) == L
    assert all(c["y"] == 0 for c in qkv)                          # the plan's Q|K|V rows
    # one token: the Q|K|V matvec (norm folded) runs inside its attention call
    assert all(bool(c["flags"] & G.CALL_IN_NEXT) == (T == 1) for c in qkv)
    assert not any(c["flags"] & G.CALL_IN_NEXT for c in calls if c not in qkv)
    for c in glu:
        assert c["N"] == 2 * cfg.n_ff and nodes[c["node"]].op == G.OP_GLU and c["y"] == nodes[c["node"]].data
    folded = [c for c in mms if c["node2"] >= 0 and nodes[c["node2"]].op == G.OP_RMS_NORM or c["node3"] >= 0]
    if T == 1:
        assert len(folded) == 2 * L + 1                            # Q|K|V and gate|up of every layer, the head
        assert all(np.float32(c["scale"]) == np.float32(cfg.eps) for c in folded)
    fas = [c for c in calls if c["name"] == "FLASH_ATTN_EXT"]
    assert all(f["n_dims"] == D and f["mode"] == cfg.rope_mode and f["x_stride"] == H * D + 2 * E for f in fas)
    assert all(f["w"] == g.k_idxs.data and f["add"] == g.kq_mask.data for f in fas)
    if T > 1:
        rk = [c for c in calls if c["name"] == "ROPE_KV"]
        assert len(rk) == L and all(r["T"] == T and r["add"] == g.k_idxs.data for r in rk)
    p.dev.close()


def test_qkv_stays_a_call_when_x_is_overwritten_before_attention():
    """The one-token Q|K|V MUL_MAT runs inside its FLASH_ATTN_EXT call only while its x (the norm's
    input) is unchanged at that node: with a node between the two writing x's bytes (ggml-alloc reusing
    them), that layer keeps the MUL_MAT as its own call, and the other layers are unchanged."""
    cfg = LL.tiny_config()
    p = Probe()
    p.kvbuf = p.dev.buffer(1 << 24)
    p.koff = 0
    W, caches = declare_model(p, cfg, 512)
    g = GL.LlamaGraph(p.dev, cfg, W, caches, 512, 1, 256, argmax=True)
    nodes = g.ctx.nodes

    def qkv_flags():
        calls = p.dev.lower(nodes)
        return [bool(c["flags"] & G.CALL_IN_NEXT) for c in calls
                if c["name"] == "MUL_MAT" and c["N"] == cfg.n_head * cfg.head_dim + 2 * cfg.E]

    assert qkv_flags() == [True] * cfg.n_layer
    x0 = next(t for t in nodes if t.name.startswith(b"inp_embd"))
    rk = next(t for t in nodes if t.op == G.OP_ROPE and t.name.startswith(b"Kcur-0"))
    rk.data = x0.data                                    # layer 0's K rotation lands on x
    assert qkv_flags() == [False] + [True] * (cfg.n_layer - 1)
    p.dev.close()


def test_fusion_refused_when_the_result_overlaps_an_input():
    """MUL_MAT + ADD is fused only when the fused result does not overlap src1 (the fused record writes
    the ADD's result while src1 is read: tsr-build.h's "not read or written in between")."""
    p = Probe()
    c = p.c
    w = p.w(G.Q8_0, [256, 256], "w")
    x = p.a(G.F32, [256, 1])
    r = p.a(G.F32, [256, 1])
    mm = p.node(c.mul_mat(w, x))
    ad = c.add(mm, r)
    ad.data, ad.buffer = x.data, x.buffer                           # ggml-alloc reused src1's bytes
    calls = p.dev.lower([mm, ad])
    assert [k["name"] for k in calls] == ["MUL_MAT", "ADD"] and calls[0]["node2"] == -1
    ad2 = p.node(c.add(p.node(c.mul_mat(w, x)), r))
    calls = p.dev.lower(c.nodes[-2:])
    assert [k["name"] for k in calls] == ["MUL_MAT"] and calls[0]["node2"] == 1 and calls[0]["y"] == ad2.data
    # a MUL_MAT whose result has a second user is not fused
    mm3 = p.node(c.mul_mat(w, x))
    ad3 = p.node(c.add(mm3, r))
    other = p.node(c.add(mm3, r))
    calls = p.dev.lower([mm3, ad3, other])
    assert [k["name"] for k in calls] == ["MUL_MAT", "ADD", "ADD"]
    p.dev.close()


def test_softcap_and_scale_fusion():
    p = Probe()
    c = p.c
    w = p.w(G.Q8_0, [256, 1000], "output.weight")
    x = p.a(G.F32, [256, 1])
    mm = p.node(c.mul_mat(w, x))
    s1 = p.node(c.scale(mm, 1.0 / 30.0))
    th = p.node(c.tanh(s1))
    s2 = p.node(c.scale(th, 30.0))
    calls = p.dev.lower([mm, s1, th, s2])
    assert len(calls) == 1 and calls[0]["flags"] == tsr_hip.MM_SOFTCAP and calls[0]["y"] == s2.data
    assert np.float32(calls[0]["scale"]) == np.float32(1.0 / 30.0) and calls[0]["scale2"] == 30.0
    mm2 = p.node(c.mul_mat(w, x))
    sc = p.node(c.scale(mm2, 0.25))
    calls = p.dev.lower([mm2, sc])
    assert len(calls) == 1 and calls[0]["flags"] == tsr_hip.MM_SCALE and calls[0]["scale2"] == 0.25
    p.dev.close()


def test_graph_key_identity():
    """The plan cache's key (ggml-tesseract.cpp:3937): the same graph built again keys the same; a
    changed shape, address or op parameter keys differently; nothing of the values enters it."""
    cfg = LL.tiny_config()

    def build(n_kv, eps=None):
        p = Probe()
        W, caches = declare_model(p, cfg, 512)
        g = GL.LlamaGraph(p.dev, cfg, W, caches, 512, 1, n_kv)
        if eps is not None:
            g.ctx.nodes[1].op_params[0] = GL.f32_bits(eps)
        k = G.graph_key(g.ctx.nodes)
        p.dev.close()
        return k

    a = build(256)
    assert build(256) == a
    assert build(512) != a
    assert build(256, eps=1e-3) != a
    assert G.graph_key([], 1) != G.graph_key([], 2)


def test_buffer_reset_forgets_the_announced_layout():
    """buffer_i.reset (ggml-tesseract.cpp:2015-2024): a buffer laid out anew before its storage is
    decided is decided from the tensors announced after the reset only. Here the tensors announced
    after it are two KV caches, so the buffer becomes KV planes; the same announcements without the
    reset (a stray f32 tensor before them) give device memory. A probe device reports no memory."""
    dev = G.Device(-1)
    c = GL.Ctx()
    assert dev.memory() == (0, 0)
    wb = dev.buffer(1 << 20, G.USAGE_WEIGHTS)
    wt = c.new(G.Q8_0, [256, 16], "w")
    c.place(wt, wb, 0)
    modes = []
    for reset in (True, False):
        b = dev.buffer(1 << 20)
        c.place(c.new(G.F32, [256], "stray"), b, 0)
        if reset:
            b.reset()
        off = c.place(c.new(G.Q8_0, [256, 64, 1], "cache_k_l0"), b, 0)
        c.place(c.new(G.Q8_0, [256, 64, 1], "cache_v_l0"), b, off)
        assert b.mode == G.MODE_UNDECIDED
        x = c.new(G.F32, [256, 1], "x")                  # not announced: its address only
        x.data, x.buffer = b.base, b.h
        ok, why = dev.supports_op(c.mul_mat(wt, x))      # reading x's bytes decides the buffer's storage
        assert not ok
        modes.append(b.mode)
    assert modes == [G.MODE_KV, G.MODE_LINEAR]
    dev.close()


def test_probe_device_has_no_memory():
    p = Probe()
    t = p.a(G.F32, [16])
    with pytest.raises(G.GGError) as e:
        p.cbuf.set_tensor(t, np.zeros(16, np.float32))
    assert e.value.code == G.E_NODEV
    with pytest.raises(G.GGError):
        p.dev.graph_compute([p.node(p.c.add(t, t))])
    p.dev.close()


def test_msum_mask_f32_matches_oracle(oc, request):
    """The library's f32 mask copy (the GENERAL path's AMASK input, tsr_msum_mask_f32 sw/sim/
    tsr_ref_at.c:704-715) against the oracle's, bit for bit; and against the compiled reference's when
    it is built. Masks with finite values, +-0, -inf, +inf, NaN and fp16 subnormals; scales around 1."""
    rng = np.random.default_rng(3)
    specials = np.array([0x0000, 0x8000, 0xFC00, 0x7C00, 0x7E00, 0xFE01, 0x0001, 0x83FF, 0x3C00, 0xBC00, 0x7BFF,
                         0x0400], np.uint16)
    cases = [rng.choice(specials, size=(3, 77)).view(np.float16),
             rng.standard_normal((2, 130)).astype(np.float16),
             (rng.random((4, 33)) * 1e-5).astype(np.float16)]
    ref = None
    try:
        ref = request.getfixturevalue("ref")
    except pytest.skip.Exception:
        pass
    for m in cases:
        for s in (0.088388346, 1.0, 3.0e-3, 0.25):
            got = tsr_hip.msum_mask_f32(m, s)
            want = oc.mask_f32(m, np.float32(s))
            assert (got.view(np.uint32) == want.view(np.uint32)).all()
            if ref is not None:
                assert (got.view(np.uint32) == ref.mask_f32(m, np.float32(s)).view(np.uint32)).all()
    with pytest.raises(tsr_hip.TsrHipError):
        tsr_hip.msum_mask_f32(cases[0], -1.0)
