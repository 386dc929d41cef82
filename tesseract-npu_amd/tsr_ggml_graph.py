"""A small stand-in for ggml's graph construction, for driving libtsr_ggml where llama.cpp is absent
(the tests, the bench's adapter leg): tensors with ggml's shapes and byte strides (ggml.c's new_tensor /
view / reshape / permute rules: a view's view_src is the base tensor and its offset accumulates), op
nodes with ggml's op_params layout, a bump allocator over the adapter's buffers, and llama.cpp's Llama
graph (src/models/llama.cpp with FLASH_ATTN_EXT over a q8_0 cache: src/llama-graph.cpp build_attn_mha,
src/llama-kv-cache.cpp cpy_k / get_k)."""
from __future__ import annotations

import struct

import numpy as np

import tsr_ggml as G

BLOCK = {G.F32: (1, 4), G.F16: (1, 2), G.BF16: (1, 2), G.Q8_0: (32, 34), G.Q4_K: (256, 144), G.I32: (1, 4),
         G.I64: (1, 8)}


def f32_bits(v: float) -> int:
    return struct.unpack("<i", struct.pack("<f", float(v)))[0]


class Ctx:
    def __init__(self, blocks=None):
        self.tensors = []              # every record (kept alive: the C side holds pointers)
        self.nodes = []                # op nodes in creation order (a topological order)
        self.blocks = dict(BLOCK)
        if blocks:
            self.blocks.update(blocks)

    # ---- tensors ------------------------------------------------------------------------------
    def _rec(self, type_, ne, name, op=G.OP_NONE):
        t = G.Tensor()
        ne4 = list(ne) + [1] * (4 - len(ne))
        blck, ts = self.blocks[type_]
        t.type, t.op = type_, op
        for i in range(4):
            t.ne[i] = ne4[i]
        nb = [ts, ts * (ne4[0] // blck)]
        nb += [nb[1] * ne4[1], nb[1] * ne4[1] * ne4[2]]
        for i in range(4):
            t.nb[i] = nb[i]
        t.name = name.encode()[:63]
        self.tensors.append(t)
        return t

    def new(self, type_, ne, name, flags=0):
        t = self._rec(type_, ne, name)
        t.flags = flags
        return t

    def _node(self, t, srcs):
        for i, s in enumerate(srcs):
            if s is not None:
                t.src[i] = G.C.pointer(s)
        self.nodes.append(t)
        return t

    def _view(self, a, type_, ne, nb, offs, name, op):
        t = self._rec(type_, ne, name, op)
        for i in range(4):
            t.nb[i] = nb[i]
        base = a
        offs0 = offs
        if a.view_src:
            base = a.view_src.contents
            offs0 += a.view_offs
        t.view_src = G.C.pointer(base)
        t.view_offs = offs0
        return self._node(t, [a])

    # ---- views ----------------------------------------------------------------------------------
    def reshape(self, a, *ne):
        ne4 = list(ne) + [1] * (4 - len(ne))
        blck, ts = self.blocks[a.type]
        nb = [ts, ts * (ne4[0] // blck)]
        nb += [nb[1] * ne4[1], nb[1] * ne4[1] * ne4[2]]
        return self._view(a, a.type, ne4, nb, 0, a.name.decode() + " (reshaped)", G.OP_RESHAPE)

    def view(self, a, ne, nb123, offs, name=None):
        ne4 = list(ne) + [1] * (4 - len(ne))
        nb = [a.nb[0]] + list(nb123) + [0] * (3 - len(nb123))
        for i in range(len(nb123) + 1, 4):
            nb[i] = nb[i - 1] * ne4[i - 1]
        return self._view(a, a.type, ne4, nb, offs, name or a.name.decode() + " (view)", G.OP_VIEW)

    def permute(self, a, ax0, ax1, ax2, ax3):
        ne, nb = [0] * 4, [0] * 4
        for i, ax in enumerate((ax0, ax1, ax2, ax3)):
            ne[ax], nb[ax] = a.ne[i], a.nb[i]
        t = self._view(a, a.type, ne, nb, 0, a.name.decode() + " (permuted)", G.OP_PERMUTE)
        t.op_params[0], t.op_params[1], t.op_params[2], t.op_params[3] = ax0, ax1, ax2, ax3
        return t

    def view_tensor(self, a, op, name):
        return self._view(a, a.type, list(a.ne), list(a.nb), 0, name, op)

    # ---- ops ------------------------------------------------------------------------------------
    def mul_mat(self, a, b, name="mul_mat"):
        t = self._rec(G.F32, [a.ne[1], b.ne[1], b.ne[2], b.ne[3]], name, G.OP_MUL_MAT)
        return self._node(t, [a, b])

    def rms_norm(self, x, eps, name="norm"):
        t = self._rec(G.F32, list(x.ne), name, G.OP_RMS_NORM)
        t.op_params[0] = f32_bits(eps)
        return self._node(t, [x])

    def mul(self, a, b, name="mul"):
        return self._node(self._rec(G.F32, list(a.ne), name, G.OP_MUL), [a, b])

    def add(self, a, b, name="add"):
        return self._node(self._rec(G.F32, list(a.ne), name, G.OP_ADD), [a, b])

    def scale(self, a, s, name="scale"):
        t = self._rec(G.F32, list(a.ne), name, G.OP_SCALE)
        t.op_params[0], t.op_params[1] = f32_bits(s), f32_bits(0.0)
        return self._node(t, [a])

    def tanh(self, a, name="tanh"):
        t = self._rec(G.F32, list(a.ne), name, G.OP_UNARY)
        t.op_params[0] = G.UNARY_TANH
        return self._node(t, [a])

    def swiglu_split(self, g, u, name="ffn_swiglu"):
        t = self._rec(G.F32, list(g.ne), name, G.OP_GLU)
        t.op_params[0], t.op_params[1] = G.GLU_SWIGLU, 0
        return self._node(t, [g, u])

    def rope_ext(self, x, pos, n_dims, mode, freq_base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0,
                 ff=None, name="rope"):
        t = self._rec(G.F32, list(x.ne), name, G.OP_ROPE)
        t.op_params[1], t.op_params[2], t.op_params[4] = n_dims, mode, 0
        for i, v in enumerate((freq_base, freq_scale, ext_factor, attn_factor, 32.0, 1.0)):
            t.op_params[5 + i] = f32_bits(v)
        return self._node(t, [x, pos, ff])

    def get_rows(self, a, ids, name="get_rows"):
        return self._node(self._rec(G.F32, [a.ne[0], ids.ne[0], 1, 1], name, G.OP_GET_ROWS), [a, ids])

    def argmax(self, a, name="argmax"):
        return self._node(self._rec(G.I32, [a.ne[1]], name, G.OP_ARGMAX), [a])

    def set_rows(self, dst, rows, idx, name="set_rows"):
        t = self._view(dst, dst.type, list(dst.ne), list(dst.nb), 0, name, G.OP_SET_ROWS)
        t.src[0] = G.C.pointer(rows)
        t.src[1] = G.C.pointer(idx)
        return t

    def flash_attn_ext(self, q, k, v, mask, scale, max_bias=0.0, softcap=0.0, name="fattn"):
        t = self._rec(G.F32, [v.ne[0], q.ne[2], q.ne[1], q.ne[3]], name, G.OP_FLASH_ATTN_EXT)
        t.op_params[0], t.op_params[1], t.op_params[2] = f32_bits(scale), f32_bits(max_bias), f32_bits(softcap)
        t.op_params[3] = 10                                      # GGML_PREC_F32 (ggml_flash_attn_ext_set_prec)
        return self._node(t, [q, k, v, mask])

    # ---- allocation -----------------------------------------------------------------------------
    def nbytes(self, t) -> int:
        blck, ts = self.blocks[t.type]
        n = t.ne[0] // blck * ts
        for i in range(1, 4):
            n += (t.ne[i] - 1) * t.nb[i]
        return n

    def place(self, t, buf, off: int) -> int:
        """t at buf.base + off; returns the next 64-aligned offset."""
        t.data = buf.base + off
        t.buffer = buf.h
        buf.init_tensor(t)
        n = self.nbytes(t)
        return off + (n + 63) // 64 * 64

    def alloc_nodes(self, buf, off: int = 0) -> int:
        """Every op node that is not a view into buf (bump allocation, no reuse); views take their base
        tensor's data + offset."""
        for t in self.nodes:
            if not t.view_src:
                off = self.place(t, buf, off)
        for t in self.nodes:
            if t.view_src:
                b = t.view_src.contents
                t.data = b.data + t.view_offs
                t.buffer = b.buffer
        return off

    def node_bytes(self) -> int:
        return sum((self.nbytes(t) + 63) // 64 * 64 for t in self.nodes if not t.view_src)


class LlamaGraph:
    """llama.cpp's graph of a Llama decoder over T tokens at positions pos0 .. pos0 + T - 1, attending to
    n_kv cache cells, with the greedy token of the last row (ARGMAX) when argmax is set."""

    def __init__(self, dev: G.Device, cfg, weights: dict, caches: dict, kv_size: int, T: int, n_kv: int,
                 argmax: bool = False):
        c = Ctx()
        self.ctx, self.cfg, self.T, self.n_kv = c, cfg, T, n_kv
        D, H, Hk, E = cfg.head_dim, cfg.n_head, cfg.n_head_kv, cfg.E
        self.inp_tokens = c.new(G.I32, [T], "inp_tokens", G.FLAG_INPUT)
        self.inp_pos = c.new(G.I32, [T], "inp_pos", G.FLAG_INPUT)
        self.k_idxs = c.new(G.I64, [T], "inp_k_idxs", G.FLAG_INPUT)
        self.v_idxs = c.new(G.I64, [T], "inp_v_idxs", G.FLAG_INPUT)
        self.kq_mask = c.new(G.F16, [n_kv, T], "attn_inp_kq_mask", G.FLAG_INPUT)
        self.out_ids = c.new(G.I32, [1], "inp_out_ids", G.FLAG_INPUT)
        W = weights
        x = c.get_rows(W["token_embd.weight"], self.inp_tokens, "inp_embd")
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
        for il in range(cfg.n_layer):
            b = f"blk.{il}."
            inpSA = x
            cur = c.mul(c.rms_norm(x, cfg.eps, f"attn_norm-{il}"), W[b + "attn_norm.weight"], f"attn_norm-{il}")
            q = c.mul_mat(W[b + "attn_q.weight"], cur, f"Qcur-{il}")
            k = c.mul_mat(W[b + "attn_k.weight"], cur, f"Kcur-{il}")
            v = c.mul_mat(W[b + "attn_v.weight"], cur, f"Vcur-{il}")
            q = c.reshape(q, D, H, T)
            k = c.reshape(k, D, Hk, T)
            v = c.reshape(v, D, Hk, T)
            q = c.rope_ext(q, self.inp_pos, D, cfg.rope_mode, cfg.rope_base, name=f"Qcur-{il}")
            k = c.rope_ext(k, self.inp_pos, D, cfg.rope_mode, cfg.rope_base, name=f"Kcur-{il}")
            kc, vc = caches[f"cache_k_l{il}"], caches[f"cache_v_l{il}"]
            c.set_rows(kc, c.view(k, [E, T], [k.nb[2]], 0), self.k_idxs, f"k_set-{il}")
            c.set_rows(vc, c.view(v, [E, T], [v.nb[2]], 0), self.v_idxs, f"v_set-{il}")
            qp = c.permute(q, 0, 2, 1, 3)
            row = E // 32 * 34
            kv4 = [D // 32 * 34, row, row * kv_size]
            kp = c.permute(c.view(kc, [D, Hk, n_kv, 1], kv4, 0), 0, 2, 1, 3)
            vp = c.permute(c.view(vc, [D, Hk, n_kv, 1], kv4, 0), 0, 2, 1, 3)
            att = c.flash_attn_ext(qp, kp, vp, self.kq_mask, scale, name=f"__fattn__-{il}")
            att = c.reshape(att, D * H, T)
            cur = c.mul_mat(W[b + "attn_output.weight"], att, f"attn_out-{il}")
            if il == cfg.n_layer - 1:
                cur = c.get_rows(cur, self.out_ids, f"attn_out_rows-{il}")
                inpSA = c.get_rows(inpSA, self.out_ids, f"inpSA_rows-{il}")
            ffn_inp = c.add(cur, inpSA, f"ffn_inp-{il}")
            cur = c.mul(c.rms_norm(ffn_inp, cfg.eps, f"ffn_norm-{il}"), W[b + "ffn_norm.weight"], f"ffn_norm-{il}")
            g = c.mul_mat(W[b + "ffn_gate.weight"], cur, f"ffn_gate-{il}")
            u = c.mul_mat(W[b + "ffn_up.weight"], cur, f"ffn_up-{il}")
            cur = c.mul_mat(W[b + "ffn_down.weight"], c.swiglu_split(g, u, f"ffn_swiglu-{il}"), f"ffn_out-{il}")
            x = c.add(cur, ffn_inp, f"l_out-{il}")
        cur = c.mul(c.rms_norm(x, cfg.eps, "result_norm"), W["output_norm.weight"], "result_norm")
        self.logits = c.mul_mat(W["output.weight"], cur, "result_output")
        self.logits.flags |= G.FLAG_OUTPUT
        self.next = c.argmax(self.logits, "result_argmax") if argmax else None
        # the compute buffer: inputs, then every op result
        leaves = [self.inp_tokens, self.inp_pos, self.k_idxs, self.v_idxs, self.kq_mask, self.out_ids]
        size = sum((c.nbytes(t) + 63) // 64 * 64 for t in leaves) + c.node_bytes()
        self.buf = dev.buffer(size, G.USAGE_COMPUTE)
        off = 0
        for t in leaves:
            off = c.place(t, self.buf, off)
        c.alloc_nodes(self.buf, off)

    def set_inputs(self, tokens, pos0: int) -> None:
        T, n_kv = self.T, self.n_kv
        tokens = np.asarray(tokens, np.int32)
        pos = pos0 + np.arange(T, dtype=np.int32)
        b = self.buf
        b.set_tensor(self.inp_tokens, tokens)
        b.set_tensor(self.inp_pos, pos)
        b.set_tensor(self.k_idxs, pos.astype(np.int64))
        b.set_tensor(self.v_idxs, pos.astype(np.int64))
        m = np.full((T, n_kv), -np.inf, np.float16)
        for r in range(T):
            m[r, :pos0 + r + 1] = 0.0
        b.set_tensor(self.kq_mask, m)
        b.set_tensor(self.out_ids, np.array([T - 1], np.int32))

    def set_position(self, pos0: int) -> None:
        """The inputs of a step at positions pos0 .. pos0 + T - 1 but the token ids (a decode loop that
        feeds the greedy token on the device)."""
        T, n_kv = self.T, self.n_kv
        pos = pos0 + np.arange(T, dtype=np.int32)
        b = self.buf
        b.set_tensor(self.inp_pos, pos)
        b.set_tensor(self.k_idxs, pos.astype(np.int64))
        b.set_tensor(self.v_idxs, pos.astype(np.int64))
        m = np.full((T, n_kv), -np.inf, np.float16)
        for r in range(T):
            m[r, :pos0 + r + 1] = 0.0
        b.set_tensor(self.kq_mask, m)

    def logits_host(self) -> np.ndarray:
        return self.buf.get_tensor(self.logits, 4 * self.cfg.n_vocab).view(np.float32)

    def free(self) -> None:
        self.buf.free()


def load_model(dev: G.Device, cfg, w, kv_size: int, images=None):
    """The weights (one weights buffer, ggml blocks) and the KV caches (one buffer of cache_k_l<n> /
    cache_v_l<n> q8_0 tensors, cleared, then images[(layer, 0 | 1)] written from cell 0 as ggml q8_0
    rows)."""
    import tsr_llama as LL
    c = Ctx()
    fmt = {0: G.Q8_0, 1: G.Q4_K}
    tens, data = {}, {}

    def add_w(name, type_, ne, arr):
        tens[name] = c.new(type_, ne, name)
        data[name] = np.ascontiguousarray(arr)

    add_w("token_embd.weight", G.F32, [cfg.n_embd, cfg.n_vocab], w.embedding())
    add_w("output_norm.weight", G.F32, [cfg.n_embd], w.norm("output_norm.weight"))
    add_w("output.weight", fmt[cfg.ofmt], [cfg.n_embd, cfg.n_vocab], w.quant("output.weight", cfg.n_vocab, cfg.n_embd, cfg.ofmt))
    for il in range(cfg.n_layer):
        for name, N, K in LL.layer_tensors(cfg, il):
            add_w(name, fmt[cfg.wfmt], [K, N], w.quant(name, N, K, cfg.wfmt))
        for nm in ("attn_norm", "ffn_norm"):
            add_w(f"blk.{il}.{nm}.weight", G.F32, [cfg.n_embd], w.norm(f"blk.{il}.{nm}.weight"))
    wbuf = dev.buffer(sum((c.nbytes(t) + 63) // 64 * 64 for t in tens.values()), G.USAGE_WEIGHTS)
    off = 0
    for name, t in tens.items():
        off = c.place(t, wbuf, off)
    for name, t in tens.items():
        wbuf.set_tensor(t, data[name])
    caches = {}
    row = cfg.E // 32 * 34
    kvbuf = dev.buffer(2 * cfg.n_layer * row * kv_size + 64 * 2 * cfg.n_layer, G.USAGE_ANY)
    off = 0
    for il in range(cfg.n_layer):
        for which in "kv":
            t = c.new(G.Q8_0, [cfg.E, kv_size, 1], f"cache_{which}_l{il}")
            caches[t.name.decode()] = t
            off = c.place(t, kvbuf, off)
    kvbuf.clear(0)
    for (il, which), img in (images or {}).items():
        kvbuf.set_tensor(caches[f"cache_{'kv'[which]}_l{il}"], np.ascontiguousarray(img, np.uint8))
    return c, tens, caches, wbuf, kvbuf
