"""A Llama-architecture decoder built from libtsr_hip's C-ABI ops: the caller side of the hot path,
in the role llama.cpp's build_llama graph plays for the reference's backend.

One decode step (T = 1) runs the op list of the reference's decoder-layer test
(sw/ctrl/tests/test_fw_m7_layer.cpp:646-686, the non-Gemma branch), layer by layer:

    Xn  = RMS_NORM(X) * attn_norm                     (RMS_NORM + MUL)
    Q|K|V = MUL_MAT(Wq|Wk|Wv, Xn)                     (one launch over the concatenated rows)
    Q, K  = ROPE(Q), ROPE(K)                          (one launch over the q and k heads)
    SET_ROWS_KV(K cache, K, pos), SET_ROWS_KV(V cache, V, pos)
    A   = FLASH_ATTN_EXT(Q, K cache, V cache, cells [0, pos], new cell pos), scale 1/sqrt(D)
    H   = MUL_MAT(Wo, A) + X                          (MUL_MAT with the residual addend)
    Hn  = RMS_NORM(H) * ffn_norm
    G|U = MUL_MAT(Wgate|Wup, Hn)                      (one launch over the concatenated rows)
    X   = MUL_MAT(Wdown, SWIGLU(G, U)) + H

then logits = MUL_MAT(Woutput, RMS_NORM(X) * output_norm) and the greedy token is the ARGMAX.

With fused=True (the default) RMS_NORM + MUL runs inside the Q|K|V and gate|up MUL_MATs
(tsr_hip_mul_mat_norm), SWIGLU in the epilogue of the gate|up MUL_MAT (TSR_HIP_MM_GLU over gate / up
rows interleaved), and ROPE with both SET_ROWS_KV inside the planned FLASH_ATTN_EXT
(tsr_hip_flash_attn_plan_rope_tab, the angles of the token's position made once per token by
tsr_hip_rope_table; eager steps, planned on the host, use tsr_hip_rope_kv), and with the planned form
the Q|K|V MUL_MAT joins that launch too (tsr_hip_attn_qkv_plan_rope_tab: one launch where each KV head's
workgroups share an XCD, else the two calls): at the Llama-3-8B shape a layer is four launches, each
fusion bit-identical to the ops it replaces. fused=False runs every op of the list as its own call.
The token embedding is a GET_ROWS of an f32 table. Row concatenation leaves every row's result
unchanged (each output row is its own dot product with the same quantized activation), and ROPE
of q and k heads in one launch is the same per-head rotation. A residual addend is one FA(add, v),
the ADD of the reference's fused "attn_out + inpSA" / "ffn_out + ffn_inp" records.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import numpy as np

import tsr_hip as H
import tsr_synth as S


class DecodeError(RuntimeError):
    """A decode launch raised the decoder's index / wait flag (LlamaDecoder.check)."""


@dataclass(frozen=True)
class LlamaConfig:
    name: str
    n_layer: int
    n_embd: int
    n_ff: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_vocab: int
    eps: float = 1e-5
    rope_base: float = 500000.0
    rope_mode: int = H.ROPE_NORMAL
    wfmt: int = H.FMT_Q4_K           # layer weights
    ofmt: int = H.FMT_Q4_K           # output head
    std: float = 0.02

    @property
    def E(self) -> int:
        return self.n_head_kv * self.head_dim

    @property
    def n_q(self) -> int:
        return self.n_head * self.head_dim

    def weight_bytes_per_token(self) -> int:
        """Quantized weight bytes one decode token reads (layers + output head), ggml block sizes."""
        def qb(fmt, N, K):
            return N * (K // 32 * 34 if fmt == H.FMT_Q8_0 else K // 256 * 144)
        per_layer = (qb(self.wfmt, self.n_q + 2 * self.E, self.n_embd) + qb(self.wfmt, self.n_embd, self.n_q) +
                     qb(self.wfmt, 2 * self.n_ff, self.n_embd) + qb(self.wfmt, self.n_embd, self.n_ff))
        return self.n_layer * per_layer + qb(self.ofmt, self.n_vocab, self.n_embd)


LLAMA3_8B = LlamaConfig("llama3-8b", 32, 4096, 14336, 32, 8, 128, 128256)


def tensor_seed(cfg: LlamaConfig, name: str) -> int:
    return S.seed_of(cfg.name, name)


def layer_tensors(cfg: LlamaConfig, il: int):
    """(name, N, K) of the quantized tensors of layer il, in ggml's GGUF names."""
    d, q, E, ff = cfg.n_embd, cfg.n_q, cfg.E, cfg.n_ff
    return [(f"blk.{il}.attn_q.weight", q, d), (f"blk.{il}.attn_k.weight", E, d), (f"blk.{il}.attn_v.weight", E, d),
            (f"blk.{il}.attn_output.weight", d, q), (f"blk.{il}.ffn_gate.weight", ff, d),
            (f"blk.{il}.ffn_up.weight", ff, d), (f"blk.{il}.ffn_down.weight", d, ff)]


class SyntheticWeights:
    """Seeded random-init weights: every quantized tensor is normal(seed_of(config, name), std) rows
    quantized to the config's format; norms are f32 N(1, 0.1); the token embedding is f32 N(0, 1)
    rows (the lookup copies rows bit for bit). Values depend only on (config name, tensor name).
    cache=True keeps every generated tensor on the host, so that a GPU model and a CPU checker built
    from the same object see the same arrays without generating them twice."""

    def __init__(self, cfg: LlamaConfig, cache: bool = False):
        self.cfg = cfg
        self.cache = {} if cache else None

    def _kept(self, key, make):
        if self.cache is None:
            return make()
        if key not in self.cache:
            self.cache[key] = make()
        return self.cache[key]

    def quant(self, name: str, N: int, K: int, fmt: int) -> np.ndarray:
        return self._kept((name, fmt), lambda: S.quant_rows(fmt, tensor_seed(self.cfg, name), N, K, self.cfg.std))

    def norm(self, name: str) -> np.ndarray:
        return self._kept(name, lambda: (1.0 + S.normal(tensor_seed(self.cfg, name), self.cfg.n_embd, 0.1))
                          .astype(np.float32))

    def embedding(self) -> np.ndarray:
        c = self.cfg
        return self._kept("token_embd.weight", lambda: S.normal(tensor_seed(c, "token_embd.weight"), c.n_vocab * c.n_embd,
                                                                1.0).reshape(c.n_vocab, c.n_embd))

    def kv_history(self, il: int, which: int, n: int) -> np.ndarray:
        """f32 rows [n, E] quantized into cells 0 .. n-1 before decoding (the prefilled context)."""
        c = self.cfg
        return S.normal(tensor_seed(c, f"kv_history.{il}.{which}"), n * c.E, 1.0).reshape(n, c.E)


def msum_decode(pos: int, n_kv: int) -> np.ndarray:
    """MSUM words of a one-row decode mask that sees cells [0, pos] of a mask n_kv cells wide (llama.cpp's
    kq_mask: 0 over the used cells, -inf elsewhere), the form tsr_hip_msum_build_f16 gives."""
    return msum_causal(pos, 1, n_kv)


def msum_causal(pos0: int, T: int, n_kv: int) -> np.ndarray:
    """MSUM words of the causal mask of a ubatch of T tokens at cells pos0 .. pos0 + T - 1: row t sees
    cells [0, pos0 + t] (one FAST run per row, the form tsr_hip_msum_build_f16 gives for llama.cpp's
    kq_mask over a cache)."""
    w = np.zeros(8 + 4 * T, np.uint32)
    w[0], w[1], w[2] = 0x4D55534D, T, n_kv
    w[9::4] = pos0 + 1 + np.arange(T, dtype=np.uint32)
    return w


class LlamaDecoder:
    """The model on one device: weights uploaded once, one q8_0 K and V cache per layer of kv_size
    cells, and the activation buffers of one decode token."""

    def __init__(self, dev: H.Device, cfg: LlamaConfig, weights: SyntheticWeights, kv_size: int, fused: bool = True,
                 qkv_in_attn: bool = True):
        self.dev, self.cfg, self.kv_size = dev, cfg, kv_size
        self.fused = fused
        self.qkv_in_attn = qkv_in_attn     # planned decode: the Q|K|V MUL_MAT inside the attention launch
        c = cfg
        f4 = 4
        self.tok_embd = dev.upload(np.ascontiguousarray(weights.embedding(), np.float32))
        self.layers = []
        for il in range(c.n_layer):
            t = {name.split(".")[2]: weights.quant(name, N, K, c.wfmt) for name, N, K in layer_tensors(c, il)}
            L = {
                "attn_norm": dev.upload(weights.norm(f"blk.{il}.attn_norm.weight")),
                "ffn_norm": dev.upload(weights.norm(f"blk.{il}.ffn_norm.weight")),
                "wqkv": dev.weight(c.wfmt, np.concatenate([t["attn_q"], t["attn_k"], t["attn_v"]]), c.n_q + 2 * c.E,
                                   c.n_embd),
                "wo": dev.weight(c.wfmt, t["attn_output"], c.n_embd, c.n_q),
                # fused: gate / up rows interleaved (row 2j = gate j, 2j + 1 = up j) for the GLU epilogue
                "wgu": dev.weight(c.wfmt, np.stack([t["ffn_gate"], t["ffn_up"]], axis=1).reshape(2 * c.n_ff, -1)
                                  if fused else np.concatenate([t["ffn_gate"], t["ffn_up"]]), 2 * c.n_ff, c.n_embd),
                "wd": dev.weight(c.wfmt, t["ffn_down"], c.n_embd, c.n_ff),
                "kc": dev.kv(c.E, kv_size),
                "vc": dev.kv(c.E, kv_size),
            }
            del t
            self.layers.append(L)
        self.out_norm = dev.upload(weights.norm("output_norm.weight"))
        self.wout = dev.weight(c.ofmt, weights.quant("output.weight", c.n_vocab, c.n_embd, c.ofmt), c.n_vocab, c.n_embd)
        # activations of one token
        self.x = dev.alloc(c.n_embd * f4)
        self.h = dev.alloc(c.n_embd * f4)
        self.xn = dev.alloc(c.n_embd * f4)
        self.qkv = dev.alloc((c.n_q + 2 * c.E) * f4)
        self.att = dev.alloc(c.n_q * f4)
        self.gu = dev.alloc(2 * c.n_ff * f4)
        self.glu = dev.alloc(c.n_ff * f4)
        self.logits = dev.alloc(c.n_vocab * f4)
        self.tok = dev.alloc(4)            # int32 token id of the step (GET_ROWS ids)
        self.next = dev.alloc(4)           # int32 greedy token (ARGMAX) of an eager step
        self.params = dev.alloc(16)        # int32 position (ROPE) at 0, int64 cell (SET_ROWS_KV) at 8
        self.bad = dev.alloc(4).fill(0)
        self.rtab = dev.alloc(4 * c.head_dim)  # ROPE angles of the token's position (tsr_hip_rope_table)
        self.scale = 1.0 / math.sqrt(c.head_dim)
        self.plan = dev.fa_plan(c.head_dim, c.n_head, c.n_head_kv, 1, kv_size)
        # the planned FLASH_ATTN_EXT can take the ROPE + SET_ROWS_KV (tsr_hip_flash_attn_plan_rope) at these shapes
        self.fa_rope = (c.head_dim in (64, 128) and (c.n_head // c.n_head_kv + 2) * c.head_dim <= 1024 and
                        c.head_dim % 8 == 0)
        self.graph = None
        self.captures = 0
        self._pf = None                    # activations of a prefill ubatch (prefill)

    @property
    def pos_ptr(self) -> int:
        return self.params.ptr

    @property
    def cell_ptr(self) -> int:
        return self.params.ptr + 8

    def prefill_history(self, weights: SyntheticWeights, n: int) -> None:
        """Cells 0 .. n-1 of every cache hold QACT'd rows of weights.kv_history (SET_ROWS_KV)."""
        idx = self.dev.upload(np.arange(n, dtype=np.int64))
        for il, L in enumerate(self.layers):
            for which, kv in ((0, L["kc"]), (1, L["vc"])):
                rows = self.dev.upload(np.ascontiguousarray(weights.kv_history(il, which, n), np.float32))
                self.dev.kv_set_rows(kv, which, rows, n, self.cfg.E, idx, self.bad)
                rows.free()
        self.dev.sync()

    def _prefill_buffers(self, U: int) -> dict:
        """Activations of a ubatch of U tokens (allocated on first use, grown when a larger one comes)."""
        if self._pf is not None and self._pf["U"] >= U:
            return self._pf
        if self._pf is not None:
            for k, b in self._pf.items():
                if k != "U":
                    b.free()
        c, d, f4 = self.cfg, self.dev, 4
        self._pf = {"U": U, "x": d.alloc(U * c.n_embd * f4), "h": d.alloc(U * c.n_embd * f4),
                    "xn": d.alloc(U * c.n_embd * f4), "qkv": d.alloc(U * (c.n_q + 2 * c.E) * f4),
                    "att": d.alloc(U * c.n_q * f4), "gu": d.alloc(U * 2 * c.n_ff * f4),
                    "glu": d.alloc(U * c.n_ff * f4), "ids": d.alloc(U * 4), "pos": d.alloc(U * 4),
                    "cell": d.alloc(U * 8)}
        return self._pf

    def prefill(self, tokens, pos0: int = 0, ubatch: int = 512) -> None:
        """The prompt tokens at positions (= cells) pos0, pos0 + 1, ... in ubatches of at most `ubatch`
        tokens, each ubatch one pass of the layers over all its tokens (llama.cpp's llama_decode of a
        ubatch): every MUL_MAT over the ubatch's rows, ROPE + SET_ROWS_KV of its cells, FLASH_ATTN_EXT
        with the causal mask (row t sees cells [0, pos0 + t]; the ubatch's cells planned newest last).
        The last token's logits end in self.logits and its greedy token in self.next and self.tok (the
        input of a following step_graph(None, ...))."""
        toks = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        if toks.size == 0:
            raise ValueError("prefill of no tokens")
        if pos0 < 0 or pos0 + toks.size > self.kv_size:
            raise ValueError(f"positions {pos0} .. {pos0 + toks.size - 1} outside the cache of {self.kv_size} cells")
        for u0 in range(0, toks.size, ubatch):
            self._prefill_ubatch(toks[u0:u0 + ubatch], pos0 + u0)
        c, d = self.cfg, self.dev
        pf, n = self._pf, c.n_embd
        last = pf["x"].ptr + ((toks.size - 1) % ubatch) * n * 4
        if self.fused:
            d.mul_mat_norm(self.wout, last, 1, n, c.eps, self.out_norm, self.logits, c.n_vocab)
        else:
            d.rms_norm(last, n, 1, n, c.eps, self.xn, n, w=self.out_norm, w_stride=n)
            d.mul_mat(self.wout, self.xn, 1, n, self.logits, c.n_vocab)
        d.argmax(self.logits, c.n_vocab, 1, c.n_vocab, self.next)
        d.copy_async(self.tok, self.next, 4)
        d.sync()

    def _prefill_ubatch(self, toks: np.ndarray, pos0: int) -> None:
        c, d = self.cfg, self.dev
        T, nq, E, n, ff = toks.size, c.n_q, c.E, c.n_embd, c.n_ff
        w3, f4 = nq + 2 * E, 4
        pf = self._prefill_buffers(T)
        x, h, xn, qkv, att, gu, glu = (pf[k] for k in ("x", "h", "xn", "qkv", "att", "gu", "glu"))
        pos = pos0 + np.arange(T, dtype=np.int64)
        pf["ids"].write(toks)
        pf["pos"].write(pos.astype(np.int32))
        pf["cell"].write(pos)
        n_kv = min(self.kv_size, (pos0 + T + 255) // 256 * 256)
        msum, runs = msum_causal(pos0, T, n_kv), np.array([[pos0, pos0 + T]], np.uint32)
        # 16 or more tokens run the MUL_MATs on the matrix cores, which take no fused RMS_NORM: there the
        # norm is its own launch (the same operations); Q4_K's matrix-core path has the GLU epilogue,
        # Q8_0's has none, so a fused Q8_0 model takes its norm / GLU matvecs 15 tokens at a time
        mma = c.wfmt == H.FMT_Q4_K and T >= 16
        step = 15 if c.wfmt == H.FMT_Q8_0 else T

        def fused_rows(fn):
            for t0 in range(0, T, step):
                fn(t0, min(step, T - t0))

        d.get_rows(self.tok_embd, n, n, c.n_vocab, pf["ids"], T, x, n, bad=self.bad)
        for L in self.layers:
            if self.fused:
                if mma:
                    d.rms_norm(x, n, T, n, c.eps, xn, n, w=L["attn_norm"], w_stride=n)
                    d.mul_mat(L["wqkv"], xn, T, n, qkv, w3)
                else:
                    fused_rows(lambda t0, tt: d.mul_mat_norm(L["wqkv"], x.ptr + t0 * n * f4, tt, n, c.eps,
                                                             L["attn_norm"], qkv.ptr + t0 * w3 * f4, w3))
                d.rope_kv(qkv, T, w3, c.head_dim, c.n_head, c.n_head_kv, c.head_dim, c.rope_mode, pf["pos"],
                          c.rope_base, L["kc"], L["vc"], pf["cell"], self.bad)
            else:
                d.rms_norm(x, n, T, n, c.eps, xn, n, w=L["attn_norm"], w_stride=n)
                d.mul_mat(L["wqkv"], xn, T, n, qkv, w3)
                d.rope(qkv, T, w3, c.head_dim, c.n_head + c.n_head_kv, c.head_dim, c.rope_mode, pf["pos"],
                       c.rope_base, qkv, w3)
                d.kv_set_rows(L["kc"], 0, qkv.ptr + nq * f4, T, w3, pf["cell"], self.bad)
                d.kv_set_rows(L["vc"], 1, qkv.ptr + (nq + E) * f4, T, w3, pf["cell"], self.bad)
            d.flash_attn(qkv, T, w3, L["kc"], L["vc"], c.head_dim, c.n_head, c.n_head_kv, self.scale, msum, att, nq,
                         new_runs=runs)
            d.mul_mat(L["wo"], att, T, nq, h, n, add=x, add_stride=n)
            if self.fused and mma:
                d.rms_norm(h, n, T, n, c.eps, xn, n, w=L["ffn_norm"], w_stride=n)
                d.mul_mat(L["wgu"], xn, T, n, glu, ff, flags=H.MM_GLU)
            elif self.fused:
                fused_rows(lambda t0, tt: d.mul_mat_norm(L["wgu"], h.ptr + t0 * n * f4, tt, n, c.eps, L["ffn_norm"],
                                                         glu.ptr + t0 * ff * f4, ff, flags=H.MM_GLU))
            else:
                d.rms_norm(h, n, T, n, c.eps, xn, n, w=L["ffn_norm"], w_stride=n)
                d.mul_mat(L["wgu"], xn, T, n, gu, 2 * ff)
                d.swiglu(gu, 2 * ff, gu.ptr + ff * f4, 2 * ff, ff, T, glu, ff)
            d.mul_mat(L["wd"], glu, T, ff, x, n, add=h, add_stride=n)

    def _mask(self, pos: int, n_kv: int | None):
        if not 0 <= pos < self.kv_size:
            raise ValueError(f"position {pos} outside the cache of {self.kv_size} cells")
        if n_kv is None:
            n_kv = min(self.kv_size, (pos + 1 + 255) // 256 * 256)
        return msum_decode(pos, n_kv), np.array([[pos, pos + 1]], np.uint32)

    @staticmethod
    def _params(pos: int) -> np.ndarray:
        p = np.zeros(2, np.int64)
        p[1] = pos
        v = p.view(np.int32)
        v[0] = pos
        return p

    def _ops(self, out_tok, msum=None, runs=None, stream=None) -> None:
        """The launches of one decode token. msum given: FLASH_ATTN_EXT planned on the host per call
        (eager); else the device-resident plan (capturable)."""
        c, d = self.cfg, self.dev
        nq, E, n = c.n_q, c.E, c.n_embd
        f4 = 4
        d.get_rows(self.tok_embd, n, n, c.n_vocab, self.tok, 1, self.x, n, bad=self.bad, stream=stream)
        w3 = nq + 2 * E
        fa_tab = self.fused and msum is None and self.fa_rope
        if fa_tab:                                                # the position's angles, once per token
            d.rope_table(self.pos_ptr, c.head_dim, c.rope_base, self.rtab, stream=stream)
        for L in self.layers:
            fa_done = False
            if fa_tab and self.qkv_in_attn:                       # Q|K|V, ROPE, SET_ROWS_KV and FA: one call
                d.attn_qkv_plan_rope_tab(self.plan, L["wqkv"], self.x, c.eps, L["attn_norm"], self.qkv, L["kc"],
                                         L["vc"], self.scale, c.head_dim, c.rope_mode, self.rtab, self.cell_ptr,
                                         self.att, nq, bad=self.bad, stream=stream)
                fa_done = True
            elif self.fused:
                d.mul_mat_norm(L["wqkv"], self.x, 1, n, c.eps, L["attn_norm"], self.qkv, w3, stream=stream)
                if fa_tab:                                        # ROPE + SET_ROWS_KV inside the FA launch
                    d.flash_attn_plan_rope_tab(self.plan, self.qkv, L["kc"], L["vc"], self.scale, c.head_dim,
                                               c.rope_mode, self.rtab, self.cell_ptr, self.att, nq, bad=self.bad,
                                               stream=stream)
                    fa_done = True
                else:
                    d.rope_kv(self.qkv, 1, w3, c.head_dim, c.n_head, c.n_head_kv, c.head_dim, c.rope_mode,
                              self.pos_ptr, c.rope_base, L["kc"], L["vc"], self.cell_ptr, self.bad, stream=stream)
            else:
                d.rms_norm(self.x, n, 1, n, c.eps, self.xn, n, w=L["attn_norm"], w_stride=n, stream=stream)
                d.mul_mat(L["wqkv"], self.xn, 1, n, self.qkv, w3, stream=stream)
                d.rope(self.qkv, 1, w3, c.head_dim, c.n_head + c.n_head_kv, c.head_dim, c.rope_mode, self.pos_ptr,
                       c.rope_base, self.qkv, w3, stream=stream)
                d.kv_set_rows(L["kc"], 0, self.qkv.ptr + nq * f4, 1, E, self.cell_ptr, self.bad, stream=stream)
                d.kv_set_rows(L["vc"], 1, self.qkv.ptr + (nq + E) * f4, 1, E, self.cell_ptr, self.bad, stream=stream)
            if fa_done:
                pass
            elif msum is not None:
                d.flash_attn(self.qkv, 1, w3, L["kc"], L["vc"], c.head_dim, c.n_head, c.n_head_kv, self.scale,
                             msum, self.att, nq, new_runs=runs, stream=stream)
            else:
                d.flash_attn_plan(self.plan, self.qkv, w3, L["kc"], L["vc"], self.scale, self.att, nq, stream=stream)
            d.mul_mat(L["wo"], self.att, 1, nq, self.h, n, add=self.x, add_stride=n, stream=stream)
            if self.fused:
                d.mul_mat_norm(L["wgu"], self.h, 1, n, c.eps, L["ffn_norm"], self.glu, c.n_ff, flags=H.MM_GLU,
                               stream=stream)
                d.mul_mat(L["wd"], self.glu, 1, c.n_ff, self.x, n, add=self.h, add_stride=n, stream=stream)
            else:
                d.rms_norm(self.h, n, 1, n, c.eps, self.xn, n, w=L["ffn_norm"], w_stride=n, stream=stream)
                d.mul_mat(L["wgu"], self.xn, 1, n, self.gu, 2 * c.n_ff, stream=stream)
                d.swiglu(self.gu, 2 * c.n_ff, self.gu.ptr + c.n_ff * f4, 2 * c.n_ff, c.n_ff, 1, self.glu, c.n_ff,
                         stream=stream)
                d.mul_mat(L["wd"], self.glu, 1, c.n_ff, self.x, n, add=self.h, add_stride=n, stream=stream)
        if self.fused:
            d.mul_mat_norm(self.wout, self.x, 1, n, c.eps, self.out_norm, self.logits, c.n_vocab, stream=stream)
        else:
            d.rms_norm(self.x, n, 1, n, c.eps, self.xn, n, w=self.out_norm, w_stride=n, stream=stream)
            d.mul_mat(self.wout, self.xn, 1, n, self.logits, c.n_vocab, stream=stream)
        d.argmax(self.logits, c.n_vocab, 1, c.n_vocab, out_tok, stream=stream)

    def step(self, token: int | None, pos: int, n_kv: int | None = None) -> None:
        """One eager decode token at position pos (cell pos): every op a separate call, FLASH_ATTN_EXT
        planned per call. token: the id to embed, or None for the previous step's greedy token. Logits
        end in self.logits, the greedy token in self.next. n_kv: the mask width (default pos + 1
        rounded up to 256, at most kv_size)."""
        msum, runs = self._mask(pos, n_kv)
        self.tok.write(np.array([token], np.int32) if token is not None else self.next.read(np.int32, (1,)))
        self.params.write(self._params(pos))
        self._ops(self.next, msum, runs)

    def step_graph(self, token: int | None, pos: int, n_kv: int | None = None) -> None:
        """One decode token as one graph replay. Per token the host only plans the attention chunks and
        queues two small stream-ordered copies (position / cell and the plan); the greedy token of the
        previous replay is embedded from the device (token None). The graph is captured on the first
        call and again whenever the plan's shape changes. Nothing waits for the device."""
        d = self.dev
        msum, runs = self._mask(pos, n_kv)
        if token is not None:
            d.write_async(self.tok, np.array([token], np.int32))
        d.write_async(self.params, self._params(pos))
        changed = self.plan.set(msum, runs)
        if self.graph is None or changed:
            if self.graph is not None:
                self.graph.free()
            d.graph_begin()
            try:
                self._ops(self.tok)
            finally:
                g = d.graph_end()
            self.graph = g
            self.captures += 1
        self.graph.launch()

    def step_async(self, token: int | None, pos: int, n_kv: int | None = None) -> None:
        """The launches of step_graph issued directly (no graph): the device-resident plan, the
        position / cell and the plan copied in stream order, the greedy token fed back on the device.
        Nothing waits for the device."""
        d = self.dev
        msum, runs = self._mask(pos, n_kv)
        if token is not None:
            d.write_async(self.tok, np.array([token], np.int32))
        d.write_async(self.params, self._params(pos))
        self.plan.set(msum, runs)
        self._ops(self.tok)

    def generate_graph(self, first_token: int, pos0: int, n_tokens: int, hist=None, check: bool = True) -> None:
        """Greedy decode of n_tokens by graph replays, queued without waiting for the device; the token
        generated at step i is copied to hist[i] (a device int32 buffer) when given. With check, the
        batch ends with check() (one wait for the device, DecodeError on a raised flag)."""
        for i in range(n_tokens):
            self.step_graph(first_token if i == 0 else None, pos0 + i)
            if hist is not None:
                self.dev.copy_async(hist.ptr + 4 * i, self.tok, 4)
        if check:
            self.check()

    BAD_RANGE, BAD_WAIT, BAD_XCD = 1, 2, 4

    def check(self) -> None:
        """Wait for the device, then raise DecodeError if a launch since the last check raised the
        decoder's flag: bit 0, a token id or cache cell was out of range (GET_ROWS / SET_ROWS_KV stored
        nothing); bit 1, a bounded wait of the one-launch FLASH_ATTN_EXT expired; bit 2, one of its
        workgroups ran on another XCD than its KV head's (for bits 1 and 2 the attention output is not
        valid). The flag is cleared when it is reported."""
        self.dev.sync()
        bad = int(self.bad.read(np.int32, (1,))[0])
        if bad == 0:
            return
        self.bad.fill(0)
        why = []
        if bad & self.BAD_RANGE:
            why.append("a token id or cache cell was out of range")
        if bad & self.BAD_WAIT:
            why.append("a wait of the one-launch FLASH_ATTN_EXT expired (attention not valid)")
        if bad & self.BAD_XCD:
            why.append("a workgroup of the one-launch FLASH_ATTN_EXT ran on another XCD than its KV head's "
                       "(attention not valid)")
        raise DecodeError(f"decode flag {bad}: " + "; ".join(why or ["unknown code"]))

    def read_logits(self) -> np.ndarray:
        """The logits of the last step (checked: raises DecodeError on a raised flag)."""
        self.check()
        return self.logits.read(np.float32, (self.cfg.n_vocab,))

    def read_next(self) -> int:
        """The greedy token of the last eager step (checked)."""
        self.check()
        return int(self.next.read(np.int32, (1,))[0])

    def read_token(self) -> int:
        """The greedy token of the last graph replay (it is also the next replay's input; checked)."""
        self.check()
        return int(self.tok.read(np.int32, (1,))[0])

    def generate(self, first_token: int, pos0: int, n_tokens: int) -> list[int]:
        """Greedy decode of n_tokens from first_token at pos0 (the previous token fed back on the device)."""
        out = []
        for i in range(n_tokens):
            self.step(first_token if i == 0 else None, pos0 + i)
            out.append(self.read_next())
        return out

    def free(self) -> None:
        if self.graph is not None:
            self.graph.free()
            self.graph = None
        self.plan.free()
        if self._pf is not None:
            for k, b in self._pf.items():
                if k != "U":
                    b.free()
            self._pf = None
        for L in self.layers:
            for k in ("wqkv", "wo", "wgu", "wd", "kc", "vc"):
                L[k].free()
        self.wout.free()


def tiny_config(name: str = "tiny-llama", **kw) -> LlamaConfig:
    """A small model with every shape rule of the 8B one (for parity tests and smoke runs)."""
    base = LlamaConfig(name, n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=64, n_vocab=384)
    return replace(base, **kw)
