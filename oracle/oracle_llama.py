"""TEST INFRASTRUCTURE ONLY: the decode step of a Llama-architecture model composed from the CPU
restatement's ops (oracle.Oracle), for checking the GPU decoder end to end. Only tests/, smoke()
and bench.py's CPU leg import it.

The op order is the reference's decoder-layer op list (sw/ctrl/tests/test_fw_m7_layer.cpp:646-686,
non-Gemma branch; each record run by its per-kind reference as sw/ctrl/ref/opl_ref.hpp:1-9 runs a
list): RMS_NORM+MUL, MUL_MAT Q / K / V, ROPE q and k, SET_ROWS_KV K and V, FLASH_ATTN_EXT (the new
cell's chunk last), MUL_MAT Wo with the residual addend, RMS_NORM+MUL, MUL_MAT gate / up, SWIGLU,
MUL_MAT down with the residual addend; then the output norm, the output head and the greedy pick.
Q, K and V are separate MUL_MATs here (the GPU decoder concatenates their rows; each row's value is
the same), and q and k are rotated by separate ROPEs."""
from __future__ import annotations

import math

import numpy as np


class OracleLlama:
    """tensors: {gguf name: quantized blocks or f32 array}; the same names as tsr_llama.layer_tensors,
    plus blk.<i>.attn_norm.weight, blk.<i>.ffn_norm.weight, output_norm.weight, output.weight and
    token_embd.weight (f32 [n_vocab, n_embd])."""

    def __init__(self, oc, *, n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_vocab, eps, rope_base,
                 rope_mode, wfmt, ofmt, tensors, kv_size, threads=1):
        self.oc = oc
        self.threads = threads
        self.n_layer, self.n_embd, self.n_ff = n_layer, n_embd, n_ff
        self.n_head, self.n_head_kv, self.D, self.n_vocab = n_head, n_head_kv, head_dim, n_vocab
        self.eps, self.rope_base, self.neox = eps, rope_base, rope_mode != 0
        self.wfmt, self.ofmt, self.t = wfmt, ofmt, tensors
        self.E = n_head_kv * head_dim
        rb = self.E // 32 * 34
        self.kc = [np.zeros((kv_size, rb), np.uint8) for _ in range(n_layer)]
        self.vc = [np.zeros((kv_size, rb), np.uint8) for _ in range(n_layer)]
        self.kv_size = kv_size
        self.scale = np.float32(1.0 / math.sqrt(head_dim))

    def set_history(self, il: int, which: int, rows) -> None:
        cache = self.kc[il] if which == 0 else self.vc[il]
        self.oc.kv_set_rows(cache, rows, np.arange(rows.shape[0], dtype=np.int64))

    def set_cache_bytes(self, il: int, which: int, image) -> None:
        """A layer's K (0) or V (1) cache as the ggml q8_0 image [kv_size][E / 32 * 34] (a copy)."""
        cache = self.kc[il] if which == 0 else self.vc[il]
        cache[:] = np.asarray(image, np.uint8).reshape(cache.shape)

    def step(self, token: int, pos: int, ts: np.float32, n_kv: int) -> np.ndarray:
        """Logits [n_vocab] of the token at position pos; ts = powf(rope_base, -2 / head_dim)."""
        return self.forward(np.array([token], np.int32), pos, ts, n_kv)

    def forward(self, tokens, pos0: int, ts: np.float32, n_kv: int) -> np.ndarray:
        """T tokens at positions pos0 .. pos0 + T - 1 (cells the same), one ubatch: row t attends to
        cells [0, pos0 + t] (llama.cpp's causal kq_mask over a cache), the ubatch's cells planned
        newest last. Returns the logits [n_vocab] of the last token."""
        oc, t, D = self.oc, self.t, self.D
        tokens = np.ascontiguousarray(tokens, np.int32)
        T = tokens.size
        x = oc.get_rows(t["token_embd.weight"], tokens)
        msum = np.zeros(8 + 4 * T, np.uint32)
        msum[0], msum[1], msum[2] = 0x4D55534D, T, n_kv
        msum[9::4] = pos0 + 1 + np.arange(T, dtype=np.uint32)        # row r: cells [0, pos0 + r + 1)
        runs = np.array([[pos0, pos0 + T]], np.uint32)
        posv = pos0 + np.arange(T, dtype=np.int32)
        cells = posv.astype(np.int64)
        for il in range(self.n_layer):
            b = f"blk.{il}."
            xn = oc.rms_norm(x, self.eps, t[b + "attn_norm.weight"])
            q = oc.mul_mat(self.wfmt, t[b + "attn_q.weight"], self.n_embd, xn, threads=self.threads)
            k = oc.mul_mat(self.wfmt, t[b + "attn_k.weight"], self.n_embd, xn, threads=self.threads)
            v = oc.mul_mat(self.wfmt, t[b + "attn_v.weight"], self.n_embd, xn, threads=self.threads)
            q = oc.rope(q, posv, D, D, self.neox, ts)
            k = oc.rope(k, posv, D, D, self.neox, ts)
            oc.kv_set_rows(self.kc[il], k, cells)
            oc.kv_set_rows(self.vc[il], v, cells)
            a = oc.flash_attn(q, self.kc[il], self.vc[il], D, self.n_head, self.n_head_kv, float(self.scale), msum,
                              new_runs=runs)
            h = oc.mul_mat(self.wfmt, t[b + "attn_output.weight"], self.n_head * D, a, add=x, threads=self.threads)
            hn = oc.rms_norm(h, self.eps, t[b + "ffn_norm.weight"])
            g = oc.mul_mat(self.wfmt, t[b + "ffn_gate.weight"], self.n_embd, hn, threads=self.threads)
            u = oc.mul_mat(self.wfmt, t[b + "ffn_up.weight"], self.n_embd, hn, threads=self.threads)
            x = oc.mul_mat(self.wfmt, t[b + "ffn_down.weight"], self.n_ff, oc.swiglu(g, u), add=h, threads=self.threads)
        xn = oc.rms_norm(x[T - 1:T], self.eps, t["output_norm.weight"])
        return oc.mul_mat(self.ofmt, t["output.weight"], self.n_embd, xn, threads=self.threads)[0]
