#!/usr/bin/env python3
"""Benchmark of the quantized-inference hot path on one MI355X.

Headline workload (the configuration the metric is quoted on): greedy
decode of a random-init Llama-3-8B-architecture model at batch 1 -- 32 layers, hidden 4096, FFN
14336 SwiGLU, 32 q / 8 KV heads, head_dim 128, vocab 128256, every weight matrix (output head
included) Q4_K from seeded N(0, 0.02), q8_0 KV caches prefilled through the model with 4096 seeded
random token ids (8 ubatches of 512 tokens, every layer's ops over the ubatch rows). One step is
one decode token: the whole decoder (embedding row, 32 x [RMS_NORM, MUL_MAT QKV, ROPE, SET_ROWS_KV,
FLASH_ATTN_EXT, MUL_MAT O + residual, RMS_NORM, MUL_MAT gate|up, SWIGLU, MUL_MAT down + residual],
output norm, output head, ARGMAX) replayed as one HIP graph, the greedy token fed back on the device.
Inputs are resident in HBM before the timed region; the 4.2 GB of weights per token exceed the
256 MB Infinity Cache many times over, so weight reads come from HBM.

Output: one JSON line with the metric (decode tokens per second), the roofline of the kernel that
takes the largest share of a token (its launch duration measured live with HIP events on the launch
stream over the model's own layers), HBM traffic of that kernel from two rocprofv3 --pmc passes, and
the CPU baseline: this repository's oracle (the reference's numerics restated in C) decoding the same
model on the host cores -- whose first-token logits are also compared bit for bit with the GPU's.
The other BASELINE configs (Q4_K FFN pair, Q8_0 matvec, flash-decode at 8192 cells, prefill) are
reported under "also".
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tesseract-npu_amd"))

import tsr_hip  # noqa: E402
import tsr_llama as LL  # noqa: E402
import tsr_synth as S  # noqa: E402

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
METRIC = "decode tok/s (8B Q4_K, ctx 4096); matvec/attn HBM GB/s as % of peak"
CTX = 4096                      # KV cells filled before the first decode token
PMC_KV_SIZE = CTX + 8 + 128     # the counter child's cache (the default bench's kv_size)
PMC_POS = CTX + 8 + 64          # and its token's cell: the timed region's middle
UBATCH = 512                    # prefill tokens per pass of the layers (llama.cpp's default n_ubatch)
PROMPT_SEED = 4096              # numpy seed of the random prompt token ids


class HipEvents:
    """hipEvent timing and hipGraph capture / replay on a given stream (libamdhip64 via ctypes)."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.h.hipDeviceSynchronize.argtypes = []
        self.h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.h.hipGraphDestroy.argtypes = [C.c_void_p]
        # device pointers are 64-bit: without argtypes ctypes would pass them as (truncated) C ints
        self.h.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]

    def event(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.h.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    def device_sync(self):
        assert self.h.hipDeviceSynchronize() == 0

    def capture(self, stream, fn, n: int):
        """A graph of fn(0) .. fn(n - 1) as launched on `stream` (relaxed capture mode)."""
        assert self.h.hipStreamBeginCapture(stream, 2) == 0
        for i in range(n):
            fn(i)
        g, ge = C.c_void_p(), C.c_void_p()
        assert self.h.hipStreamEndCapture(stream, C.byref(g)) == 0
        assert self.h.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
        return g, ge

    def eager_ms(self, stream, fn, n: int, replays: int = 3) -> float:
        """Milliseconds per call of fn over n direct launches: the median of `replays` timed rounds
        after one untimed round."""
        a, b = self.event(), self.event()
        for i in range(n):
            fn(i)
        times = []
        for _ in range(replays):
            self.record(a, stream)
            for i in range(n):
                fn(i)
            self.record(b, stream)
            times.append(self.elapsed_ms(a, b) / n)
        return float(np.median(times))

    def graph_ms(self, stream, fn, n: int, replays: int = 3) -> tuple:
        """Milliseconds per call of fn over n calls replayed from one graph: the median of `replays`
        timed replays after one untimed replay; also the eager (host-launched) time of n calls."""
        g, ge = self.capture(stream, fn, n)
        try:
            assert self.h.hipGraphLaunch(ge, stream) == 0
            self.device_sync()
            a, b = self.event(), self.event()
            times = []
            for _ in range(replays):
                self.record(a, stream)
                assert self.h.hipGraphLaunch(ge, stream) == 0
                self.record(b, stream)
                times.append(self.elapsed_ms(a, b) / n)
            self.record(a, stream)
            for i in range(n):
                fn(i)
            self.record(b, stream)
            eager = self.elapsed_ms(a, b) / n
            return float(np.median(times)), eager
        finally:
            self.h.hipGraphExecDestroy(ge)
            self.h.hipGraphDestroy(g)


def q4k_bytes(N: int, K: int) -> int:
    return N * (K // 256) * 144


def mv_bytes(N: int, K: int) -> int:
    """Algorithmic bytes of one Q4_K matvec: weights + f32 x + f32 y."""
    return q4k_bytes(N, K) + 4 * K + 4 * N


def token_bytes(cfg, n_kv_read: int) -> int:
    """Algorithmic bytes of one decode token: every quantized weight once, the q8_0 K and V of the
    visible cells of every layer, the embedding row and the norm vectors."""
    E = cfg.E
    kv = cfg.n_layer * 2 * n_kv_read * (E // 32) * 34
    return cfg.weight_bytes_per_token() + kv + 4 * cfg.n_embd * (2 * cfg.n_layer + 2)


def e2e_decode(dev, ev, steps: int, warmup: int, eager: bool = False) -> dict:
    """Llama-3-8B-architecture Q4_K decode with CTX cells of context.

    Cells 0 .. CTX-1 of every layer's caches are filled by the prefill of CTX random token ids in
    ubatches of UBATCH (untimed; its rate is reported); token 0, the prompt's greedy token, is decoded
    at position CTX eagerly (its logits are kept for the CPU leg's bit comparison), tokens 1 .. warmup-1
    by graph replays (the first replay captures), then `steps` timed graph replays at positions
    CTX+warmup .. CTX+warmup+steps-1; with `eager`, direct launches instead of every replay. Every
    greedy token is copied to a device history buffer."""
    cfg = LL.LLAMA3_8B
    wts = LL.SyntheticWeights(cfg, cache=True)
    kv_size = CTX + warmup + steps
    stream = dev.stream
    t0 = time.perf_counter()
    m = LL.LlamaDecoder(dev, cfg, wts, kv_size)
    setup_s = time.perf_counter() - t0
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg.n_vocab, CTX).astype(np.int32)
    t0 = time.perf_counter()
    m.prefill(prompt, 0, UBATCH)
    prefill_s = time.perf_counter() - t0
    tok0 = m.read_next()
    print(f"[bench] prefill of {CTX} random ids in ubatches of {UBATCH}: {prefill_s:.2f} s", flush=True)
    hist = dev.alloc(4 * (warmup + steps))
    m.step(tok0, CTX)
    logits0 = m.read_logits().copy()
    tok1 = m.read_next()
    hist.write(np.array([tok1], np.int32))
    for i in range(1, warmup):
        if eager:   # no decode graph at all (the profiler's kernel trace of this process)
            m.step_async(tok1 if i == 1 else None, CTX + i)
        else:
            m.step_graph(tok1 if i == 1 else None, CTX + i)
        dev.copy_async(hist.ptr + 4 * i, m.tok, 4)
    dev.sync()
    captures = m.captures
    e0, e1 = ev.event(), ev.event()
    ev.device_sync()
    h0 = time.perf_counter()
    ev.record(e0, stream)
    for i in range(steps):
        if eager:
            m.step_async(None, CTX + warmup + i)
        else:
            m.step_graph(None, CTX + warmup + i)
        dev.copy_async(hist.ptr + 4 * (warmup + i), m.tok, 4)
    ev.record(e1, stream)
    host_enqueue_s = time.perf_counter() - h0
    ms = ev.elapsed_ms(e0, e1)
    wall_s = time.perf_counter() - h0
    if m.captures != captures:
        raise RuntimeError("the decode graph was re-captured inside the timed region")
    m.check()                   # DecodeError: an index out of range (1) or an expired FA wait (2)
    toks = hist.read(np.int32, (warmup + steps,))
    ms_tok = ms / steps
    mid_kv = CTX + warmup + steps // 2 + 1
    tb = token_bytes(cfg, mid_kv)

    # each op class alone, launched over the model's own 32 layers (graph replay, or direct launches
    # with `eager`; HIP events on the launch stream): what a token spends where
    n, E, nq, ff, d = cfg.n_embd, cfg.E, cfg.n_q, cfg.n_ff, dev
    L = m.layers
    nl = cfg.n_layer
    f4 = 4
    w3 = nq + 2 * E
    kv_b = 2 * kv_size * (E // 32) * 34 + 4 * w3 + 4 * nq
    if m.qkv_in_attn:           # the decoder's attention half: one launch with the Q|K|V rows
        ops = {"mul_mat_norm qkv+rope+set_rows_kv+flash_attn (one launch)": (
            lambda i: d.attn_qkv_plan_rope_tab(m.plan, L[i % nl]["wqkv"], m.x, cfg.eps, L[i % nl]["attn_norm"], m.qkv,
                                               L[i % nl]["kc"], L[i % nl]["vc"], m.scale, cfg.head_dim, cfg.rope_mode,
                                               m.rtab, m.cell_ptr, m.att, nq, bad=m.bad, stream=stream),
            nl, mv_bytes(w3, n) + 4 * n + kv_b, "k_fa_dec<qkv>")}
    else:
        ops = {
            "mul_mat_norm qkv Q4_K 6144x4096": (
                lambda i: d.mul_mat_norm(L[i % nl]["wqkv"], m.x, 1, n, cfg.eps, L[i % nl]["attn_norm"], m.qkv, w3,
                                         stream=stream), nl, mv_bytes(w3, n) + 4 * n, "k_mv_q4k<norm>"),
            "rope+set_rows_kv+flash_attn": (
                lambda i: d.flash_attn_plan_rope_tab(m.plan, m.qkv, L[i % nl]["kc"], L[i % nl]["vc"], m.scale,
                                                     cfg.head_dim, cfg.rope_mode, m.rtab, m.cell_ptr, m.att, nq,
                                                     bad=m.bad, stream=stream),
                nl, kv_b, "k_fa_dec")}
    ops.update({
        "mul_mat o Q4_K 4096x4096 +res": (lambda i: d.mul_mat(L[i % nl]["wo"], m.att, 1, nq, m.h, n, add=m.x, add_stride=n,
                                                              stream=stream), nl, mv_bytes(n, nq) + 4 * n, "k_mv_q4k"),
        "mul_mat_norm+glu gate|up Q4_K 28672x4096": (
            lambda i: d.mul_mat_norm(L[i % nl]["wgu"], m.h, 1, n, cfg.eps, L[i % nl]["ffn_norm"], m.glu, ff,
                                     flags=tsr_hip.MM_GLU, stream=stream),
            nl, q4k_bytes(2 * ff, n) + 8 * n + 4 * ff, "k_mv_q4k<norm,glu>"),
        "mul_mat down Q4_K 4096x14336 +res": (
            lambda i: d.mul_mat(L[i % nl]["wd"], m.glu, 1, ff, m.x, n, add=m.h, add_stride=n, stream=stream),
            nl, mv_bytes(n, ff) + 4 * n, "k_mv_q4k"),
        "mul_mat_norm output Q4_K 128256x4096": (
            lambda i: d.mul_mat_norm(m.wout, m.x, 1, n, cfg.eps, m.out_norm, m.logits, cfg.n_vocab, stream=stream),
            1, mv_bytes(cfg.n_vocab, n) + 4 * n, "k_mv_q4k<norm>"),
        "rope_table": (lambda i: d.rope_table(m.pos_ptr, cfg.head_dim, cfg.rope_base, m.rtab, stream=stream), 1,
                       4 * cfg.head_dim, "k_rope_table"),
        "argmax": (lambda i: d.argmax(m.logits, cfg.n_vocab, 1, cfg.n_vocab, m.next, stream=stream), 1,
                   4 * cfg.n_vocab, "k_argmax"),
        "get_rows": (lambda i: d.get_rows(m.tok_embd, n, n, cfg.n_vocab, m.tok, 1, m.h, n, bad=m.bad, stream=stream), 1,
                     8 * n, "k_get_rows"),
    })
    per_op = {}
    for name, (fn, count, nbytes, kname) in ops.items():
        for i in range(3):
            fn(i)
        ev.device_sync()
        t = ev.eager_ms(stream, fn, 2 * nl) if eager else ev.graph_ms(stream, fn, 2 * nl)[0]
        per_op[name] = {"launch_us": round(t * 1e3, 3), "per_token": count, "us_per_token": round(t * 1e3 * count, 1),
                        "GB/s": round(nbytes / (t * 1e-3) / 1e9, 1), "algorithmic_bytes": nbytes, "kernel": kname}
    ev.device_sync()
    out = {
        "cfg": cfg, "wts": wts, "model": m, "kv_size": kv_size, "logits0": logits0, "tokens": toks.tolist(),
        "ms_per_token": ms_tok, "tok_s": 1e3 / ms_tok, "token_bytes": tb,
        "host_enqueue_ms_per_token": host_enqueue_s * 1e3 / steps, "wall_ms_per_token": wall_s * 1e3 / steps,
        "setup_s": setup_s, "per_op": per_op, "captures": captures, "tok0": tok0, "prefill_s": prefill_s,
    }
    return out


def cpu_decode(e2e: dict, max_seconds: float = 40.0, max_tokens: int = 5) -> dict:
    """The oracle's decode of the same model (the reference numerics restated in C, MUL_MAT on all the
    host cores available, up to 16) from the same cache state (the GPU's prefilled cache bytes, read
    back): token 0 at position CTX with the same first id, then the oracle's own greedy tokens, for
    about max_seconds. Its logits of token 0 are compared bit for bit with the GPU's, and its greedy
    tokens with the GPU's. (The prefill itself is checked against the oracle on small models by the
    tests; at 8B it would take the oracle hours.)"""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    from oracle_llama import OracleLlama
    cfg, wts = e2e["cfg"], e2e["wts"]
    oc = oracle.Oracle()
    threads = min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1))
    t = {"token_embd.weight": wts.embedding(), "output_norm.weight": wts.norm("output_norm.weight")[None],
         "output.weight": wts.quant("output.weight", cfg.n_vocab, cfg.n_embd, cfg.ofmt)}
    for il in range(cfg.n_layer):
        for name, N, K in LL.layer_tensors(cfg, il):
            t[name] = wts.quant(name, N, K, cfg.wfmt)
        for nm in ("attn_norm", "ffn_norm"):
            t[f"blk.{il}.{nm}.weight"] = wts.norm(f"blk.{il}.{nm}.weight")[None]
    kv_size = e2e["kv_size"]
    ref = OracleLlama(oc, n_layer=cfg.n_layer, n_embd=cfg.n_embd, n_ff=cfg.n_ff, n_head=cfg.n_head,
                      n_head_kv=cfg.n_head_kv, head_dim=cfg.head_dim, n_vocab=cfg.n_vocab, eps=cfg.eps,
                      rope_base=cfg.rope_base, rope_mode=cfg.rope_mode, wfmt=cfg.wfmt, ofmt=cfg.ofmt, tensors=t,
                      kv_size=kv_size, threads=threads)
    for il, caches in enumerate(e2e["caches"]):
        for which in (0, 1):
            ref.set_cache_bytes(il, which, caches[which])
    e2e["caches"] = None
    libm = C.CDLL("libm.so.6")
    libm.powf.argtypes = [C.c_float, C.c_float]
    libm.powf.restype = C.c_float
    ts = np.float32(libm.powf(float(np.float32(cfg.rope_base)), float(np.float32(-2.0) / np.float32(cfg.head_dim))))
    gpu_toks = e2e["tokens"]
    tok, n, times, same_tokens, logits_equal = e2e["tok0"], 0, [], True, None
    while n < max_tokens:
        pos = CTX + n
        t0 = time.perf_counter()
        logits = ref.step(tok, pos, ts, min(kv_size, (pos + 1 + 255) // 256 * 256))
        times.append(time.perf_counter() - t0)
        nxt = int(oc.argmax(logits[None])[0])
        if n == 0:
            logits_equal = bool(np.array_equal(logits.view(np.uint32), e2e["logits0"].view(np.uint32)))
        same_tokens &= nxt == gpu_toks[n]
        tok, n = nxt, n + 1
        if sum(times) >= max_seconds:
            break
    per = float(np.median(times))
    # the same first token on one thread (position CTX again: it rewrites its cell with the same rows)
    ref.threads = 1
    t0 = time.perf_counter()
    logits1 = ref.step(e2e["tok0"], CTX, ts, min(kv_size, (CTX + 1 + 255) // 256 * 256))
    one_s = time.perf_counter() - t0
    one_equal = bool(np.array_equal(logits1.view(np.uint32), e2e["logits0"].view(np.uint32)))
    return {"value": round(1.0 / per, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"{n} decode tokens of the same Llama-3-8B-arch Q4_K model at positions {CTX}..{CTX + n - 1} "
                       f"by oracle/oracle_llama.py over oracle/oc_*.c ({threads} threads in MUL_MAT), "
                       f"median {per:.2f} s per token"),
            "statistic": f"median of {n} tokens",
            "single_thread": {"value": round(1.0 / one_s, 4), "unit": "tok/s", "cores": 1,
                              "sample": f"token 0 again at position {CTX} on one thread, {one_s:.2f} s",
                              "token0_logits_bit_equal": one_equal},
            "host": host_info(),
            "ggml_cpu": "not measured (unavailable offline: llama.cpp/ggml is an un-vendored submodule)",
            "parity": {"token0_logits_bit_equal": logits_equal, "greedy_tokens_equal": bool(same_tokens),
                       "tokens_compared": n}}


def cpu_configs(threads: int, runs: int = 5) -> dict:
    """The oracle (the reference's numerics restated in C, oracle/oc_*.c) on BASELINE configs[0]-[3]'s
    workloads, drawn from the same seeds as the GPU legs under "also", on the host cores: each at one
    thread and at `threads` threads, the median of `runs` timed runs after one untimed run. MUL_MAT is
    threaded over output rows (like the reference's mvm_rows pool, sw/sim/tsr_sim.c:1608-1647); the
    causal prefill FLASH_ATTN_EXT over query rows (each row is planned and computed on its own, so the
    row blocks give the whole call's bits); the decode FLASH_ATTN_EXT is one sequential call (its chunk
    plan depends on all of a token's KV heads: a split by head would be another computation). The
    prefill MUL_MATs time a sample of 32 of the 512 token rows (rows are independent) and report the
    full call's rate."""
    import concurrent.futures as cf
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    oc = oracle.Oracle()

    def med(fn):
        t0 = time.perf_counter()
        fn()
        first = time.perf_counter() - t0
        ts = [first] if first > 0.25 else []       # a long run is its own warm-up: it counts
        while len(ts) < runs:
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def both(fn_of_threads, unit_of):
        r = {}
        for th in sorted({1, threads}):
            s = med(lambda: fn_of_threads(th))
            r[f"threads_{th}"] = {"seconds": round(s, 6), **unit_of(s)}
        return r

    out = {"runs": runs, "statistic": "median", "kind": "port", "threads_all": threads, "host": host_info()}
    # Q8_0 matvec 4864 x 896 (the GPU leg's seeds)
    N, K = 4864, 896
    w = S.quant_rows(0, S.seed_of("cfg1", "w"), N, K)
    x = S.normal(S.seed_of("cfg1", "x"), K)
    nb = N * (K // 32) * 34 + 4 * K + 4 * N
    out["q8_0_matvec_4864x896"] = both(lambda th: oc.mul_mat(0, w, K, x, threads=th),
                                       lambda s: {"us_per_call": round(s * 1e6, 1), "GB/s": round(nb / s / 1e9, 3)})
    # Q4_K up 14336 x 4096 then down 4096 x 14336
    up = S.quant_rows(1, S.seed_of("cfg2", "w_up"), 14336, 4096)
    dn = S.quant_rows(1, S.seed_of("cfg2", "w_down"), 4096, 14336)
    xu = S.normal(S.seed_of("cfg2", "x"), 4096)

    def pair(th):
        h = oc.mul_mat(1, up, 4096, xu, threads=th)
        oc.mul_mat(1, dn, 14336, h, threads=th)
    nb = 2 * (14336 * 16 * 144) + 4 * (4096 + 14336) * 2
    out["ffn_pair_q4k_14336x4096_4096x14336"] = both(pair, lambda s: {"us_per_step": round(s * 1e6, 1),
                                                                      "GB/s": round(nb / s / 1e9, 3)})
    del up, dn
    # FLASH_ATTN_EXT decode, 8192 cells, 32 q / 8 KV heads, D 128
    n_kv, E = 8192, 1024
    kc = np.zeros((n_kv, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    oc.kv_set_rows(kc, S.normal(S.seed_of("cfg3", "k"), n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    oc.kv_set_rows(vc, S.normal(S.seed_of("cfg3", "v"), n_kv * E).reshape(n_kv, E), np.arange(n_kv))
    q = S.normal(S.seed_of("cfg3", "q"), 32 * 128).astype(np.float16).astype(np.float32).reshape(1, -1)
    ms = oc.msum(np.zeros((1, n_kv), np.float16))
    scale = np.float32(1.0 / np.sqrt(128))
    s = med(lambda: oc.flash_attn(q, kc, vc, 128, 32, 8, scale, ms))
    nb = 2 * n_kv * E // 32 * 34 + 2 * 32 * 128 + 4 * 32 * 128
    out["fa_decode_q8kv_8192_32q8kv_d128"] = {"threads_1": {"seconds": round(s, 6), "us_per_call": round(s * 1e6, 1),
                                                            "GB/s": round(nb / s / 1e9, 3)},
                                              "note": "one sequential call (the plan spans all KV heads)"}
    del kc, vc
    # prefill MUL_MATs (a 32-row sample of the 512 token rows) and the causal FA over 512 tokens
    T, K, Ts = 512, 4096, 32
    xs = S.normal(S.seed_of("cfg4", "x"), T * K).reshape(T, K)[:: T // Ts][:Ts]
    for name, N in (("prefill_q8_0_512x4096x4096", 4096), ("prefill_q8_0_512x14336x4096", 14336)):
        w = S.quant_rows(0, S.seed_of("cfg4", "w_" + str(N)), N, K)
        ops = 2 * T * N * K
        out[name] = both(lambda th: oc.mul_mat(0, w, K, xs, threads=th),
                         lambda s, ops=ops: {"seconds_per_512_rows": round(s * T / Ts, 4),
                                             "int8_GOPS": round(ops / (s * T / Ts) / 1e9, 2)})
        out[name]["sample"] = f"{Ts} of the {T} token rows (every {T // Ts}th)"
        del w
    T, E = 512, 1024
    kc = np.zeros((T, E // 32 * 34), np.uint8)
    vc = np.zeros_like(kc)
    oc.kv_set_rows(kc, S.normal(S.seed_of("cfg4", "fa_k"), T * E).reshape(T, E), np.arange(T))
    oc.kv_set_rows(vc, S.normal(S.seed_of("cfg4", "fa_v"), T * E).reshape(T, E), np.arange(T))
    qp = S.normal(S.seed_of("cfg4", "fa_q"), T * 4096).reshape(T, 4096).astype(np.float16).astype(np.float32)
    mask = np.full((T, T), -np.inf, np.float16)
    mask[np.tril_indices(T)] = 0

    def fa_rows(th):
        cuts = np.linspace(0, T, th + 1).astype(int)
        blocks = [(a, b) for a, b in zip(cuts[:-1], cuts[1:]) if b > a]
        run = lambda ab: oc.flash_attn(qp[ab[0]:ab[1]], kc, vc, 128, 32, 8, scale, oc.msum(mask[ab[0]:ab[1]]), None,
                                       [[0, T]])
        if len(blocks) == 1:
            return run(blocks[0])
        with cf.ThreadPoolExecutor(len(blocks)) as ex:        # ctypes calls release the GIL
            return list(ex.map(run, blocks))
    out["fa_prefill_causal_512_32q8kv_d128"] = both(fa_rows, lambda s: {"ms_per_call": round(s * 1e3, 2)})
    return out


def host_info() -> dict:
    """The CPU the baseline ran on: model name, online CPUs and the CPUs this process may use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc_online": os.cpu_count(),
            "nproc_affinity": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}


def adapter_decode(ev, e2e, caches, steps: int) -> dict:
    """The same decode through the ggml-backend adapter (libtsr_ggml): llama.cpp's graph of the
    Llama-3-8B-architecture model (tsr_ggml_graph.LlamaGraph: separate Q / K / V MUL_MATs, ROPE,
    SET_ROWS into cache tensors recognized by name, permuted FLASH_ATTN_EXT views, inp_out_ids), the
    weights set as ggml blocks into a weights buffer, the caches as the decoder's q8_0 images into a KV
    buffer. Token 0 is decoded at position CTX (its logits compared bit for bit with the decoder's), then
    `steps` timed tokens at CTX + 1 .., one graph_compute each: the adapter replays its captured graph,
    the greedy token fed back on the device (cpy_tensor from the ARGMAX result to inp_tokens)."""
    import tsr_ggml as G
    import tsr_ggml_graph as GL
    cfg, wts, kv_size = e2e["cfg"], e2e["wts"], e2e["kv_size"]
    gd = G.Device(0)
    t0 = time.perf_counter()
    images = {}
    for il, (k, v) in enumerate(caches):
        images[(il, 0)], images[(il, 1)] = k, v
    _, W, kvt, wbuf, kvbuf = GL.load_model(gd, cfg, wts, kv_size, images)
    g = GL.LlamaGraph(gd, cfg, W, kvt, kv_size, 1, kv_size, argmax=True)
    nodes = gd.prepare(g.ctx.nodes)
    g.set_inputs([e2e["tok0"]], CTX)
    gd.graph_compute(nodes)                                # lowers, converts the weights, runs
    logits0 = g.logits_host()
    setup_s = time.perf_counter() - t0
    same = bool((logits0.view(np.uint32) == e2e["logits0"].view(np.uint32)).all())
    hstream = C.c_void_p(tsr_hip.load().tsr_hip_stream(gd.L.tsr_gg_hip_ctx(gd.h)))
    pos = CTX + 1
    for i in range(2):                                     # the capture, one replay
        g.buf.cpy_tensor(g.next, g.inp_tokens)
        g.set_position(pos)
        gd.graph_compute(nodes)
        pos += 1
    gd.synchronize()
    e0, e1 = ev.event(), ev.event()
    s0 = gd.stats()
    ev.record(e0, hstream)
    h0 = time.perf_counter()
    hs = []
    for i in range(steps):
        g.buf.cpy_tensor(g.next, g.inp_tokens)
        g.set_position(pos)
        gd.graph_compute(nodes)
        hs.append(time.perf_counter())
        pos += 1
    ev.record(e1, hstream)
    host_wall_ms = (time.perf_counter() - h0) * 1e3 / steps
    # the host's own cost per token: the first tokens after the synchronize, while the host runs ahead
    # of the device (later ones wait for the staging slots that the device has not consumed yet: 4
    # input copies a token through 64 slots, so from token 16 on the loop runs at the device's pace)
    dts = np.diff(np.array([h0] + hs[:12])) * 1e3
    host_ms = float(np.median(dts))
    ms = ev.elapsed_ms(e0, e1)
    gd.synchronize()                                       # TSR_GG_E_FLAG if a kernel raised a flag
    s1 = gd.stats()
    calls = [c["name"] for c in gd.lower(g.ctx.nodes) if not c["flags"] & G.CALL_IN_NEXT]
    out = {"tok_s": round(steps / (ms * 1e-3), 2), "ms_per_token": round(ms / steps, 5),
           "host_ms_per_token": round(host_ms, 4),
           "host_ms_per_token_note": "median over the first 12 tokens (the host ahead of the device)",
           "host_wall_ms_per_token": round(host_wall_ms, 4), "replays": s1["replays"] - s0["replays"],
           "plan_hits": s1["plan_hits"] - s0["plan_hits"], "launches_per_token": len(calls),
           "graph_nodes": len(g.ctx.nodes), "token0_logits_bit_equal_to_decoder": same,
           "setup_s": round(setup_s, 2),
           "path": "tsr_gg_graph_compute over llama.cpp's graph (fused: Q|K|V + norm + ROPE+SET_ROWS+FA, "
                   "gate|up + norm + GLU), captured once, replayed per token"}
    g.free()
    kvbuf.free()
    wbuf.free()
    gd.close()
    return out


def extra_workloads(dev, ev, stream, n: int, eager: bool = False) -> dict:
    """The other single-GPU BASELINE configs, each timed over rotating device copies (> 2x MALL):
    configs[1] the Q4_K FFN up/down pair, configs[0] Q8_0 matvec 4864x896, configs[2] q8-KV
    flash-decode (32 q / 8 KV heads, D 128, n_kv 8192, batch 1), configs[3] the prefill matmuls and
    the causal prefill attention. Per-call time from HIP events on the launch stream (graph replay
    and direct launches; with `eager`, direct launches only)."""
    out = {}

    def timed(fn, nn=None):
        for i in range(5):
            fn(i)
        ev.device_sync()
        if eager:
            t = ev.eager_ms(stream, fn, nn or n)
            return t, t
        return ev.graph_ms(stream, fn, nn or n)

    def timed_eager(fn, nn):
        for i in range(3):
            fn(i)
        ev.device_sync()
        a, b = ev.event(), ev.event()
        ev.record(a, stream)
        for i in range(nn):
            fn(i)
        ev.record(b, stream)
        return ev.elapsed_ms(a, b) / nn

    # the Llama-3-8B FFN up / down Q4_K matvec pair
    N_up, K_up, N_dn, K_dn = 14336, 4096, 4096, 14336
    up_blocks = S.quant_rows(1, S.seed_of("cfg2", "w_up"), N_up, K_up)
    dn_blocks = S.quant_rows(1, S.seed_of("cfg2", "w_down"), N_dn, K_dn)
    x = S.normal(S.seed_of("cfg2", "x"), K_up)
    per_copy = up_blocks.nbytes + dn_blocks.nbytes
    copies = max(2, -(-2 * MALL_BYTES // per_copy))
    ups = [dev.weight(1, up_blocks, N_up, K_up) for _ in range(copies)]
    dns = [dev.weight(1, dn_blocks, N_dn, K_dn) for _ in range(copies)]
    xb, hb, yb = dev.upload(x), dev.alloc(4 * N_up), dev.alloc(4 * N_dn)

    def step(i):
        dev.mul_mat(ups[i % copies], xb, 1, K_up, hb, N_up, stream=stream)
        dev.mul_mat(dns[i % copies], hb, 1, K_dn, yb, N_dn, stream=stream)

    ms, ms_eager = timed(step)
    up_ms, _ = timed(lambda i: dev.mul_mat(ups[i % copies], xb, 1, K_up, hb, N_up, stream=stream))
    dn_ms, _ = timed(lambda i: dev.mul_mat(dns[i % copies], hb, 1, K_dn, yb, N_dn, stream=stream))
    sb = mv_bytes(N_up, K_up) + mv_bytes(N_dn, K_dn)
    out["ffn_pair_q4k_14336x4096_4096x14336"] = {
        "us_per_step": round(ms * 1e3, 3), "us_per_step_eager": round(ms_eager * 1e3, 3),
        "GB/s": round(sb / (ms * 1e-3) / 1e9, 1), "frac_of_hbm_peak": round(sb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "up_us": round(up_ms * 1e3, 3), "up_GB/s": round(mv_bytes(N_up, K_up) / (up_ms * 1e-3) / 1e9, 1),
        "down_us": round(dn_ms * 1e3, 3), "down_GB/s": round(mv_bytes(N_dn, K_dn) / (dn_ms * 1e-3) / 1e9, 1),
        "copies": copies}
    del ups, dns

    # Q8_0 4864 x 896
    N, K = 4864, 896
    blocks = S.quantize_q8_0(S.normal(S.seed_of("cfg1", "w"), N * K, 0.02).reshape(N, K))
    per = blocks.nbytes
    copies = -(-2 * MALL_BYTES // per)
    ws = [dev.weight(0, blocks, N, K) for _ in range(copies)]
    xb = dev.upload(S.normal(S.seed_of("cfg1", "x"), K))
    yb = dev.alloc(4 * N)
    ms, ms_eager = timed(lambda i: dev.mul_mat(ws[i % copies], xb, 1, K, yb, N, stream=stream))
    nbytes = N * (K // 32) * 34 + 4 * K + 4 * N
    out["q8_0_matvec_4864x896"] = {"us_per_call": round(ms * 1e3, 3), "us_per_call_eager": round(ms_eager * 1e3, 3),
                                   "algorithmic_bytes": nbytes,
                                   "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                   "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                   "copies": copies}
    del ws

    # flash-decode over a q8_0 KV cache
    n_head, n_kv_head, D, n_kv = 32, 8, 128, 8192
    E = n_kv_head * D
    kf = dev.upload(S.normal(S.seed_of("cfg3", "k"), n_kv * E))
    vf = dev.upload(S.normal(S.seed_of("cfg3", "v"), n_kv * E))
    idx = dev.upload(np.arange(n_kv, dtype=np.int64))
    k0, v0 = dev.kv(E, n_kv), dev.kv(E, n_kv)
    dev.kv_set_rows(k0, 0, kf, n_kv, E, idx)
    dev.kv_set_rows(v0, 1, vf, n_kv, E, idx)
    kimg, vimg = k0.get_bytes(0), v0.get_bytes(1)
    per = kimg.nbytes + vimg.nbytes
    copies = max(2, -(-2 * MALL_BYTES // per))
    caches = [(k0, v0)]
    for _ in range(copies - 1):
        kc, vc = dev.kv(E, n_kv), dev.kv(E, n_kv)
        kc.set_bytes(0, kimg)
        vc.set_bytes(1, vimg)
        caches.append((kc, vc))
    q = S.normal(S.seed_of("cfg3", "q"), n_head * D).astype(np.float16).astype(np.float32)
    qb = dev.upload(q)
    ob = dev.alloc(4 * n_head * D)
    msum = tsr_hip.msum_build_f16(np.zeros((1, n_kv), np.float16))
    scale = np.float32(1.0 / np.sqrt(D))
    nbytes = 2 * n_kv * E // 32 * 34 + 2 * n_head * D + 4 * n_head * D
    # the planned entry point (the decode form: one launch, k_fa_dec), the plan set once for the mask
    plan = dev.fa_plan(D, n_head, n_kv_head, 1, n_kv)
    plan.set(msum)
    # outside the timed loops: the planned launch's bits against the unplanned entry point's (both bit-exact
    # against the oracle in the GPU tests)
    dev.flash_attn_plan(plan, qb, n_head * D, k0, v0, scale, ob, n_head * D, stream=stream)
    dev.sync(stream)
    planned_out = ob.read(np.float32, (n_head * D,))
    dev.flash_attn(qb, 1, n_head * D, k0, v0, D, n_head, n_kv_head, scale, msum, ob, n_head * D, stream=stream)
    dev.sync(stream)
    planned_equal = bool((planned_out.view(np.uint32) == ob.read(np.float32, (n_head * D,)).view(np.uint32)).all())
    if not planned_equal:
        raise SystemExit("bench: the planned FLASH_ATTN_EXT launch differs from the unplanned entry point")
    ms, ms_eager = timed(lambda i: dev.flash_attn_plan(plan, qb, n_head * D, caches[i % copies][0], caches[i % copies][1],
                                                       scale, ob, n_head * D, stream=stream))
    # the unplanned entry point (work list planned per call on the host: QK, P.V and merge launches)
    ms3, ms3_eager = timed(lambda i: dev.flash_attn(qb, 1, n_head * D, caches[i % copies][0], caches[i % copies][1], D,
                                                    n_head, n_kv_head, scale, msum, ob, n_head * D, stream=stream))
    out["fa_decode_q8kv_8192_32q8kv_d128"] = {"us_per_call": round(ms * 1e3, 3), "us_per_call_eager": round(ms_eager * 1e3, 3),
                                              "algorithmic_bytes": nbytes,
                                              "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                              "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                              "copies": copies, "launches_per_call": 1, "kernel": "k_fa_dec",
                                              "unplanned_us_per_call": round(ms3 * 1e3, 3),
                                              "unplanned_launches_per_call": 3,
                                              "planned_bits_equal_unplanned": planned_equal}
    plan.free()
    del caches

    # prefill at Llama-3-8B shapes, 512 tokens: Q8_0 MUL_MAT on the int8 matrix cores
    T, K = 512, 4096
    xq = dev.upload(S.normal(S.seed_of("cfg4", "x"), T * K))
    for name, N in (("prefill_q8_0_512x4096x4096", 4096), ("prefill_q8_0_512x14336x4096", 14336)):
        blocks = S.quant_rows(0, S.seed_of("cfg4", "w_" + str(N)), N, K)
        ws = [dev.weight(0, blocks, N, K) for _ in range(2)]
        yb = dev.alloc(4 * T * N)
        ms, ms_eager = timed(lambda i: dev.mul_mat(ws[i % 2], xq, T, K, yb, N, stream=stream), 20)
        ops = 2 * T * N * K
        out[name] = {"us_per_call": round(ms * 1e3, 2), "us_per_call_eager": round(ms_eager * 1e3, 2),
                     "int8_TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                     "frac_of_int8_mfma_peak": round(ops / (ms * 1e-3) / 5.0e15, 4),
                     "launches_per_call": 2, "note": "QACT of the 512 rows + the matrix-core kernel"}
        del ws, yb
    # the same on Q4_K weights (the headline model's format): QACT A256 + the Q4_K matrix-core kernel;
    # 512 x 14336 x 4096 with the GLU epilogue is the 8B ubatch's gate|up (28672 interleaved rows)
    for name, N, K4, flags in (("prefill_q4_k_512x4096x4096", 4096, 4096, 0),
                               ("prefill_q4_k_512x4096x14336", 4096, 14336, 0),
                               ("prefill_q4_k_glu_512x28672x4096", 28672, 4096, tsr_hip.MM_GLU)):
        blocks = S.quant_rows(1, S.seed_of("cfg4", "w4_" + name), N, K4)
        ws = [dev.weight(1, blocks, N, K4) for _ in range(2)]
        x4 = dev.upload(S.normal(S.seed_of("cfg4", "x4"), T * K4))
        ny = N // 2 if flags else N
        yb = dev.alloc(4 * T * ny)
        ms, ms_eager = timed(lambda i: dev.mul_mat(ws[i % 2], x4, T, K4, yb, ny, flags=flags, stream=stream), 20)
        ops = 2 * T * N * K4
        out[name] = {"us_per_call": round(ms * 1e3, 2), "us_per_call_eager": round(ms_eager * 1e3, 2),
                     "int8_TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                     "frac_of_int8_mfma_peak": round(ops / (ms * 1e-3) / 5.0e15, 4),
                     "launches_per_call": 2, "note": "QACT A256 of the 512 rows + the Q4_K matrix-core kernel"}
        del ws, yb, x4

    # causal flash attention over 512 tokens (32 q / 8 KV heads, D 128, q8_0 KV); the
    # work list of 512 rows is copied to the device per call, so this one is timed eagerly
    T, n_head, n_kv_head, D = 512, 32, 8, 128
    E = n_kv_head * D
    kf = dev.upload(S.normal(S.seed_of("cfg4", "k"), T * E))
    vf = dev.upload(S.normal(S.seed_of("cfg4", "v"), T * E))
    idx = dev.upload(np.arange(T, dtype=np.int64))
    kc, vc = dev.kv(E, T), dev.kv(E, T)
    dev.kv_set_rows(kc, 0, kf, T, E, idx)
    dev.kv_set_rows(vc, 1, vf, T, E, idx)
    mask = np.full((T, T), -np.inf, np.float16)
    mask[np.tril_indices(T)] = 0
    msum = tsr_hip.msum_build_f16(mask)
    qb = dev.upload(S.normal(S.seed_of("cfg4", "q"), T * n_head * D).astype(np.float16).astype(np.float32))
    ob = dev.alloc(4 * T * n_head * D)
    scale = np.float32(1.0 / np.sqrt(D))
    ms = timed_eager(lambda i: dev.flash_attn(qb, T, n_head * D, kc, vc, D, n_head, n_kv_head, scale, msum, ob,
                                              n_head * D, new_runs=[[0, T]], stream=stream), 20)
    out["fa_prefill_causal_512_32q8kv_d128"] = {"us_per_call": round(ms * 1e3, 2), "launches_per_call": 3,
                                                "timing": "eager (host-built work list of 512 rows)"}
    return out


COPY_BYTES = 256 << 20          # calibration copy (device to device)
# the launches of the counter child, in dispatch order, and the per_op entry each one stands for
PMC_TAGS = {"gate|up": "gate|up", "down": "mul_mat down", "fa": "flash_attn"}


def pmc_child(reps: int = 3) -> int:
    """Counter-collection child (run under rocprofv3 --pmc): a device-to-device copy of COPY_BYTES,
    then, `reps` dispatches each, the decode model's layer-0 gate|up (28672x4096, RMS_NORM and SWIGLU
    fused) and down (4096x14336, residual addend) Q4_K matvecs as the decoder launches them, and the
    planned one-launch ROPE + SET_ROWS_KV + FLASH_ATTN_EXT of one layer at the bench's mid-run context
    (cells [0, pos] visible, the new cell pos), on the model's seeded weights and seeded cache rows."""
    cfg = LL.LLAMA3_8B
    wts = LL.SyntheticWeights(cfg)
    dev = tsr_hip.Device(0)
    ev = HipEvents()
    src, dst = dev.alloc(COPY_BYTES), dev.alloc(COPY_BYTES)
    src.fill(1)
    gu = np.stack([wts.quant("blk.0.ffn_gate.weight", cfg.n_ff, cfg.n_embd, cfg.wfmt),
                   wts.quant("blk.0.ffn_up.weight", cfg.n_ff, cfg.n_embd, cfg.wfmt)], axis=1).reshape(2 * cfg.n_ff, -1)
    w_gu = dev.weight(cfg.wfmt, gu, 2 * cfg.n_ff, cfg.n_embd)
    w_dn = dev.weight(cfg.wfmt, wts.quant("blk.0.ffn_down.weight", cfg.n_embd, cfg.n_ff, cfg.wfmt), cfg.n_embd, cfg.n_ff)
    xb, gb, yb = dev.upload(S.normal(S.seed_of("pmc", "x"), cfg.n_embd)), dev.alloc(8 * cfg.n_ff), dev.alloc(4 * cfg.n_embd)
    nw = dev.upload(wts.norm("blk.0.ffn_norm.weight"))
    # one layer's caches at the e2e shape, cells [0, pos) filled, the token at cell pos
    kv_size, pos = PMC_KV_SIZE, PMC_POS
    E, nq, w3 = cfg.E, cfg.n_q, cfg.n_q + 2 * cfg.E
    kc, vc = dev.kv(E, kv_size), dev.kv(E, kv_size)
    idx = dev.upload(np.arange(pos, dtype=np.int64))
    for which, kv in ((0, kc), (1, vc)):
        rows = dev.upload(S.normal(S.seed_of("pmc", f"kv{which}"), pos * E))
        dev.kv_set_rows(kv, which, rows, pos, E, idx)
        rows.free()
    qkv = dev.alloc(4 * w3)
    w_qkv = dev.weight(cfg.wfmt, np.concatenate([wts.quant(f"blk.0.attn_{t}.weight", N, cfg.n_embd, cfg.wfmt)
                                                 for t, N in (("q", nq), ("k", E), ("v", E))]), w3, cfg.n_embd)
    an = dev.upload(wts.norm("blk.0.attn_norm.weight"))
    params = dev.upload(LL.LlamaDecoder._params(pos))
    rtab, att, bad = dev.alloc(4 * cfg.head_dim), dev.alloc(4 * nq), dev.alloc(4).fill(0)
    plan = dev.fa_plan(cfg.head_dim, cfg.n_head, cfg.n_head_kv, 1, kv_size)
    plan.set(LL.msum_decode(pos, min(kv_size, (pos + 1 + 255) // 256 * 256)), np.array([[pos, pos + 1]], np.uint32))
    dev.rope_table(params.ptr, cfg.head_dim, cfg.rope_base, rtab)
    dev.sync()
    for _ in range(reps):
        assert ev.h.hipMemcpyAsync(dst.ptr, src.ptr, COPY_BYTES, 3, dev.stream) == 0   # 3: device to device
    ev.device_sync()
    for _ in range(reps):      # the decoder's gate|up: RMS_NORM + MUL in front, SWIGLU behind
        dev.mul_mat_norm(w_gu, xb, 1, cfg.n_embd, cfg.eps, nw, gb, cfg.n_ff, flags=tsr_hip.MM_GLU, stream=dev.stream)
    for _ in range(reps):      # the decoder's down, residual addend
        dev.mul_mat(w_dn, gb, 1, cfg.n_ff, yb, cfg.n_embd, add=xb, add_stride=cfg.n_embd, stream=dev.stream)
    for _ in range(reps):      # the decoder's attention launch (with its Q|K|V rows)
        dev.attn_qkv_plan_rope_tab(plan, w_qkv, xb, cfg.eps, an, qkv, kc, vc, np.float32(1.0 / np.sqrt(cfg.head_dim)),
                                   cfg.head_dim, cfg.rope_mode, rtab, params.ptr + 8, att, nq, bad=bad,
                                   stream=dev.stream)
    ev.device_sync()
    assert int(bad.read(np.int32, (1,))[0]) == 0
    plan.free()
    dev.close()
    return 0


# BASELINE configs[0]-[2] in the configs counter child: (name, kernel substring, algorithmic bytes per launch)
PMC_CONFIGS = [("q8_0_matvec_4864x896", "k_mv_q80", 4864 * 28 * 34 + 4 * 896 + 4 * 4864),
               ("q4k_up_14336x4096", "k_mv_q4k", 14336 * 16 * 144 + 4 * 4096 + 4 * 14336),
               ("q4k_down_4096x14336", "k_mv_q4k", 4096 * 56 * 144 + 4 * 14336 + 4 * 4096),
               ("fa_decode_q8kv_8192_32q8kv_d128", "k_fa_dec", 2 * 8192 * 1024 // 32 * 34 + 2 * 4096 + 4 * 4096)]


def pmc_configs_child(reps: int = 3) -> int:
    """Counter child for BASELINE configs[0]-[2] (run under rocprofv3 --pmc): the calibration copy, then
    `reps` launches each, over device copies that rotate (no launch finds its bytes in a cache the one
    before filled), of the Q8_0 matvec 4864 x 896, the Q4_K up 14336 x 4096 and down 4096 x 14336
    matvecs, and the planned FLASH_ATTN_EXT decode at 8192 cells (one k_fa_dec launch), with the seeds
    of the timed legs."""
    dev = tsr_hip.Device(0)
    ev = HipEvents()
    src, dst = dev.alloc(COPY_BYTES), dev.alloc(COPY_BYTES)
    src.fill(1)
    dev.sync()
    for _ in range(reps):
        assert ev.h.hipMemcpyAsync(dst.ptr, src.ptr, COPY_BYTES, 3, dev.stream) == 0
    ev.device_sync()
    src.free()
    dst.free()
    w8 = S.quant_rows(0, S.seed_of("cfg1", "w"), 4864, 896)
    ws = [dev.weight(0, w8, 4864, 896) for _ in range(reps)]
    xb, yb = dev.upload(S.normal(S.seed_of("cfg1", "x"), 896)), dev.alloc(4 * 14336)
    for i in range(reps):
        dev.mul_mat(ws[i], xb, 1, 896, yb, 4864)
    dev.sync()
    del ws
    for name, N, K in (("w_up", 14336, 4096), ("w_down", 4096, 14336)):
        blocks = S.quant_rows(1, S.seed_of("cfg2", name), N, K)
        ws = [dev.weight(1, blocks, N, K) for _ in range(reps)]
        xk = dev.upload(S.normal(S.seed_of("cfg2", "x" + name), K))
        for i in range(reps):
            dev.mul_mat(ws[i], xk, 1, K, yb, N)
        dev.sync()
        del ws
    n_kv, E, n_head, D = 8192, 1024, 32, 128
    idx = dev.upload(np.arange(n_kv, dtype=np.int64))
    caches = []
    for i in range(reps):
        kc, vc = dev.kv(E, n_kv), dev.kv(E, n_kv)
        for which, kv in ((0, kc), (1, vc)):
            rows = dev.upload(S.normal(S.seed_of("cfg3", "kv"[which]), n_kv * E))
            dev.kv_set_rows(kv, which, rows, n_kv, E, idx)
            rows.free()
        caches.append((kc, vc))
    qb = dev.upload(S.normal(S.seed_of("cfg3", "q"), n_head * D).astype(np.float16).astype(np.float32))
    ob = dev.alloc(4 * n_head * D)
    plan = dev.fa_plan(D, n_head, 8, 1, n_kv)
    plan.set(tsr_hip.msum_build_f16(np.zeros((1, n_kv), np.float16)))
    for i in range(reps):
        dev.flash_attn_plan(plan, qb, n_head * D, caches[i][0], caches[i][1], np.float32(1.0 / np.sqrt(D)), ob, n_head * D)
    dev.sync()
    assert dev.get_flags() == 0
    plan.free()
    dev.close()
    return 0


def measure_config_traffic(reps: int = 3) -> dict:
    """HBM bytes per launch of the configs[0]-[2] kernels: FETCH_SIZE and WRITE_SIZE (two rocprofv3
    --pmc passes over the configs child), each scaled by the counter's reading for the calibration copy;
    with each kernel's algorithmic bytes and their ratio."""
    if shutil.which("rocprofv3") is None:
        return {"error": "rocprofv3 not found"}
    workdir = tempfile.mkdtemp(prefix="tsr_pmc_")
    try:
        res = {name: {"algorithmic_bytes": ab} for name, _, ab in PMC_CONFIGS}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            rows = _pmc_pass(counter, workdir, "--pmc-configs-child")
            copy = sorted((v for _, k, v in rows if "copyBuffer" in k), reverse=True)[:reps]
            cal = COPY_BYTES / (float(np.median(copy)) * 1024.0)
            seen = {}
            for _, k, v in rows:
                for name, kern, _ in PMC_CONFIGS:
                    if kern in k:
                        seen.setdefault(kern, []).append(v)
                        break
            q4 = seen.get("k_mv_q4k", [])
            per = {"q8_0_matvec_4864x896": seen.get("k_mv_q80", []), "q4k_up_14336x4096": q4[:reps],
                   "q4k_down_4096x14336": q4[reps:], "fa_decode_q8kv_8192_32q8kv_d128": seen.get("k_fa_dec", [])}
            for name, vals in per.items():
                if len(vals) != reps:
                    raise RuntimeError(f"{counter}: {name}: {len(vals)} dispatches")
                res[name][counter] = round(float(np.median(vals)) * 1024.0 * cal)
            res["calibration_" + counter] = round(cal, 4)
        for name, _, ab in PMC_CONFIGS:
            r = res[name]
            r["traffic"] = r["FETCH_SIZE"] + r["WRITE_SIZE"]
            r["traffic_ratio"] = round(r["traffic"] / ab, 4)
        return res
    finally:
        shutil.rmtree(workdir, ignore_errors=True)


def _pmc_pass(counter: str, workdir: str, child: str = "--pmc-child") -> list:
    """One rocprofv3 --pmc pass over a child; returns [(dispatch id, kernel name, value)] of the
    counter in dispatch order. counter may name several counters (space separated): the rows then
    carry the counter's name as a fourth field."""
    names = counter.split()
    out = os.path.join(workdir, "pmc_" + "_".join(names))
    cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", *names, "--output-format", "csv",
           "-d", out, "-o", "pmc", "--", sys.executable, os.path.abspath(__file__), child]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, cwd=workdir)
    files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
    if r.returncode != 0 and not files:
        raise RuntimeError(f"rocprofv3 --pmc {counter} failed ({r.returncode}): {r.stdout[-400:]}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") in names:
                    rec = (int(row["Dispatch_Id"]), row["Kernel_Name"], float(row["Counter_Value"]))
                    rows.append(rec if len(names) == 1 else rec + (row["Counter_Name"],))
    return sorted(rows)


PREFILL_PMC = [("q8_0 512x4096x4096", 0, 4096, 4096, 0), ("q4_K 512x4096x14336", 1, 4096, 14336, 0),
               ("q4_K+GLU 512x28672x4096", 1, 28672, 4096, tsr_hip.MM_GLU)]


def pmc_prefill_child(reps: int = 2) -> int:
    """Counter child for the prefill matmuls of BASELINE configs[3]: `reps` launches each of the Q8_0
    512x4096x4096, Q4_K 512x4096x14336 and Q4_K + GLU 512x28672x4096 MUL_MATs (activation QACT kernel +
    matrix-core kernel), in that order."""
    dev = tsr_hip.Device(0)
    T = 512
    for name, fmt, N, K, flags in PREFILL_PMC:
        w = dev.weight(fmt, S.quant_rows(fmt, S.seed_of("pmc-prefill", name), N, K), N, K)
        x = dev.upload(S.normal(S.seed_of("pmc-prefill", "x" + name), T * K))
        ny = N // 2 if flags else N
        y = dev.alloc(4 * T * ny)
        for _ in range(reps):
            dev.mul_mat(w, x, T, K, y, ny, flags=flags)
        dev.sync()
        del w, x, y
    dev.close()
    return 0


def measure_prefill_counters(reps: int = 2) -> dict:
    """MFMA and VALU use of the prefill matrix-core kernels (one rocprofv3 --pmc pass: rocprofv3's
    derived MfmaUtil = MFMA-busy cycles / (GPU-active cycles x SIMDs) and VALUBusy = active VALU
    instruction cycles / CUs / GPU-active cycles, plus the MFMA and VALU instruction counts)."""
    if shutil.which("rocprofv3") is None:
        return {"error": "rocprofv3 not found"}
    workdir = tempfile.mkdtemp(prefix="tsr_pmc_")
    try:
        rows = _pmc_pass("MfmaUtil VALUBusy SQ_INSTS_MFMA SQ_INSTS_VALU", workdir, "--pmc-prefill-child")
        by = {}
        for did, k, v, name in rows:
            if "k_mm_" in k:
                by.setdefault(did, {"kernel": k.split("(")[0].replace("void ", "")})[name] = v
        disp = [by[d] for d in sorted(by)]
        if len(disp) != reps * len(PREFILL_PMC):
            raise RuntimeError(f"unexpected matrix-core dispatches: {len(disp)}")
        out = {}
        for i, (name, *_r) in enumerate(PREFILL_PMC):
            ds = disp[reps * i:reps * (i + 1)]
            out[name] = {"kernel": ds[-1]["kernel"],
                         "MfmaUtil_pct": round(float(np.median([d["MfmaUtil"] for d in ds])), 2),
                         "VALUBusy_pct": round(float(np.median([d["VALUBusy"] for d in ds])), 2),
                         "SQ_INSTS_MFMA": int(np.median([d["SQ_INSTS_MFMA"] for d in ds])),
                         "SQ_INSTS_VALU": int(np.median([d["SQ_INSTS_VALU"] for d in ds]))}
        return out
    finally:
        shutil.rmtree(workdir, ignore_errors=True)


def measure_traffic(reps: int = 3) -> dict:
    """HBM bytes per launch of the gate|up and down matvecs and of the decode attention launch (with the
    layer's Q|K|V rows):
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch, two separate rocprofv3 passes), each scaled by the
    same counter's reading for the calibration copy (COPY_BYTES read and COPY_BYTES written)."""
    if shutil.which("rocprofv3") is None:
        return {"error": "rocprofv3 not found"}
    workdir = tempfile.mkdtemp(prefix="tsr_pmc_")
    try:
        res = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            rows = _pmc_pass(counter, workdir)
            # the calibration copies: the `reps` largest copy dispatches (the uploads before them are
            # copies too, of at most a few MiB)
            copy = sorted((v for _, k, v in rows if "copyBuffer" in k), reverse=True)[:reps]
            mv = [v for _, k, v in rows if "k_mv_q4k" in k]
            fa = [v for _, k, v in rows if "k_fa" in k]
            if not copy or len(mv) != 2 * reps or len(fa) != reps:
                raise RuntimeError(f"{counter}: unexpected dispatches {[(k, v) for _, k, v in rows][:12]}")
            cal = COPY_BYTES / (float(np.median(copy)) * 1024.0)   # true bytes per counted byte
            res[counter] = {"calibration_factor": round(cal, 4), "copy_KiB": float(np.median(copy)),
                            "gate|up": float(np.median(mv[:reps])) * 1024.0 * cal,
                            "down": float(np.median(mv[reps:])) * 1024.0 * cal,
                            "fa": float(np.median(fa)) * 1024.0 * cal}
        return res
    finally:
        shutil.rmtree(workdir, ignore_errors=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode tokens before them (>= 2)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the other BASELINE configs")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc traffic passes")
    ap.add_argument("--eager", action="store_true",
                    help="time everything as direct launches: no HIP graph is built (so the adapter leg, which "
                         "replays a captured graph, is skipped too)")
    ap.add_argument("--no-adapter", action="store_true", help="skip the decode through the ggml-backend adapter")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-prefill-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-configs-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.pmc_child:
        return pmc_child()
    if args.pmc_configs_child:
        return pmc_configs_child()
    if args.pmc_prefill_child:
        return pmc_prefill_child()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (multi-GPU sharding is "
                                   "designed, not built or measured)"}))
        return 2
    if args.warmup < 2 or args.steps < 1:
        print(json.dumps({"error": "--warmup must be >= 2 (an eager token and the capturing replay) and --steps >= 1"}))
        return 2

    # traffic passes first: child processes under rocprofv3, before this process touches the GPU
    traffic = prefill_counters = config_traffic = None
    if not args.no_traffic:
        try:
            traffic = measure_traffic()
        except Exception as e:  # reported, not fatal: the timing below does not depend on it
            traffic = {"error": str(e)[:300]}
        if not args.no_extra:
            try:
                prefill_counters = measure_prefill_counters()
            except Exception as e:
                prefill_counters = {"error": str(e)[:300]}
            try:
                config_traffic = measure_config_traffic()
            except Exception as e:
                config_traffic = {"error": str(e)[:300]}

    dev = tsr_hip.Device(0)
    info = dev.info()
    stream = dev.stream
    ev = HipEvents()
    print(f"bench: e2e decode, {args.warmup} warmup + {args.steps} timed tokens after {CTX} cells", file=sys.stderr,
          flush=True)
    e2e = e2e_decode(dev, ev, args.steps, args.warmup, eager=args.eager)
    print(f"bench: {e2e['tok_s']:.1f} tok/s", file=sys.stderr, flush=True)
    per_op = e2e["per_op"]
    # the roofline kernel: the op class (one kernel each) with the largest share of a token
    dom = max(per_op, key=lambda k: per_op[k]["us_per_token"])
    dv = per_op[dom]
    tag = next((t for t, key in PMC_TAGS.items() if key in dom), None)
    traffic_bytes = None
    if tag and traffic and "error" not in traffic:
        traffic_bytes = round(traffic["FETCH_SIZE"][tag] + traffic["WRITE_SIZE"][tag])
    achieved = dv["algorithmic_bytes"] / (dv["launch_us"] * 1e-6) / 1e9
    m = e2e.pop("model")
    # the CPU leg decodes from the GPU's prefilled caches (the ggml q8_0 images, read back)
    caches = [(L["kc"].get_bytes(0), L["vc"].get_bytes(1)) for L in m.layers]
    e2e["caches"] = None if args.no_cpu else caches
    m.free()
    # the adapter always replays a captured graph: --eager (the kernel-trace profile's form) skips it
    adapter = None if (args.no_adapter or args.eager) else adapter_decode(ev, e2e, caches, args.steps)
    del caches

    also = {} if args.no_extra else extra_workloads(dev, ev, stream, 200, eager=args.eager)
    if prefill_counters is not None:
        also["prefill_counters"] = prefill_counters
    if config_traffic is not None:
        also["config_traffic"] = config_traffic
    if adapter is not None:
        also["adapter_decode_llama3_8b_q4k"] = adapter
    cpu = None if args.no_cpu else cpu_decode(e2e)
    if cpu is not None:
        print("bench: CPU baselines of configs[0]-[3]", file=sys.stderr, flush=True)
        cpu["per_config"] = cpu_configs(cpu["cores"])
    ms_tok = e2e["ms_per_token"]
    out = {
        "metric": METRIC,
        "value": round(e2e["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_tok, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q8_0 int8 dot products, f32 accumulate (spec f32 rules)",
        "data": ("synthetic: random-init weights N(0,0.02) quantized to Q4_K, KV prefilled from seeded random "
                 "token ids, greedy tokens"),
        "config": {"workload": "Llama-3-8B-arch Q4_K decode, batch 1, ctx 4096 (BASELINE configs[4])",
                   "layers": 32, "n_embd": 4096, "n_ff": 14336, "heads": "32 q / 8 kv, head_dim 128",
                   "n_vocab": 128256, "kv": "q8_0", "kv_cells_before_decode": CTX,
                   "timed_positions": [CTX + args.warmup, CTX + args.warmup + args.steps - 1],
                   "timing": ("direct launches per token (--eager)" if args.eager else
                              "one captured HIP graph per token, replayed") + "; HIP events on the launch stream",
                   "device": info["arch"], "n_cu": info["n_cu"]},
        "token": {"algorithmic_bytes": e2e["token_bytes"],
                  "GB/s": round(e2e["token_bytes"] / (ms_tok * 1e-3) / 1e9, 1),
                  "frac_of_hbm_peak": round(e2e["token_bytes"] / (ms_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "host_enqueue_ms": round(e2e["host_enqueue_ms_per_token"], 4),
                  "wall_ms": round(e2e["wall_ms_per_token"], 4),
                  "sum_of_ops_us": round(sum(v["us_per_token"] for v in per_op.values()), 1),
                  "per_op": per_op, "setup_s": round(e2e["setup_s"], 1)},
        "prefill": {"tokens": CTX, "ubatch": UBATCH, "seconds": round(e2e["prefill_s"], 3),
                    "tok_s": round(CTX / e2e["prefill_s"], 1),
                    "note": "untimed setup of the decode workload, wall clock including host planning"},
        "roofline": {"bound": "hbm", "kernel": f"{dv['kernel']} ({dom})", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes, "traffic_detail": traffic,
                     "launch_us": dv["launch_us"], "algorithmic_bytes": dv["algorithmic_bytes"]},
        "cpu_baseline": cpu,
        "also": also,
    }
    print(json.dumps(out))
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
