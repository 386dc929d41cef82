"""End-to-end decode on the GPU (tsr_llama.LlamaDecoder over the C ABI) against the same decode
composed from the oracle's ops (oracle/oracle_llama.py): logits bit for bit at every step and the
same greedy tokens, on small models with the 8B model's shape rules."""
import ctypes as C

import numpy as np
import pytest

import tsr_hip as H
import tsr_llama as LL
from helpers import assert_bits_equal
from oracle_llama import OracleLlama

pytestmark = pytest.mark.gpu

_libm = C.CDLL("libm.so.6")
_libm.powf.argtypes = [C.c_float, C.c_float]
_libm.powf.restype = C.c_float


def oracle_model(oc, cfg, w, kv_size, hist, threads=1):
    t = {"token_embd.weight": w.embedding(), "output_norm.weight": w.norm("output_norm.weight")[None],
         "output.weight": w.quant("output.weight", cfg.n_vocab, cfg.n_embd, cfg.ofmt)}
    for il in range(cfg.n_layer):
        for name, N, K in LL.layer_tensors(cfg, il):
            t[name] = w.quant(name, N, K, cfg.wfmt)
        for nm in ("attn_norm", "ffn_norm"):
            t[f"blk.{il}.{nm}.weight"] = w.norm(f"blk.{il}.{nm}.weight")[None]
    m = OracleLlama(oc, n_layer=cfg.n_layer, n_embd=cfg.n_embd, n_ff=cfg.n_ff, n_head=cfg.n_head,
                    n_head_kv=cfg.n_head_kv, head_dim=cfg.head_dim, n_vocab=cfg.n_vocab, eps=cfg.eps,
                    rope_base=cfg.rope_base, rope_mode=cfg.rope_mode, wfmt=cfg.wfmt, ofmt=cfg.ofmt, tensors=t,
                    kv_size=kv_size, threads=threads)
    for il in range(cfg.n_layer):
        for which in (0, 1):
            m.set_history(il, which, w.kv_history(il, which, hist))
    return m


@pytest.mark.parametrize("cfg,kv_size,hist,n_steps", [
    (LL.tiny_config(), 512, 100, 5),
    (LL.tiny_config("tiny-qwen", wfmt=H.FMT_Q8_0, ofmt=H.FMT_Q8_0, rope_mode=H.ROPE_NEOX, eps=1e-6,
                    rope_base=1000000.0), 640, 300, 4),
    (LL.tiny_config("tiny-gqa8", n_head=8, n_head_kv=1, head_dim=128, n_embd=512, n_ff=768, n_vocab=1000), 300, 255, 3),
], ids=["q4k-norm", "q80-neox", "gqa8-d128"])
@pytest.mark.parametrize("fused", [True, False], ids=["fused", "separate"])
def test_decode_matches_oracle(dev, oc, cfg, kv_size, hist, n_steps, fused):
    w = LL.SyntheticWeights(cfg)
    print(f"\ndecode parity {cfg.name} fused={fused}: kv {kv_size} history {hist} steps {n_steps}", flush=True)
    gpu = LL.LlamaDecoder(dev, cfg, w, kv_size, fused=fused)
    gpu.prefill_history(w, hist)
    ref = oracle_model(oc, cfg, w, kv_size, hist)
    ts = np.float32(_libm.powf(float(np.float32(cfg.rope_base)), float(np.float32(-2.0) / np.float32(cfg.head_dim))))
    tok = 7
    for i in range(n_steps):
        pos = hist + i
        n_kv = min(kv_size, (pos + 1 + 255) // 256 * 256)
        gpu.step(tok if i == 0 else None, pos)
        got = gpu.read_logits()
        want = ref.step(tok, pos, ts, n_kv)
        assert_bits_equal(got, want, f"{cfg.name} step {i} (pos {pos})")
        nxt = gpu.read_next()
        assert nxt == int(oc.argmax(want[None])[0])
        tok = nxt
    for il in range(cfg.n_layer):                                 # the caches hold the same bytes
        assert (gpu.layers[il]["kc"].get_bytes(0).reshape(kv_size, -1) == ref.kc[il]).all()
        assert (gpu.layers[il]["vc"].get_bytes(1).reshape(kv_size, -1) == ref.vc[il]).all()
    assert gpu.bad.read(np.int32, (1,))[0] == 0
    gpu.free()


@pytest.mark.parametrize("cfg,kv_size,hist,n_steps", [
    (LL.tiny_config(), 300, 254, 5),              # cells 255 .. 259: the plan grows a second chunk at 257
    (LL.tiny_config("tiny-qwen", wfmt=H.FMT_Q8_0, ofmt=H.FMT_Q8_0, rope_mode=H.ROPE_NEOX, eps=1e-6,
                    rope_base=1000000.0), 640, 300, 3),
    (LL.tiny_config("tiny-kv8", n_head=16, n_head_kv=8, head_dim=64, n_embd=512, n_ff=768, n_vocab=1000), 300, 254,
     4),                                          # 8 KV heads: Q|K|V inside the attention launch
], ids=["q4k-norm-grow", "q80-neox", "q4k-kv8"])
def test_decode_graph_matches_oracle(dev, oc, cfg, kv_size, hist, n_steps):
    """The same decode as one graph replay per token: FLASH_ATTN_EXT from the device-resident plan, the
    position / cell and the plan copied in stream order, the greedy token fed back on the device."""
    w = LL.SyntheticWeights(cfg)
    print(f"\ngraph decode parity {cfg.name}: kv {kv_size} history {hist} steps {n_steps}", flush=True)
    gpu = LL.LlamaDecoder(dev, cfg, w, kv_size)
    gpu.prefill_history(w, hist)
    ref = oracle_model(oc, cfg, w, kv_size, hist)
    ts = np.float32(_libm.powf(float(np.float32(cfg.rope_base)), float(np.float32(-2.0) / np.float32(cfg.head_dim))))
    tok = 11
    for i in range(n_steps):
        pos = hist + i
        n_kv = min(kv_size, (pos + 1 + 255) // 256 * 256)
        gpu.step_graph(tok if i == 0 else None, pos)
        got = gpu.read_logits()
        want = ref.step(tok, pos, ts, n_kv)
        assert_bits_equal(got, want, f"{cfg.name} graph step {i} (pos {pos})")
        tok = gpu.read_token()
        assert tok == int(oc.argmax(want[None])[0])
    assert gpu.captures == (2 if hist < 256 < hist + n_steps else 1)
    gpu.free()


def test_decode_graph_runs_ahead(dev):
    """Tokens queued without waiting (generate_graph) equal tokens decoded one replay at a time."""
    cfg = LL.tiny_config()
    w = LL.SyntheticWeights(cfg)
    a = LL.LlamaDecoder(dev, cfg, w, 256)
    a.prefill_history(w, 40)
    hist = dev.alloc(4 * 12)
    a.generate_graph(3, 40, 12, hist)
    dev.sync()
    fast = hist.read(np.int32, (12,))
    a.free()
    b = LL.LlamaDecoder(dev, cfg, w, 256)
    b.prefill_history(w, 40)
    slow = []
    for i in range(12):
        b.step(3 if i == 0 else None, 40 + i)
        slow.append(b.read_next())
    b.free()
    assert list(fast) == slow


@pytest.mark.parametrize("cfg,kv_size,hist,n_prompt,ubatch,fused", [
    (LL.tiny_config(), 512, 0, 70, 32, True),                  # ubatches of 32, 32, 6 from cell 0
    (LL.tiny_config(), 400, 40, 50, 512, False),               # one ubatch after a history, separate ops
    (LL.tiny_config("tiny-qwen", wfmt=H.FMT_Q8_0, ofmt=H.FMT_Q8_0, rope_mode=H.ROPE_NEOX, eps=1e-6,
                    rope_base=1000000.0), 640, 200, 90, 40, True),   # Q8_0: the matrix-core MUL_MATs
    (LL.tiny_config("tiny-gqa8", n_head=8, n_head_kv=1, head_dim=128, n_embd=512, n_ff=768, n_vocab=1000),
     300, 0, 260, 256, True),                                  # a second chunk of the causal rows
], ids=["q4k-3ub", "q4k-separate-hist", "q80-neox-hist", "gqa8-d128-2ub"])
def test_prefill_matches_oracle(dev, oc, cfg, kv_size, hist, n_prompt, ubatch, fused):
    """Prefill of a prompt in ubatches (every op over the ubatch's rows, the causal mask) against the
    oracle's forward of the same ubatches: the last token's logits bit for bit, the same cache bytes, the
    same greedy token; then one graph-replayed decode token from the prefilled caches."""
    w = LL.SyntheticWeights(cfg)
    print(f"\nprefill parity {cfg.name} fused={fused}: kv {kv_size} history {hist} prompt {n_prompt} "
          f"ubatch {ubatch}", flush=True)
    gpu = LL.LlamaDecoder(dev, cfg, w, kv_size, fused=fused)
    if hist:
        gpu.prefill_history(w, hist)
    ref = oracle_model(oc, cfg, w, kv_size, hist)
    ts = np.float32(_libm.powf(float(np.float32(cfg.rope_base)), float(np.float32(-2.0) / np.float32(cfg.head_dim))))
    toks = np.random.default_rng(n_prompt).integers(0, cfg.n_vocab, n_prompt).astype(np.int32)
    gpu.prefill(toks, hist, ubatch=ubatch)
    for u0 in range(0, n_prompt, ubatch):
        T = min(ubatch, n_prompt - u0)
        want = ref.forward(toks[u0:u0 + T], hist + u0, ts, min(kv_size, (hist + u0 + T + 255) // 256 * 256))
    assert_bits_equal(gpu.read_logits(), want, f"{cfg.name} prefill logits")
    nxt = int(oc.argmax(want[None])[0])
    assert gpu.read_next() == nxt and gpu.read_token() == nxt
    for il in range(cfg.n_layer):
        assert (gpu.layers[il]["kc"].get_bytes(0).reshape(kv_size, -1) == ref.kc[il]).all(), f"K cache, layer {il}"
        assert (gpu.layers[il]["vc"].get_bytes(1).reshape(kv_size, -1) == ref.vc[il]).all(), f"V cache, layer {il}"
    pos = hist + n_prompt
    gpu.step_graph(None, pos)
    want = ref.step(nxt, pos, ts, min(kv_size, (pos + 1 + 255) // 256 * 256))
    assert_bits_equal(gpu.read_logits(), want, f"{cfg.name} decode after prefill")
    assert gpu.bad.read(np.int32, (1,))[0] == 0
    gpu.free()


def test_prefill_refusals(dev):
    cfg = LL.tiny_config()
    gpu = LL.LlamaDecoder(dev, cfg, LL.SyntheticWeights(cfg), 64)
    with pytest.raises(ValueError):
        gpu.prefill(np.zeros(0, np.int32))
    with pytest.raises(ValueError):
        gpu.prefill(np.zeros(10, np.int32), 60)
    gpu.free()


def test_decode_llama3_8b_token_matches_oracle(dev, oc):
    """BASELINE configs[4] at its full shape: the Llama-3-8B-architecture Q4_K model (32 layers, n_embd
    4096, n_ff 14336, 32 q / 8 KV heads of 128, vocabulary 128256), q8_0 caches holding a short history,
    one decode token eagerly and the same token by graph replay (the form the bench times): all 128256
    logits bit-equal to the oracle composition's step, and the same greedy token."""
    cfg = LL.LLAMA3_8B
    hist, kv_size = 100, 256
    w = LL.SyntheticWeights(cfg, cache=True)        # one generation of the 4.5 GB of blocks for both sides
    print(f"\n8B decode parity: history {hist}, kv {kv_size}", flush=True)
    gpu = LL.LlamaDecoder(dev, cfg, w, kv_size)
    gpu.prefill_history(w, hist)
    ref = oracle_model(oc, cfg, w, kv_size, hist, threads=16)
    ts = np.float32(_libm.powf(float(np.float32(cfg.rope_base)), float(np.float32(-2.0) / np.float32(cfg.head_dim))))
    tok, pos = 1234, hist
    n_kv = min(kv_size, (pos + 1 + 255) // 256 * 256)
    want = ref.step(tok, pos, ts, n_kv)
    print("8B decode parity: oracle token done", flush=True)
    gpu.step(tok, pos)
    assert_bits_equal(gpu.read_logits(), want, "8B eager step")
    assert gpu.read_next() == int(oc.argmax(want[None])[0])
    gpu.step_graph(tok, pos)                        # rewrites cell pos with the same rows
    assert_bits_equal(gpu.read_logits(), want, "8B graph step")
    assert gpu.read_token() == int(oc.argmax(want[None])[0])
    for il in (0, cfg.n_layer - 1):                 # the new cell's K / V bytes
        assert (gpu.layers[il]["kc"].get_bytes(0).reshape(kv_size, -1)[pos] == ref.kc[il][pos]).all()
        assert (gpu.layers[il]["vc"].get_bytes(1).reshape(kv_size, -1)[pos] == ref.vc[il][pos]).all()
    gpu.free()
    w.cache.clear()


def test_decode_flag_raises(dev):
    """A token id outside the embedding table raises the decoder's flag (GET_ROWS stores nothing): the
    next read raises DecodeError naming it, and the flag is cleared for the steps after it."""
    cfg = LL.tiny_config()
    gpu = LL.LlamaDecoder(dev, cfg, LL.SyntheticWeights(cfg), 64)
    gpu.step_graph(cfg.n_vocab + 5, 3)
    with pytest.raises(LL.DecodeError, match="out of range"):
        gpu.read_token()
    gpu.step_graph(5, 4)
    gpu.read_token()
    gpu.free()
