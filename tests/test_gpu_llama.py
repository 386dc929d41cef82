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


def oracle_model(oc, cfg, w, kv_size, hist):
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
                    kv_size=kv_size)
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
], ids=["q4k-norm-grow", "q80-neox"])
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
