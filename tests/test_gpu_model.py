"""End-to-end parity of the gfx950 runtime (C ABI am_runtime / am_model / am_session)
against the CPU oracle model: greedy token ids identical for the first 32 decode
steps on the tiny config, through the fused decode plan
replayed as a HIP graph and through the one-kernel-per-reference-node plan."""

import ctypes as C
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402

L = N.lib()
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "tiny_fp32_seed0.npz")


class Runtime:
    def __init__(self):
        self.rt = N.vp()
        L.call("am_runtime_open", 0, C.byref(self.rt))

    def model(self, cfg: dict, seed: int):
        mc = N.ModelConfig(cfg["num_layers"], cfg["hidden"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                           cfg["ffn"], cfg["vocab"], cfg["rms_eps"], cfg["rope_theta"],
                           N.AM_DT_BF16 if cfg["act"] == "bf16" else N.AM_DT_F32, cfg["weight_format"],
                           cfg.get("group_size", 128), cfg["max_tokens"], cfg.get("chunk", 64))
        m = N.vp()
        L.call("am_model_create_synthetic", self.rt, C.byref(mc), seed, C.byref(m))
        return m

    def session(self, m, fused=1, graph=1):
        s = N.vp()
        L.call("am_session_open", m, C.byref(N.SessionOptions(fused, graph)), C.byref(s))
        return s


def gpu_generate(rt, m, prompt, n_new, fused=1, graph=1):
    s = rt.session(m, fused, graph)
    toks = np.zeros(n_new, np.int64)
    nout = N.i64()
    L.call("am_session_generate_ids", s, prompt.ctypes.data, prompt.size, n_new, -1, toks.ctypes.data, C.byref(nout))
    logits = np.zeros(m_vocab(rt, m), np.float32)
    L.call("am_session_logits", s, logits.ctypes.data)
    L.am_session_destroy(s)
    return toks, logits


_vocab = {}


def m_vocab(rt, m):
    return _vocab[m.value]


@pytest.fixture(scope="module")
def tiny():
    rt = Runtime()
    cfg = dict(O.TINY)
    cfg["chunk"] = 16
    m = rt.model(cfg, 0)
    _vocab[m.value] = cfg["vocab"]
    prompt = O.token_ids(0, 0, cfg["vocab"], 16)
    g = np.load(GOLDEN)
    yield rt, m, prompt, g
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt.rt)


def test_tiny_prompt_matches_golden(tiny):
    rt, m, prompt, g = tiny
    assert np.array_equal(prompt, g["prompt"])


@pytest.mark.parametrize("fused,graph", [(1, 1), (0, 1), (1, 0), (0, 0)])
def test_tiny_greedy_tokens_match_oracle(tiny, fused, graph):
    rt, m, prompt, g = tiny
    toks, logits = gpu_generate(rt, m, prompt, 33, fused, graph)
    assert np.array_equal(toks, g["tokens"][:33]), (toks, g["tokens"])
    ref = g["last_logits"]
    err = np.max(np.abs(logits - ref)) / np.max(np.abs(ref))
    assert err < 1e-3, err


def test_tiny_chunked_prefill_matches(tiny):
    """A prompt longer than the prefill chunk is processed in chunks (KV positions carry over)."""
    rt, m, prompt, g = tiny
    long_prompt = O.token_ids(0, 5, 32000, 40)
    orc = O.OracleModel(O.TINY, 0)
    ref, _ = orc.generate(long_prompt, 8)
    toks, _ = gpu_generate(rt, m, long_prompt, 8)
    assert np.array_equal(toks, ref)


@pytest.mark.parametrize("act,fmt", [("bf16", N.AM_WF_BF16), ("bf16", N.AM_WF_INT8), ("bf16", N.AM_WF_INT4),
                                     ("f32", N.AM_WF_INT4)])
def test_small_quantized_model_logits(act, fmt):
    """Tiny-shaped model with bf16 activations / quantized weights: logits after a
    prefill and 4 decode steps within the bf16 bar of the oracle fed the same tokens."""
    cfg = dict(O.TINY, act=act, weight_format=fmt, ffn=1536, vocab=4096, num_layers=2, max_tokens=64, chunk=8)
    rt = Runtime()
    m = rt.model(cfg, 3)
    _vocab[m.value] = cfg["vocab"]
    prompt = O.token_ids(3, 0, cfg["vocab"], 12)
    s = rt.session(m, 1, 1)
    first = N.i64()
    L.call("am_session_prefill", s, prompt.ctypes.data, prompt.size, C.byref(first))
    orc = O.OracleModel(cfg, 3)
    ref_logits = orc.forward(prompt, 0)
    got = np.zeros(cfg["vocab"], np.float32)
    L.call("am_session_logits", s, got.ctypes.data)
    tol = 2e-2 if act == "bf16" else 1e-3
    assert np.max(np.abs(got - ref_logits)) / np.max(np.abs(ref_logits)) < tol
    tok = int(first.value)
    pos = prompt.size
    for _ in range(4):
        out = np.zeros(1, np.int64)
        L.call("am_session_decode", s, 1, out.ctypes.data)
        ref_logits = orc.forward(np.array([tok], np.int64), pos)
        L.call("am_session_logits", s, got.ctypes.data)
        assert np.max(np.abs(got - ref_logits)) / np.max(np.abs(ref_logits)) < tol
        tok = int(out[0])
        pos += 1
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt.rt)
