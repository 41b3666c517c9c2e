"""Which gain buffer each RMSNorm applies, on the GPU.

Every synthetic model has unit gains, so a decode or prefill plan that binds the input
norm's gain where the post-attention gain belongs, or the final norm to a layer's
gain, or drops one, passes every test that uses them.  Here the tiny model is written
out as a Hugging Face checkpoint with a different non-unit gain on every norm
(1 + N(0, 0.1), oracle_lib.norm_gains) and loaded through am_model_load_hf:

- fp32 (BASELINE.json configs[0] with gains): the 33 greedy tokens equal the ones
  transformers' LlamaForCausalLM produces on the same checkpoint
  (tests/golden/hf_tiny_gains_fp32_seed0.npz), and every step's logits are within 1e-3
  of the golden's largest |logit|;
- bf16 activations with INT4 g128 weights quantized while loading (the fused decode
  plan: norms in the q/k/v, gate/up and lm_head GEMV prologues): every step's logits
  are within the bf16 bar 2e-2 of the oracle built with the same gains, and the greedy
  tokens equal the oracle's.

The oracle's gain wiring is pinned against the same transformers golden, with planted
swaps that fail it (tests/test_oracle.py)."""

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
from test_hf_checkpoint import _model_tensors, bf16_bytes, make_dir  # noqa: E402

L = N.lib()
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "hf_tiny_gains_fp32_seed0.npz")


def _with_gains(tensors, gains, n_layers):
    t = dict(tensors)
    t["model.norm.weight"] = gains["final"].astype(np.float32)
    for l in range(n_layers):
        t[f"model.layers.{l}.input_layernorm.weight"] = gains["input"][l].astype(np.float32)
        t[f"model.layers.{l}.post_attention_layernorm.weight"] = gains["post"][l].astype(np.float32)
    return t


def _synthetic(rt, c, act, fmt, seed):
    mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                       c["vocab"], c["rms_eps"], c["rope_theta"], act, fmt, 128, c["max_tokens"], 16)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), seed, C.byref(m))
    return m


def _steps(m, prompt, n_steps, vocab):
    """Prefill, then one decode step at a time: (token, logits) of every step."""
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1)), C.byref(s))
    logits = np.zeros(vocab, np.float32)
    out = []
    try:
        tok = N.i64()
        L.call("am_session_prefill", s, prompt.ctypes.data, prompt.size, C.byref(tok))
        t = int(tok.value)
        for step in range(n_steps):
            if step > 0:
                one = np.zeros(1, np.int64)
                L.call("am_session_decode", s, 1, one.ctypes.data)
                t = int(one[0])
            L.call("am_session_logits", s, logits.ctypes.data)
            out.append((t, logits.copy()))
    finally:
        L.am_session_destroy(s)
    return out


def test_fp32_checkpoint_with_norm_gains_matches_transformers(tmp_path):
    g = np.load(GOLDEN)
    c = dict(O.TINY)
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    try:
        ms = _synthetic(rt, c, N.AM_DT_F32, N.AM_WF_F32, 0)
        tensors = _model_tensors(L, ms, c, torch)
        L.am_model_destroy(ms)
        gains = O.norm_gains(0, c["num_layers"], c["hidden"])
        d = str(tmp_path / "tiny_gains")
        make_dir(d, c, tensors=_with_gains(tensors, gains, c["num_layers"]),
                 cfg_kw={"rms_norm_eps": c["rms_eps"], "rope_theta": c["rope_theta"]})
        m = N.vp()
        L.call("am_model_load_hf", rt, d.encode(),
               C.byref(N.ModelLoadOptions(N.AM_DT_F32, N.AM_WF_F32, 128, c["max_tokens"], 16)), C.byref(m))
        # the gains reached their buffers
        hip = C.CDLL("libamdhip64.so.7")
        hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        for kind, layer, want in ((N.AM_BUF_IN_NORM, 1, gains["input"][1]), (N.AM_BUF_POST_NORM, 2, gains["post"][2]),
                                  (N.AM_BUF_FINAL_NORM, 0, gains["final"])):
            ptr, nb = N.vp(), N.i64()
            L.call("am_model_buffer", m, kind, layer, C.byref(ptr), C.byref(nb))
            got = np.empty(c["hidden"], np.float32)
            assert nb.value == got.nbytes and hip.hipMemcpy(got.ctypes.data, ptr.value, got.nbytes, 2) == 0
            assert np.array_equal(got, want.astype(np.float32)), kind
        prompt = np.ascontiguousarray(g["prompt"], np.int64)
        steps = _steps(m, prompt, len(g["tokens"]), c["vocab"])
        L.am_model_destroy(m)
    finally:
        L.am_runtime_destroy(rt)
    toks = [t for t, _ in steps]
    stride = int(g["sample_stride"])
    for step, (t, lg) in enumerate(steps):
        scale = float(np.max(np.abs(g["top_val"][step])))
        err = max(float(np.max(np.abs(lg[g["top_idx"][step]] - g["top_val"][step]))),
                  float(np.max(np.abs(lg[::stride] - g["sample"][step])))) / scale
        assert err <= 1e-3, f"step {step}: logits off by {err:.3e} of max |logit|"
    assert np.array_equal(np.array(toks), g["tokens"]), (toks, g["tokens"].tolist())


@pytest.mark.parametrize("graph", [1, 0])
def test_bf16_int4_checkpoint_with_norm_gains_matches_oracle(tmp_path, graph):
    c = dict(O.TINY, act="bf16", weight_format=N.AM_WF_INT4, ffn=1536, vocab=4096, num_layers=3, max_tokens=96)
    seed = 5
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    orc = O.OracleModel(c, seed)
    try:
        mb = _synthetic(rt, c, N.AM_DT_BF16, N.AM_WF_BF16, seed)  # bf16 values the INT4 weights quantize from
        tensors = _model_tensors(L, mb, c, torch)
        L.am_model_destroy(mb)
        gains = O.norm_gains(seed, c["num_layers"], c["hidden"])
        # the device stores gains in the activation dtype: give the oracle the same values
        gains = {k: O.round_bf16(v) for k, v in gains.items()}
        t = _with_gains(tensors, gains, c["num_layers"])
        tb = {n: (bf16_bytes(a), "BF16", list(a.shape)) for n, a in t.items()}  # exact: the values are bf16
        d = str(tmp_path / "tiny_gains_bf16")
        make_dir(d, c, tensors=tb, cfg_kw={"rms_norm_eps": c["rms_eps"], "rope_theta": c["rope_theta"]})
        m = N.vp()
        L.call("am_model_load_hf", rt, d.encode(),
               C.byref(N.ModelLoadOptions(N.AM_DT_BF16, N.AM_WF_INT4, 128, c["max_tokens"], 16)), C.byref(m))
        prompt = O.token_ids(seed, 3, c["vocab"], 21)
        n_steps = 24
        s = N.vp()
        L.call("am_session_open", m, C.byref(N.SessionOptions(1, graph)), C.byref(s))
        orc.set_gains(gains)
        logits = np.zeros(c["vocab"], np.float32)
        try:
            tok = N.i64()
            L.call("am_session_prefill", s, prompt.ctypes.data, prompt.size, C.byref(tok))
            got = int(tok.value)
            ref = orc.forward(prompt, 0)
            for step in range(n_steps):
                if step > 0:
                    one = np.zeros(1, np.int64)
                    L.call("am_session_decode", s, 1, one.ctypes.data)
                    got = int(one[0])
                    ref = orc.forward(np.array([want], np.int64), prompt.size + step - 1)
                L.call("am_session_logits", s, logits.ctypes.data)
                scale = float(np.max(np.abs(ref)))
                err = float(np.max(np.abs(logits - ref))) / scale
                assert err <= 2e-2, f"step {step}: logits off by {err:.3e} of max |logit|"
                want = O.argmax(ref)
                assert got == want, f"step {step}: token {got} != oracle {want}"
        finally:
            L.am_session_destroy(s)
        L.am_model_destroy(m)
    finally:
        orc.close()
        L.am_runtime_destroy(rt)
