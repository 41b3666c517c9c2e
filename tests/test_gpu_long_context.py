"""The long-context workload of BASELINE.json configs[4], run through the session
against an oracle fixture (tests/golden/make_long_golden.py): a 2-layer model with
the full Llama-3-8B layer shape and vocabulary (INT4 g128, bf16 activations, seed 1),
a 32768-position KV cache, four 8192-token prompts (streams 1..4) each prefilled into
its own sequence with am_session_prefill_row in 2048-token chunks (chunk carry-over
across four chunks), then 16 greedy steps decoded together at batch 4
(am_session_decode) at context 8192..8208.  Once with contiguous per-sequence KV
slots, once with a paged cache of 64-position blocks.

Bars, per sequence and step: logits within the north star's bf16 bar, 2e-2 of the
step's largest |logit| (the top-16 entries and every 257th vocabulary entry the
fixture holds); greedy tokens identical to the oracle's, except at a step the oracle
itself cannot rank (its own top-2 gap within its own fp64-vs-AVX2 error at that step,
self_err): that sequence is then no longer compared (its context has left the
fixture's), and such divergences may number at most twice the oracle's own flips on
this workload (self_flip; 2 of 68 steps, at 2 of the 8 steps it cannot rank)."""

import ctypes as C
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402

L = N.lib()
FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "llama8b_long_int4_seed1.npz")
SHAPE = dict(num_layers=2, hidden=4096, num_q_heads=32, num_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
             rms_eps=1e-5, rope_theta=500000.0)
TOL = 2e-2


def _errors(logits, g, r, step):
    scale = float(np.max(np.abs(g["top_val"][r, step])))
    e_top = float(np.max(np.abs(logits[g["top_idx"][r, step]] - g["top_val"][r, step])))
    e_smp = float(np.max(np.abs(logits[::int(g["sample_stride"])] - g["sample"][r, step])))
    return max(e_top, e_smp) / scale, float(g["top2_gap"][r, step]) / scale


@pytest.mark.parametrize("kv_block", [0, 64])
def test_long_context_batch4_session_matches_oracle(kv_block):
    if not os.path.exists(FIXTURE):
        pytest.skip(f"no fixture {FIXTURE}")
    g = np.load(FIXTURE)
    prompts = g["prompts"].astype(np.int64)
    B, P = prompts.shape
    steps = g["tokens"].shape[1]
    chunk = int(g["chunk"])
    V = SHAPE["vocab"]
    for r in range(B):  # the fixture's prompts are the synthetic-data SPEC's streams 1..4
        ids = np.zeros(P, np.int64)
        L.call("am_synth_token_ids_host", 1, 1 + r, V, P, ids.ctypes.data)
        assert np.array_equal(ids, prompts[r]), r
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    mc = N.ModelConfig(SHAPE["num_layers"], SHAPE["hidden"], SHAPE["num_q_heads"], SHAPE["num_kv_heads"],
                       SHAPE["head_dim"], SHAPE["ffn"], V, SHAPE["rms_eps"], SHAPE["rope_theta"], N.AM_DT_BF16,
                       N.AM_WF_INT4, 128, 32768, chunk)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 1, C.byref(m))
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1, B, 0, kv_block, 0)), C.byref(s))
    report = []
    live = [True] * B
    divergences = 0
    worst = 0.0
    try:
        got = np.zeros((B, V), np.float32)

        def check(r, step, token):
            nonlocal divergences, worst
            err, gap = _errors(got[r], g, r, step)
            worst = max(worst, err)
            want = int(g["tokens"][r, step])
            report.append((r, step, token, want, round(err, 5), round(gap, 5)))
            assert err <= TOL, f"seq {r} step {step}: logits off by {err:.3e} of max |logit| ({report[-8:]})"
            if token != want:
                own = float(g["self_err"][r, step])
                assert gap <= own, (f"seq {r} step {step}: token {token} != oracle {want} where the oracle's top-2 "
                                    f"gap {gap:.3e} exceeds its own error {own:.3e} at that step (GPU error {err:.3e})")
                divergences += 1
                live[r] = False

        for r in range(B):
            first = N.i64()
            L.call("am_session_prefill_row", s, r, prompts[r].ctypes.data, P, C.byref(first))
            assert L.am_session_row_position(s, r) == P
            L.call("am_session_logits", s, got.ctypes.data)
            check(r, 0, int(first.value))
        for step in range(1, steps):
            out = np.zeros((B, 1), np.int64)
            L.call("am_session_decode", s, 1, out.ctypes.data)
            L.call("am_session_logits", s, got.ctypes.data)
            for r in range(B):
                assert L.am_session_row_position(s, r) == P + step
                if live[r]:
                    check(r, step, int(out[r, 0]))
        self_flips = int(np.sum(g["self_flip"]))
        print(f"[long context kv_block={kv_block}] {B} sequences x {steps} steps: max logit error {worst:.3e} "
              f"(oracle fp64 vs AVX2: {float(np.max(g['self_err'])):.3e}), near-tie divergences {divergences} "
              f"(oracle fp64 vs AVX2 flips: {self_flips})", flush=True)
        assert divergences <= 2 * self_flips, (f"{divergences} divergences, oracle's own flips {self_flips}, max "
                                               f"error {worst:.3e}: {report}")
    finally:
        L.am_session_destroy(s)
        L.am_model_destroy(m)
        L.am_runtime_destroy(rt)
