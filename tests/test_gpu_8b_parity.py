"""Full-depth token parity at the benchmark's model: the 32-layer Llama-3-8B-shaped
model (BASELINE.json configs[1..3]: hidden 4096, 32/8 heads of 128, FFN 14336, vocab
128256, theta 5e5; seeded synthetic weights, seed 1) run through the runtime's C ABI
(am_model_create_synthetic, am_session_prefill / am_session_decode with the fused
decode plan replayed as a HIP graph) against fixtures the CPU oracle wrote on its
AVX2 path (tests/golden/make_8b_golden.py): the 512 prompt ids of stream 0, the
prefill token and the next 32 greedy tokens.

Bars.  Greedy token ids identical to the oracle's, except at steps the oracle itself
cannot rank: a token may differ only at a step where the oracle's own top-two gap
(recorded in the fixture) is within the oracle's own measured error at that step; the
test then continues from the oracle's token by prefilling prompt + the oracle's tokens
so far, and every later step is held to the same bars.

The bars are calibrated by the oracle itself.  The fixture also holds the same 33
steps recomputed on the oracle's fp64-accumulation path: two valid summation orders of
the same bf16 composition, 32 layers deep, differ by 2-5% of the largest |logit|
(self_err, per step) and pick different greedy tokens at some near-ties (self_flip).
The GPU's summation order is a third one.  Its logit error may exceed the oracle's
largest self error by at most 25% at any step.  Which near-ties flip is chance: each of
the 12-15 steps the oracle cannot rank flips with some probability under any change of
order, so the count of divergences may be at most twice the oracle's own count (a
doubling of the flip rate fails).  Measured on the MI355X (divergences / oracle flips,
largest error / oracle's largest), register-staged prefill GEMM for INT8 and bf16:
int4 4 / 3, 4.05e-2 / 3.65e-2; int8 2 / 3, 4.53e-2 / 4.33e-2; bf16 3 / 5, 4.44e-2 /
4.32e-2; with the DMA-ring prefill GEMM and its fused epilogues for every format: bf16
7 / 5, 3.98e-2 / 4.32e-2; every divergence at a step the oracle cannot rank.  The
per-op 2e-2 bf16 bar of the north star holds op by op (test_gpu_decode_shapes.py); it
does not compose over 32 layers."""

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
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
SHAPE = dict(num_layers=32, hidden=4096, num_q_heads=32, num_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
             rms_eps=1e-5, rope_theta=500000.0)
FORMATS = {"int4": N.AM_WF_INT4, "int8": N.AM_WF_INT8, "bf16": N.AM_WF_BF16}
ERR_FACTOR = 1.25  # GPU logit error / the oracle's largest self error, per step


def _fixture(fmt):
    path = os.path.join(GOLDEN, f"llama8b_{fmt}_seed1.npz")
    if not os.path.exists(path):
        pytest.skip(f"no fixture {path}")
    return np.load(path)


def _logit_errors(logits, g, step):
    scale = float(np.max(np.abs(g["top_val"][step])))
    e_top = float(np.max(np.abs(logits[g["top_idx"][step]] - g["top_val"][step]))) / scale
    e_smp = float(np.max(np.abs(logits[::int(g["sample_stride"])] - g["sample"][step]))) / scale
    return max(e_top, e_smp), scale


@pytest.mark.parametrize("fmt", ["int4", "int8", "bf16"])
def test_8b_greedy_tokens_match_oracle(fmt):
    g = _fixture(fmt)
    prompt = np.ascontiguousarray(g["prompt"], np.int64)
    want = g["tokens"]
    n_steps = len(want)
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    mc = N.ModelConfig(SHAPE["num_layers"], SHAPE["hidden"], SHAPE["num_q_heads"], SHAPE["num_kv_heads"],
                       SHAPE["head_dim"], SHAPE["ffn"], SHAPE["vocab"], SHAPE["rms_eps"], SHAPE["rope_theta"],
                       N.AM_DT_BF16, FORMATS[fmt], 128, 1024, 512)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 1, C.byref(m))
    logits = np.zeros(SHAPE["vocab"], np.float32)
    self_err = g["self_err"].astype(np.float64)
    self_flips = int(np.sum(g["self_flip"]))
    tol = ERR_FACTOR * float(np.max(self_err))
    report = []
    try:
        step = 0
        divergences = 0
        while step < n_steps:
            # (re)start from the prompt plus the oracle's tokens before `step`
            s = N.vp()
            L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1)), C.byref(s))
            ctx = np.ascontiguousarray(np.concatenate([prompt, want[:step]]).astype(np.int64))
            tok = N.i64()
            L.call("am_session_prefill", s, ctx.ctypes.data, ctx.size, C.byref(tok))
            got = int(tok.value)
            restarted = False
            while True:
                L.call("am_session_logits", s, logits.ctypes.data)
                err, scale = _logit_errors(logits, g, step)
                gap = float(g["top2_gap"][step]) / scale
                report.append((step, got, int(want[step]), round(err, 5), round(gap, 5)))
                assert err <= tol, (f"{fmt} step {step}: logits off by {err:.3e} of max |logit|, above "
                                    f"{ERR_FACTOR} x the oracle's own {float(np.max(self_err)):.3e} ({report})")
                if got != int(want[step]):
                    assert gap <= self_err[step], (
                        f"{fmt} step {step}: token {got} != oracle {int(want[step])} where the oracle's top-2 gap "
                        f"{gap:.3e} exceeds its own error {self_err[step]:.3e} at that step ({report})")
                    divergences += 1
                    print(f"[8b parity {fmt}] divergence at step {step}: gap {gap:.4f}, gpu error {err:.4f}, "
                          f"oracle self error {self_err[step]:.4f}", flush=True)
                    step += 1
                    restarted = True
                    break
                step += 1
                if step >= n_steps:
                    break
                one = np.zeros(1, np.int64)
                L.call("am_session_decode", s, 1, one.ctypes.data)
                got = int(one[0])
            L.am_session_destroy(s)
            if not restarted:
                break
        worst = max(r[3] for r in report)
        summary = (f"[8b parity {fmt}] steps {n_steps}: near-tie divergences {divergences} (oracle fp64 vs AVX2: "
                   f"{self_flips}), max logit error {worst:.3e} (oracle fp64 vs AVX2: {float(np.max(self_err)):.3e})")
        print(summary, flush=True)
        assert divergences <= 2 * self_flips, f"{summary}: {report}"
    finally:
        L.am_model_destroy(m)
        L.am_runtime_destroy(rt)
