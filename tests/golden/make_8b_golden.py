"""Writes tests/golden/llama8b_<fmt>_seed1.npz: greedy decode of the Llama-3-8B-shaped
model (BASELINE.json configs[1..3]: 32 layers, hidden 4096, 32/8 heads, head_dim 128,
FFN 14336, vocab 128256, theta 5e5, eps 1e-5) computed by the CPU oracle on its AVX2
path (the reference's fp32 dot-product kernel, cpu_dot_product_avx2.cpp:8-40, with
bf16 rounding at every op boundary), for the GPU token-parity test
tests/test_gpu_8b_parity.py.

Workload: seeded synthetic weights (seed 1, N(0, 0.02) as bf16, quantized by the
build SPEC for int8 / int4), the 512 prompt ids of stream 0, the prefill token and 32
decode steps (33 tokens).  Stored per step: the greedy token, the top-16 (index, value)
logits, the gap between the two largest logits (a near-tie tells the test where a
divergence is admissible) and the logits at every 257th vocabulary index.

The same steps are then recomputed on the oracle's fp64-accumulation path, fed the same
tokens: the per-step error between the two paths (same metric as the GPU test) and
the steps where their greedy tokens differ measure how far two valid summation orders
of the same bf16 composition drift apart over 32 layers.  That spread sets the GPU
test's logit bar.

CPU only, all host cores; about 15 minutes per format:
    python tests/golden/make_8b_golden.py int4 [int8 bf16]
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

SHAPE = dict(num_layers=32, hidden=4096, num_q_heads=32, num_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
             rms_eps=1e-5, rope_theta=500000.0)
FORMATS = {"bf16": 1, "int8": 2, "int4": 3}
PROMPT = 512
STEPS = 33
TOPK = 16
SAMPLE_STRIDE = 257


def main(fmts):
    O.lib().orc_set_threads(os.cpu_count() or 8)
    prompt = O.token_ids(1, 0, SHAPE["vocab"], PROMPT)
    for fmt in fmts:
        t0 = time.time()
        cfg = dict(SHAPE, act="bf16", weight_format=FORMATS[fmt], group_size=128, max_tokens=PROMPT + STEPS + 8)
        m = O.OracleModel(cfg, 1)
        m.set_fast(True)
        print(f"[{fmt}] model built in {time.time() - t0:.0f} s", flush=True)
        toks, top_idx, top_val, gap, sample = [], [], [], [], []
        logits = m.forward(prompt, 0)
        for step in range(STEPS):
            if step > 0:
                logits = m.forward(np.array([toks[-1]], np.int64), PROMPT + step - 1)
            t = O.argmax(logits)
            order = np.argsort(-logits, kind="stable")[:TOPK]
            toks.append(t)
            top_idx.append(order)
            top_val.append(logits[order])
            gap.append(logits[order[0]] - logits[order[1]])
            sample.append(logits[::SAMPLE_STRIDE].copy())
            print(f"[{fmt}] step {step}: token {t} gap {gap[-1]:.4g} ({time.time() - t0:.0f} s)", flush=True)
        # the fp64 path over the same tokens (it rewrites every cache row it reads)
        m.set_fast(False)
        self_err, self_flip = [], []
        for step in range(STEPS):
            if step == 0:
                lg = m.forward(prompt, 0)
            else:
                lg = m.forward(np.array([toks[step - 1]], np.int64), PROMPT + step - 1)
            scale = float(np.max(np.abs(top_val[step])))
            e = max(float(np.max(np.abs(lg[top_idx[step]] - top_val[step]))),
                    float(np.max(np.abs(lg[::SAMPLE_STRIDE] - sample[step])))) / scale
            self_err.append(e)
            self_flip.append(int(O.argmax(lg) != toks[step]))
            print(f"[{fmt}] fp64 step {step}: error {e:.4g} token {'differs' if self_flip[-1] else 'same'} "
                  f"({time.time() - t0:.0f} s)", flush=True)
        m.close()
        np.savez(os.path.join(HERE, f"llama8b_{fmt}_seed1.npz"), prompt=prompt, tokens=np.array(toks, np.int64),
                 top_idx=np.array(top_idx, np.int64), top_val=np.array(top_val, np.float32),
                 top2_gap=np.array(gap, np.float32), sample=np.array(sample, np.float32),
                 sample_stride=np.int64(SAMPLE_STRIDE), self_err=np.array(self_err, np.float32),
                 self_flip=np.array(self_flip, np.int64))
        print(f"[{fmt}] tokens {toks}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or ["int4"])
