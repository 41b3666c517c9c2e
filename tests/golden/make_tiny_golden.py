"""Writes tests/golden/tiny_fp32_seed0.npz from the CPU oracle.

tiny Llama (4 layers, hidden 512, 8/2 heads, head_dim 64,
FFN 1376, vocab 32000, theta 1e4, eps 1e-5), fp32, synthetic weights seed 0
(N(0, 0.02), RMSNorm gains 1.0), 16 uniform prompt ids (stream 0), greedy decode
33 tokens (the prefill token + 32 decode steps), KV capacity 256.  The reference
itself cannot run this (its Linear/RoPE/Attention kernels do not exist), so the
fixture comes from the oracle restatement; the oracle is pinned separately by the
reference's known-answer tests (tests/test_oracle.py).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402


def main():
    prompt = O.token_ids(0, 0, 32000, 16)
    m = O.OracleModel(O.TINY, 0)
    toks, logits = m.generate(prompt, 33)
    m.set_fast(True)
    fast_toks, _ = m.generate(prompt, 33)
    assert np.array_equal(toks, fast_toks), "fp64 and AVX2 oracle paths disagree"
    np.savez(os.path.join(HERE, "tiny_fp32_seed0.npz"), prompt=prompt, tokens=toks, last_logits=logits)
    print("tokens", toks.tolist())


if __name__ == "__main__":
    main()
