"""Writes tests/golden/llama8b_long_int4_seed1.npz: the long-context workload of
BASELINE.json configs[4] on a 2-layer model with the full Llama-3-8B layer shape
(hidden 4096, 32/8 heads of 128, FFN 14336, vocab 128256, theta 5e5, eps 1e-5; INT4
g128 weights quantized from the seed-1 N(0, 0.02) bf16 stream, bf16 activations), for
the GPU session test tests/test_gpu_long_context.py.

Workload: four sequences, each an 8192-token prompt (seed 1, streams 1..4) prefilled in
2048-token chunks into a 32768-position cache (the oracle forward runs chunk by chunk
at positions 0, 2048, 4096, 6144), then 16 greedy decode steps; the GPU test decodes the
four together at batch 4.  Stored per sequence and step (17 steps: the prefill token
and 16 decode tokens): the greedy token, the top-16 (index, value) logits, the gap
between the two largest logits and the logits at every 257th vocabulary index.

The sequences are independent, so each one runs through the oracle on its own; a
forward at position 0 overwrites every cache row the next sequence reads.

The same steps are then recomputed on the oracle's fp64-accumulation path fed the same
tokens (self_err, self_flip): how far two valid summation orders of the same bf16
composition drift apart at this depth and context, which the GPU test reports beside
its own error.

CPU only; about an hour with 6 threads:
    python tests/golden/make_long_golden.py [threads]
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

SHAPE = dict(num_layers=2, hidden=4096, num_q_heads=32, num_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
             rms_eps=1e-5, rope_theta=500000.0, act="bf16", weight_format=3, group_size=128, max_tokens=32768)
SEED = 1
BATCH = 4
PROMPT = 8192
CHUNK = 2048
STEPS = 17
TOPK = 16
SAMPLE_STRIDE = 257


def run(m, prompt, toks=None):
    """Chunked prefill then decode; with `toks`, feeds those tokens instead of the
    argmax (the fp64 recomputation).  Returns the logits of every step."""
    out = []
    logits = None
    for c in range(0, PROMPT, CHUNK):
        logits = m.forward(prompt[c:c + CHUNK], c)
    out.append(logits)
    cur = O.argmax(logits) if toks is None else int(toks[0])
    for step in range(1, STEPS):
        logits = m.forward(np.array([cur], np.int64), PROMPT + step - 1)
        out.append(logits)
        cur = O.argmax(logits) if toks is None else int(toks[step])
    return out


def main(threads):
    O.lib().orc_set_threads(threads)
    t0 = time.time()
    m = O.OracleModel(SHAPE, SEED)
    print(f"model built in {time.time() - t0:.0f} s", flush=True)
    prompts = np.stack([O.token_ids(SEED, 1 + r, SHAPE["vocab"], PROMPT) for r in range(BATCH)])
    toks = np.zeros((BATCH, STEPS), np.int64)
    top_idx = np.zeros((BATCH, STEPS, TOPK), np.int64)
    top_val = np.zeros((BATCH, STEPS, TOPK), np.float32)
    gap = np.zeros((BATCH, STEPS), np.float32)
    sample = np.zeros((BATCH, STEPS, (SHAPE["vocab"] + SAMPLE_STRIDE - 1) // SAMPLE_STRIDE), np.float32)
    m.set_fast(True)
    for r in range(BATCH):
        for step, lg in enumerate(run(m, prompts[r])):
            order = np.argsort(-lg, kind="stable")[:TOPK]
            toks[r, step] = O.argmax(lg)
            top_idx[r, step] = order
            top_val[r, step] = lg[order]
            gap[r, step] = lg[order[0]] - lg[order[1]]
            sample[r, step] = lg[::SAMPLE_STRIDE]
        print(f"seq {r}: tokens {toks[r].tolist()} min gap {gap[r].min():.4g} ({time.time() - t0:.0f} s)",
              flush=True)
    self_err = np.zeros((BATCH, STEPS), np.float32)
    self_flip = np.zeros((BATCH, STEPS), np.int64)
    m.set_fast(False)
    for r in range(BATCH):
        for step, lg in enumerate(run(m, prompts[r], toks[r])):
            scale = float(np.max(np.abs(top_val[r, step])))
            self_err[r, step] = max(float(np.max(np.abs(lg[top_idx[r, step]] - top_val[r, step]))),
                                    float(np.max(np.abs(lg[::SAMPLE_STRIDE] - sample[r, step])))) / scale
            self_flip[r, step] = int(O.argmax(lg) != toks[r, step])
        print(f"seq {r} fp64: max error {self_err[r].max():.4g} flips {int(self_flip[r].sum())} "
              f"({time.time() - t0:.0f} s)", flush=True)
    m.close()
    np.savez(os.path.join(HERE, "llama8b_long_int4_seed1.npz"), prompts=prompts.astype(np.int32), tokens=toks,
             top_idx=top_idx, top_val=top_val, top2_gap=gap, sample=sample, sample_stride=np.int64(SAMPLE_STRIDE),
             chunk=np.int64(CHUNK), self_err=self_err, self_flip=self_flip)
    print(f"done in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else (os.cpu_count() or 8))
