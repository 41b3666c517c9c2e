"""Writes tests/golden/hf_tiny_fp32_seed0.npz: an independent pin of the whole-model
composition, computed by Hugging Face transformers' LlamaForCausalLM (CPU, fp32, eager
attention) on the tiny config of BASELINE.json configs[0] with the build's seeded
synthetic weights.

transformers is a third-party implementation of the Llama architecture the reference
builds (model_graph_builder.cpp:133-415 follows the HF Llama layout: split-half RoPE,
repeat_kv GQA, RMSNorm with gain, SiLU-gated MLP, untied head).  Nothing of the
oracle's composition is reused here: only the weight values (the synthetic-data SPEC)
and the prompt ids come from the oracle library, so a wiring slip in the oracle (a
residual taken at the wrong point, RoPE after the KV write, a wrong GQA mapping) makes
tests/test_oracle.py disagree with this file.

Stored: the prompt, the 33 greedy tokens (prefill token + 32 decode steps), the full
logits of the prefill step, and per step the top-16 (index, value) pairs plus the
logits at every 97th vocabulary index.

With `gains`, writes tests/golden/hf_tiny_gains_fp32_seed0.npz instead: the same model
with non-unit RMSNorm gains, 1 + N(0, 0.1) from the synthetic stream, a different vector
for every norm (oracle_lib.norm_gains).  Unit gains cannot show which gain buffer a
norm applies; these pin the wiring (input vs post-attention gain of each layer, the
final norm's own gain).

Runs on the CPU in a few seconds:
    python tests/golden/make_hf_tiny_golden.py [gains]
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

N_TOKENS = 33
SAMPLE_STRIDE = 97
TOPK = 16

# tensor ids of the synthetic-data SPEC: ((layer + 1) << 8) | role
ROLES = {"self_attn.q_proj": 1, "self_attn.k_proj": 2, "self_attn.v_proj": 3, "self_attn.o_proj": 4,
         "mlp.gate_proj": 5, "mlp.up_proj": 6, "mlp.down_proj": 7}


def build_model(cfg, seed, gains=None):
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    hc = LlamaConfig(vocab_size=cfg["vocab"], hidden_size=cfg["hidden"], intermediate_size=cfg["ffn"],
                     num_hidden_layers=cfg["num_layers"], num_attention_heads=cfg["num_q_heads"],
                     num_key_value_heads=cfg["num_kv_heads"], head_dim=cfg["head_dim"],
                     max_position_embeddings=cfg["max_tokens"], rms_norm_eps=cfg["rms_eps"],
                     rope_theta=cfg["rope_theta"], tie_word_embeddings=False, attention_bias=False,
                     mlp_bias=False, hidden_act="silu")
    hc._attn_implementation = "eager"
    model = LlamaForCausalLM(hc).to(torch.float32).eval()
    sd = {}
    H, V = cfg["hidden"], cfg["vocab"]
    sd["model.embed_tokens.weight"] = O.synth_f32(seed, 0x01, V * H).reshape(V, H)
    sd["lm_head.weight"] = O.synth_f32(seed, 0x02, V * H).reshape(V, H)
    sd["model.norm.weight"] = np.ones(H, np.float32) if gains is None else gains["final"].astype(np.float32)
    for l in range(cfg["num_layers"]):
        for name, role in ROLES.items():
            shape = tuple(model.state_dict()[f"model.layers.{l}.{name}.weight"].shape)
            sd[f"model.layers.{l}.{name}.weight"] = O.synth_f32(seed, ((l + 1) << 8) | role,
                                                               shape[0] * shape[1]).reshape(shape)
        if gains is None:
            sd[f"model.layers.{l}.input_layernorm.weight"] = np.ones(H, np.float32)
            sd[f"model.layers.{l}.post_attention_layernorm.weight"] = np.ones(H, np.float32)
        else:
            sd[f"model.layers.{l}.input_layernorm.weight"] = gains["input"][l].astype(np.float32)
            sd[f"model.layers.{l}.post_attention_layernorm.weight"] = gains["post"][l].astype(np.float32)
    missing, unexpected = model.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=False)
    # rotary inv_freq buffers are not weights
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return model


def hf_greedy(model, prompt, n_new):
    """Greedy decode by full re-forward of the whole sequence each step (no KV cache:
    the HF cache is not under test)."""
    import torch

    ids = list(int(t) for t in prompt)
    toks, steps = [], []
    with torch.no_grad():
        for _ in range(n_new):
            out = model(torch.tensor([ids], dtype=torch.long), use_cache=False)
            logits = out.logits[0, -1].to(torch.float32).numpy().copy()
            t = int(np.argmax(logits))
            toks.append(t)
            steps.append(logits)
            ids.append(t)
    return np.array(toks, np.int64), steps


def main(with_gains=False):
    import torch

    torch.manual_seed(0)
    cfg = dict(O.TINY)
    prompt = O.token_ids(0, 0, cfg["vocab"], 16)
    gains = O.norm_gains(0, cfg["num_layers"], cfg["hidden"]) if with_gains else None
    model = build_model(cfg, 0, gains)
    toks, steps = hf_greedy(model, prompt, N_TOKENS)
    top_idx = np.stack([np.argsort(-s, kind="stable")[:TOPK] for s in steps]).astype(np.int64)
    top_val = np.stack([s[i] for s, i in zip(steps, top_idx)]).astype(np.float32)
    sample = np.stack([s[::SAMPLE_STRIDE] for s in steps]).astype(np.float32)
    gap = np.array([np.sort(s)[-1] - np.sort(s)[-2] for s in steps], np.float32)
    name = "hf_tiny_gains_fp32_seed0.npz" if with_gains else "hf_tiny_fp32_seed0.npz"
    np.savez(os.path.join(HERE, name), prompt=prompt, tokens=toks, prefill_logits=steps[0],
             top_idx=top_idx, top_val=top_val, sample=sample, sample_stride=np.int64(SAMPLE_STRIDE), top2_gap=gap)
    print("tokens", toks.tolist())
    print("min top-2 gap", float(gap.min()))


if __name__ == "__main__":
    main("gains" in sys.argv[1:])
