#!/usr/bin/env python3
"""Benchmark: batch-1 greedy decode tokens/s of the Llama-3-8B-shaped INT4 model on one
MI355X (32 layers, hidden 4096, 32/8 heads, head_dim 128,
FFN 14336, vocab 128256, theta 5e5, INT4 group-128 fp16 scales, batch 1, prompt 512,
decode 256), plus the weight-GEMV HBM roofline and the CPU oracle baseline.

One "step" = one decode token through the fused decode plan (embedding, 32 x
[norm+qkv+rope+kv, attention, o+add, norm+gate/up+silu, down+add], norm+lm_head+argmax),
replayed as a HIP graph from device-resident state.  Inputs (weights, KV cache, prompt
state) are resident in HBM before the timed region; the timed region is K graph replays
bracketed by device synchronisation.

Prints ONE JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.
"""

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth

FORMAT_LABEL = {"int4": "INT4", "int8": "INT8", "bf16": "bf16"}
GEMV_KIND = {"int4": "weight-only INT4 g128 dequant", "int8": "weight-only INT8 per-channel dequant",
             "bf16": "bf16-weight"}
CONFIGS = {
    "int4": dict(weight_format=3, name="llama3-8b-shape-int4-g128", decode=256),
    "int8": dict(weight_format=2, name="llama3-8b-shape-int8-perchannel", decode=128),
    "bf16": dict(weight_format=1, name="llama3-8b-shape-bf16", decode=128),
}
SHAPE = dict(num_layers=32, hidden=4096, num_q_heads=32, num_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
             rms_eps=1e-5, rope_theta=500000.0)
# OpType values of the fused decode steps (host/am_core.h)
OP_NAMES = {1: "Embedding", 2: "RmsNorm", 3: "Linear", 5: "RoPE", 6: "Attention", 8: "SiluMul", 10: "KVCacheUpdate",
            11: "Add", 13: "Argmax", 17: "FusedRmsNormQkvRoPEKVUpdate", 18: "FusedLinearAdd",
            19: "FusedRmsNormGateUpSiluMul", 20: "FusedRmsNormLmHeadArgmax", 21: "EmbedToken"}
GEMV_OPS = (17, 18, 19, 20)
GATE_UP_OP = 19  # the dominant decode kernel: the gate/up GEMV, 2 x ffn rows per layer
# the gate/up GEMV's kernel in the committed PMC traffic summary, per weight format
GATE_UP_KERNEL = {3: "gemv_kernel<ActBF16, 3, true, 3,", 2: "gemv_kernel<ActBF16, 2, true, 3,",
                  1: "gemv_kernel<ActBF16, 1, true, 3,"}


def weight_row_bytes(weight_format: int, k: int, group: int = 128) -> int:
    """HBM bytes of one weight row of k values in the device formats (INT4: nibbles plus
    one fp16 scale per group; INT8: bytes plus an fp32 row scale; bf16: 2 bytes)."""
    if weight_format == 3:
        return k // 2 + 2 * (k // group)
    if weight_format == 2:
        return k + 4
    return 2 * k


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def cpu_baseline(weight_format: int, seconds_budget: float = 20.0, pos: int = 512, sequences: int = 1):
    """Oracle restatement of the reference CPU path (AVX2 dot product inner loop,
    dequantize-on-the-fly rows), 1 thread, on a bounded sample of the same decode
    workload: one 8B-shape layer + the full lm_head, timed per decode token at
    position ~pos, then scaled to the 32-layer token (t_token = t_rest + 32 * t_layer).
    The cache rows before pos are left as the model allocated them (zeros): a decode
    step's cost does not depend on their values.  With sequences > 1 the reference's
    CPU path decodes each sequence on its own, so the aggregate rate equals the
    single-sequence rate (reported as such)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np

    import oracle_lib as O

    L = O.lib()
    res = {}
    for layers in (1, 2):
        cfg = dict(SHAPE, num_layers=layers, act="bf16", weight_format=weight_format, group_size=128,
                   max_tokens=pos + 88)
        L.orc_set_threads(min(16, os.cpu_count() or 1))     # weight generation only (untimed)
        m = O.OracleModel(cfg, 1)
        m.set_fast(True)
        L.orc_set_threads(1)
        prompt = O.token_ids(1, 0, SHAPE["vocab"], 4)
        m.forward(prompt, pos - 4)                            # fill a few cache rows before pos
        times = []
        t_start = time.perf_counter()
        tok = np.array([int(prompt[-1])], np.int64)
        p = pos
        while len(times) < 3 and time.perf_counter() - t_start < seconds_budget / 2:
            t0 = time.perf_counter()
            m.forward(tok, p)
            times.append(time.perf_counter() - t0)
            p += 1
        res[layers] = min(times)
        m.close()
    t_layer = max(res[2] - res[1], 1e-9)
    t_rest = max(res[1] - t_layer, 0.0)
    t_token = t_rest + SHAPE["num_layers"] * t_layer
    cpu = _cpu_model_name()
    return {
        "value": round(1.0 / t_token, 4),
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle AVX2 path, 1 thread on {cpu} (nproc={os.cpu_count()}): decode tokens at pos {pos} of "
                   f"1-layer and 2-layer 8B-shape models with the full lm_head; t_layer={t_layer*1e3:.1f} ms, "
                   f"t_rest={t_rest*1e3:.1f} ms, scaled to 32 layers = {t_token*1e3:.0f} ms/token" +
                   (f"; {sequences} sequences decode one after another, so the aggregate rate is the same"
                    if sequences > 1 else "")),
    }


GEMV_SHAPES = [(4096, 4096, "q/o"), (1024, 4096, "k/v"), (14336, 4096, "gate or up"), (4096, 14336, "down"),
               (128256, 4096, "lm_head")]


def _cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_plan(all_cores: int):
    """The rest of the CPU-baseline plan, on the same oracle restatement of the
    reference CPU path (AVX2 dot product and RMSNorm, rows dequantized on the fly):
    - the tiny fp32 config end to end (prefill 16, greedy
      decode 32) on one thread, with its tokens checked against the committed golden;
    - the decode GEMV of each 8B shape in bf16, INT8 and INT4 (the reference's
      benchmark harness pattern: benchmark_cpu_dot_product_avx2.cpp:21-36, timed
      repeats of one kernel), one thread, and again on `all_cores` threads, labelled
      apart (the reference's OpenMP pragmas are inert in its build, so one thread is
      the reference's own figure)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np

    import oracle_lib as O

    L = O.lib()
    out = {"cpu": _cpu_model_name(), "nproc": os.cpu_count()}
    # tiny end to end
    L.orc_set_threads(1)
    m = O.OracleModel(O.TINY, 0)
    m.set_fast(True)
    prompt = O.token_ids(0, 0, O.TINY["vocab"], 16)
    t0 = time.perf_counter()
    logits = m.forward(prompt, 0)
    t_prefill = time.perf_counter() - t0
    toks = [O.argmax(logits)]
    t0 = time.perf_counter()
    for i in range(32):
        logits = m.forward(np.array([toks[-1]], np.int64), 16 + i)
        toks.append(O.argmax(logits))
    t_decode = time.perf_counter() - t0
    m.close()
    golden = None
    try:
        g = np.load(os.path.join(ROOT, "tests", "golden", "tiny_fp32_seed0.npz"))
        golden = bool(np.array_equal(np.array(toks, np.int64), g["tokens"]))
    except OSError:
        pass
    out["tiny_end_to_end"] = {"threads": 1, "prefill_tokens": 16, "prefill_ms": round(t_prefill * 1e3, 2),
                              "decode_tokens": 32, "decode_tokens_per_s": round(32 / t_decode, 2),
                              "tokens": toks, "tokens_equal_committed_golden": golden}

    def sweep(threads):
        L.orc_set_threads(threads)
        rows = []
        for n, k, role in GEMV_SHAPES:
            x = np.random.default_rng(n + k).standard_normal(k).astype(np.float32)
            y = np.empty(n, np.float32)
            for fmt, fname in ((1, "bf16"), (2, "int8"), (3, "int4")):
                q = L.orc_qweight_create(n, k, fmt, 128, 1)
                if not q:
                    raise RuntimeError("orc_qweight_create failed")
                L.orc_qweight_gemv(q, O.ptr(x), O.ptr(y))  # first touch
                best = 1e9
                for _ in range(2):
                    t0 = time.perf_counter()
                    L.orc_qweight_gemv(q, O.ptr(x), O.ptr(y))
                    best = min(best, time.perf_counter() - t0)
                nb = int(L.orc_qweight_bytes(q))
                L.orc_qweight_destroy(q)
                rows.append({"n": n, "k": k, "role": role, "format": fname, "bytes": nb, "ms": round(best * 1e3, 3),
                             "gbs": round(nb / best / 1e9, 3)})
        return rows

    out["gemv_1_thread"] = sweep(1)
    out["gemv_all_cores"] = {"threads": all_cores, "label": "all cores (not the reference's configuration)",
                             "results": sweep(all_cores)}
    L.orc_set_threads(1)
    return out


def calibrate_copy(mib: int) -> None:
    """Device-to-device copy of a known size (the HIP runtime's copy kernel), three
    times: the reference dispatch for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipFree.argtypes = [C.c_void_p]
    n = mib << 20
    a, b = C.c_void_p(), C.c_void_p()
    if hip.hipMalloc(C.byref(a), n) != 0 or hip.hipMalloc(C.byref(b), n) != 0:
        raise SystemExit("hipMalloc failed")
    for _ in range(3):
        if hip.hipMemcpy(b, a, n, 3) != 0:  # hipMemcpyDeviceToDevice
            raise SystemExit("hipMemcpy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)
    print(json.dumps({"calibrate_copy_bytes": n}), flush=True)


def measured_traffic(name: str):
    """The committed rocprofv3 PMC summary profiles/<name>.json of this workload, as
    (summary dict or None, provenance).  Provenance names the commit the counters were
    taken at and whether the native library's sources have changed since (the summary
    records their digest), in which case the byte counts describe older code."""
    path = os.path.join(ROOT, "profiles", f"{name}.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None, {"source": None}
    from aethermind_amd.profiling import source_digest
    return d, {"source": f"profiles/{name}.json", "commit": d.get("commit"),
               "stale": d.get("source_digest") != source_digest()}


def attention_pmc(summary):
    """PMC bytes and measured GB/s of the decode attention kernel from a traffic summary"""
    if not summary:
        return None
    for name, k in summary.get("per_kernel", {}).items():
        if name.startswith("attention_decode_kernel"):
            out = {"kernel": name, "pmc_bytes_per_launch": round(k["fetch_bytes_avg"] + k["write_bytes_avg"])}
            if "duration_ns_avg" in k:
                out["trace_us_per_launch"] = round(k["duration_ns_avg"] / 1e3, 2)
                out["measured_gbs"] = round(k["achieved_gbs"], 1)
            return out
    return None


def run_long(args, N, L):
    """8B-shape INT4, static KV cache of 32768 bf16 positions
    per sequence, four sequences of 8192 prompt ids (seed 1, streams 1..4) prefilled in
    2048-token chunks, then batch-4 greedy decode.  Reports aggregate decode tokens/s,
    the decode-attention KV bandwidth and the weight-GEMV bandwidth."""
    import numpy as np
    B, P, CHUNK, CAP = 4, args.prompt if args.prompt != 512 else 8192, 2048, 32768
    steps = args.steps if args.steps is not None else 256
    if P + args.warmup + steps + args.profile_steps + 2 > CAP:
        raise SystemExit("prompt + warmup + steps + profile exceed the 32768-token KV cache")
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    mc = N.ModelConfig(SHAPE["num_layers"], SHAPE["hidden"], SHAPE["num_q_heads"], SHAPE["num_kv_heads"],
                       SHAPE["head_dim"], SHAPE["ffn"], SHAPE["vocab"], SHAPE["rms_eps"], SHAPE["rope_theta"],
                       N.AM_DT_BF16, 3, 128, CAP, CHUNK)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 1, C.byref(m))
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1, B, 0, args.kv_block, 0)), C.byref(s))
    prompts = []
    for r in range(B):
        pr = np.empty(P, np.int64)
        L.call("am_synth_token_ids_host", 1, r + 1, SHAPE["vocab"], P, pr.ctypes.data)
        prompts.append(pr)
    first = N.i64()
    L.call("am_session_prefill_row", s, 0, prompts[0].ctypes.data, P, C.byref(first))  # warm
    t0 = time.perf_counter()
    for r in range(B):
        L.call("am_session_prefill_row", s, r, prompts[r].ctypes.data, P, C.byref(first))
        log(f"prefill seq {r}: {P} tokens in {CHUNK}-token chunks, first token {first.value}")
    prefill_s = time.perf_counter() - t0
    log(f"prefill {B} x {P} tokens: {prefill_s:.2f} s ({B * P / prefill_s:.0f} tok/s)")
    warm = np.zeros((B, max(args.warmup, 1)), np.int64)
    L.call("am_session_decode", s, max(args.warmup, 1), warm.ctypes.data)
    L.call("am_runtime_synchronize", rt)
    t0 = time.perf_counter()
    L.call("am_session_decode_async", s, steps)
    L.call("am_runtime_synchronize", rt)
    L.call("am_session_decode", s, 0, None)
    dt = time.perf_counter() - t0
    ms_per_step = dt * 1e3 / steps
    tok_s = B * steps / dt
    ctx_mid = P + max(args.warmup, 1) + steps / 2
    log(f"decode: {steps} steps x {B} sequences in {dt*1e3:.1f} ms -> {tok_s:.1f} tok/s aggregate "
        f"({ms_per_step:.3f} ms/step, context ~{ctx_mid:.0f})")
    ms_by_op = (C.c_double * 64)()
    cnt_by_op = (C.c_int64 * 64)()
    L.call("am_session_profile_decode", s, args.profile_steps, ms_by_op, cnt_by_op)
    ctx_prof = P + max(args.warmup, 1) + steps + args.profile_steps / 2
    breakdown = {OP_NAMES.get(i, str(i)): {"ms_per_step": round(ms_by_op[i] / args.profile_steps, 4),
                                           "launches_per_step": cnt_by_op[i] // args.profile_steps}
                 for i in range(64) if cnt_by_op[i]}
    for k, v in breakdown.items():
        log(f"  {k:32s} {v['ms_per_step']:8.4f} ms/step  x{v['launches_per_step']}")
    attn_ms = ms_by_op[6] / args.profile_steps
    kv_bytes = B * ctx_prof * SHAPE["num_layers"] * SHAPE["num_kv_heads"] * SHAPE["head_dim"] * 2 * 2
    attn_gbs = kv_bytes / (attn_ms * 1e-3) / 1e9
    gemv_ms = sum(ms_by_op[i] for i in GEMV_OPS) / args.profile_steps
    weight_bytes = L.am_model_weight_bytes_total(m)
    gemv_gbs = weight_bytes / (gemv_ms * 1e-3) / 1e9
    log(f"decode attention: {attn_ms:.3f} ms/step for {kv_bytes/1e9:.2f} GB of KV -> {attn_gbs:.0f} GB/s; "
        f"weight GEMVs {gemv_ms:.3f} ms/step -> {gemv_gbs:.0f} GB/s")
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)
    step_bytes = weight_bytes + kv_bytes
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(3, pos=P + 64, sequences=B)
            log(f"cpu baseline: {cpu['value']} tok/s ({cpu['sample']})")
        except Exception as e:  # the GPU figures stand without it
            log(f"cpu baseline failed: {e}")
    pmc, prov = measured_traffic("attention_long_decode_traffic")
    att = attention_pmc(pmc)
    out = {
        "metric": "batch-4 long-context decode tokens/sec (aggregate), Llama-3-8B-shape INT4, KV 32768",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-w/bf16-act/fp32-acc",
        "data": "synthetic (seeded N(0,0.02) weights generated on device, seeded uniform prompt ids)",
        "config": {"workload": f"llama3-8b-shape-int4-g128, {B} sequences x {P} prompt ids prefilled in {CHUNK}-token "
                               f"chunks, batch-{B} greedy decode, {steps} timed steps, KV cache {CAP} bf16",
                   "kv": f"paged, {args.kv_block}-position blocks" if args.kv_block else "contiguous slot per sequence",
                   "model": "llama3-8b-shape-int4-g128", "global_batch": B, "seq_len": P,
                   "parallelism": "none (1 GPU)", "prefill_s": round(prefill_s, 3),
                   "prefill_tokens_per_s": round(B * P / prefill_s, 1)},
        "roofline": {"bound": "hbm", "achieved": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": (att["pmc_bytes_per_launch"] * SHAPE["num_layers"]) if att else None,
                     "traffic_unit": "HBM bytes per step of the decode attention launches (rocprofv3 PMC, "
                                     "copy-scaled, one launch per layer)",
                     "traffic_provenance": prov, "attention_pmc": att,
                     "bytes_per_step": int(step_bytes), "attention_ms_per_step": round(attn_ms, 4),
                     "attention_kv_gbs": round(attn_gbs, 1), "gemv_ms_per_step": round(gemv_ms, 4),
                     "gemv_weight_gbs": round(gemv_gbs, 1)},
        "breakdown": breakdown,
        "cpu_baseline": cpu,
        "host": platform.node(),
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode tokens (default: config decode length)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="int4", choices=sorted(CONFIGS) + ["long"],
                    help="int4 (the headline), int8, bf16, or long (configs[4]: batch-4 decode over 8192-token prompts)")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--profile-steps", type=int, default=16)
    ap.add_argument("--kv-block", type=int, default=0,
                    help="paged KV with blocks of this many positions (0: one contiguous slot per sequence)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (PMC counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs the decode path on one GPU only; --gpus must be 1 "
              "(multi-GPU sharding is described in DESIGN.md, not implemented)", file=sys.stderr)
        sys.exit(2)

    import aethermind_amd.native as N

    L = N.lib()
    if args.config == "long":
        run_long(args, N, L)
        return
    cfgd = CONFIGS[args.config]
    steps = args.steps if args.steps is not None else cfgd["decode"]
    max_tokens = 4096
    if args.prompt + args.warmup + steps + args.profile_steps + 2 > max_tokens:
        raise SystemExit("prompt + warmup + steps + profile exceed the 4096-token KV cache")

    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    mc = N.ModelConfig(SHAPE["num_layers"], SHAPE["hidden"], SHAPE["num_q_heads"], SHAPE["num_kv_heads"],
                       SHAPE["head_dim"], SHAPE["ffn"], SHAPE["vocab"], SHAPE["rms_eps"], SHAPE["rope_theta"],
                       N.AM_DT_BF16, cfgd["weight_format"], 128, max_tokens, 512)
    t0 = time.perf_counter()
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 1, C.byref(m))
    log(f"model {cfgd['name']} created in {time.perf_counter() - t0:.1f}s; linear weight bytes/token "
        f"{L.am_model_weight_bytes_total(m)}")
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1, 1, 0, args.kv_block, 0)), C.byref(s))

    import numpy as np
    prompt = np.empty(args.prompt, np.int64)
    # prompt ids of the build SPEC (seed 1, stream 0)
    L.call("am_synth_token_ids_host", 1, 0, SHAPE["vocab"], args.prompt, prompt.ctypes.data)

    def sync():
        L.call("am_runtime_synchronize", rt)

    first = N.i64()
    L.call("am_session_prefill", s, prompt.ctypes.data, prompt.size, C.byref(first))  # warm (JIT/caches)
    t0 = time.perf_counter()
    L.call("am_session_prefill", s, prompt.ctypes.data, prompt.size, C.byref(first))
    prefill_s = time.perf_counter() - t0
    log(f"prefill {args.prompt} tokens: {prefill_s*1e3:.1f} ms ({args.prompt/prefill_s:.0f} tok/s), first token "
        f"{first.value}")

    warm = np.zeros(max(args.warmup, 1), np.int64)
    L.call("am_session_decode", s, max(args.warmup, 1), warm.ctypes.data)  # captures + replays the graph
    L.call("am_session_decode", s, 0, None)
    sync()

    t0 = time.perf_counter()
    L.call("am_session_decode_async", s, steps)
    sync()
    L.call("am_session_decode", s, 0, None)
    dt = time.perf_counter() - t0
    ms_per_step = dt * 1e3 / steps
    tok_s = steps / dt
    log(f"decode: {steps} tokens in {dt*1e3:.1f} ms -> {tok_s:.1f} tok/s ({ms_per_step:.3f} ms/token), "
        f"{L.am_session_decode_plan_size(s)} kernels/token")

    # Per-kernel durations of the same decode plan right after the timed region: each
    # weight GEMV launch carries start/stop HIP events bound to its dispatch on the
    # session stream (hipExtLaunchKernelGGL); other steps are bracketed by events.
    ms_by_op = (C.c_double * 64)()
    cnt_by_op = (C.c_int64 * 64)()
    L.call("am_session_profile_decode", s, args.profile_steps, ms_by_op, cnt_by_op)
    breakdown = {OP_NAMES.get(i, str(i)): {"ms_per_token": round(ms_by_op[i] / args.profile_steps, 4),
                                           "launches_per_token": cnt_by_op[i] // args.profile_steps}
                 for i in range(64) if cnt_by_op[i]}
    gemv_ms = sum(ms_by_op[i] for i in GEMV_OPS) / args.profile_steps
    gemv_launches = sum(cnt_by_op[i] for i in GEMV_OPS) // args.profile_steps
    weight_bytes = L.am_model_weight_bytes_total(m)
    if gemv_ms <= 0.0:
        raise SystemExit("profile pass returned no GEMV time")
    achieved = weight_bytes / (gemv_ms * 1e-3) / 1e9
    log(f"weight GEMVs: {gemv_ms:.3f} ms/token over {gemv_launches} launches -> {achieved:.0f} GB/s "
        f"({achieved / HBM_PEAK_GBS:.1%} of {HBM_PEAK_GBS:.0f})")
    for k, v in breakdown.items():
        log(f"  {k:32s} {v['ms_per_token']:8.4f} ms/token  x{v['launches_per_token']}")

    plan_size = L.am_session_decode_plan_size(s)
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(cfgd["weight_format"])
            log(f"cpu baseline: {cpu['value']} tok/s ({cpu['sample']})")
        except Exception as e:  # the GPU figures stand without it
            log(f"cpu baseline failed: {e}")
        if cpu is not None:
            try:
                t0 = time.perf_counter()
                cpu["plan"] = cpu_baseline_plan(min(16, os.cpu_count() or 1))
                te = cpu["plan"]["tiny_end_to_end"]
                log(f"cpu tiny end to end (1 thread): prefill 16 in {te['prefill_ms']} ms, decode "
                    f"{te['decode_tokens_per_s']} tok/s, tokens equal golden: {te['tokens_equal_committed_golden']}")
                for r in cpu["plan"]["gemv_1_thread"]:
                    log(f"cpu gemv 1 thread {r['n']}x{r['k']} {r['format']}: {r['ms']} ms, {r['gbs']} GB/s")
                log(f"cpu baseline plan took {time.perf_counter() - t0:.1f} s")
            except Exception as e:
                log(f"cpu baseline plan failed: {e}")

    pmc, prov = measured_traffic(f"gemv_{args.config}_decode_traffic")
    # The dominant kernel (the bench contract's roofline): the gate/up GEMV, timed by
    # the dispatch-bound events of the profile pass; algorithmic bytes per launch = its
    # 2 x ffn weight rows of hidden values.
    gu_launches = cnt_by_op[GATE_UP_OP] // args.profile_steps
    if gu_launches <= 0:
        raise SystemExit("profile pass returned no gate/up GEMV launches")
    gu_us = ms_by_op[GATE_UP_OP] / args.profile_steps / gu_launches * 1e3
    gu_bytes = 2 * SHAPE["ffn"] * weight_row_bytes(cfgd["weight_format"], SHAPE["hidden"])
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    gu_pmc = None
    if pmc:
        for name, k in pmc.get("per_kernel", {}).items():
            if name.startswith(GATE_UP_KERNEL[cfgd["weight_format"]]):
                gu_pmc = round(k["fetch_bytes_avg"] + k["write_bytes_avg"])
    dominant = max(GEMV_OPS, key=lambda i: ms_by_op[i])
    if dominant != GATE_UP_OP:
        log(f"note: the slowest GEMV step this run is {OP_NAMES.get(dominant)}, not the gate/up GEMV")
    log(f"gate/up GEMV: {gu_us:.2f} us per launch, {gu_bytes} B -> {gu_gbs:.0f} GB/s "
        f"({gu_gbs / HBM_PEAK_GBS:.1%} of {HBM_PEAK_GBS:.0f})")
    out = {
        "metric": (f"batch-1 decode tokens/sec, Llama-3-8B-shape {FORMAT_LABEL[args.config]}; "
                   "GEMV HBM GB/s vs peak"),
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"int4": "int4-w/bf16-act/fp32-acc", "int8": "int8-w/bf16-act/fp32-acc",
                  "bf16": "bf16"}[args.config],
        "data": "synthetic (seeded N(0,0.02) weights generated on device, seeded uniform prompt ids)",
        "config": {"workload": f"{cfgd['name']} batch-1 greedy decode, prompt {args.prompt}, "
                               f"{steps} timed decode tokens after {args.warmup} warmup, KV cache 4096 bf16",
                   "model": cfgd["name"], "global_batch": 1, "seq_len": args.prompt, "parallelism": "none (1 GPU)",
                   "prefill_ms": round(prefill_s * 1e3, 2), "kernels_per_token": plan_size,
                   "kv": f"paged, {args.kv_block}-position blocks" if args.kv_block else "contiguous"},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": gu_pmc,
                     "traffic_unit": "HBM bytes per gate/up launch (rocprofv3 PMC, copy-scaled)",
                     "traffic_provenance": prov,
                     "kernel": f"gate/up GEMV ({GEMV_KIND[args.config]}; RMSNorm prologue, SiLU-Mul epilogue), "
                               f"the dominant decode kernel",
                     "bytes_per_launch": gu_bytes, "us_per_launch": round(gu_us, 3),
                     "launches_per_token": gu_launches,
                     "all_gemv": {"achieved": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                                  "traffic": pmc.get("hbm_bytes_per_token") if pmc else None,
                                  "traffic_unit": "HBM bytes per token over the GEMV launches",
                                  "kernel": f"every weight GEMV ({GEMV_KIND[args.config]}, all 4 fused epilogues)",
                                  "bytes_per_token": weight_bytes, "gemv_ms_per_token": round(gemv_ms, 4),
                                  "launches_per_token": gemv_launches},
                     "attention_pmc": attention_pmc(pmc)},
        "breakdown": breakdown,
        "cpu_baseline": cpu,
        "host": platform.node(),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
