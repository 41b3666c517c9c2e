"""Quantized (GPTQ) checkpoint ingestion under allow_quantized_tensors, and the
reference's tensor-name rules (ModelValidationOptions, model_validation_options.h:7-16;
DetectUnsupportedTensors / ValidateUnknownTensorPolicy, hf_model_validator.cpp:168-385;
its tests test_hf_model_validator.cpp:955-1010).

The GPTQ layout is restated here from the published AutoGPTQ / optimum format (this
file's gptq_pack is the test's own writer, independent of the library's reader):
  qweight I32 [k/8][n]: nibble t of word (i, j) = q[8i + t][j], q in 0..15
  qzeros  I32 [groups][n/8]: nibble t of word (g, j) = stored zero of column 8j + t,
          stored = z - 1 (mod 16) for checkpoint_format "gptq", z for "gptq_v2"
  scales  [groups][n]; g_idx I32 [k]
  w[j][k] = scales[g_idx[k]][j] * (q[k][j] - z[g_idx[k]][j])
AutoGPTQ's torch dequant evaluates that product in fp16; the library evaluates it in
fp32, where it is exact (|q - z| <= 15, fp16 scales), so the checks below are exact.

CPU: the host-only inspector (am_hf_inspect_ex) applies the rules.
GPU: (1) the unpack kernel against numpy, both outputs; (2) a GPTQ checkpoint whose
grid is this library's INT4 grid (zeros 8, fp16 scales, group 128, in-order groups)
loads to the same device bytes as the dense bf16 checkpoint it was made from,
quantized on load, in both checkpoint formats; (3) an asymmetric act-order checkpoint
loads to s * (q - z) exactly as F32, to its RNE rounding as BF16, and to the build
SPEC quantization of it as INT4."""

import ctypes as C

import numpy as np
import pytest

import aethermind_amd.native as N
from test_hf_checkpoint import SMALL, bf16_bytes, make_dir, tensor_shapes

PROJ = {"self_attn.q_proj": ("q", "h"), "self_attn.k_proj": ("kv", "h"), "self_attn.v_proj": ("kv", "h"),
        "self_attn.o_proj": ("h", "q"), "mlp.gate_proj": ("f", "h"), "mlp.up_proj": ("f", "h"),
        "mlp.down_proj": ("h", "f")}


def gptq_pack(q, zeros, fmt="gptq"):
    """q int [k][n] in 0..15, zeros int [groups][n] in 0..15 -> (qweight, qzeros) as int32"""
    k, n = q.shape
    qw = np.zeros((k // 8, n), np.uint32)
    for t in range(8):
        qw |= (q[t::8].astype(np.uint32) & 0xF) << np.uint32(4 * t)
    stored = (zeros.astype(np.int64) - (1 if fmt == "gptq" else 0)) & 0xF
    qz = np.zeros((zeros.shape[0], n // 8), np.uint32)
    for t in range(8):
        qz |= stored[:, t::8].astype(np.uint32) << np.uint32(4 * t)
    return qw.view(np.int32), qz.view(np.int32)


def gptq_dequant(q, zeros, scales, g_idx):
    """w [n][k] fp32 = scales[g_idx] * (q - zeros[g_idx]), exact"""
    s = scales.astype(np.float32)[g_idx]  # [k][n]
    d = (q.astype(np.int64) - zeros.astype(np.int64)[g_idx]).astype(np.float32)
    return np.ascontiguousarray((s * d).T)


def dims(c):
    return {"h": c["hidden"], "q": c["num_q_heads"] * c["head_dim"], "kv": c["num_kv_heads"] * c["head_dim"],
            "f": c["ffn"]}


def random_gptq(rng, n, k, group, act_order):
    q = rng.integers(0, 16, size=(k, n))
    groups = k // group
    zeros = rng.integers(0, 16, size=(groups, n))
    scales = (rng.random((groups, n)) * 0.01 + 1e-3).astype(np.float16)
    if act_order:
        g_idx = np.empty(k, np.int32)
        g_idx[rng.permutation(k)] = np.arange(k) // group
    else:
        g_idx = (np.arange(k) // group).astype(np.int32)
    return q, zeros, scales, g_idx


def gptq_tensors(prefix, q, zeros, scales, g_idx, fmt="gptq", with_gidx=True):
    qw, qz = gptq_pack(q, zeros, fmt)
    t = {prefix + ".qweight": qw, prefix + ".qzeros": qz, prefix + ".scales": scales}
    if with_gidx:
        t[prefix + ".g_idx"] = g_idx.astype(np.int32)
    return t


def qcfg(group=32, fmt="gptq", desc_act=False, **kw):
    d = {"quant_method": "gptq", "bits": 4, "group_size": group, "desc_act": desc_act, "sym": False,
         "checkpoint_format": fmt}
    d.update(kw)
    return d


def inspect(d, flags=0):
    L = N.lib()
    cfg = N.ModelConfig()
    nt, nb = N.i64(), N.i64()
    rc = L.dll.am_hf_inspect_ex(d.encode(), flags, C.byref(cfg), C.byref(nt), C.byref(nb))
    return rc, nt.value, L.last_error()


def small_gptq_dir(tmp, rng, fmt="gptq", group=32, mutate=None, cfg_kw=None):
    """SMALL with every projection of layer 0 stored as GPTQ, the rest dense"""
    c = SMALL
    D = dims(c)
    t = {n: (rng.standard_normal(s) * 0.02).astype(np.float32) for n, s in tensor_shapes(c).items()}
    for name, (nd, kd) in PROJ.items():
        prefix = f"model.layers.0.{name}"
        del t[prefix + ".weight"]
        t.update(gptq_tensors(prefix, *random_gptq(rng, D[nd], D[kd], group, False), fmt=fmt))
    if mutate:
        mutate(t)
    make_dir(tmp, c, tensors=t, cfg_kw=dict({"quantization_config": qcfg(group, fmt)}, **(cfg_kw or {})))
    return t


# ---------------------------------------------------------------- CPU: rules

def test_gptq_checkpoint_needs_the_flag(tmp_path):
    d = str(tmp_path / "g")
    t = small_gptq_dir(d, np.random.default_rng(0))
    rc, _, msg = inspect(d)
    assert rc == N.AM_STATUS_INVALID_ARGUMENT and "allow_quantized_tensors" in msg
    rc, nt, msg = inspect(d, N.AM_LOAD_ALLOW_QUANTIZED_TENSORS)
    assert rc == N.AM_STATUS_OK, msg
    assert nt == len(t)


def test_quantized_tensor_names_follow_the_reference_rules(tmp_path):
    rng = np.random.default_rng(1)
    base = {n: (rng.standard_normal(s) * 0.02).astype(np.float32) for n, s in tensor_shapes(SMALL).items()}

    def check(extra, flags, ok, name):
        d = str(tmp_path / name)
        make_dir(d, SMALL, tensors=dict(base, **extra))
        rc, nt, msg = inspect(d, flags)
        assert (rc == N.AM_STATUS_OK) == ok, (name, rc, msg)
        if ok:
            assert nt == len(base)  # tensors outside the model are dropped
        return msg

    z4 = np.zeros(4, np.float32)
    # RejectsQuantizedTensorByDefault / AllowsQuantizedTensorWhenOptionEnabled
    msg = check({"model.layers.0.self_attn.q_proj.qweight": z4}, 0, False, "qw_default")
    assert "qweight" in msg
    check({"model.layers.0.self_attn.q_proj.qweight": z4}, N.AM_LOAD_ALLOW_QUANTIZED_TENSORS, True, "qw_allowed")
    # RejectsScalesQuantizedTensor / AllowsNonQuantizedTensorNameContainingScales
    assert "scales" in check({"model.layers.0.mlp.gate_proj.scales": z4}, 0, False, "scales")
    check({"model.layers.0.mlp.gate_proj.scales.weight": z4}, 0, True, "scales_weight")
    # unknown tensors: ignored by default, errors when strict or not allowed
    check({"some.extra.tensor": z4, "model.rotary_emb.inv_freq": z4}, 0, True, "unknown_default")
    assert "unexpected" in check({"some.extra.tensor": z4}, N.AM_LOAD_STRICT_TENSOR_NAMES, False, "unknown_strict")
    check({"some.extra.tensor": z4}, N.AM_LOAD_REJECT_UNKNOWN_TENSORS, False, "unknown_rejected")
    check({"model.rotary_emb.inv_freq": z4}, N.AM_LOAD_STRICT_TENSOR_NAMES, True, "inv_freq_strict")
    # always refused: MoE, LoRA, layer index past num_hidden_layers
    check({"model.layers.0.mlp.experts.0.weight": z4}, 0, False, "moe")
    check({"model.layers.0.self_attn.q_proj.lora_A.weight": z4}, 0, False, "lora")
    assert "layer index" in check({"model.layers.2.mlp.gate_proj.weight": z4}, 0, False, "layer_past_end")


@pytest.mark.parametrize("case,code,text", [
    ("bits8", "UNIMPLEMENTED", "4-bit"), ("awq", "UNIMPLEMENTED", "gptq"), ("group_odd", "INVALID_ARGUMENT", "group_size"),
    ("format_marlin", "UNIMPLEMENTED", "checkpoint_format"), ("qweight_shape", "INVALID_ARGUMENT", "qweight"),
    ("qzeros_dtype", "INVALID_ARGUMENT", "qzeros"), ("scales_int", "INVALID_ARGUMENT", "scales"),
    ("gidx_range", "INVALID_ARGUMENT", "g_idx"), ("missing_qzeros", "INVALID_ARGUMENT", "q_proj"),
    ("group_not_dividing", "INVALID_ARGUMENT", "group_size")])
def test_gptq_rejects(tmp_path, case, code, text):
    rng = np.random.default_rng(2)
    d = str(tmp_path / case)
    cfg_kw = {}
    mutate = None
    p0 = "model.layers.0.self_attn.q_proj"
    if case == "bits8":
        cfg_kw = {"quantization_config": qcfg(bits=8)}
    elif case == "awq":
        cfg_kw = {"quantization_config": qcfg(quant_method="awq")}
    elif case == "group_odd":
        cfg_kw = {"quantization_config": qcfg(group=12)}
    elif case == "format_marlin":
        cfg_kw = {"quantization_config": qcfg(fmt="marlin")}
    elif case == "qweight_shape":
        def mutate(t):
            t[p0 + ".qweight"] = t[p0 + ".qweight"][:-1]
    elif case == "qzeros_dtype":
        def mutate(t):
            t[p0 + ".qzeros"] = t[p0 + ".qzeros"].astype(np.float32)
    elif case == "scales_int":
        def mutate(t):
            t[p0 + ".scales"] = t[p0 + ".scales"].astype(np.int32)
    elif case == "gidx_range":
        def mutate(t):
            t[p0 + ".g_idx"] = np.full_like(t[p0 + ".g_idx"], 2)  # 2 groups of 32 over k = 64
    elif case == "missing_qzeros":
        def mutate(t):
            del t[p0 + ".qzeros"]
    elif case == "group_not_dividing":
        cfg_kw = {"quantization_config": qcfg(group=48)}
    small_gptq_dir(d, rng, mutate=mutate, cfg_kw=cfg_kw)
    rc, _, msg = inspect(d, N.AM_LOAD_ALLOW_QUANTIZED_TENSORS)
    assert rc == getattr(N, "AM_STATUS_" + code), (case, rc, msg)
    assert text in msg, (case, msg)


def test_gptq_pack_round_trip():
    """the test's writer against its own reader (a slip in either shows up here)"""
    rng = np.random.default_rng(3)
    q, z, s, g = random_gptq(rng, 16, 64, 16, True)
    for fmt in ("gptq", "gptq_v2"):
        qw, qz = gptq_pack(q, z, fmt)
        u = qw.view(np.uint32)
        back = np.stack([(u >> np.uint32(4 * t)) & 0xF for t in range(8)], 1).reshape(64, 16)
        assert np.array_equal(back, q)
        zu = qz.view(np.uint32)
        off = 1 if fmt == "gptq" else 0
        zb = np.stack([((zu >> np.uint32(4 * t)) + off) & 0xF for t in range(8)], 2).reshape(4, 16)
        assert np.array_equal(zb, z)
    w = gptq_dequant(q, z, s, g)
    assert w[5, 7] == np.float32(s[g[7], 5]) * np.float32(q[7, 5] - z[g[7], 5])


# ---------------------------------------------------------------- GPU

def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2"])
@pytest.mark.parametrize("act_order", [False, True])
def test_unpack_kernel_matches_numpy(fmt, act_order):
    _gpu()
    from gpu_util import dev, empty, p, stream
    import torch
    rng = np.random.default_rng(4)
    n, k, group = 96, 256, 64
    q, z, s, g = random_gptq(rng, n, k, group, act_order)
    qw, qz = gptq_pack(q, z, fmt)
    dq, dz, ds, dg = dev(qw), dev(qz), dev(s.view(np.uint16)), dev(g)
    out = empty((n, k), torch.float32)
    a = N.GptqArgs(p(dq), p(dz), p(ds), N.AM_DT_F16, 1 if fmt == "gptq" else 0, p(dg), n, k, group, p(out), None, None)
    N.lib().call("am_gfx950_gptq_unpack", C.byref(a), stream())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), gptq_dequant(q, z, s, g))
    # logical INT4 output: q - z as two's complement nibbles, low nibble = even k
    lg = empty((n, k // 2), torch.uint8)
    sc = empty((n, k // group), torch.int16)
    a = N.GptqArgs(p(dq), p(dz), p(ds), N.AM_DT_F16, 1 if fmt == "gptq" else 0, None, n, k, group, None, p(lg), p(sc))
    N.lib().call("am_gfx950_gptq_unpack", C.byref(a), stream())
    torch.cuda.synchronize()
    gi = np.arange(k) // group
    d = (q - z[gi]).T & 0xF  # [n][k]
    assert np.array_equal(lg.cpu().numpy(), (d[:, 0::2] | (d[:, 1::2] << 4)).astype(np.uint8))
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), s.view(np.uint16).T)


def _load(L, rt, d, act, wf, flags=N.AM_LOAD_ALLOW_QUANTIZED_TENSORS):
    m = N.vp()
    L.call("am_model_load_hf_ex", rt, d.encode(), C.byref(N.ModelLoadOptions(act, wf, 128, 128, 16)), flags,
           C.byref(m))
    return m


def _weight_bytes(L, m, layer, role):
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    w = N.Weight()
    L.call("am_model_weight", m, layer, role, C.byref(w))
    db, sb = N.i64(), N.i64()
    L.call("am_gfx950_weight_bytes", w.n, w.k, w.format, w.group_size, C.byref(db), C.byref(sb))
    out = []
    for ptr, nb in ((w.data, db.value), (w.scales, sb.value)):
        if nb:
            x = np.empty(nb, np.uint8)
            assert hip.hipMemcpy(x.ctypes.data, ptr, nb, 2) == 0
            out.append(x)
    return out


def _proj_weight(L, m, layer, name, torch):
    """fp32 [n][k] of one projection read back through the C ABI (dequantized)"""
    from gpu_util import p, stream
    role = {"self_attn.q_proj": 5, "self_attn.k_proj": 6, "self_attn.v_proj": 7, "self_attn.o_proj": 1,
            "mlp.gate_proj": 8, "mlp.up_proj": 9, "mlp.down_proj": 3}[name]
    w = N.Weight()
    L.call("am_model_weight", m, layer, role, C.byref(w))
    out = torch.empty((w.n, w.k), dtype=torch.float32, device="cuda")
    L.call("am_gfx950_dequant", N.DequantArgs(w, p(out)), stream())
    torch.cuda.synchronize()
    return out.cpu().numpy()


CFG = dict(num_layers=2, hidden=256, num_q_heads=4, num_kv_heads=2, head_dim=64, ffn=512, vocab=512)


def _dense(rng, c):
    return {n: (rng.standard_normal(s) * 0.02).astype(np.float32) for n, s in tensor_shapes(c).items()}


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2"])
def test_symmetric_gptq_repacks_exactly_to_the_int4_grid(tmp_path, fmt):
    torch = _gpu()
    import oracle_lib as O
    from test_hf_checkpoint import _generate
    L = N.lib()
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    c = CFG
    rng = np.random.default_rng(5)
    dense = _dense(rng, c)
    # the dense checkpoint in bf16 (its values are what both models quantize)
    for n in dense:
        dense[n] = (np.frombuffer(bf16_bytes(dense[n]), np.uint16).astype(np.uint32) << 16).view(np.float32) \
            .reshape(dense[n].shape)
    tb = {n: (bf16_bytes(a), "BF16", list(a.shape)) for n, a in dense.items()}
    d_dense = str(tmp_path / "dense")
    make_dir(d_dense, c, tensors=tb)
    # the same weights as GPTQ: the SPEC INT4 quantization (oracle) written as q + 8, zero 8
    tq = dict(tb)
    for layer in range(c["num_layers"]):
        for name in PROJ:
            prefix = f"model.layers.{layer}.{name}"
            w = dense[prefix + ".weight"]
            packed, sc = O.quant_int4(w, 128)
            lo, hi = packed & 0xF, packed >> 4
            qs = np.empty(w.shape, np.int64)
            qs[:, 0::2], qs[:, 1::2] = lo, hi
            qs = np.where(qs >= 8, qs - 16, qs)  # two's complement nibble -> -8..7
            del tq[prefix + ".weight"]
            groups = w.shape[1] // 128
            trivial = (np.arange(w.shape[1]) // 128).astype(np.int32)  # in-order groups, written for layer 0 only
            tq.update(gptq_tensors(prefix, (qs + 8).T, np.full((groups, w.shape[0]), 8),
                                   sc.view(np.float16).T.copy(), trivial, fmt=fmt, with_gidx=layer == 0))
    d_q = str(tmp_path / "gptq")
    make_dir(d_q, c, tensors=tq, cfg_kw={"quantization_config": qcfg(128, fmt, sym=True)})
    ma = _load(L, rt, d_dense, N.AM_DT_BF16, N.AM_WF_INT4, 0)
    mb = _load(L, rt, d_q, N.AM_DT_BF16, N.AM_WF_INT4)
    for layer in range(c["num_layers"]):
        for role in range(4):
            for x, y in zip(_weight_bytes(L, ma, layer, role), _weight_bytes(L, mb, layer, role)):
                assert np.array_equal(x, y), (layer, role)
    prompt = np.arange(7, 19, dtype=np.int64)
    assert np.array_equal(_generate(L, ma, prompt, 8), _generate(L, mb, prompt, 8))
    L.am_model_destroy(ma)
    L.am_model_destroy(mb)
    L.am_runtime_destroy(rt)


@pytest.mark.gpu
@pytest.mark.parametrize("target", ["f32", "bf16", "int4", "int8"])
def test_asymmetric_act_order_gptq_dequantizes_exactly(tmp_path, target):
    torch = _gpu()
    import oracle_lib as O
    L = N.lib()
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    c = CFG
    D = dims(c)
    rng = np.random.default_rng(6)
    t = _dense(rng, c)
    want = {}
    for layer in range(c["num_layers"]):
        for name, (nd, kd) in PROJ.items():
            prefix = f"model.layers.{layer}.{name}"
            q, z, s, g = random_gptq(rng, D[nd], D[kd], 64, True)
            want[prefix] = gptq_dequant(q, z, s, g)
            del t[prefix + ".weight"]
            t.update(gptq_tensors(prefix, q, z, s, g))
    d = str(tmp_path / "asym")
    make_dir(d, c, tensors=t, cfg_kw={"quantization_config": qcfg(64, "gptq", desc_act=True)})
    act = N.AM_DT_F32 if target == "f32" else N.AM_DT_BF16
    wf = {"f32": N.AM_WF_F32, "bf16": N.AM_WF_BF16, "int4": N.AM_WF_INT4, "int8": N.AM_WF_INT8}[target]
    m = _load(L, rt, d, act, wf)
    for prefix, w in want.items():
        layer, name = int(prefix.split(".")[2]), prefix.split(".", 3)[3]
        got = _proj_weight(L, m, layer, name, torch)
        if target == "f32":
            exp = w
        elif target == "bf16":
            exp = (np.frombuffer(bf16_bytes(w), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(w.shape)
        elif target == "int4":
            exp = O.dequant_int4(*O.quant_int4(w, 128), w.shape[1], 128)
        else:
            exp = O.dequant_int8(*O.quant_int8(w))
        assert np.array_equal(got, exp), (target, prefix, np.max(np.abs(got - exp)))
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)
