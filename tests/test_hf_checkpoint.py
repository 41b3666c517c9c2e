"""Hugging Face checkpoint loading (am_model_load_hf / am_hf_inspect), the counterpart of
the reference's HfDirectoryReader + HfSafetensorsFile + HfModelValidator +
ResolveWeights (src/model/formats/hf/hf_directory_reader.cpp:333-412,
hf_safetensors_file.cpp:64-382, hf_model_validator.cpp:168-644,
hf_weight_resolver.cpp:17-110).

CPU: the host-only reader accepts single-file and sharded checkpoints (F32, F16, BF16,
tied heads) and rejects what the reference rejects (missing / misshapen / unknown
tensors, bias, RoPE scaling, other model types, other dtypes, bad offsets, shards
outside the directory).
GPU: BASELINE configs[0] as an fp32 safetensors checkpoint (the build's seeded weights
written out through the C ABI) reproduces the committed golden greedy tokens, and a
bf16 checkpoint quantized to INT4 while loading gives the same device weights, bit for
bit, as the synthetic INT4 model built from the same bf16 values."""

import ctypes as C
import json
import os
import struct

import numpy as np
import pytest

import aethermind_amd.native as N

SMALL = dict(num_layers=2, hidden=64, num_q_heads=4, num_kv_heads=2, head_dim=16, ffn=128, vocab=100)


def hf_config(c, **kw):
    d = {"model_type": "llama", "architectures": ["LlamaForCausalLM"], "hidden_size": c["hidden"],
         "intermediate_size": c["ffn"], "num_hidden_layers": c["num_layers"],
         "num_attention_heads": c["num_q_heads"], "num_key_value_heads": c["num_kv_heads"],
         "vocab_size": c["vocab"], "rms_norm_eps": 1e-5, "rope_theta": 10000.0, "hidden_act": "silu",
         "max_position_embeddings": 256, "tie_word_embeddings": False, "torch_dtype": "float32"}
    d.update(kw)
    return d


def tensor_shapes(c, tied=False):
    H, Q, KV, F, V = c["hidden"], c["num_q_heads"] * c["head_dim"], c["num_kv_heads"] * c["head_dim"], c["ffn"], c["vocab"]
    t = {"model.embed_tokens.weight": (V, H), "model.norm.weight": (H,)}
    if not tied:
        t["lm_head.weight"] = (V, H)
    for l in range(c["num_layers"]):
        p = f"model.layers.{l}"
        t.update({f"{p}.input_layernorm.weight": (H,), f"{p}.post_attention_layernorm.weight": (H,),
                  f"{p}.self_attn.q_proj.weight": (Q, H), f"{p}.self_attn.k_proj.weight": (KV, H),
                  f"{p}.self_attn.v_proj.weight": (KV, H), f"{p}.self_attn.o_proj.weight": (H, Q),
                  f"{p}.mlp.gate_proj.weight": (F, H), f"{p}.mlp.up_proj.weight": (F, H),
                  f"{p}.mlp.down_proj.weight": (H, F)})
    return t


_ST_DTYPE = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int32): "I32"}


def write_safetensors(path, tensors, dtype_override=None):
    """tensors: name -> (numpy array | (bytes, st_dtype, shape)).  Written by hand (the
    format is an 8-byte header length, a JSON header and the raw data) so tests can also
    produce BF16 data and malformed files."""
    header, blobs, off = {}, [], 0
    for name, t in tensors.items():
        if isinstance(t, tuple):
            raw, dt, shape = t
        else:
            raw, dt, shape = np.ascontiguousarray(t).tobytes(), _ST_DTYPE[t.dtype], list(t.shape)
        if dtype_override and name in dtype_override:
            dt = dtype_override[name]
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def bf16_bytes(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even
    return r.tobytes()


def make_dir(tmp, c, tensors=None, shards=1, cfg_kw=None, tied=False):
    os.makedirs(tmp, exist_ok=True)
    with open(os.path.join(tmp, "config.json"), "w") as f:
        json.dump(hf_config(c, tie_word_embeddings=tied, **(cfg_kw or {})), f)
    if tensors is None:
        rng = np.random.default_rng(0)
        tensors = {n: (rng.standard_normal(s) * 0.02).astype(np.float32) for n, s in tensor_shapes(c, tied).items()}
    names = list(tensors)
    if shards == 1:
        write_safetensors(os.path.join(tmp, "model.safetensors"), tensors)
    else:
        wm = {}
        for i in range(shards):
            part = {n: tensors[n] for n in names[i::shards]}
            fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(os.path.join(tmp, fn), part)
            wm.update({n: fn for n in part})
        with open(os.path.join(tmp, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {"total_size": 0}, "weight_map": wm}, f)
    return tensors


def inspect(d):
    L = N.lib()
    cfg = N.ModelConfig()
    nt, nb = N.i64(), N.i64()
    rc = L.dll.am_hf_inspect(d.encode(), C.byref(cfg), C.byref(nt), C.byref(nb))
    msg = L.dll.am_last_error_message()
    return rc, cfg, nt.value, (msg.decode() if msg else "")


def test_inspect_single_and_sharded(tmp_path):
    for shards in (1, 3):
        d = str(tmp_path / f"s{shards}")
        t = make_dir(d, SMALL, shards=shards)
        rc, cfg, nt, msg = inspect(d)
        assert rc == 0, msg
        assert (cfg.num_layers, cfg.hidden, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab) == \
            (2, 64, 4, 2, 16, 128, 100)
        assert abs(cfg.rms_eps - 1e-5) < 1e-12 and cfg.rope_theta == 10000.0
        assert nt == len(t)


def test_inspect_dtypes_and_tied_head(tmp_path):
    """Each checkpoint has one linear dtype (embedding, head and projections; the
    reference's require_uniform_linear_dtype default); norm gains may use any of F32,
    F16 and BF16."""
    rng = np.random.default_rng(1)
    shapes = tensor_shapes(SMALL, tied=True)
    norm_dt = ["f16", "bf16", "f32"]
    for lin in ("f32", "f16", "bf16"):
        t = {}
        for i, (n, s) in enumerate(shapes.items()):
            a = (rng.standard_normal(s) * 0.02).astype(np.float32)
            dt = norm_dt[i % 3] if len(s) == 1 else lin
            t[n] = a.astype(np.float16) if dt == "f16" else (bf16_bytes(a), "BF16", list(s)) if dt == "bf16" else a
        d = str(tmp_path / f"tied_{lin}")
        make_dir(d, SMALL, tensors=t, tied=True)
        rc, _, nt, msg = inspect(d)
        assert rc == 0, msg
        assert nt == len(shapes)
    d2 = str(tmp_path / "untied_missing_head")
    make_dir(d2, SMALL, tensors=t, tied=False)
    rc, _, _, msg = inspect(d2)
    assert rc != 0 and "lm_head" in msg


def test_inspect_reads_rope_parameters_object(tmp_path):
    """transformers >= 5 writes RoPE as rope_parameters={rope_theta, rope_type:
    'default'} with no top-level rope_theta; the reader takes theta from it
    (hf_directory_reader.cpp:145-155) and treats 'default' as no scaling."""
    for i, kw in enumerate([{"rope_parameters": {"rope_theta": 500000.0, "rope_type": "default"}},
                            {"rope_scaling": {"rope_theta": 500000.0, "type": ""}},
                            {"rope_theta": 1.0, "rope_parameters": {"rope_theta": 500000.0}},
                            {"rope_scaling": None, "rope_theta": 500000.0}]):
        d = str(tmp_path / f"r{i}")
        make_dir(d, SMALL)
        cfgd = hf_config(SMALL, **kw)
        if "rope_theta" not in kw:
            del cfgd["rope_theta"]
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(cfgd, f)
        rc, cfg, _, msg = inspect(d)
        assert rc == 0, (kw, msg)
        assert cfg.rope_theta == 500000.0, kw


def test_inspect_transformers_written_config(tmp_path):
    """A config.json written by transformers' own LlamaConfig (CPU only)."""
    tr = pytest.importorskip("transformers")
    c = tr.LlamaConfig(vocab_size=SMALL["vocab"], hidden_size=SMALL["hidden"], intermediate_size=SMALL["ffn"],
                       num_hidden_layers=SMALL["num_layers"], num_attention_heads=SMALL["num_q_heads"],
                       num_key_value_heads=SMALL["num_kv_heads"], max_position_embeddings=128, rms_norm_eps=1e-6,
                       rope_theta=500000.0, tie_word_embeddings=False)
    d = str(tmp_path / "tf")
    make_dir(d, SMALL)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(c.to_dict(), f)
    rc, cfg, _, msg = inspect(d)
    assert rc == 0, msg
    assert cfg.rope_theta == 500000.0 and abs(cfg.rms_eps - 1e-6) < 1e-12


@pytest.mark.parametrize("case", ["missing", "shape", "unknown", "bias_cfg", "rope_scaling", "model_type",
                                  "dtype", "head_dim", "gap", "size", "truncated", "shard_escape",
                                  "not_in_index", "rope_params_scaling", "rope_params_factor", "int_2p31",
                                  "eps_missing", "eps_zero", "maxpos_missing", "dtype_hint_int8",
                                  "dtype_hint_f64", "dtype_hint_number", "mixed_linear", "tied_head_dtype",
                                  "ffn_small"])
def test_inspect_rejects(tmp_path, case):
    d = str(tmp_path / case)
    rng = np.random.default_rng(2)
    shapes = tensor_shapes(SMALL)
    t = {n: (rng.standard_normal(s) * 0.02).astype(np.float32) for n, s in shapes.items()}
    cfg_kw = {}
    if case == "missing":
        del t["model.layers.1.mlp.up_proj.weight"]
    elif case == "shape":
        t["model.layers.0.self_attn.k_proj.weight"] = np.zeros((16, 64), np.float32)
    elif case == "unknown":
        t["model.layers.0.self_attn.q_proj.bias"] = np.zeros(64, np.float32)
    elif case == "bias_cfg":
        cfg_kw = {"attention_bias": True}
    elif case == "rope_scaling":
        cfg_kw = {"rope_scaling": {"type": "linear", "factor": 2.0}}
    elif case == "model_type":
        cfg_kw = {"model_type": "mistral"}
    elif case == "dtype":
        t["model.norm.weight"] = np.zeros(64, np.int32)
    elif case == "head_dim":
        cfg_kw = {"head_dim": 32}
    elif case == "rope_params_scaling":
        cfg_kw = {"rope_parameters": {"rope_theta": 1e4, "rope_type": "llama3"}}
    elif case == "rope_params_factor":
        cfg_kw = {"rope_parameters": {"rope_theta": 1e4, "factor": 8.0}}
    elif case == "int_2p31":
        cfg_kw = {"max_position_embeddings": 2 ** 31}
    elif case == "eps_zero":
        cfg_kw = {"rms_norm_eps": 0.0}
    elif case == "dtype_hint_int8":
        cfg_kw = {"torch_dtype": "int8"}
    elif case == "dtype_hint_f64":
        cfg_kw = {"torch_dtype": "float64"}
    elif case == "dtype_hint_number":
        cfg_kw = {"dtype": 16}
    elif case == "mixed_linear":
        t["model.layers.1.mlp.up_proj.weight"] = t["model.layers.1.mlp.up_proj.weight"].astype(np.float16)
    elif case == "ffn_small":
        cfg_kw = {"intermediate_size": 32}
        for l in range(SMALL["num_layers"]):
            for nm, shp in ((f"model.layers.{l}.mlp.gate_proj.weight", (32, 64)),
                            (f"model.layers.{l}.mlp.up_proj.weight", (32, 64)),
                            (f"model.layers.{l}.mlp.down_proj.weight", (64, 32))):
                t[nm] = np.zeros(shp, np.float32)
    if case == "tied_head_dtype":
        t["lm_head.weight"] = t["lm_head.weight"].astype(np.float16)
        make_dir(d, SMALL, tensors=t, tied=True)
    else:
        make_dir(d, SMALL, tensors=t, cfg_kw=cfg_kw, shards=2 if case in ("shard_escape", "not_in_index") else 1)
    if case in ("eps_missing", "maxpos_missing"):
        p = os.path.join(d, "config.json")
        cj = json.load(open(p))
        del cj["rms_norm_eps" if case == "eps_missing" else "max_position_embeddings"]
        json.dump(cj, open(p, "w"))
    if case == "gap":  # 4 data bytes that no tensor covers
        with open(os.path.join(d, "model.safetensors"), "ab") as f:
            f.write(b"\0\0\0\0")
    elif case == "size":  # a tensor whose offsets disagree with its shape x dtype
        p = os.path.join(d, "model.safetensors")
        raw = open(p, "rb").read()
        hl = struct.unpack("<Q", raw[:8])[0]
        h = json.loads(raw[8:8 + hl])
        h["model.norm.weight"]["shape"] = [32]
        hb = json.dumps(h).encode()
        open(p, "wb").write(struct.pack("<Q", len(hb)) + hb + raw[8 + hl:])
    elif case == "truncated":
        p = os.path.join(d, "model.safetensors")
        raw = open(p, "rb").read()
        open(p, "wb").write(raw[:-100])
    elif case == "shard_escape":
        p = os.path.join(d, "model.safetensors.index.json")
        idx = json.load(open(p))
        k = next(iter(idx["weight_map"]))
        idx["weight_map"][k] = "../" + idx["weight_map"][k]
        json.dump(idx, open(p, "w"))
    elif case == "not_in_index":
        p = os.path.join(d, "model.safetensors.index.json")
        idx = json.load(open(p))
        del idx["weight_map"]["model.norm.weight"]
        json.dump(idx, open(p, "w"))
    rc, _, _, msg = inspect(d)
    assert rc != 0, case
    assert msg, case
    expect = {"rope_params_scaling": "RoPE scaling", "rope_params_factor": "RoPE scaling", "int_2p31": "2^31",
              "eps_missing": "rms_norm_eps", "eps_zero": "rms_norm_eps", "maxpos_missing": "max_position_embeddings",
              "dtype_hint_int8": "torch_dtype", "dtype_hint_f64": "torch_dtype", "dtype_hint_number": "dtype",
              "mixed_linear": "mixed linear", "tied_head_dtype": "tied", "ffn_small": "intermediate_size"}
    if case in expect:
        assert expect[case] in msg, (case, msg)


# ---------------------------------------------------------------- GPU

def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch


def _model_tensors(L, m, c, torch):
    """The model's logical weights (fp32 numpy) read back through the C ABI."""
    from gpu_util import p, stream

    def weight(layer, role):
        w = N.Weight()
        L.call("am_model_weight", m, layer, role, C.byref(w))
        out = torch.empty((w.n, w.k), dtype=torch.float32, device="cuda")
        L.call("am_gfx950_dequant", N.DequantArgs(w, p(out)), stream())
        torch.cuda.synchronize()
        return out.cpu().numpy()

    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]

    def buf(kind, layer, shape):
        ptr, nb = N.vp(), N.i64()
        L.call("am_model_buffer", m, kind, layer, C.byref(ptr), C.byref(nb))
        raw = np.empty(nb.value, np.uint8)
        assert hip.hipMemcpy(raw.ctypes.data, ptr.value, raw.nbytes, 2) == 0  # device -> host
        if raw.nbytes == int(np.prod(shape)) * 4:
            return raw.view(np.float32).reshape(shape)
        bits = raw.view(np.uint16).astype(np.uint32) << 16  # bf16 activations: exact widening
        return bits.view(np.float32).reshape(shape)

    H = c["hidden"]
    t = {"model.embed_tokens.weight": buf(N.AM_BUF_EMBED, 0, (c["vocab"], H)),
         "model.norm.weight": buf(N.AM_BUF_FINAL_NORM, 0, (H,)), "lm_head.weight": weight(0, 4)}
    for l in range(c["num_layers"]):
        p_ = f"model.layers.{l}"
        t[f"{p_}.input_layernorm.weight"] = buf(N.AM_BUF_IN_NORM, l, (H,))
        t[f"{p_}.post_attention_layernorm.weight"] = buf(N.AM_BUF_POST_NORM, l, (H,))
        for name, role in (("self_attn.q_proj", 5), ("self_attn.k_proj", 6), ("self_attn.v_proj", 7),
                           ("self_attn.o_proj", 1), ("mlp.gate_proj", 8), ("mlp.up_proj", 9), ("mlp.down_proj", 3)):
            t[f"{p_}.{name}.weight"] = weight(l, role)
    return t


def _runtime():
    L = N.lib()
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    return L, rt


def _generate(L, m, prompt, n_new):
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1)), C.byref(s))
    toks = np.zeros(n_new, np.int64)
    nout = N.i64()
    L.call("am_session_generate_ids", s, prompt.ctypes.data, prompt.size, n_new, -1, toks.ctypes.data, C.byref(nout))
    L.am_session_destroy(s)
    return toks


@pytest.mark.gpu
def test_tiny_fp32_checkpoint_reproduces_golden_tokens(tmp_path):
    """the tiny fp32 Llama as a (sharded) safetensors checkpoint."""
    torch = _gpu()
    import oracle_lib as O
    L, rt = _runtime()
    c = dict(O.TINY)
    mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                       c["vocab"], c["rms_eps"], c["rope_theta"], N.AM_DT_F32, N.AM_WF_F32, 128, c["max_tokens"], 16)
    ms = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 0, C.byref(ms))
    tensors = _model_tensors(L, ms, c, torch)
    L.am_model_destroy(ms)
    d = str(tmp_path / "tiny")
    make_dir(d, c, tensors=tensors, shards=2, cfg_kw={"rms_norm_eps": c["rms_eps"], "rope_theta": c["rope_theta"]})
    m = N.vp()
    L.call("am_model_load_hf", rt, d.encode(), C.byref(N.ModelLoadOptions(N.AM_DT_F32, N.AM_WF_F32, 128,
                                                                         c["max_tokens"], 16)), C.byref(m))
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tiny_fp32_seed0.npz"))
    toks = _generate(L, m, g["prompt"], 32)
    assert np.array_equal(toks, g["tokens"][:32]), (toks, g["tokens"][:32])
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)


@pytest.mark.gpu
def test_bf16_checkpoint_quantized_on_load_matches_synthetic_int4(tmp_path):
    torch = _gpu()
    from gpu_util import p, stream
    L, rt = _runtime()
    c = dict(num_layers=2, hidden=512, num_q_heads=8, num_kv_heads=2, head_dim=64, ffn=1536, vocab=4096,
             rms_eps=1e-5, rope_theta=10000.0)

    def synth(fmt):
        mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                           c["vocab"], c["rms_eps"], c["rope_theta"], N.AM_DT_BF16, fmt, 128, 128, 16)
        m = N.vp()
        L.call("am_model_create_synthetic", rt, C.byref(mc), 9, C.byref(m))
        return m

    mb = synth(N.AM_WF_BF16)  # the bf16 values the INT4 model is quantized from
    t = _model_tensors(L, mb, c, torch)
    L.am_model_destroy(mb)
    tb = {n: (bf16_bytes(a), "BF16", list(a.shape)) for n, a in t.items()}  # exact: the values are bf16
    d = str(tmp_path / "bf16")
    make_dir(d, c, tensors=tb, cfg_kw={"rms_norm_eps": c["rms_eps"]})
    mq = synth(N.AM_WF_INT4)
    ml = N.vp()
    L.call("am_model_load_hf", rt, d.encode(), C.byref(N.ModelLoadOptions(N.AM_DT_BF16, N.AM_WF_INT4, 128, 128, 16)),
           C.byref(ml))
    for layer, role in [(0, 0), (0, 1), (0, 2), (1, 3), (1, 2), (0, 4)]:
        wa, wb = N.Weight(), N.Weight()
        L.call("am_model_weight", mq, layer, role, C.byref(wa))
        L.call("am_model_weight", ml, layer, role, C.byref(wb))
        db, sb = N.i64(), N.i64()
        L.call("am_gfx950_weight_bytes", wa.n, wa.k, wa.format, wa.group_size, db, sb)
        hip = C.CDLL("libamdhip64.so.7")
        hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        for pa, pb, nbytes in ((wa.data, wb.data, db.value), (wa.scales, wb.scales, sb.value)):
            x, y = np.empty(nbytes, np.uint8), np.empty(nbytes, np.uint8)
            assert hip.hipMemcpy(x.ctypes.data, pa, nbytes, 2) == 0 and hip.hipMemcpy(y.ctypes.data, pb, nbytes, 2) == 0
            assert np.array_equal(x, y), (layer, role)
    prompt = np.arange(5, 17, dtype=np.int64)
    assert np.array_equal(_generate(L, mq, prompt, 8), _generate(L, ml, prompt, 8))
    L.am_model_destroy(mq)
    L.am_model_destroy(ml)
    L.am_runtime_destroy(rt)


@pytest.mark.gpu
def test_f16_linear_with_mixed_norm_dtypes_loads_exactly(tmp_path):
    """F16 projections with F32 / BF16 / F16 norm gains (one linear dtype, any norm
    dtype): every tensor reaches the device exactly (F16 and BF16 widen to fp32 without
    rounding), through a staging area sized for the largest tensor."""
    torch = _gpu()
    L, rt = _runtime()
    c = dict(SMALL)
    rng = np.random.default_rng(4)
    shapes = tensor_shapes(c)
    src, t = {}, {}
    for i, (n, s) in enumerate(shapes.items()):
        a = (rng.standard_normal(s) * 0.02).astype(np.float16).astype(np.float32)
        if len(s) == 1:
            a = (1.0 + a).astype(np.float32)
            kind = i % 3
            if kind == 1:
                b = np.frombuffer(bf16_bytes(a), np.uint16)
                a = (b.astype(np.uint32) << 16).view(np.float32).reshape(s)
                t[n] = (bf16_bytes(a), "BF16", list(s))
            else:
                t[n] = a.astype(np.float16) if kind == 2 else a
        else:
            t[n] = a.astype(np.float16)
        src[n] = a
    d = str(tmp_path / "mixed_norms")
    make_dir(d, c, tensors=t)
    m = N.vp()
    L.call("am_model_load_hf", rt, d.encode(), C.byref(N.ModelLoadOptions(N.AM_DT_F32, N.AM_WF_F32, 128, 64, 16)),
           C.byref(m))
    got = _model_tensors(L, m, dict(c, rms_eps=1e-5), torch)
    for n, a in src.items():
        assert np.array_equal(got[n], a), n
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)


@pytest.mark.gpu
def test_prd_session_abi_generates_golden_tokens(tmp_path):
    """The PRD's Phase-1 C ABI (aethermind_prd.md:298-320): am_runtime_create(config),
    am_model_load(runtime, path, &error), am_session_create(model, config) and
    am_session_generate with uint32 token ids, output capacity and an error object.
    The tiny fp32 checkpoint generates the golden tokens (prefill token + 32 decode
    steps); the generation limits and the error path behave as specified."""
    torch = _gpu()
    import oracle_lib as O
    L, rt0 = _runtime()
    c = dict(O.TINY)
    mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                       c["vocab"], c["rms_eps"], c["rope_theta"], N.AM_DT_F32, N.AM_WF_F32, 128, c["max_tokens"], 16)
    ms = N.vp()
    L.call("am_model_create_synthetic", rt0, C.byref(mc), 0, C.byref(ms))
    tensors = _model_tensors(L, ms, c, torch)
    L.am_model_destroy(ms)
    L.am_runtime_destroy(rt0)
    d = str(tmp_path / "tiny")
    make_dir(d, c, tensors=tensors, cfg_kw={"rms_norm_eps": c["rms_eps"], "rope_theta": c["rope_theta"]})
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tiny_fp32_seed0.npz"))

    dll = L.dll
    cfg = N.Config(C.sizeof(N.Config), 0, N.AM_DT_F32, N.AM_WF_F32, 128, c["max_tokens"], 16)
    rt = dll.am_runtime_create(C.byref(cfg))
    assert rt, dll.am_last_error_message()
    err = N.vp()
    bad = dll.am_model_load(rt, str(tmp_path / "missing").encode(), C.byref(err))
    assert not bad and err.value, "a missing directory must fail with an error object"
    assert dll.am_gfx950_error_code(err) == N.STATUS_NAMES.index("NOT_FOUND")
    assert b"missing" in dll.am_gfx950_error_message(err)
    dll.am_error_free(err)
    m = dll.am_model_load(rt, d.encode(), C.byref(err))
    assert m and not err.value, dll.am_last_error_message()
    prompt = np.ascontiguousarray(g["prompt"].astype(np.uint32))
    out = np.zeros(64, np.uint32)
    n = C.c_size_t()
    # no session limit: the output capacity (33) bounds the generation
    s = dll.am_session_create(m, C.byref(N.SessionConfig(C.sizeof(N.SessionConfig), 0, -1, 1)))
    assert s, dll.am_last_error_message()
    rc = dll.am_session_generate(s, prompt.ctypes.data, prompt.size, out.ctypes.data, 33, C.byref(n), C.byref(err))
    assert rc == 0 and not err.value and n.value == 33
    assert np.array_equal(out[:33].astype(np.int64), g["tokens"]), (out[:33], g["tokens"])
    dll.am_session_destroy(s)
    # the session's max_tokens bounds it, and generation stops after eos
    eos = int(g["tokens"][4])
    s = dll.am_session_create(m, C.byref(N.SessionConfig(C.sizeof(N.SessionConfig), 3, -1, 0)))
    rc = dll.am_session_generate(s, prompt.ctypes.data, prompt.size, out.ctypes.data, 64, C.byref(n), C.byref(err))
    assert rc == 0 and n.value == 3 and np.array_equal(out[:3].astype(np.int64), g["tokens"][:3])
    dll.am_session_destroy(s)
    s = dll.am_session_create(m, C.byref(N.SessionConfig(C.sizeof(N.SessionConfig), 0, eos, 1)))
    rc = dll.am_session_generate(s, prompt.ctypes.data, prompt.size, out.ctypes.data, 64, C.byref(n), C.byref(err))
    first = int(np.flatnonzero(g["tokens"] == eos)[0])
    assert rc == 0 and n.value == first + 1 and int(out[first]) == eos
    # an out-of-vocabulary id is an error with an error object
    badp = prompt.copy()
    badp[3] = c["vocab"]
    rc = dll.am_session_generate(s, badp.ctypes.data, badp.size, out.ctypes.data, 64, C.byref(n), C.byref(err))
    assert rc == N.STATUS_NAMES.index("OUT_OF_RANGE") and err.value and n.value == 0
    dll.am_error_free(err)
    dll.am_session_destroy(s)
    dll.am_model_unload(m)
    dll.am_runtime_destroy(rt)
