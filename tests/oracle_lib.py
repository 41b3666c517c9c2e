"""ctypes access to the CPU oracle (oracle/liboracle.so) for tests, smoke() and the
benchmark's cpu_baseline leg.  Test infrastructure only: the product never loads it."""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_DOT_SO = os.path.join(ROOT, "oracle", "_ref", "libref_dot.so")

vp, i32, i64, u64, f32, f64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double


class OrcConfig(C.Structure):
    _fields_ = [(n, i32) for n in ("num_layers", "hidden", "num_q_heads", "num_kv_heads", "head_dim", "ffn",
                                   "vocab", "act_bf16", "weight_format", "group_size", "max_tokens")] + \
               [("rms_eps", f32), ("rope_theta", f64)]


_SIGS = {
    "orc_f32_to_bf16": (C.c_uint16, [f32]),
    "orc_bf16_to_f32": (f32, [C.c_uint16]),
    "orc_f32_to_f16": (C.c_uint16, [f32]),
    "orc_f16_to_f32": (f32, [C.c_uint16]),
    "orc_portable_log": (f64, [f64]),
    "orc_portable_sincos_turns": (None, [f64, C.POINTER(f64), C.POINTER(f64)]),
    "orc_portable_sqrt": (f64, [f64]),
    "orc_splitmix64": (u64, [u64]),
    "orc_tensor_key": (u64, [u64, u64]),
    "orc_synth_normal_f32": (None, [u64, u64, f64, i64, i64, vp]),
    "orc_synth_normal_bf16": (None, [u64, u64, f64, i64, i64, vp]),
    "orc_synth_token_ids": (None, [u64, u64, i64, i64, vp]),
    "orc_quant_int8": (i32, [vp, i64, i64, vp, vp]),
    "orc_dequant_int8": (i32, [vp, vp, i64, i64, vp]),
    "orc_quant_int4": (i32, [vp, i64, i64, i64, vp, vp]),
    "orc_dequant_int4": (i32, [vp, vp, i64, i64, i64, vp]),
    "orc_embedding_i64": (i32, [vp, i64, vp, i64, i64, vp]),
    "orc_rmsnorm_scalar": (i32, [vp, vp, i64, i64, f32, vp]),
    "orc_rmsnorm_avx2": (i32, [vp, vp, i64, i64, f32, vp]),
    "orc_dot_avx2": (f32, [vp, vp, i64]),
    "orc_linear": (None, [vp, vp, i64, i64, i64, vp]),
    "orc_linear_avx2": (None, [vp, vp, i64, i64, i64, vp]),
    "orc_rope_table": (None, [i64, i64, f64, vp, vp]),
    "orc_rope": (None, [vp, i64, i64, i64, vp, vp, vp]),
    "orc_attention": (None, [vp, vp, vp, i64, i64, i64, i64, i64, i64, vp]),
    "orc_silu_mul": (None, [vp, vp, i64, vp]),
    "orc_argmax": (i64, [vp, i64]),
    "orc_round_bf16_inplace": (None, [vp, i64]),
    "orc_model_create_synthetic": (vp, [C.POINTER(OrcConfig), u64, i32]),
    "orc_model_destroy": (None, [vp]),
    "orc_model_generate": (i32, [vp, vp, i64, i64, vp, vp]),
    "orc_model_forward": (i32, [vp, vp, i64, i64, vp]),
    "orc_model_set_fast": (None, [vp, i32]),
    "orc_model_set_slip": (None, [vp, i32]),
    "orc_model_set_norm_gain": (i32, [vp, i32, i32, vp]),
    "orc_set_threads": (None, [i32]),
    "orc_qweight_create": (vp, [i64, i64, i32, i64, u64]),
    "orc_qweight_destroy": (None, [vp]),
    "orc_qweight_bytes": (i64, [vp]),
    "orc_qweight_gemv": (None, [vp, vp, vp]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle not built: run `make -C oracle` (or __graft_entry__.build())")
        _lib = C.CDLL(ORACLE_SO)
        for n, (r, a) in _SIGS.items():
            f = getattr(_lib, n)
            f.restype = r
            f.argtypes = a
    return _lib


def ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(vp)


# ---------------------------------------------------------------- numpy helpers
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits (RNE, NaN -> 0x7FC0) through the oracle."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    L = lib()
    flat, of = x.reshape(-1), out.reshape(-1)
    for i in range(flat.size):
        of[i] = L.orc_f32_to_bf16(float(flat[i]))
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_round_bf16_inplace(ptr(x), x.size)
    return x


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def synth_f32(seed: int, tid: int, n: int, offset: int = 0, std: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_normal_f32(seed, tid, std, offset, n, ptr(out))
    return out


def synth_bf16(seed: int, tid: int, n: int, offset: int = 0, std: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().orc_synth_normal_bf16(seed, tid, std, offset, n, ptr(out))
    return out


def token_ids(seed: int, stream: int, vocab: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int64)
    lib().orc_synth_token_ids(seed, stream, vocab, n, ptr(out))
    return out


def quant_int8(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    assert lib().orc_quant_int8(ptr(w), n, k, ptr(q), ptr(s)) == 0
    return q, s


def dequant_int8(q, s):
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    lib().orc_dequant_int8(ptr(np.ascontiguousarray(q)), ptr(np.ascontiguousarray(s)), n, k, ptr(out))
    return out


def quant_int4(w: np.ndarray, group: int = 128):
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    packed = np.empty((n, k // 2), np.uint8)
    sc = np.empty((n, k // group), np.uint16)
    rc = lib().orc_quant_int4(ptr(w), n, k, group, ptr(packed), ptr(sc))
    assert rc == 0, rc
    return packed, sc


def dequant_int4(packed, sc, k: int, group: int = 128):
    n = packed.shape[0]
    out = np.empty((n, k), np.float32)
    lib().orc_dequant_int4(ptr(np.ascontiguousarray(packed)), ptr(np.ascontiguousarray(sc)), n, k, group, ptr(out))
    return out


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_linear(ptr(x), ptr(w), m, n, k, ptr(out))
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    assert lib().orc_rmsnorm_scalar(ptr(x), ptr(np.ascontiguousarray(w, np.float32)), x.shape[0], x.shape[1],
                                    eps, ptr(out)) == 0
    return out


def rope_tables(max_pos: int, d: int, theta: float):
    c = np.empty((max_pos, d // 2), np.float32)
    s = np.empty((max_pos, d // 2), np.float32)
    lib().orc_rope_table(max_pos, d, theta, ptr(c), ptr(s))
    return c, s


def rope(x: np.ndarray, heads: int, d: int, pos: np.ndarray, cos_t, sin_t) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    pos = np.ascontiguousarray(pos, np.int64)
    lib().orc_rope(ptr(x), x.shape[0], heads, d, ptr(pos), ptr(cos_t), ptr(sin_t))
    return x


def attention(q, kc, vc, seq, hq, hkv, d, cap, start):
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty((seq, hq * d), np.float32)
    lib().orc_attention(ptr(q), ptr(np.ascontiguousarray(kc, np.float32)), ptr(np.ascontiguousarray(vc, np.float32)),
                        seq, hq, hkv, d, cap, start, ptr(out))
    return out


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    out = np.empty_like(g)
    lib().orc_silu_mul(ptr(g), ptr(np.ascontiguousarray(u, np.float32)), g.size, ptr(out))
    return out


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().orc_argmax(ptr(x), x.size))


class OracleModel:
    """Whole-model Llama forward on the CPU (model_graph_builder.cpp:133-415 order)."""

    def __init__(self, cfg: dict, seed: int):
        c = OrcConfig(cfg["num_layers"], cfg["hidden"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                      cfg["ffn"], cfg["vocab"], 1 if cfg["act"] == "bf16" else 0, cfg["weight_format"],
                      cfg.get("group_size", 128), cfg["max_tokens"], cfg["rms_eps"], cfg["rope_theta"])
        self.cfg = cfg
        self.h = lib().orc_model_create_synthetic(C.byref(c), seed, 0)
        if not self.h:
            raise RuntimeError("oracle model creation failed")

    def set_fast(self, fast: bool):
        lib().orc_model_set_fast(self.h, 1 if fast else 0)

    def set_slip(self, slip: int):
        lib().orc_model_set_slip(self.h, slip)

    def set_norm_gain(self, kind: int, layer: int, gain: np.ndarray):
        """kind 0 = input norm of `layer`, 1 = post-attention norm, 2 = final norm."""
        g = np.ascontiguousarray(gain, np.float32)
        assert g.size == self.cfg["hidden"]
        assert lib().orc_model_set_norm_gain(self.h, kind, layer, ptr(g)) == 0

    def set_gains(self, gains: dict):
        """gains: {"input": [L][H], "post": [L][H], "final": [H]} (norm_gains())."""
        for l in range(self.cfg["num_layers"]):
            self.set_norm_gain(0, l, gains["input"][l])
            self.set_norm_gain(1, l, gains["post"][l])
        self.set_norm_gain(2, 0, gains["final"])

    def generate(self, prompt: np.ndarray, n_new: int):
        prompt = np.ascontiguousarray(prompt, np.int64)
        toks = np.empty(n_new, np.int64)
        logits = np.empty(self.cfg["vocab"], np.float32)
        rc = lib().orc_model_generate(self.h, ptr(prompt), prompt.size, n_new, ptr(toks), ptr(logits))
        assert rc == 0, rc
        return toks, logits

    def forward(self, ids: np.ndarray, pos: int):
        ids = np.ascontiguousarray(ids, np.int64)
        logits = np.empty(self.cfg["vocab"], np.float32)
        rc = lib().orc_model_forward(self.h, ptr(ids), ids.size, pos, ptr(logits))
        assert rc == 0, rc
        return logits

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def norm_gains(seed: int, num_layers: int, hidden: int, std: float = 0.1) -> dict:
    """Non-unit RMSNorm gains of the synthetic-data SPEC's stream: 1 + N(0, std) with
    tensor id ((layer + 1) << 8) | 8 for the input norm, | 9 for the post-attention norm
    and 0x03 for the final norm, so every gain vector differs from every other."""
    return {"input": np.stack([1.0 + synth_f32(seed, ((l + 1) << 8) | 8, hidden, std=std) for l in range(num_layers)]),
            "post": np.stack([1.0 + synth_f32(seed, ((l + 1) << 8) | 9, hidden, std=std) for l in range(num_layers)]),
            "final": 1.0 + synth_f32(seed, 0x03, hidden, std=std)}


TINY = dict(num_layers=4, hidden=512, num_q_heads=8, num_kv_heads=2, head_dim=64, ffn=1376, vocab=32000,
            act="f32", weight_format=0, group_size=128, max_tokens=256, rms_eps=1e-5, rope_theta=10000.0)
