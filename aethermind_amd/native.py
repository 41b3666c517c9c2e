"""ctypes bindings of the gfx950 C ABI (include/am_c_api.h, am_gfx950.h, am_runtime.h).

Struct layouts mirror the C headers field for field.  Nothing here computes: every
call goes to ``libaethermind_gfx950.so`` and a missing library is an error.
"""

from __future__ import annotations

import ctypes as C
import os

AM_DT_F32, AM_DT_BF16, AM_DT_F16, AM_DT_I8, AM_DT_I4, AM_DT_I32, AM_DT_I64, AM_DT_U32, AM_DT_U8 = range(9)
AM_WF_F32, AM_WF_BF16, AM_WF_INT8, AM_WF_INT4 = range(4)
AM_PREFILL_SPLIT, AM_PREFILL_SILU_MUL, AM_PREFILL_QKV_ROPE_KV = 0, 1, 2
AM_LOAD_STRICT_TENSOR_NAMES, AM_LOAD_REJECT_UNKNOWN_TENSORS, AM_LOAD_ALLOW_QUANTIZED_TENSORS = 1, 2, 4
(AM_ROLE_QKV, AM_ROLE_O, AM_ROLE_GATE_UP, AM_ROLE_DOWN, AM_ROLE_LM_HEAD, AM_ROLE_Q, AM_ROLE_K, AM_ROLE_V,
 AM_ROLE_GATE, AM_ROLE_UP) = range(10)
AM_BUF_EMBED, AM_BUF_IN_NORM, AM_BUF_POST_NORM, AM_BUF_FINAL_NORM, AM_BUF_ROPE_COS, AM_BUF_ROPE_SIN = range(6)

STATUS_NAMES = ["OK", "CANCELLED", "UNKNOWN", "INVALID_ARGUMENT", "DEADLINE_EXCEEDED", "NOT_FOUND",
                "ALREADY_EXISTS", "PERMISSION_DENIED", "RESOURCE_EXHAUSTED", "FAILED_PRECONDITION", "ABORTED",
                "OUT_OF_RANGE", "UNIMPLEMENTED", "INTERNAL", "UNAVAILABLE", "DATA_LOSS", "OVERFLOW",
                "UNAUTHENTICATED"]

(AM_STATUS_OK, AM_STATUS_CANCELLED, AM_STATUS_UNKNOWN, AM_STATUS_INVALID_ARGUMENT, AM_STATUS_DEADLINE_EXCEEDED,
 AM_STATUS_NOT_FOUND, AM_STATUS_ALREADY_EXISTS, AM_STATUS_PERMISSION_DENIED, AM_STATUS_RESOURCE_EXHAUSTED,
 AM_STATUS_FAILED_PRECONDITION, AM_STATUS_ABORTED, AM_STATUS_OUT_OF_RANGE, AM_STATUS_UNIMPLEMENTED, AM_STATUS_INTERNAL,
 AM_STATUS_UNAVAILABLE, AM_STATUS_DATA_LOSS, AM_STATUS_OVERFLOW, AM_STATUS_UNAUTHENTICATED) = range(len(STATUS_NAMES))

vp, i32, i64, u64, f32, f64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double


class Weight(C.Structure):
    _fields_ = [("data", vp), ("scales", vp), ("n", i64), ("k", i64), ("format", i32), ("group_size", i32)]


class EmbeddingArgs(C.Structure):
    _fields_ = [("ids", vp), ("ids_dtype", i32), ("n_tokens", i64), ("table", vp), ("table_dtype", i32),
                ("vocab", i64), ("hidden", i64), ("out", vp), ("out_dtype", i32), ("err_flag", vp), ("check", i32)]


class RmsNormArgs(C.Structure):
    _fields_ = [("x", vp), ("w", vp), ("out", vp), ("rows", i64), ("hidden", i64), ("x_stride", i64),
                ("out_stride", i64), ("eps", f32), ("x_dtype", i32), ("w_dtype", i32), ("out_dtype", i32)]


class LinearArgs(C.Structure):
    _fields_ = [("x", vp), ("x_dtype", i32), ("m", i64), ("w", Weight), ("out", vp), ("out_dtype", i32),
                ("residual", vp), ("mode", i32), ("workspace", vp), ("workspace_bytes", i64)]


class KvPages(C.Structure):
    _fields_ = [("block_table", vp), ("block_size", i32), ("table_stride", i32), ("num_blocks", i64),
                ("err_flag", vp)]


class PrefillRopeKv(C.Structure):
    _fields_ = [("cos_tab", vp), ("sin_tab", vp), ("max_pos", i64), ("start_pos_dev", vp), ("k_cache", vp),
                ("v_cache", vp), ("hq", i64), ("hkv", i64), ("head_dim", i64), ("capacity", i64),
                ("pages", C.POINTER(KvPages)), ("err_flag", vp)]


class PrefillLinearArgs(C.Structure):
    _fields_ = [("x", vp), ("m", i64), ("w", Weight), ("epilogue", i32), ("out", vp * 3), ("split", i64 * 2),
                ("workspace", vp), ("workspace_bytes", i64), ("rope_kv", C.POINTER(PrefillRopeKv))]


class RopeArgs(C.Structure):
    _fields_ = [("q", vp), ("k", vp), ("q_out", vp), ("k_out", vp), ("pos", vp), ("cos_tab", vp), ("sin_tab", vp),
                ("seq", i64), ("hq", i64), ("hkv", i64), ("head_dim", i64), ("max_pos", i64), ("dtype", i32)]


class KvUpdateArgs(C.Structure):
    _fields_ = [("k", vp), ("v", vp), ("k_cache", vp), ("v_cache", vp), ("seq", i64), ("hkv", i64),
                ("head_dim", i64), ("capacity", i64), ("start_pos", i64), ("start_pos_dev", vp), ("dtype", i32),
                ("err_flag", vp), ("pages", C.POINTER(KvPages))]


class AttentionArgs(C.Structure):
    _fields_ = [("q", vp), ("k_cache", vp), ("v_cache", vp), ("out", vp), ("seq", i64), ("hq", i64), ("hkv", i64),
                ("head_dim", i64), ("capacity", i64), ("start_pos", i64), ("start_pos_dev", vp), ("batch", i64),
                ("cache_batch_stride", i64), ("dtype", i32), ("num_splits", i32), ("workspace", vp),
                ("workspace_bytes", i64), ("pages", C.POINTER(KvPages))]


class SiluMulArgs(C.Structure):
    _fields_ = [("gate", vp), ("up", vp), ("out", vp), ("n", i64), ("dtype", i32)]


class AddArgs(C.Structure):
    _fields_ = [("a", vp), ("b", vp), ("out", vp), ("n", i64), ("dtype", i32)]


class ArgmaxArgs(C.Structure):
    _fields_ = [("x", vp), ("dtype", i32), ("rows", i64), ("n", i64), ("out", vp), ("workspace", vp),
                ("workspace_bytes", i64)]


class QuantizeArgs(C.Structure):
    _fields_ = [("src", vp), ("src_dtype", i32), ("src_rows", i64), ("dst", Weight), ("dst_row_offset", i64),
                ("dst_row_stride", i64)]


class PackInt4Args(C.Structure):
    _fields_ = [("logical", vp), ("scales", vp), ("dst", Weight)]


class GptqArgs(C.Structure):
    _fields_ = [("qweight", vp), ("qzeros", vp), ("scales", vp), ("scales_dtype", i32), ("zero_offset", i32),
                ("g_idx", vp), ("n", i64), ("k", i64), ("group_size", i64), ("out_f32", vp), ("out_logical", vp),
                ("out_scales", vp)]


class DequantArgs(C.Structure):
    _fields_ = [("w", Weight), ("out", vp)]


class SynthArgs(C.Structure):
    _fields_ = [("seed", u64), ("tensor_id", u64), ("stddev", f64), ("offset", i64), ("n", i64), ("out", vp),
                ("dtype", i32)]


class FusedQkvArgs(C.Structure):
    _fields_ = [("h", vp), ("norm_w", vp), ("eps", f32), ("w_qkv", Weight), ("cos_tab", vp), ("sin_tab", vp),
                ("pos", vp), ("q_out", vp), ("k_cache", vp), ("v_cache", vp), ("hq", i64), ("hkv", i64),
                ("head_dim", i64), ("capacity", i64), ("dtype", i32), ("rows", i64), ("cache_batch_stride", i64),
                ("pages", C.POINTER(KvPages))]


class FusedLinearResidualArgs(C.Structure):
    _fields_ = [("x", vp), ("w", Weight), ("h", vp), ("dtype", i32), ("rows", i64)]


class FusedGateUpArgs(C.Structure):
    _fields_ = [("h", vp), ("norm_w", vp), ("eps", f32), ("w_gate_up", Weight), ("act_out", vp), ("dtype", i32),
                ("rows", i64)]


class FusedLmHeadArgs(C.Structure):
    _fields_ = [("h", vp), ("norm_w", vp), ("eps", f32), ("w", Weight), ("logits", vp), ("token_out", vp),
                ("tokens_hist", vp), ("pos", vp), ("step", vp), ("dtype", i32), ("workspace", vp),
                ("workspace_bytes", i64), ("rows", i64), ("hist_stride", i64)]


class LaunchInfo(C.Structure):
    _fields_ = [("kernel", C.c_char * 96), ("grid", i64), ("block_threads", i32), ("lds_bytes", i32)]


class DecodeLayer(C.Structure):
    _fields_ = [("w_qkv", Weight), ("w_o", Weight), ("w_gate_up", Weight), ("w_down", Weight), ("in_norm", vp),
                ("post_norm", vp), ("k_cache", vp), ("v_cache", vp)]


class DecodeLayersArgs(C.Structure):
    _fields_ = [("layers", vp), ("num_layers", i64), ("hidden", i64), ("hq", i64), ("hkv", i64), ("head_dim", i64),
                ("ffn", i64), ("capacity", i64), ("eps", f32), ("cos_tab", vp), ("sin_tab", vp), ("pos", vp),
                ("h", vp), ("workspace", vp), ("workspace_bytes", i64), ("dtype", i32), ("timeline", vp)]


class ModelConfig(C.Structure):
    _fields_ = [("num_layers", i32), ("hidden", i32), ("num_q_heads", i32), ("num_kv_heads", i32),
                ("head_dim", i32), ("ffn", i32), ("vocab", i32), ("rms_eps", f32), ("rope_theta", f64),
                ("act_dtype", i32), ("weight_format", i32), ("group_size", i32), ("max_tokens", i32),
                ("max_prefill_chunk", i32)]


class ModelLoadOptions(C.Structure):
    _fields_ = [("act_dtype", i32), ("weight_format", i32), ("group_size", i32), ("max_tokens", i32),
                ("max_prefill_chunk", i32)]


class Config(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("device", i32), ("act_dtype", i32), ("weight_format", i32),
                ("group_size", i32), ("max_tokens", i32), ("max_prefill_chunk", i32), ("load_flags", C.c_uint32)]


class SessionConfig(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("max_tokens", C.c_uint32), ("eos_token_id", i64), ("use_graph", i32)]


class AllocStats(C.Structure):
    _fields_ = [("device_allocs", i64), ("device_frees", i64), ("device_bytes_live", i64), ("pinned_allocs", i64),
                ("pinned_frees", i64), ("pinned_bytes_live", i64), ("graph_instantiations", i64)]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


class SessionOptions(C.Structure):
    _fields_ = [("fused_decode", i32), ("use_graph", i32), ("batch", i32), ("persistent_decode", i32),
                ("kv_block_size", i32), ("kv_pool_blocks", i32)]


_SIGS = {
    # name: (restype, argtypes)
    "am_last_error_message": (C.c_char_p, []),
    "am_gfx950_error_create": (vp, [i32, C.c_char_p]),
    "am_gfx950_error_destroy": (None, [vp]),
    "am_gfx950_error_code": (i32, [vp]),
    "am_gfx950_error_message": (C.c_char_p, [vp]),
    "am_gfx950_device_count": (i32, []),
    "am_gfx950_last_launch": (i32, [C.POINTER(LaunchInfo)]),
    "am_gfx950_version": (C.c_char_p, []),
    "am_gfx950_embedding": (i32, [C.POINTER(EmbeddingArgs), vp]),
    "am_gfx950_embed_token": (i32, [vp, vp, i32, i64, i64, vp, vp, vp]),
    "am_gfx950_rmsnorm": (i32, [C.POINTER(RmsNormArgs), vp]),
    "am_gfx950_linear": (i32, [C.POINTER(LinearArgs), vp]),
    "am_gfx950_prefill_linear": (i32, [C.POINTER(PrefillLinearArgs), vp]),
    "am_gfx950_gemm_workspace_bytes": (i64, [i64, i64, i64, i64]),
    "am_gfx950_rope": (i32, [C.POINTER(RopeArgs), vp]),
    "am_gfx950_rope_table": (i32, [i64, i64, f64, vp, vp]),
    "am_gfx950_kv_update": (i32, [C.POINTER(KvUpdateArgs), vp]),
    "am_gfx950_attention": (i32, [C.POINTER(AttentionArgs), vp]),
    "am_gfx950_attention_workspace_bytes": (i64, [i64, i64, i64, i64, i64, i64, i32]),
    "am_gfx950_attention_noalloc": (i32, [C.POINTER(AttentionArgs), vp]),
    "am_gfx950_attention_noalloc_max_bytes": (i64, []),
    "am_gfx950_silu_mul": (i32, [C.POINTER(SiluMulArgs), vp]),
    "am_gfx950_add": (i32, [C.POINTER(AddArgs), vp]),
    "am_gfx950_argmax": (i32, [C.POINTER(ArgmaxArgs), vp]),
    "am_gfx950_argmax_workspace_bytes": (i64, [i64]),
    "am_gfx950_quantize": (i32, [C.POINTER(QuantizeArgs), vp]),
    "am_gfx950_pack_plain": (i32, [C.POINTER(QuantizeArgs), vp]),
    "am_gfx950_pack_int4": (i32, [C.POINTER(PackInt4Args), vp]),
    "am_gfx950_dequant": (i32, [C.POINTER(DequantArgs), vp]),
    "am_gfx950_gptq_unpack": (i32, [C.POINTER(GptqArgs), vp]),
    "am_gfx950_weight_bytes": (i32, [i64, i64, i32, i32, C.POINTER(i64), C.POINTER(i64)]),
    "am_gfx950_synth_normal": (i32, [C.POINTER(SynthArgs), vp]),
    "am_gfx950_synth_token_ids": (i32, [u64, u64, i64, i64, vp, vp]),
    "am_gfx950_fill": (i32, [vp, i32, i64, f32, vp]),
    "am_gfx950_fused_qkv": (i32, [C.POINTER(FusedQkvArgs), vp]),
    "am_gfx950_fused_linear_residual": (i32, [C.POINTER(FusedLinearResidualArgs), vp]),
    "am_gfx950_fused_gate_up": (i32, [C.POINTER(FusedGateUpArgs), vp]),
    "am_gfx950_fused_lm_head": (i32, [C.POINTER(FusedLmHeadArgs), vp]),
    "am_gfx950_lm_head_workspace_bytes": (i64, []),
    "am_gfx950_decode_layers": (i32, [C.POINTER(DecodeLayersArgs), vp]),
    "am_gfx950_decode_layers_workspace_bytes": (i64, [i64, i64, i64, i64, i64]),
    "am_gfx950_decode_layers_validate": (i32, [C.POINTER(DecodeLayersArgs), C.POINTER(DecodeLayer)]),
    "am_gfx950_decode_layers_aborted": (i32, [vp, C.POINTER(i32)]),
    "am_gfx950_decode_advance": (i32, [vp, vp, vp, vp, vp]),
    "am_gfx950_decode_advance_rows": (i32, [vp, i64, vp, i64, vp, vp, vp]),
    "am_runtime_open": (i32, [i32, C.POINTER(vp)]),
    "am_runtime_destroy": (None, [vp]),
    "am_runtime_stream": (vp, [vp]),
    "am_runtime_synchronize": (i32, [vp]),
    "am_synth_token_ids_host": (i32, [u64, u64, i64, i64, vp]),
    "am_model_create_synthetic": (i32, [vp, C.POINTER(ModelConfig), u64, C.POINTER(vp)]),
    "am_model_destroy": (None, [vp]),
    "am_model_weight": (i32, [vp, i32, i32, C.POINTER(Weight)]),
    "am_model_load_hf": (i32, [vp, C.c_char_p, C.POINTER(ModelLoadOptions), C.POINTER(vp)]),
    "am_hf_inspect": (i32, [C.c_char_p, C.POINTER(ModelConfig), C.POINTER(i64), C.POINTER(i64)]),
    "am_model_load_hf_ex": (i32, [vp, C.c_char_p, C.POINTER(ModelLoadOptions), C.c_uint32, C.POINTER(vp)]),
    "am_hf_inspect_ex": (i32, [C.c_char_p, C.c_uint32, C.POINTER(ModelConfig), C.POINTER(i64), C.POINTER(i64)]),
    "am_model_save_packed_cache": (i32, [vp, C.c_char_p]),
    "am_packed_cache_inspect": (i32, [C.c_char_p, C.POINTER(ModelConfig), C.POINTER(i64)]),
    "am_model_load_packed_cache": (i32, [vp, C.c_char_p, C.POINTER(ModelLoadOptions), C.POINTER(vp)]),
    "am_model_buffer": (i32, [vp, i32, i32, C.POINTER(vp), C.POINTER(i64)]),
    "am_model_weight_bytes_total": (i64, [vp]),
    "am_debug_alloc_stats": (i32, [C.POINTER(AllocStats)]),
    "am_session_open": (i32, [vp, C.POINTER(SessionOptions), C.POINTER(vp)]),
    "am_session_destroy": (None, [vp]),
    "am_session_prefill": (i32, [vp, vp, i64, C.POINTER(i64)]),
    "am_session_prefill_row": (i32, [vp, i64, vp, i64, C.POINTER(i64)]),
    "am_session_batch": (i64, [vp]),
    "am_session_row_position": (i64, [vp, i64]),
    "am_session_decode": (i32, [vp, i64, vp]),
    "am_session_decode_async": (i32, [vp, i64]),
    "am_session_generate_ids": (i32, [vp, vp, i64, i64, i64, vp, C.POINTER(i64)]),
    "am_runtime_create": (vp, [C.POINTER(Config)]),
    "am_model_load": (vp, [vp, C.c_char_p, C.POINTER(vp)]),
    "am_model_unload": (None, [vp]),
    "am_session_create": (vp, [vp, C.POINTER(SessionConfig)]),
    "am_session_generate": (i32, [vp, vp, C.c_size_t, vp, C.c_size_t, C.POINTER(C.c_size_t), C.POINTER(vp)]),
    "am_error_free": (None, [vp]),
    "am_session_logits": (i32, [vp, vp]),
    "am_session_position": (i64, [vp]),
    "am_session_decode_plan_size": (i64, [vp]),
    "am_session_persistent_decode": (i32, [vp]),
    "am_session_profile_decode": (i32, [vp, i64, vp, vp]),
}


class NativeError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        name = STATUS_NAMES[code] if 0 <= code < len(STATUS_NAMES) else str(code)
        super().__init__(f"{fn} -> {name}: {msg}")
        self.code = code
        self.status = name


def lib_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "libaethermind_gfx950.so")


class Lib:
    """Loaded library with typed functions; ``call`` raises NativeError on non-OK."""

    def __init__(self, path: str | None = None):
        path = path or lib_path()
        if not os.path.exists(path):
            raise RuntimeError(f"gfx950 library not built ({path}); run __graft_entry__.build()")
        self.path = path
        self.dll = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(self.dll, name)
            fn.restype = res
            fn.argtypes = args

    def __getattr__(self, name):
        return getattr(self.dll, name)

    def last_error(self) -> str:
        """this thread's last error text (am_last_error_message)"""
        msg = self.dll.am_last_error_message()
        return msg.decode() if msg else ""

    def call(self, name: str, *args) -> None:
        rc = getattr(self.dll, name)(*args)
        if rc != 0:
            msg = self.dll.am_last_error_message()
            raise NativeError(name, rc, msg.decode() if msg else "")


_LIB: Lib | None = None


def lib() -> Lib:
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB


def last_launch() -> LaunchInfo:
    """The last kernel an entry point launched on this thread (name and launch shape)."""
    info = LaunchInfo()
    lib().call("am_gfx950_last_launch", C.byref(info))
    return info


def header_functions(include_dir: str) -> list[str]:
    """Names of every function declared in the C headers (for the export check)."""
    import re
    names = []
    for fn in sorted(os.listdir(include_dir)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(include_dir, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(am_\w+)\s*\(", text, flags=re.M):
            names.append(m.group(1))
    return sorted(set(names))
