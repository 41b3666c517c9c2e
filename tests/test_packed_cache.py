"""On-disk packed weight cache (am_model_save_packed_cache / am_model_load_packed_cache /
am_packed_cache_inspect), the SavePackedCache / LoadPackedCache of the reference's
weight-packing design (docs/designs/model_loader/model_weight_packing_strategy.md:390-394,
design-only there).

CPU: a cache header written here from the documented byte layout (this file restates
the format and its checksum independently of the C++ writer) is accepted by the
library's inspector, and each kind of damage is refused with its status code.
GPU: a model saved and loaded back has the same device weights byte for byte and
generates the same tokens; a payload corruption or a format mismatch is refused."""

import ctypes as C
import os
import struct

import numpy as np
import pytest

import aethermind_amd.native as N

MASK = (1 << 64) - 1
MUL = 0x9E3779B97F4A7C15
LANES0 = (0x243F6A8885A308D3, 0x13198A2E03707344, 0xA4093822299F31D0, 0x082EFA98EC4E6C89)


def _mix(h, w):
    x = ((h ^ w) * MUL) & MASK
    return ((x << 29) | (x >> 35)) & MASK


def checksum(data: bytes) -> int:
    """Four multiply-rotate lanes over 8-byte little-endian words, 32 bytes per round
    (a short tail zero-padded), folded with the byte length."""
    lanes = list(LANES0)
    n = len(data)
    padded = data + b"\0" * ((-n) % 32)
    for i in range(0, len(padded), 32):
        for lane in range(4):
            lanes[lane] = _mix(lanes[lane], struct.unpack_from("<Q", padded, i + 8 * lane)[0])
    h = (n * MUL) & MASK
    for lane in range(4):
        h = _mix(h, lanes[lane])
    return h ^ (h >> 31)


CFG = dict(num_layers=2, hidden=64, num_q_heads=4, num_kv_heads=2, head_dim=16, ffn=128, vocab=100, rms_eps=1e-5,
           rope_theta=500000.0, act_dtype=N.AM_DT_BF16, weight_format=N.AM_WF_INT4, group_size=32)


def header(payload: bytes, cfg=CFG, magic=b"AMPKGFX1", version=1, arch=b"gfx950", layout=1) -> bytes:
    b = bytearray(256)
    b[0:8] = magic
    struct.pack_into("<IIQQ", b, 8, version, 256, len(payload), checksum(payload))
    b[32:32 + len(arch)] = arch
    struct.pack_into("<I7i", b, 48, layout, cfg["num_layers"], cfg["hidden"], cfg["num_q_heads"],
                     cfg["num_kv_heads"], cfg["head_dim"], cfg["ffn"], cfg["vocab"])
    struct.pack_into("<f", b, 80, cfg["rms_eps"])
    struct.pack_into("<d", b, 88, cfg["rope_theta"])
    struct.pack_into("<3i", b, 96, cfg["act_dtype"], cfg["weight_format"], cfg["group_size"])
    struct.pack_into("<Q", b, 248, checksum(bytes(b[:248])))
    return bytes(b)


def _inspect(path):
    L = N.lib()
    cfg = N.ModelConfig()
    nb = N.i64()
    rc = L.dll.am_packed_cache_inspect(str(path).encode(), C.byref(cfg), C.byref(nb))
    return rc, cfg, nb.value


def test_inspect_accepts_a_header_written_from_the_documented_layout(tmp_path):
    payload = bytes(range(256)) * 16
    p = tmp_path / "ok.ampk"
    p.write_bytes(header(payload) + payload)
    rc, cfg, nb = _inspect(p)
    assert rc == N.AM_STATUS_OK, N.lib().last_error()
    assert nb == len(payload)
    assert (cfg.num_layers, cfg.hidden, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab) == \
        (2, 64, 4, 2, 16, 128, 100)
    assert cfg.rms_eps == pytest.approx(1e-5) and cfg.rope_theta == 500000.0
    assert (cfg.act_dtype, cfg.weight_format, cfg.group_size) == (N.AM_DT_BF16, N.AM_WF_INT4, 32)


@pytest.mark.parametrize("case,code", [
    ("missing", "NOT_FOUND"), ("magic", "INVALID_ARGUMENT"), ("version", "FAILED_PRECONDITION"),
    ("arch", "FAILED_PRECONDITION"), ("layout", "FAILED_PRECONDITION"), ("header_bit", "DATA_LOSS"),
    ("truncated", "DATA_LOSS"), ("padded", "DATA_LOSS"), ("short_header", "DATA_LOSS"),
    ("heads", "INVALID_ARGUMENT"), ("dtype", "INVALID_ARGUMENT")])
def test_inspect_refuses(tmp_path, case, code):
    payload = bytes(4096)
    h = header(payload)
    body = h + payload
    if case == "magic":
        body = header(payload, magic=b"AMPKGFX2") + payload
    elif case == "version":
        body = header(payload, version=2) + payload
    elif case == "arch":
        body = header(payload, arch=b"gfx942") + payload
    elif case == "layout":
        body = header(payload, layout=7) + payload
    elif case == "header_bit":
        body = bytearray(body)
        body[120] ^= 1
        body = bytes(body)
    elif case == "truncated":
        body = body[:-1]
    elif case == "padded":
        body = body + b"\0" * 256
    elif case == "short_header":
        body = h[:100]
    elif case == "heads":
        body = header(payload, cfg=dict(CFG, num_kv_heads=3)) + payload
    elif case == "dtype":
        body = header(payload, cfg=dict(CFG, act_dtype=N.AM_DT_F16)) + payload
    p = tmp_path / "c.ampk"
    if case != "missing":
        p.write_bytes(body)
    rc, _, _ = _inspect(p)
    assert rc == getattr(N, "AM_STATUS_" + code), (case, rc, N.lib().last_error())


# ---------------------------------------------------------------- GPU

def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch


def _slab_bytes(L, m, c):
    """every weight of the model as raw device bytes, in a fixed order"""
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]

    def raw(ptr, n):
        out = np.empty(n, np.uint8)
        assert hip.hipMemcpy(out.ctypes.data, ptr, n, 2) == 0
        return out

    parts = []
    for kind, layers in ((N.AM_BUF_EMBED, [0]), (N.AM_BUF_IN_NORM, range(c["num_layers"])),
                         (N.AM_BUF_POST_NORM, range(c["num_layers"])), (N.AM_BUF_FINAL_NORM, [0])):
        for layer in layers:
            ptr, nb = N.vp(), N.i64()
            L.call("am_model_buffer", m, kind, layer, C.byref(ptr), C.byref(nb))
            parts.append(raw(ptr.value, nb.value))
    roles = [(layer, r) for layer in range(c["num_layers"]) for r in (0, 1, 2, 3)] + [(0, 4)]
    for layer, role in roles:
        w = N.Weight()
        L.call("am_model_weight", m, layer, role, C.byref(w))
        db, sb = N.i64(), N.i64()
        L.call("am_gfx950_weight_bytes", w.n, w.k, w.format, w.group_size, C.byref(db), C.byref(sb))
        parts.append(raw(w.data, db.value))
        if sb.value:
            parts.append(raw(w.scales, sb.value))
    return parts


def _tokens(L, m, n=12):
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1)), C.byref(s))
    prompt = np.arange(3, 20, dtype=np.int64)
    toks, nout = np.zeros(n, np.int64), N.i64()
    L.call("am_session_generate_ids", s, prompt.ctypes.data, prompt.size, n, -1, toks.ctypes.data, C.byref(nout))
    logits = np.zeros(512, np.float32)  # [vocab]
    L.call("am_session_logits", s, logits.ctypes.data)
    L.am_session_destroy(s)
    return toks, logits


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int4", "int8", "bf16"])
def test_save_load_round_trip(tmp_path, fmt):
    _gpu()
    L = N.lib()
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    wf = {"int4": N.AM_WF_INT4, "int8": N.AM_WF_INT8, "bf16": N.AM_WF_BF16}[fmt]
    c = dict(num_layers=3, hidden=256, num_q_heads=4, num_kv_heads=2, head_dim=64, ffn=512, vocab=512)
    mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                       c["vocab"], 1e-5, 10000.0, N.AM_DT_BF16, wf, 128, 256, 16)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 5, C.byref(m))
    path = str(tmp_path / f"model_{fmt}.ampk")
    L.call("am_model_save_packed_cache", m, path.encode())
    assert not os.path.exists(path + ".tmp")
    rc, cfg, nb = _inspect(path)
    assert rc == N.AM_STATUS_OK and (cfg.hidden, cfg.weight_format, cfg.max_tokens) == (256, wf, 0)
    assert os.path.getsize(path) == 256 + nb
    opt = N.ModelLoadOptions(N.AM_DT_BF16, wf, 128, 256, 16)
    m2 = N.vp()
    L.call("am_model_load_packed_cache", rt, path.encode(), C.byref(opt), C.byref(m2))
    a, b = _slab_bytes(L, m, c), _slab_bytes(L, m2, c)
    assert len(a) == len(b) and all(np.array_equal(x, y) for x, y in zip(a, b))
    assert L.am_model_weight_bytes_total(m) == L.am_model_weight_bytes_total(m2)
    t1, l1 = _tokens(L, m)
    t2, l2 = _tokens(L, m2)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)
    L.am_model_destroy(m2)

    # a format the cache does not hold
    other = N.AM_WF_BF16 if wf != N.AM_WF_BF16 else N.AM_WF_INT8
    m3 = N.vp()
    rc = L.dll.am_model_load_packed_cache(rt, path.encode(), C.byref(N.ModelLoadOptions(N.AM_DT_BF16, other, 128,
                                                                                          256, 16)), C.byref(m3))
    assert rc == N.AM_STATUS_INVALID_ARGUMENT and "cache holds" in L.last_error()
    # one payload byte flipped
    with open(path, "r+b") as f:
        f.seek(256 + nb // 2)
        v = f.read(1)
        f.seek(256 + nb // 2)
        f.write(bytes([v[0] ^ 0x40]))
    rc = L.dll.am_model_load_packed_cache(rt, path.encode(), C.byref(opt), C.byref(m3))
    assert rc == N.AM_STATUS_DATA_LOSS, L.last_error()
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)
