"""Device-memory plumbing for the GPU tests: torch tensors hold the buffers, the
gfx950 library (through ctypes) does every computation under test."""

from __future__ import annotations

import numpy as np
import torch

import aethermind_amd.native as N


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def empty(shape, dtype) -> torch.Tensor:
    return torch.empty(shape, dtype=dtype, device="cuda:0")


def zeros(shape, dtype) -> torch.Tensor:
    return torch.zeros(shape, dtype=dtype, device="cuda:0")


def p(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream():
    return torch.cuda.current_stream().cuda_stream


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bf16_dev(bits: np.ndarray) -> torch.Tensor:
    """bf16 bit patterns (uint16) -> device int16 buffer with the same bytes."""
    return dev(np.asarray(bits, np.uint16).view(np.int16))


def bits_host(t: torch.Tensor) -> np.ndarray:
    return host(t).view(np.uint16)


def alloc_weight(n: int, k: int, fmt: int, group: int = 128):
    L = N.lib()
    db, sb = N.i64(), N.i64()
    L.call("am_gfx950_weight_bytes", n, k, fmt, group, db, sb)
    data = zeros((db.value,), torch.uint8)
    scales = zeros((max(sb.value, 1),), torch.uint8)
    w = N.Weight(p(data), p(scales) if sb.value else None, n, k, fmt, group)
    return w, data, scales


def pack_weight(src_f32: np.ndarray, fmt: int, group: int = 128, src_bf16_bits: np.ndarray | None = None):
    """Device-repack a logical fp32 (or bf16) matrix with the library's loader kernels."""
    L = N.lib()
    n, k = src_f32.shape
    if src_bf16_bits is not None:
        src = bf16_dev(src_bf16_bits)
        sdt = N.AM_DT_BF16
    else:
        src = dev(src_f32.astype(np.float32))
        sdt = N.AM_DT_F32
    w, data, scales = alloc_weight(n, k, fmt, group)
    qa = N.QuantizeArgs(p(src), sdt, n, w, 0, 1)
    if fmt in (N.AM_WF_INT8, N.AM_WF_INT4):
        L.call("am_gfx950_quantize", qa, stream())
    else:
        L.call("am_gfx950_pack_plain", qa, stream())
    torch.cuda.synchronize()
    return w, (data, scales, src)


def dequant(w: N.Weight) -> np.ndarray:
    out = empty((w.n, w.k), torch.float32)
    N.lib().call("am_gfx950_dequant", N.DequantArgs(w, p(out)), stream())
    return host(out)
