"""aethermind_amd -- MI355X (gfx950) prefill/decode path for AetherMind.

The product is the in-tree shared library ``libaethermind_gfx950.so`` (HIP kernels,
C ABI in ``include/am_gfx950.h`` / ``include/am_runtime.h``, C++20 host runtime).
This package only binds it with ctypes so tests and the benchmark can drive it; it
holds no compute of its own and raises when the library is missing.
"""

from .native import (  # noqa: F401
    AM_DT_BF16,
    AM_DT_F32,
    AM_DT_I32,
    AM_DT_I64,
    AM_DT_U32,
    AM_WF_BF16,
    AM_WF_F32,
    AM_WF_INT4,
    AM_WF_INT8,
    Lib,
    ModelConfig,
    NativeError,
    Weight,
    lib,
    lib_path,
)
