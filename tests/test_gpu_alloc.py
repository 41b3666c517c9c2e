"""Steady-state decode allocates nothing (docs/products/aethermind_prd.md:152: after
warm-up the decode path takes no memory beyond the weight mapping and the static KV
growth).

Every device allocation (hipMalloc), pinned host allocation (hipHostMalloc) and HIP
graph instantiation the library makes goes through one counted wrapper
(am_debug_alloc_stats).  After a session's prefill and first decode step (where the
decode graph is captured and instantiated), 64 more decode steps, taken one call at a
time and then as one multi-step call, leave every counter where it was: for a
contiguous-cache session with and without the graph, a paged-KV session whose decode
crosses block boundaries (blocks come from the session's pool, and the device block
table is refreshed from its pinned mirror), and a batch-4 session."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402

L = N.lib()


def stats():
    s = N.AllocStats()
    L.call("am_debug_alloc_stats", C.byref(s))
    return s.as_dict()


@pytest.mark.parametrize("batch,graph,kv_block", [(1, 1, 0), (1, 0, 0), (1, 1, 32), (4, 1, 0), (4, 1, 32)])
def test_decode_steady_state_allocates_nothing(batch, graph, kv_block):
    c = dict(O.TINY, ffn=1536, vocab=4096, num_layers=2)
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    before_model = stats()
    mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                       c["vocab"], c["rms_eps"], c["rope_theta"], N.AM_DT_BF16, N.AM_WF_INT4, 128, 256, 16)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), 3, C.byref(m))
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, graph, batch, 0, kv_block, 0)), C.byref(s))
    try:
        assert stats()["device_allocs"] > before_model["device_allocs"]  # the counter sees the setup
        first = N.i64()
        for r in range(batch):
            prompt = O.token_ids(3, r, c["vocab"], 20 + 3 * r)
            L.call("am_session_prefill_row", s, r, prompt.ctypes.data, prompt.size, C.byref(first))
        out = np.zeros((batch, 1), np.int64)
        L.call("am_session_decode", s, 1, out.ctypes.data)  # warm-up: the decode graph is built here
        warm = stats()
        for _ in range(32):
            L.call("am_session_decode", s, 1, out.ctypes.data)
        many = np.zeros((batch, 32), np.int64)
        L.call("am_session_decode", s, 32, many.ctypes.data)
        L.call("am_runtime_synchronize", rt)
        after = stats()
        assert after == warm, {k: (warm[k], after[k]) for k in warm if warm[k] != after[k]}
        for r in range(batch):
            assert L.am_session_row_position(s, r) == 20 + 3 * r + 65
    finally:
        L.am_session_destroy(s)
        L.am_model_destroy(m)
        L.am_runtime_destroy(rt)
    end = stats()
    # everything the model and session took is returned
    assert end["device_bytes_live"] == before_model["device_bytes_live"]
    assert end["pinned_bytes_live"] == before_model["pinned_bytes_live"]
