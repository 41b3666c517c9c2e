"""am_gfx950_attention_noalloc: the attention entry point that allocates nothing (its
split tickets and records live in the library's file-scope device scratch).  Checked
through the C ABI against am_gfx950_attention with a caller workspace on the same
inputs: identical bits, on two calls in a row with the second one smaller, for the
8B decode shape (split merge in use), the batch-4 long-context decode and a prefill
chunk; a shape beyond the scratch maximum is rejected cleanly, and so is a call that
passes a workspace."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402
from gpu_util import bf16_dev, bits_host, dev, empty, p, stream, zeros  # noqa: E402

L = N.lib()


def _case(seed, B, seq, hq, hkv, d, cap, starts):
    rng = np.random.default_rng(seed)

    def bf(shape):
        a = rng.standard_normal(shape, dtype=np.float32)
        u = a.view(np.uint32)
        return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)

    q = bf16_dev(bf((B, seq, hq * d)))
    kc = bf16_dev(bf((B, hkv, cap, d)))
    vc = bf16_dev(bf((B, hkv, cap, d)))
    posd = dev(np.array(starts, np.int64))
    return q, kc, vc, posd


def _run_both(B, seq, hq, hkv, d, cap, starts, seed):
    q, kc, vc, posd = _case(seed, B, seq, hq, hkv, d, cap, starts)
    out_ref = zeros((B, seq, hq * d), torch.int16)
    out_na = zeros((B, seq, hq * d), torch.int16)
    wsb = L.am_gfx950_attention_workspace_bytes(B, seq, hq, hkv, d, cap, 0)
    ws = zeros((max(wsb, 1),), torch.uint8)
    start_dev = p(posd) if seq == 1 else None
    start_host = 0 if seq == 1 else starts[0]
    a_ref = N.AttentionArgs(p(q), p(kc), p(vc), p(out_ref), seq, hq, hkv, d, cap, start_host, start_dev, B,
                            hkv * cap * d, N.AM_DT_BF16, 0, p(ws), wsb)
    a_na = N.AttentionArgs(p(q), p(kc), p(vc), p(out_na), seq, hq, hkv, d, cap, start_host, start_dev, B,
                           hkv * cap * d, N.AM_DT_BF16, 0, None, 0)
    L.call("am_gfx950_attention", a_ref, stream())
    L.call("am_gfx950_attention_noalloc", a_na, stream())
    got, want = bits_host(out_na), bits_host(out_ref)
    assert want.any(), "reference output is empty"
    assert np.array_equal(got, want), (B, seq, hq, hkv, cap, np.flatnonzero(got != want)[:8])
    return wsb


def test_noalloc_matches_workspace_entry_point_twice_second_smaller():
    print("[noalloc] 8B decode batch 1 ctx 700, then batch 1 ctx 300", flush=True)
    wsb = _run_both(1, 1, 32, 8, 128, 4096, [700], seed=1)
    assert wsb > 0  # the split merge (tickets + records) is in use
    _run_both(1, 1, 32, 8, 128, 1024, [300], seed=2)


def test_noalloc_long_context_batch4_then_smaller():
    print("[noalloc] batch 4 ctx ~8.3k cap 16384, then batch 2 cap 2048", flush=True)
    _run_both(4, 1, 32, 8, 128, 16384, [8300, 8200, 8190, 16383], seed=3)
    _run_both(2, 1, 32, 8, 128, 2048, [2000, 10], seed=4)


def test_noalloc_prefill_chunk_then_decode():
    print("[noalloc] prefill 64 rows at 100, then decode", flush=True)
    _run_both(1, 64, 8, 2, 64, 512, [100], seed=5)
    _run_both(1, 1, 8, 2, 64, 512, [163], seed=6)


def test_noalloc_rejects_oversize_and_workspace():
    big_cap = 1 << 20  # 16 splits x 16 rows x 64 heads x 130 x 4 B > 8 MiB
    need = L.am_gfx950_attention_workspace_bytes(16, 1, 64, 8, 128, big_cap, 0)
    assert need > L.am_gfx950_attention_noalloc_max_bytes()
    dummy = zeros((16,), torch.int16)
    a = N.AttentionArgs(p(dummy), p(dummy), p(dummy), p(dummy), 1, 64, 8, 128, big_cap, 0, p(dummy), 16, 0,
                        N.AM_DT_BF16, 0, None, 0)
    with pytest.raises(N.NativeError) as e:
        L.call("am_gfx950_attention_noalloc", a, stream())
    assert e.value.status == "RESOURCE_EXHAUSTED" and "maximum" in str(e.value)
    ws = zeros((1024,), torch.uint8)
    a2 = N.AttentionArgs(p(dummy), p(dummy), p(dummy), p(dummy), 1, 8, 2, 64, 512, 0, p(dummy), 1, 0,
                         N.AM_DT_BF16, 0, p(ws), 1024)
    with pytest.raises(N.NativeError) as e:
        L.call("am_gfx950_attention_noalloc", a2, stream())
    assert e.value.status == "INVALID_ARGUMENT"
