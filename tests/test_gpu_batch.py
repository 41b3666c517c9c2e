"""Batched decode: up to 16 sequences advanced one token per step together.

The batched kernels (one read of the weights for all token rows, MFMA skinny GEMM)
are checked through the C ABI against the CPU oracle ops on the same inputs: Linear
(store, fp32 out, residual), the fused RMSNorm+q/k/v+RoPE+KV write at per-row
positions into per-sequence cache planes, RMSNorm+gate/up+SiLU-Mul, Linear+Add and
RMSNorm+lm_head+Argmax with the per-row decode-state update.  A batched session is
checked sequence by sequence against oracle models fed the same tokens.  Bars: bf16
paths within 2e-2 of the largest reference magnitude, per row;
argmax and state updates exact.
"""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402
from gpu_util import bf16_dev, bits_host, dev, empty, host, p, pack_weight, stream, zeros  # noqa: E402
from test_gpu_decode_shapes import launched  # noqa: E402

L = N.lib()
TOL = 2e-2


def close(got, ref, tol, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.max(np.abs(ref)), 1e-30)
    err = np.max(np.abs(got - ref)) / scale
    assert err <= tol, f"{what}: max rel err {err:.3e} > {tol}"


def rows_close(got, ref, tol, what):
    for r in range(ref.shape[0]):
        close(got[r], ref[r], tol, f"{what} row {r}")


def weights(n, k, fmt, seed):
    bits = O.synth_bf16(seed, 0x55, n * k).reshape(n, k)
    w = O.bf16_to_f32(bits).copy()
    dw, keep = pack_weight(w, fmt, 128, src_bf16_bits=bits)
    if fmt == N.AM_WF_INT8:
        w = O.dequant_int8(*O.quant_int8(w))
    elif fmt == N.AM_WF_INT4:
        pk, sc = O.quant_int4(w, 128)
        w = O.dequant_int4(pk, sc, k, 128)
    return w, dw, keep


def rbf(x):
    return O.round_bf16(np.asarray(x, np.float32))


def bf_rows(seed, tid, m, k, std=1.0):
    return rbf(O.synth_f32(seed, tid, m * k, std=std).reshape(m, k))


def rd(t):
    return O.bf16_to_f32(bits_host(t))


FMTS = [N.AM_WF_BF16, N.AM_WF_INT8, N.AM_WF_INT4]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m,n,k", [(1, 1376, 512), (2, 1040, 4096), (4, 200, 14336), (7, 130, 1024),
                                   (16, 4096, 4096), (16, 33, 256)])
def test_linear_batched(fmt, m, n, k):
    """am_gfx950_linear mode 3: every row against the oracle Linear, bf16 and fp32
    outputs, and the residual form; feature counts that are not a multiple of the
    16-feature tile and row counts that are not a multiple of 4."""
    wref, dw, keep = weights(n, k, fmt, seed=21 + m)
    x = bf_rows(22, m, m, k)
    xd = bf16_dev(O.bf16_bits(x))
    ref = O.linear(x, wref)
    out = empty((m, n), torch.int16)
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(out), N.AM_DT_BF16, None, 3), stream())
    rows_close(rd(out), ref, TOL, f"batched linear fmt={fmt} {m}x{n}x{k}")
    lo = empty((m, n), torch.float32)
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(lo), N.AM_DT_F32, None, 3), stream())
    rows_close(host(lo), ref, 5e-3, "fp32 out")
    res = bf_rows(23, m, m, n)
    rdv = bf16_dev(O.bf16_bits(res))
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(out), N.AM_DT_BF16, p(rdv), 3), stream())
    rows_close(rd(out), rbf(res + rbf(ref)), TOL, "residual")


def test_linear_auto_mode_takes_batched_kernel():
    """mode 0 with 2..16 bf16 rows gives the batched kernel's result (identical bits
    to mode 3)."""
    m, n, k = 5, 300, 512
    wref, dw, keep = weights(n, k, N.AM_WF_INT4, seed=30)
    x = bf_rows(31, 0, m, k)
    xd = bf16_dev(O.bf16_bits(x))
    a, b = empty((m, n), torch.int16), empty((m, n), torch.int16)
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(a), N.AM_DT_BF16, None, 0), stream())
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(b), N.AM_DT_BF16, None, 3), stream())
    assert np.array_equal(bits_host(a), bits_host(b))


def test_linear_batched_rejects_unsupported():
    wref, dw, keep = weights(64, 4096, N.AM_WF_INT4, seed=32)
    x = bf16_dev(O.bf16_bits(bf_rows(33, 0, 17, 4096)))
    out = empty((17, 64), torch.int16)
    with pytest.raises(N.NativeError) as e:  # 17 rows
        L.call("am_gfx950_linear", N.LinearArgs(p(x), N.AM_DT_BF16, 17, dw, p(out), N.AM_DT_BF16, None, 3), stream())
    assert e.value.status == "INVALID_ARGUMENT"


def test_linear_batched_row_groups():
    """8 rows x 16384 bf16 values do not fit one block's LDS: the launch runs in row
    groups (each re-reading the weights), with outputs and residuals at their rows."""
    w2, dw2, keep2 = weights(64, 16384, N.AM_WF_BF16, seed=34)
    x2 = bf_rows(35, 0, 8, 16384)
    x2d = bf16_dev(O.bf16_bits(x2))
    ref = O.linear(x2, w2)
    out2 = empty((8, 64), torch.int16)
    L.call("am_gfx950_linear", N.LinearArgs(p(x2d), N.AM_DT_BF16, 8, dw2, p(out2), N.AM_DT_BF16, None, 3), stream())
    rows_close(rd(out2), ref, TOL, "row groups")
    res = bf_rows(36, 0, 8, 64)
    rdv = bf16_dev(O.bf16_bits(res))
    L.call("am_gfx950_linear", N.LinearArgs(p(x2d), N.AM_DT_BF16, 8, dw2, p(rdv), N.AM_DT_BF16, p(rdv), 3), stream())
    rows_close(rd(rdv), rbf(res + rbf(ref)), TOL, "row groups residual")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("d", [64, 128])
def test_fused_qkv_batched(fmt, d):
    """RMSNorm -> q|k|v -> RoPE -> KV write for B sequences at different positions:
    q rows, the K/V rows at each sequence's position in its own cache planes (planes
    cbs elements apart), and nothing else in the caches written."""
    B, H, hq, hkv, cap = 3, 512, 8, 2, 64
    n = (hq + 2 * hkv) * d
    wref, dw, keep = weights(n, H, fmt, seed=40 + d)
    h = bf_rows(41, d, B, H)
    nw = rbf(1.0 + 0.25 * O.synth_f32(42, 0, H, std=1.0))
    pos = np.array([5, 17, 63], np.int64)
    ct, st = O.rope_tables(cap, d, 10000.0)
    cbs = hkv * cap * d + 96  # per-sequence plane stride with padding
    kc = zeros((B * cbs,), torch.int16)
    vc = zeros((B * cbs,), torch.int16)
    qo = empty((B, hq * d), torch.int16)
    hd, nwd, pd, ctd, std_ = bf16_dev(O.bf16_bits(h)), bf16_dev(O.bf16_bits(nw)), dev(pos), dev(ct), dev(st)
    a = N.FusedQkvArgs(p(hd), p(nwd), 1e-5, dw, p(ctd), p(std_), p(pd), p(qo), p(kc), p(vc), hq, hkv, d, cap,
                       N.AM_DT_BF16, B, cbs)
    L.call("am_gfx950_fused_qkv", a, stream())
    xn = rbf(O.rmsnorm(h, nw, 1e-5))
    y = rbf(O.linear(xn, wref))
    Q, KV = hq * d, hkv * d
    qr = rbf(O.rope(y[:, :Q], hq, d, pos, ct, st))
    kr = rbf(O.rope(y[:, Q:Q + KV], hkv, d, pos, ct, st))
    vr = y[:, Q + KV:]
    rows_close(rd(qo), qr, TOL, "q")
    kh, vh = rd(kc), rd(vc)
    for b in range(B):
        kplane = kh[b * cbs:b * cbs + hkv * cap * d].reshape(hkv, cap, d)
        vplane = vh[b * cbs:b * cbs + hkv * cap * d].reshape(hkv, cap, d)
        close(kplane[:, pos[b], :].reshape(-1), kr[b], TOL, f"k row {b}")
        close(vplane[:, pos[b], :].reshape(-1), vr[b], TOL, f"v row {b}")
        kplane[:, pos[b], :] = 0
        vplane[:, pos[b], :] = 0
        assert not kplane.any() and not vplane.any(), f"stray cache writes in sequence {b}"
        assert not kh[b * cbs + hkv * cap * d:(b + 1) * cbs].any(), "write into the plane padding"


@pytest.mark.parametrize("fmt", FMTS)
def test_fused_gate_up_and_residual_batched(fmt):
    B, H, F = 5, 512, 1536
    wgu, dgu, k1 = weights(2 * F, H, fmt, seed=50)
    wdn, ddn, k2 = weights(H, F, fmt, seed=51)
    h = bf_rows(52, 0, B, H)
    nw = rbf(1.0 + 0.25 * O.synth_f32(53, 0, H, std=1.0))
    hd, nwd = bf16_dev(O.bf16_bits(h)), bf16_dev(O.bf16_bits(nw))
    act = empty((B, F), torch.int16)
    L.call("am_gfx950_fused_gate_up", N.FusedGateUpArgs(p(hd), p(nwd), 1e-5, dgu, p(act), N.AM_DT_BF16, B), stream())
    xn = rbf(O.rmsnorm(h, nw, 1e-5))
    gu = rbf(O.linear(xn, wgu))
    aref = rbf(O.silu_mul(gu[:, :F], gu[:, F:]))
    rows_close(rd(act), aref, TOL, "gate/up silu")
    # down projection + residual, in place on h, fed the device activations
    a_dev = rd(act)
    L.call("am_gfx950_fused_linear_residual", N.FusedLinearResidualArgs(p(act), ddn, p(hd), N.AM_DT_BF16, B),
           stream())
    rows_close(rd(hd), rbf(h + rbf(O.linear(a_dev, wdn))), TOL, "down + residual")


def test_fused_lm_head_batched_argmax_and_state():
    """RMSNorm -> lm_head logits (fp32) -> per-row argmax, tokens_hist[r][step],
    pos[r] + 1, step + 1 once."""
    B, H, V = 4, 512, 5000
    w, dw, keep = weights(V, H, N.AM_WF_INT4, seed=60)
    h = bf_rows(61, 0, B, H)
    nw = rbf(np.ones(H, np.float32))
    hd, nwd = bf16_dev(O.bf16_bits(h)), bf16_dev(O.bf16_bits(nw))
    logits = empty((B, V), torch.float32)
    tok = zeros((B,), torch.int64)
    hs = 9
    hist = zeros((B, hs), torch.int64)
    pos = dev(np.array([3, 10, 20, 30], np.int64))
    step = dev(np.array([2], np.int64))
    ws = zeros((L.am_gfx950_lm_head_workspace_bytes(),), torch.uint8)
    a = N.FusedLmHeadArgs(p(hd), p(nwd), 1e-5, dw, p(logits), p(tok), p(hist), p(pos), p(step), N.AM_DT_BF16,
                          p(ws), ws.numel(), B, hs)
    for it in range(2):
        L.call("am_gfx950_fused_lm_head", a, stream())
        lg = host(logits)
        rows_close(lg, O.linear(rbf(O.rmsnorm(h, nw, 1e-5)), w), 5e-3, "logits")
        want = np.array([O.argmax(lg[r]) for r in range(B)])
        assert np.array_equal(host(tok), want)
        assert np.array_equal(host(hist)[:, 2 + it], want)
        assert np.array_equal(host(pos), np.array([3, 10, 20, 30]) + it + 1)
        assert int(host(step)[0]) == 3 + it
    assert not host(ws)[:256].any(), "argmax tickets must be left zero"


@pytest.mark.parametrize("B", [4, 2])
def test_attention_decode_long_context_batch4(B):
    """The long-context decode of BASELINE configs[4]: four sequences at positions near
    8k (and one at the last cache row) over their own cache planes, 8B head shape.  A
    grid that gives every CU a block (8 splits x 8 kv heads x 4 rows = 256) runs the
    8-wave block (two waves per SIMD); batch 2 keeps the 4-wave block."""
    hq, hkv, d, cap = 32, 8, 128, 8448
    starts = [8191, 8300, 5000, cap - 1][:B]
    q = rbf(O.synth_f32(70, 1, B * hq * d, std=1.0).reshape(B, hq * d))
    kc = rbf(O.synth_f32(70, 2, B * hkv * cap * d, std=1.0).reshape(B, hkv, cap, d))
    vc = rbf(O.synth_f32(70, 3, B * hkv * cap * d, std=1.0).reshape(B, hkv, cap, d))
    qd, kd, vd = bf16_dev(O.bf16_bits(q)), bf16_dev(O.bf16_bits(kc)), bf16_dev(O.bf16_bits(vc))
    out = empty((B, hq * d), torch.int16)
    posd = dev(np.array(starts, np.int64))
    wsb = L.am_gfx950_attention_workspace_bytes(B, 1, hq, hkv, d, cap, 0)
    ws = zeros((max(wsb, 1),), torch.uint8)
    a = N.AttentionArgs(p(qd), p(kd), p(vd), p(out), 1, hq, hkv, d, cap, 0, p(posd), B, hkv * cap * d, 1, 0,
                        p(ws), wsb)
    L.call("am_gfx950_attention", a, stream())
    name = launched()
    wide = 8 * hkv * B >= torch.cuda.get_device_properties(0).multi_processor_count
    assert name == f"attention_decode<d=128,g=4,splits=8{',waves=8' if wide else ''}>", name
    got = rd(out)
    for r in range(B):
        ref = O.attention(q[r:r + 1], kc[r], vc[r], 1, hq, hkv, d, cap, starts[r])[0]
        close(got[r], ref, TOL, f"row {r} start {starts[r]}")


# ---------------------------------------------------------------- batched session
class _Rt:
    def __init__(self):
        self.rt = N.vp()
        L.call("am_runtime_open", 0, C.byref(self.rt))

    def close(self):
        L.am_runtime_destroy(self.rt)


@pytest.mark.parametrize("fmt", [N.AM_WF_INT4, N.AM_WF_BF16])
@pytest.mark.parametrize("graph", [1, 0])
def test_batched_session_matches_oracle_per_sequence(fmt, graph):
    """Three sequences with prompts of different lengths prefilled into their own KV
    reservations and decoded together: every sequence's logits after the prefill and
    after each decode step match an oracle model of that sequence fed the same
    tokens, and the batched decode gives each sequence the tokens its own logits pick."""
    cfg = dict(O.TINY, act="bf16", weight_format=fmt, ffn=1536, vocab=4096, num_layers=2, max_tokens=64)
    B, seed = 3, 7
    rt = _Rt()
    mc = N.ModelConfig(cfg["num_layers"], cfg["hidden"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                       cfg["ffn"], cfg["vocab"], cfg["rms_eps"], cfg["rope_theta"], N.AM_DT_BF16, fmt, 128,
                       cfg["max_tokens"], 8)
    m = N.vp()
    L.call("am_model_create_synthetic", rt.rt, C.byref(mc), seed, C.byref(m))
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, graph, B)), C.byref(s))
    assert L.am_session_batch(s) == B
    prompts = [O.token_ids(seed, 10 + r, cfg["vocab"], n) for r, n in enumerate((12, 5, 19))]
    orcs = [O.OracleModel(cfg, seed) for _ in range(B)]
    toks = []
    V = cfg["vocab"]
    got = np.zeros((B, V), np.float32)
    for r in range(B):
        first = N.i64()
        L.call("am_session_prefill_row", s, r, prompts[r].ctypes.data, prompts[r].size, C.byref(first))
        L.call("am_session_logits", s, got.ctypes.data)
        ref = orcs[r].forward(prompts[r], 0)
        close(got[r], ref, TOL, f"prefill logits seq {r}")
        assert int(first.value) == O.argmax(got[r])
        toks.append(int(first.value))
        assert L.am_session_row_position(s, r) == prompts[r].size
    posn = [pr.size for pr in prompts]
    for step in range(4):
        out = np.zeros((B, 1), np.int64)
        L.call("am_session_decode", s, 1, out.ctypes.data)
        L.call("am_session_logits", s, got.ctypes.data)
        for r in range(B):
            ref = orcs[r].forward(np.array([toks[r]], np.int64), posn[r])
            close(got[r], ref, TOL, f"decode step {step} seq {r}")
            assert int(out[r, 0]) == O.argmax(got[r])
            toks[r] = int(out[r, 0])
            posn[r] += 1
            assert L.am_session_row_position(s, r) == posn[r]
    # a multi-step call returns [B][n] tokens, sequence-major, and each sequence keeps
    # following its own logits
    out = np.zeros((B, 3), np.int64)
    L.call("am_session_decode", s, 3, out.ctypes.data)
    L.call("am_session_logits", s, got.ctypes.data)
    for r in range(B):
        assert int(out[r, 2]) == O.argmax(got[r])
    for o in orcs:
        o.close()
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    rt.close()


def test_batched_session_rows_in_groups_match_oracle():
    """Eight sequences with a 14336-wide FFN: the down projection's token rows (8 x 14336
    bf16) exceed one block's LDS, so its batched launches run in row groups (5 + 3),
    each re-reading the weights; every sequence's logits still match its own oracle."""
    cfg = dict(O.TINY, act="bf16", weight_format=N.AM_WF_INT4, ffn=14336, vocab=4096, num_layers=2, max_tokens=48)
    B, seed = 8, 9
    rt = _Rt()
    mc = N.ModelConfig(cfg["num_layers"], cfg["hidden"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                       cfg["ffn"], cfg["vocab"], cfg["rms_eps"], cfg["rope_theta"], N.AM_DT_BF16, N.AM_WF_INT4, 128,
                       cfg["max_tokens"], 8)
    m = N.vp()
    L.call("am_model_create_synthetic", rt.rt, C.byref(mc), seed, C.byref(m))
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1, B)), C.byref(s))
    prompts = [O.token_ids(seed, 20 + r, cfg["vocab"], 3 + 2 * r) for r in range(B)]
    orcs = [O.OracleModel(cfg, seed) for _ in range(B)]
    V = cfg["vocab"]
    got = np.zeros((B, V), np.float32)
    toks = []
    for r in range(B):
        first = N.i64()
        L.call("am_session_prefill_row", s, r, prompts[r].ctypes.data, prompts[r].size, C.byref(first))
        orcs[r].forward(prompts[r], 0)
        toks.append(int(first.value))
    posn = [pr.size for pr in prompts]
    for step in range(3):
        out = np.zeros((B, 1), np.int64)
        L.call("am_session_decode", s, 1, out.ctypes.data)
        L.call("am_session_logits", s, got.ctypes.data)
        for r in range(B):
            ref = orcs[r].forward(np.array([toks[r]], np.int64), posn[r])
            close(got[r], ref, TOL, f"decode step {step} seq {r}")
            assert int(out[r, 0]) == O.argmax(got[r])
            toks[r] = int(out[r, 0])
            posn[r] += 1
    for o in orcs:
        o.close()
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    rt.close()


def test_batched_session_needs_every_sequence_prefilled():
    cfg = dict(O.TINY, act="bf16", weight_format=N.AM_WF_INT4, ffn=1536, vocab=4096, num_layers=1, max_tokens=32)
    rt = _Rt()
    mc = N.ModelConfig(1, cfg["hidden"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"], cfg["ffn"],
                       cfg["vocab"], 1e-5, 10000.0, N.AM_DT_BF16, N.AM_WF_INT4, 128, 32, 8)
    m = N.vp()
    L.call("am_model_create_synthetic", rt.rt, C.byref(mc), 1, C.byref(m))
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1, 2)), C.byref(s))
    pr = O.token_ids(1, 0, cfg["vocab"], 4)
    first = N.i64()
    L.call("am_session_prefill_row", s, 0, pr.ctypes.data, pr.size, C.byref(first))
    out = np.zeros((2, 1), np.int64)
    with pytest.raises(N.NativeError) as e:
        L.call("am_session_decode", s, 1, out.ctypes.data)
    assert e.value.status == "FAILED_PRECONDITION"
    with pytest.raises(N.NativeError) as e:
        L.call("am_session_prefill_row", s, 2, pr.ctypes.data, pr.size, C.byref(first))
    assert e.value.status == "OUT_OF_RANGE"
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    rt.close()
