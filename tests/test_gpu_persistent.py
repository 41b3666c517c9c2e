"""Parity of the persistent all-layers decode kernel (am_gfx950_decode_layers, one launch
runs the per-layer node sequence of model_graph_builder.cpp:133-290 for every layer of a
batch-1 decode token) against the CPU oracle and against the per-op fused decode plan
(am_gfx950_fused_qkv / am_gfx950_attention / am_gfx950_fused_linear_residual /
am_gfx950_fused_gate_up), through the C ABI:

* the kernel entry point itself on layer inputs built by the library (random KV cache
  prefix, position 37): output hidden vector and the KV rows it writes;
* a host-preset abort flag: the launch returns without touching h and the flag reads back;
* sessions (am_session_* with persistent_decode required) against the oracle fed the
  same tokens, for GQA groups of 4 and 8 and hidden 2048 / 4096, as a HIP graph and
  eagerly, and against the per-op plan at contexts that take several 64-position
  passes per attention split.

Tolerance: the bf16 bar of the build (2e-2 of the largest magnitude)."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402
from gpu_util import p, stream, zeros  # noqa: E402

L = N.lib()
TOL = 2e-2


def small(hkv, **kw):
    c = dict(num_layers=2, hidden=2048, num_q_heads=16, num_kv_heads=hkv, head_dim=128, ffn=5632, vocab=8192,
             rms_eps=1e-5, rope_theta=10000.0, act="bf16", weight_format=N.AM_WF_INT4, group_size=128, max_tokens=256,
             chunk=64)
    c.update(kw)
    return c


B8_2L = dict(num_layers=2, hidden=4096, num_q_heads=32, num_kv_heads=8, head_dim=128, ffn=14336, vocab=32000,
             rms_eps=1e-5, rope_theta=500000.0, act="bf16", weight_format=N.AM_WF_INT4, group_size=128,
             max_tokens=4096, chunk=1024)


class Runtime:
    def __init__(self):
        self.rt = N.vp()
        L.call("am_runtime_open", 0, C.byref(self.rt))
        self.models = []

    def model(self, cfg, seed):
        mc = N.ModelConfig(cfg["num_layers"], cfg["hidden"], cfg["num_q_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                           cfg["ffn"], cfg["vocab"], cfg["rms_eps"], cfg["rope_theta"], N.AM_DT_BF16,
                           cfg["weight_format"], cfg["group_size"], cfg["max_tokens"], cfg["chunk"])
        m = N.vp()
        L.call("am_model_create_synthetic", self.rt, C.byref(mc), seed, C.byref(m))
        self.models.append(m)
        return m

    def session(self, m, persistent, graph=1):
        s = N.vp()
        try:
            L.call("am_session_open", m, C.byref(N.SessionOptions(1, graph, 1, persistent)), C.byref(s))
        except N.NativeError as e:  # pragma: no cover - other CU counts
            if "256-CU" in str(e):
                pytest.skip("persistent decode needs a 256-CU device")
            raise
        return s

    def close(self):
        for m in self.models:
            L.am_model_destroy(m)
        L.am_runtime_destroy(self.rt)


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def logits(s, vocab):
    out = np.zeros(vocab, np.float32)
    L.call("am_session_logits", s, out.ctypes.data)
    return out


def prefill(s, prompt):
    first = N.i64()
    L.call("am_session_prefill", s, prompt.ctypes.data, prompt.size, C.byref(first))
    return int(first.value)


def decode1(s):
    out = np.zeros(1, np.int64)
    L.call("am_session_decode", s, 1, out.ctypes.data)
    return int(out[0])


# ---------------------------------------------------------------- entry point itself

def bf16_bits(x):
    return (torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16)).view(torch.int16)


def weight(m, layer, role):
    w = N.Weight()
    L.call("am_model_weight", m, layer, role, C.byref(w))
    return w


def buf(m, kind, layer=0):
    ptr, nb = N.vp(), N.i64()
    L.call("am_model_buffer", m, kind, layer, C.byref(ptr), C.byref(nb))
    return ptr.value


@pytest.mark.parametrize("hkv", [4, 2])
def test_entry_point_matches_per_op_kernels(hkv):
    """am_gfx950_decode_layers vs the per-op fused kernels on the same layer inputs:
    position 37 over a random bf16 KV prefix, two layers."""
    cfg = small(hkv, max_tokens=128)
    rt = Runtime()
    m = rt.model(cfg, 11)
    H, hq, d, F, cap, nl = cfg["hidden"], cfg["num_q_heads"], cfg["head_dim"], cfg["ffn"], cfg["max_tokens"], 2
    pos = 37
    rng = np.random.default_rng(5)
    h0 = bf16_bits(rng.standard_normal(H) * 0.5).cuda()
    kv_init = [bf16_bits(rng.standard_normal((hkv, cap, d)) * 0.8).cuda() for _ in range(2 * nl)]
    for t in kv_init:
        t.view(hkv, cap, d)[:, pos:, :] = 0
    cos, sin = buf(m, N.AM_BUF_ROPE_COS), buf(m, N.AM_BUF_ROPE_SIN)
    pos_dev = torch.tensor([pos], dtype=torch.int64, device="cuda")

    # per-op reference
    h_ref = h0.clone()
    kv_ref = [t.clone() for t in kv_init]
    q = zeros((hq * d,), torch.int16)
    att = zeros((hq * d,), torch.int16)
    act = zeros((F,), torch.int16)
    ws_b = L.am_gfx950_attention_workspace_bytes(1, 1, hq, hkv, d, cap, 0)
    aws = zeros((max(ws_b, 16),), torch.uint8)
    for li in range(nl):
        kc, vc = kv_ref[2 * li], kv_ref[2 * li + 1]
        qa = N.FusedQkvArgs(p(h_ref), buf(m, N.AM_BUF_IN_NORM, li), cfg["rms_eps"], weight(m, li, 0), cos, sin,
                            p(pos_dev), p(q), p(kc), p(vc), hq, hkv, d, cap, N.AM_DT_BF16, 1, 0)
        L.call("am_gfx950_fused_qkv", C.byref(qa), stream())
        aa = N.AttentionArgs(p(q), p(kc), p(vc), p(att), 1, hq, hkv, d, cap, pos, None, 1, 0, N.AM_DT_BF16, 0, p(aws),
                             ws_b)
        L.call("am_gfx950_attention", C.byref(aa), stream())
        L.call("am_gfx950_fused_linear_residual", C.byref(N.FusedLinearResidualArgs(p(att), weight(m, li, 1), p(h_ref),
                                                                                    N.AM_DT_BF16, 1)), stream())
        ga = N.FusedGateUpArgs(p(h_ref), buf(m, N.AM_BUF_POST_NORM, li), cfg["rms_eps"], weight(m, li, 2), p(act),
                               N.AM_DT_BF16, 1)
        L.call("am_gfx950_fused_gate_up", C.byref(ga), stream())
        L.call("am_gfx950_fused_linear_residual", C.byref(N.FusedLinearResidualArgs(p(act), weight(m, li, 3), p(h_ref),
                                                                                    N.AM_DT_BF16, 1)), stream())

    # persistent kernel
    h_p = h0.clone()
    kv_p = [t.clone() for t in kv_init]
    table = (N.DecodeLayer * nl)()
    for li in range(nl):
        table[li] = N.DecodeLayer(weight(m, li, 0), weight(m, li, 1), weight(m, li, 2), weight(m, li, 3),
                                  buf(m, N.AM_BUF_IN_NORM, li), buf(m, N.AM_BUF_POST_NORM, li), p(kv_p[2 * li]),
                                  p(kv_p[2 * li + 1]))
    table_dev = torch.frombuffer(bytearray(bytes(table)), dtype=torch.uint8).cuda()
    wsb = L.am_gfx950_decode_layers_workspace_bytes(H, hq, hkv, d, F)
    ws = zeros((wsb,), torch.uint8)
    args = N.DecodeLayersArgs(p(table_dev), nl, H, hq, hkv, d, F, cap, cfg["rms_eps"], cos, sin, p(pos_dev), p(h_p),
                              p(ws), wsb, N.AM_DT_BF16)
    try:
        L.call("am_gfx950_decode_layers_validate", C.byref(args), table)
    except N.NativeError as e:  # pragma: no cover
        if "256-CU" in str(e):
            pytest.skip("persistent decode needs a 256-CU device")
        raise
    L.call("am_gfx950_decode_layers", C.byref(args), stream())
    torch.cuda.synchronize()
    ab = N.i32()
    L.call("am_gfx950_decode_layers_aborted", p(ws), C.byref(ab))
    assert ab.value == 0

    hr = h_ref.view(torch.bfloat16).float().cpu().numpy()
    hp = h_p.view(torch.bfloat16).float().cpu().numpy()
    assert rel(hp, hr) < TOL, rel(hp, hr)
    for li in range(2 * nl):
        a = kv_p[li].view(torch.bfloat16).float().view(hkv, cap, d)
        b = kv_ref[li].view(torch.bfloat16).float().view(hkv, cap, d)
        assert torch.equal(a[:, :pos], b[:, :pos])  # the prefix is untouched
        assert torch.count_nonzero(a[:, pos + 1:]) == 0
        assert rel(a[:, pos].cpu().numpy(), b[:, pos].cpu().numpy()) < TOL

    # a second call on the same workspace (next epoch) at the next position
    pos_dev.fill_(pos + 1)
    h2 = h0.clone()
    args.h = p(h2)
    L.call("am_gfx950_decode_layers", C.byref(args), stream())
    torch.cuda.synchronize()
    L.call("am_gfx950_decode_layers_aborted", p(ws), C.byref(ab))
    assert ab.value == 0
    assert torch.count_nonzero(kv_p[0].view(hkv, cap, d)[:, pos + 1]) > 0

    # abort preset by the host: every block returns at once, h is left as it was
    ws[64:68] = torch.tensor([1, 0, 0, 0], dtype=torch.uint8, device="cuda")
    h3 = h0.clone()
    args.h = p(h3)
    L.call("am_gfx950_decode_layers", C.byref(args), stream())
    torch.cuda.synchronize()
    L.call("am_gfx950_decode_layers_aborted", p(ws), C.byref(ab))
    assert ab.value == 1
    assert torch.equal(h3, h0)
    rt.close()


def test_entry_point_rejects_unsupported_shapes():
    args = N.DecodeLayersArgs()
    args.dtype = N.AM_DT_BF16
    args.head_dim, args.hq, args.hkv, args.hidden, args.ffn = 64, 16, 4, 2048, 5632
    with pytest.raises(N.NativeError):
        L.call("am_gfx950_decode_layers_validate", C.byref(args), None)
    args.head_dim, args.hq, args.hkv, args.hidden = 128, 16, 16, 2048  # group of 1
    with pytest.raises(N.NativeError):
        L.call("am_gfx950_decode_layers_validate", C.byref(args), None)
    args.hkv, args.hidden = 4, 1024
    with pytest.raises(N.NativeError):
        L.call("am_gfx950_decode_layers_validate", C.byref(args), None)


# ---------------------------------------------------------------- sessions

@pytest.mark.parametrize("hkv,graph", [(4, 1), (2, 1), (4, 0)])
def test_session_logits_match_oracle(hkv, graph):
    """Persistent-decode session vs the oracle fed the same tokens: prefill 24, 6 steps."""
    cfg = small(hkv)
    rt = Runtime()
    m = rt.model(cfg, 7)
    s = rt.session(m, 1, graph)
    assert L.am_session_persistent_decode(s) == 1
    assert L.am_session_decode_plan_size(s) == 3
    prompt = O.token_ids(7, 0, cfg["vocab"], 24)
    tok = prefill(s, prompt)
    orc = O.OracleModel(cfg, 7)
    orc.forward(prompt, 0)
    pos = prompt.size
    for step in range(6):
        nxt = decode1(s)
        ref = orc.forward(np.array([tok], np.int64), pos)
        got = logits(s, cfg["vocab"])
        assert rel(got, ref) < TOL, (step, rel(got, ref))
        tok, pos = nxt, pos + 1
    L.am_session_destroy(s)
    rt.close()


def compare_with_per_op(cfg, seed, n_prompt, steps):
    """Two sessions on one model (persistent, per-op fused plan), the same prompt: the
    logits of every step agree; the tokens agree unless the per-op top-2 gap is within
    the tolerance (a genuine near-tie), after which the inputs differ and the check stops."""
    rt = Runtime()
    m = rt.model(cfg, seed)
    sp = rt.session(m, 1)
    sr = rt.session(m, -1)
    assert L.am_session_persistent_decode(sp) == 1 and L.am_session_persistent_decode(sr) == 0
    prompt = O.token_ids(seed, 1, cfg["vocab"], n_prompt)
    tp, tr = prefill(sp, prompt), prefill(sr, prompt)
    assert tp == tr
    for step in range(steps):
        tp, tr = decode1(sp), decode1(sr)
        a, b = logits(sp, cfg["vocab"]), logits(sr, cfg["vocab"])
        assert rel(a, b) < TOL, (step, rel(a, b))
        if tp != tr:
            top2 = np.sort(b)[-2:]
            assert top2[1] - top2[0] < TOL * np.max(np.abs(b)), (step, tp, tr)
            break
    L.am_session_destroy(sp)
    L.am_session_destroy(sr)
    rt.close()


@pytest.mark.parametrize("hkv", [4, 2])
def test_session_matches_per_op_plan(hkv):
    compare_with_per_op(small(hkv), 21, 40, 16)


def test_session_long_context_small():
    """ctx ~4400 with 4 kv heads: 64 splits of ~69 positions, two passes per split."""
    compare_with_per_op(small(4, max_tokens=4608, chunk=1024), 23, 4400, 3)


def test_session_8b_shape_two_layers_long_context():
    """hidden 4096, 32/8 heads, ffn 14336 (the 8B layer shape), ctx ~3000: 32 splits of
    ~94 positions per kv head."""
    compare_with_per_op(B8_2L, 25, 3000, 4)
