"""Layer-by-layer parity: one decoder layer of a synthetic model executed node by node
(model_graph_builder.cpp:133-290 order) through the per-op C ABI on the model's own
repacked device weights, every intermediate compared with the CPU oracle op fed the
oracle's previous intermediate.  Localises a model-level mismatch to one node."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402
from gpu_util import bf16_dev, bits_host, dev, empty, host, p, stream, zeros  # noqa: E402

L = N.lib()


def rel(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("act,fmt,S", [("f32", N.AM_WF_F32, 5), ("bf16", N.AM_WF_BF16, 5), ("bf16", N.AM_WF_INT4, 12),
                                       ("bf16", N.AM_WF_INT8, 1)])
def test_layer0_node_by_node(act, fmt, S):
    cfg = dict(O.TINY, act=act, weight_format=fmt, ffn=1536, vocab=4096, num_layers=1, max_tokens=64)
    H, F, d, hq, hkv, cap = cfg["hidden"], cfg["ffn"], cfg["head_dim"], cfg["num_q_heads"], cfg["num_kv_heads"], 64
    Q, KV = hq * d, hkv * d
    bf = act == "bf16"
    dt = N.AM_DT_BF16 if bf else N.AM_DT_F32
    tdt = torch.int16 if bf else torch.float32
    tol = 2e-2 if bf else 1e-3
    seed = 3

    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    mc = N.ModelConfig(1, H, hq, hkv, d, F, cfg["vocab"], 1e-5, 10000.0, dt, fmt, 128, cap, 16)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), seed, C.byref(m))
    torch.cuda.synchronize()

    def weight(role):
        w = N.Weight()
        L.call("am_model_weight", m, 0, role, C.byref(w))
        return w

    def buf(kind):
        ptr, nb = N.vp(), N.i64()
        L.call("am_model_buffer", m, kind, 0, C.byref(ptr), C.byref(nb))
        return ptr.value

    def rd(t):  # device activation -> fp32 numpy
        return O.bf16_to_f32(bits_host(t)) if bf else host(t)

    def rnd(x):
        return O.round_bf16(x) if bf else np.asarray(x, np.float32)

    def oracle_w(tid, n, k):
        if fmt == N.AM_WF_F32:
            return O.synth_f32(seed, tid, n * k).reshape(n, k)
        w = O.bf16_to_f32(O.synth_bf16(seed, tid, n * k)).reshape(n, k).copy()
        if fmt == N.AM_WF_INT8:
            return O.dequant_int8(*O.quant_int8(w))
        if fmt == N.AM_WF_INT4:
            pk, sc = O.quant_int4(w, 128)
            return O.dequant_int4(pk, sc, k, 128)
        return w

    tid = lambda r: (1 << 8) | r  # noqa: E731  (layer 0, roles q=1..down=7)
    s = stream()
    ids = O.token_ids(seed, 0, cfg["vocab"], S)
    idd = dev(ids)
    pos = np.arange(S, dtype=np.int64)
    posd = dev(pos)

    # Embedding
    h = empty((S, H), tdt)
    L.call("am_gfx950_embedding", N.EmbeddingArgs(p(idd), N.AM_DT_I64, S, buf(N.AM_BUF_EMBED), dt, cfg["vocab"], H,
                                                  p(h), dt, None, 0), s)
    emb = (O.bf16_to_f32(O.synth_bf16(seed, 1, cfg["vocab"] * H)) if bf else O.synth_f32(seed, 1, cfg["vocab"] * H))
    h_ref = emb.reshape(-1, H)[ids]
    assert np.array_equal(rd(h), h_ref), "embedding"
    errs = {}

    # RmsNorm
    xn = empty((S, H), tdt)
    L.call("am_gfx950_rmsnorm", N.RmsNormArgs(p(h), buf(N.AM_BUF_IN_NORM), p(xn), S, H, H, H, 1e-5, dt, dt, dt), s)
    xn_ref = rnd(O.rmsnorm(h_ref, np.ones(H, np.float32), 1e-5))
    errs["rmsnorm"] = rel(rd(xn), xn_ref)

    def lin(x_dev, x_ref, role, n, tidv, k):
        out = empty((S, n), tdt)
        L.call("am_gfx950_linear", N.LinearArgs(p(x_dev), dt, S, weight(role), p(out), dt, None, 0), s)
        ref = rnd(O.linear(x_ref, oracle_w(tidv, n, k)))
        return out, ref

    q, q_ref = lin(xn, xn_ref, N.AM_ROLE_Q, Q, tid(1), H)
    errs["q"] = rel(rd(q), q_ref)
    k, k_ref = lin(xn, xn_ref, N.AM_ROLE_K, KV, tid(2), H)
    errs["k"] = rel(rd(k), k_ref)
    v, v_ref = lin(xn, xn_ref, N.AM_ROLE_V, KV, tid(3), H)
    errs["v"] = rel(rd(v), v_ref)

    # RoPE (in place)
    ct, st = O.rope_tables(cap, d, 10000.0)
    ra = N.RopeArgs(p(q), p(k), p(q), p(k), p(posd), buf(N.AM_BUF_ROPE_COS), buf(N.AM_BUF_ROPE_SIN), S, hq, hkv, d, cap,
                    dt)
    L.call("am_gfx950_rope", ra, s)
    q_ref = rnd(O.rope(q_ref, hq, d, pos, ct, st))
    k_ref = rnd(O.rope(k_ref, hkv, d, pos, ct, st))
    errs["rope_q"] = rel(rd(q), q_ref)
    errs["rope_k"] = rel(rd(k), k_ref)

    # KVCacheUpdate + Attention
    kc = zeros((hkv, cap, d), tdt)
    vc = zeros((hkv, cap, d), tdt)
    L.call("am_gfx950_kv_update", N.KvUpdateArgs(p(k), p(v), p(kc), p(vc), S, hkv, d, cap, 0, None, dt, None), s)
    kc_ref = np.zeros((hkv, cap, d), np.float32)
    vc_ref = np.zeros((hkv, cap, d), np.float32)
    kk, vv = rd(k), rd(v)
    for srow in range(S):
        for g in range(hkv):
            kc_ref[g, srow] = kk[srow, g * d:(g + 1) * d]
            vc_ref[g, srow] = vv[srow, g * d:(g + 1) * d]
    assert np.array_equal(rd(kc), kc_ref), "kv_update"
    attn = empty((S, Q), tdt)
    wsb = L.am_gfx950_attention_workspace_bytes(1, S, hq, hkv, d, cap, 0)
    ws = zeros((wsb,), torch.uint8)
    L.call("am_gfx950_attention", N.AttentionArgs(p(q), p(kc), p(vc), p(attn), S, hq, hkv, d, cap, 0, None, 1, 0, dt,
                                                  0, p(ws), wsb), s)
    attn_ref = rnd(O.attention(rd(q), kc_ref, vc_ref, S, hq, hkv, d, cap, 0))
    errs["attention"] = rel(rd(attn), attn_ref)

    o, o_ref = lin(attn, attn_ref, N.AM_ROLE_O, H, tid(4), Q)
    errs["o"] = rel(rd(o), o_ref)
    h2 = empty((S, H), tdt)
    L.call("am_gfx950_add", N.AddArgs(p(h), p(o), p(h2), S * H, dt), s)
    h2_ref = rnd(h_ref + o_ref)
    errs["add"] = rel(rd(h2), h2_ref)

    L.call("am_gfx950_rmsnorm", N.RmsNormArgs(p(h2), buf(N.AM_BUF_POST_NORM), p(xn), S, H, H, H, 1e-5, dt, dt, dt), s)
    xn2_ref = rnd(O.rmsnorm(h2_ref, np.ones(H, np.float32), 1e-5))
    errs["rmsnorm2"] = rel(rd(xn), xn2_ref)
    g_, g_ref = lin(xn, xn2_ref, N.AM_ROLE_GATE, F, tid(5), H)
    errs["gate"] = rel(rd(g_), g_ref)
    u_, u_ref = lin(xn, xn2_ref, N.AM_ROLE_UP, F, tid(6), H)
    errs["up"] = rel(rd(u_), u_ref)
    a_ = empty((S, F), tdt)
    L.call("am_gfx950_silu_mul", N.SiluMulArgs(p(g_), p(u_), p(a_), S * F, dt), s)
    a_ref = rnd(O.silu_mul(g_ref, u_ref))
    errs["silu_mul"] = rel(rd(a_), a_ref)
    dn, dn_ref = lin(a_, a_ref, N.AM_ROLE_DOWN, H, tid(7), F)
    errs["down"] = rel(rd(dn), dn_ref)

    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)
    print(act, fmt, S, {k_: f"{v_:.2e}" for k_, v_ in errs.items()})
    bad = {k_: v_ for k_, v_ in errs.items() if not v_ <= tol}
    assert not bad, f"nodes over {tol}: {bad}"
