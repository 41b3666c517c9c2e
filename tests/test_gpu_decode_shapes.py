"""The kernels the 8B benchmark runs, at the benchmark's own shapes, against the CPU
oracle (BASELINE.json configs[1..4]: hidden 4096, 32/8 heads of 128, FFN 14336, vocab
128256).

Each decode GEMV entry point picks its kernel variant by shape (block of 4, 8 or 12
waves, one or two weight buffers, split-K rows), so the small-shape tests of
test_gpu_kernels.py do not reach the variants the benchmark runs.  Here every fused
decode entry point runs at its 8B shape for INT4 (group 128), INT8 (per channel) and
bf16 weights, the variant reached is read back (am_gfx950_last_launch) and asserted,
and the output is compared with the oracle ops on the same inputs:

  am_gfx950_fused_qkv            RMSNorm -> q|k|v 6144x4096 -> RoPE (theta 5e5, d 128)
                                 -> K/V rows at position 600 of a 4096-position cache
  am_gfx950_fused_linear_residual  o 4096x4096 and down 4096x14336, + residual
  am_gfx950_fused_gate_up        RMSNorm -> gate|up 28672x4096 -> SiLU-Mul
  am_gfx950_fused_lm_head        RMSNorm -> 128256x4096 fp32 logits -> argmax, token
                                 history, position and step update (twice in a row)
  am_gfx950_linear (MFMA GEMM)   prefill 512x28672x4096 and 512x4096x14336
  am_gfx950_attention (prefill)  a 2048-row chunk at position 6144 of a 32768 cache

Bars: bf16 outputs within 2e-2 of the largest reference magnitude (north-star
tolerance), checked per row / head; fp32 logits within 1e-3; the greedy token equals
the oracle's argmax unless the oracle's top two are within the logit tolerance.
Weights are N(0, 0.02) rounded to bf16 (numpy RNG: the synthetic-data SPEC stream is
pinned elsewhere and is slow on the CPU at these sizes), quantized on the device and by
the oracle from the same values (bit-exact, test_quantize_dequant_bitexact)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402
from gpu_util import bf16_dev, bits_host, dev, empty, host, p, pack_weight, stream, zeros  # noqa: E402

L = N.lib()
TOL = 2e-2
H, HQ, HKV, D, F, V = 4096, 32, 8, 128, 14336, 128256
THETA = 500000.0
FMTS = {"int4": N.AM_WF_INT4, "int8": N.AM_WF_INT8, "bf16": N.AM_WF_BF16}


def close(got, ref, tol, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    err = float(np.max(np.abs(got - ref))) / scale
    assert err <= tol, f"{what}: max rel err {err:.3e} > {tol}"


def rows_close(got, ref, tol, what):
    for r in range(ref.shape[0]):
        close(got[r], ref[r], tol, f"{what} row {r}")


def bf16_rne_bits(a):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bits_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def rbf(x):
    return O.round_bf16(np.asarray(x, np.float32))


def big_weight(n, k, fmt, seed):
    """bf16-valued N(0, 0.02) weight [n][k] repacked on the device; returns the oracle's
    dequantized fp32 copy, the device weight and the buffers that keep it alive."""
    rng = np.random.default_rng(seed)
    bits = bf16_rne_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    w = bits_f32(bits)
    dw, keep = pack_weight(w, fmt, 128, src_bf16_bits=bits)
    keep = keep[:2]  # the bf16 source is no longer needed on the device
    if fmt == N.AM_WF_INT8:
        w = O.dequant_int8(*O.quant_int8(w))
    elif fmt == N.AM_WF_INT4:
        pk, sc = O.quant_int4(w, 128)
        w = O.dequant_int4(pk, sc, k, 128)
    return w, dw, keep


def act_rows(seed, m, k, std=1.0):
    rng = np.random.default_rng(seed)
    return bits_f32(bf16_rne_bits(rng.standard_normal((m, k), dtype=np.float32) * np.float32(std)))


def rd(t):
    return O.bf16_to_f32(bits_host(t))


def launched():
    return N.last_launch().kernel.decode()


def gains(seed):
    rng = np.random.default_rng(seed)
    return rbf(1.0 + 0.25 * rng.standard_normal(H).astype(np.float32))


# ------------------------------------------------------------------ decode GEMVs
@pytest.mark.parametrize("fmt", sorted(FMTS))
def test_fused_gate_up_8b(fmt):
    wf = FMTS[fmt]
    w, dw, keep = big_weight(2 * F, H, wf, seed=101)
    h = act_rows(102, 1, H)
    nw = gains(103)
    hd, nwd = bf16_dev(bf16_rne_bits(h)), bf16_dev(bf16_rne_bits(nw))
    act = empty((1, F), torch.int16)
    L.call("am_gfx950_fused_gate_up", N.FusedGateUpArgs(p(hd), p(nwd), 1e-5, dw, p(act), N.AM_DT_BF16, 1), stream())
    k = launched()
    assert k.startswith("gemv<bf16,") and "gate_up,norm=1" in k and ",nw=8," in k, k  # one 8-wave block per CU
    xn = rbf(O.rmsnorm(h, nw, 1e-5))
    gu = rbf(O.linear(xn, w))
    ref = rbf(O.silu_mul(gu[:, :F], gu[:, F:]))
    got = rd(act)
    close(got, ref, TOL, f"gate/up {fmt} [{k}]")
    for seg in range(0, F, 2048):  # every slice of features, so no block's rows escape
        close(got[0, seg:seg + 2048], ref[0, seg:seg + 2048], 3 * TOL, f"gate/up {fmt} features {seg}+")


@pytest.mark.parametrize("fmt", sorted(FMTS))
def test_fused_qkv_rope_kv_8b(fmt):
    wf = FMTS[fmt]
    n = (HQ + 2 * HKV) * D
    w, dw, keep = big_weight(n, H, wf, seed=111)
    h = act_rows(112, 1, H)
    nw = gains(113)
    cap, pos = 4096, 600
    ct, st = O.rope_tables(cap, D, THETA)
    kc = zeros((HKV * cap * D,), torch.int16)
    vc = zeros((HKV * cap * D,), torch.int16)
    qo = empty((1, HQ * D), torch.int16)
    hd, nwd = bf16_dev(bf16_rne_bits(h)), bf16_dev(bf16_rne_bits(nw))
    pd, ctd, std_ = dev(np.array([pos], np.int64)), dev(ct), dev(st)
    a = N.FusedQkvArgs(p(hd), p(nwd), 1e-5, dw, p(ctd), p(std_), p(pd), p(qo), p(kc), p(vc), HQ, HKV, D, cap,
                       N.AM_DT_BF16, 1, 0)
    L.call("am_gfx950_fused_qkv", a, stream())
    k = launched()
    assert k.startswith("gemv<bf16,") and "qkv,norm=1" in k, k
    if wf == N.AM_WF_INT4:
        assert ",nw=4," in k and k.endswith("one=1>"), k  # one weight block per wave
    xn = rbf(O.rmsnorm(h, nw, 1e-5))
    y = rbf(O.linear(xn, w))
    Q, KV = HQ * D, HKV * D
    posv = np.array([pos], np.int64)
    qr = rbf(O.rope(y[:, :Q], HQ, D, posv, ct, st))
    kr = rbf(O.rope(y[:, Q:Q + KV], HKV, D, posv, ct, st))
    vr = y[:, Q + KV:]
    got_q = rd(qo)
    for hh in range(HQ):
        close(got_q[0, hh * D:(hh + 1) * D], qr[0, hh * D:(hh + 1) * D], TOL, f"q head {hh} {fmt} [{k}]")
    kh, vh = rd(kc).reshape(HKV, cap, D), rd(vc).reshape(HKV, cap, D)
    for g in range(HKV):
        close(kh[g, pos], kr[0, g * D:(g + 1) * D], TOL, f"k head {g} {fmt}")
        close(vh[g, pos], vr[0, g * D:(g + 1) * D], TOL, f"v head {g} {fmt}")
    kh[:, pos] = 0
    vh[:, pos] = 0
    assert not kh.any() and not vh.any(), "cache rows other than the position were written"


@pytest.mark.parametrize("fmt", sorted(FMTS))
@pytest.mark.parametrize("proj", ["o", "down"])
def test_fused_linear_residual_8b(fmt, proj):
    wf = FMTS[fmt]
    kdim = H if proj == "o" else F
    w, dw, keep = big_weight(H, kdim, wf, seed=121 + kdim)
    x = act_rows(122, 1, kdim)
    h = act_rows(123, 1, H)
    xd, hd = bf16_dev(bf16_rne_bits(x)), bf16_dev(bf16_rne_bits(h))
    L.call("am_gfx950_fused_linear_residual", N.FusedLinearResidualArgs(p(xd), dw, p(hd), N.AM_DT_BF16, 1), stream())
    k = launched()
    if proj == "down" and wf == N.AM_WF_INT4:
        assert k.startswith("gemv_ksplit<bf16,int4,residual>"), k  # split-K rows
    else:
        assert k.startswith("gemv<bf16,") and "residual,norm=0" in k, k
    wx = rbf(O.linear(x, w))
    ref = rbf(h + wx)
    got = rd(hd)
    close(got, ref, TOL, f"{proj} + residual {fmt} [{k}]")
    # every element within one bf16 step of each of the two roundings
    bad = np.abs(got - ref) > 2.0 ** -7 * (np.abs(ref) + np.abs(wx)) + 1e-6
    assert not bad.any(), (proj, fmt, np.flatnonzero(bad)[:8])


@pytest.mark.parametrize("fmt", sorted(FMTS))
def test_fused_lm_head_argmax_state_8b(fmt):
    wf = FMTS[fmt]
    w, dw, keep = big_weight(V, H, wf, seed=131)
    h = act_rows(132, 1, H)
    nw = gains(133)
    hd, nwd = bf16_dev(bf16_rne_bits(h)), bf16_dev(bf16_rne_bits(nw))
    logits = empty((V,), torch.float32)
    tok = zeros((1,), torch.int64)
    hist = zeros((8,), torch.int64)
    posd = dev(np.array([600], np.int64))
    step = dev(np.array([3], np.int64))
    ws = zeros((L.am_gfx950_lm_head_workspace_bytes(),), torch.uint8)
    a = N.FusedLmHeadArgs(p(hd), p(nwd), 1e-5, dw, p(logits), p(tok), p(hist), p(posd), p(step), N.AM_DT_BF16,
                          p(ws), ws.numel(), 1, 0)
    ref = O.linear(rbf(O.rmsnorm(h, nw, 1e-5)), w)[0]
    top = O.argmax(ref)
    for it in range(2):
        L.call("am_gfx950_fused_lm_head", a, stream())
        k = launched()
        assert k.startswith("gemv<bf16,") and "lm_head,norm=1" in k, k
        if wf == N.AM_WF_INT4:
            assert ",p=2,nw=12," in k, k  # two pairs per iteration, 12-wave per-CU blocks
        lg = host(logits)
        close(lg, ref, 1e-3, f"logits {fmt} [{k}]")
        t = int(host(tok)[0])
        assert t == O.argmax(lg), "token is not the argmax of the kernel's own logits"
        scale = float(np.max(np.abs(ref)))
        assert t == top or ref[top] - ref[t] <= 1e-3 * scale, (t, top)
        assert int(host(hist)[3 + it]) == t
        assert int(host(posd)[0]) == 601 + it and int(host(step)[0]) == 4 + it
    assert not host(ws)[:256].any(), "the argmax ticket must be left zero"


# ------------------------------------------------------------------ prefill GEMM
@pytest.mark.parametrize("fmt", sorted(FMTS))
@pytest.mark.parametrize("shape", ["gate_up", "down"])
def test_prefill_gemm_8b(fmt, shape):
    """The 512-token prefill GEMMs; the oracle computes a sample of 12 rows (spread
    over every 128-row tile) in full."""
    wf = FMTS[fmt]
    m = 512
    n, kdim = (2 * F, H) if shape == "gate_up" else (H, F)
    w, dw, keep = big_weight(n, kdim, wf, seed=141 + n)
    x = act_rows(142, m, kdim)
    xd = bf16_dev(bf16_rne_bits(x))
    out = empty((m, n), torch.int16)
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(out), N.AM_DT_BF16, None, 2), stream())
    k = launched()
    assert k.startswith({N.AM_WF_INT4: "gemm_i4", N.AM_WF_INT8: "gemm_i8", N.AM_WF_BF16: "gemm_bf16"}[wf] + "<store,"), k
    got = rd(out)
    rows = [0, 1, 127, 128, 200, 255, 256, 300, 383, 384, 450, 511]
    ref = O.linear(np.ascontiguousarray(x[rows]), w)
    for i, r in enumerate(rows):
        close(got[r], ref[i], TOL, f"gemm {shape} {fmt} row {r} [{k}]")
        for seg in range(0, n, 4096):
            close(got[r, seg:seg + 4096], ref[i, seg:seg + 4096], 3 * TOL, f"row {r} cols {seg}+")


# ------------------------------------------------------------------ prefill attention
def test_prefill_attention_prompt_512_two_key_groups():
    """BASELINE configs[1..3]'s 512-token prompt at the 8B shape: 16 positions per block
    (256 blocks), each block as two 4-wave key groups over alternate key tiles whose
    softmax states merge in LDS.  The oracle checks rows at both ends of a block, of a
    32-key tile and of the prompt, in all 32 heads: the first block (one key tile, so the
    second group has none) and the last (16 tiles, eight per group)."""
    cap, S = 4096, 512
    rng = np.random.default_rng(152)
    kv = [bits_f32(bf16_rne_bits(rng.standard_normal((HKV, S, D), dtype=np.float32))) for _ in range(2)]
    kc = zeros((HKV, cap, D), torch.int16)
    vc = zeros((HKV, cap, D), torch.int16)
    kc[:, :S] = dev(bf16_rne_bits(kv[0]).view(np.int16))
    vc[:, :S] = dev(bf16_rne_bits(kv[1]).view(np.int16))
    q = bits_f32(bf16_rne_bits(rng.standard_normal((S, HQ * D), dtype=np.float32)))
    qd = bf16_dev(bf16_rne_bits(q))
    out = empty((S, HQ * D), torch.int16)
    a = N.AttentionArgs(p(qd), p(kc), p(vc), p(out), S, HQ, HKV, D, cap, 0, None, 1, 0, N.AM_DT_BF16, 0, None, 0)
    L.call("am_gfx950_attention", a, stream())
    k = launched()
    assert k == "attention_prefill<d=128,g=4,qb=16,ks=2>", k
    got = rd(out)
    kf = np.zeros((HKV, cap, D), np.float32)
    vf = np.zeros((HKV, cap, D), np.float32)
    kf[:, :S] = kv[0]
    vf[:, :S] = kv[1]
    for s in (0, 1, 15, 16, 31, 32, 33, 255, 496, 510, 511):
        ref = O.attention(np.ascontiguousarray(q[s:s + 1]), kf, vf, 1, HQ, HKV, D, cap, s)
        for hh in range(HQ):
            close(got[s, hh * D:(hh + 1) * D], ref[0, hh * D:(hh + 1) * D], TOL, f"row {s} head {hh}")


def test_prefill_attention_chunk_2048_at_6144_cap_32768():
    """BASELINE configs[4]'s chunked prefill: the fourth 2048-token chunk (positions
    6144..8191) of a 32768-position cache attends to 6144 committed positions plus its
    own causal prefix.  The oracle checks 8 query rows x all 32 heads."""
    cap, start, S = 32768, 6144, 2048
    rng = np.random.default_rng(151)
    n_rows = start + S
    kv = [bits_f32(bf16_rne_bits(rng.standard_normal((HKV, n_rows, D), dtype=np.float32))) for _ in range(2)]
    kc = zeros((HKV, cap, D), torch.int16)
    vc = zeros((HKV, cap, D), torch.int16)
    kc[:, :n_rows] = dev(bf16_rne_bits(kv[0]).view(np.int16))
    vc[:, :n_rows] = dev(bf16_rne_bits(kv[1]).view(np.int16))
    q = bits_f32(bf16_rne_bits(rng.standard_normal((S, HQ * D), dtype=np.float32)))
    qd = bf16_dev(bf16_rne_bits(q))
    out = empty((S, HQ * D), torch.int16)
    nb = L.am_gfx950_attention_workspace_bytes(1, S, HQ, HKV, D, cap, 0)
    ws = zeros((max(nb, 1),), torch.uint8)
    a = N.AttentionArgs(p(qd), p(kc), p(vc), p(out), S, HQ, HKV, D, cap, start, None, 1, 0, N.AM_DT_BF16, 0,
                        p(ws), nb)
    L.call("am_gfx950_attention", a, stream())
    k = launched()
    assert k == "attention_prefill<d=128,g=4,qb=64>", k  # 64 positions per block at 2048 rows
    got = rd(out)
    kf = np.zeros((HKV, cap, D), np.float32)
    vf = np.zeros((HKV, cap, D), np.float32)
    kf[:, :n_rows] = kv[0]
    vf[:, :n_rows] = kv[1]
    for s in (0, 1, 31, 32, 777, 1024, 2046, 2047):
        ref = O.attention(np.ascontiguousarray(q[s:s + 1]), kf, vf, 1, HQ, HKV, D, cap, start + s)
        for hh in range(HQ):
            close(got[s, hh * D:(hh + 1) * D], ref[0, hh * D:(hh + 1) * D], TOL, f"row {s} head {hh}")
