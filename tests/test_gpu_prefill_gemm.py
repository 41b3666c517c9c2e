"""The prefill GEMM (gemm_i4.hip: INT4 g128, INT8 per-channel and bf16 weights on one
kernel template) and its fused epilogues, through the C ABI, against the CPU oracle: am_gfx950_linear (store, residual) and
am_gfx950_prefill_linear (q|k|v column split, gate|up SiLU-Mul) at the 8B prefill
shapes (512 rows; q|k|v 6144x4096, gate|up 28672x4096, down 4096x14336) and at ragged
shapes (rows and columns that are not tile multiples, a k of one group, groups of 256).
With a workspace, shapes whose tiles leave CUs idle split K; the split launches are
checked against the oracle and repeated to show that they are deterministic and leave
their tickets at zero.

Bar: bf16 outputs within 2e-2 of the largest reference magnitude per row (north-star
tolerance); the oracle computes a sample of rows in full, covering every 128-row tile.
The roundings are the reference op boundaries: each Linear output rounded to bf16,
the residual sum rounded again, SiLU-Mul from the rounded gate and up."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a GPU", allow_module_level=True)

import aethermind_amd.native as N  # noqa: E402
import oracle_lib as O  # noqa: E402
from gpu_util import bf16_dev, bits_host, empty, host, p, pack_weight, stream  # noqa: E402
from test_gpu_decode_shapes import act_rows, bf16_rne_bits, bits_f32, close, launched, rbf  # noqa: E402

L = N.lib()
TOL = 2e-2


FMTS = [N.AM_WF_INT4, N.AM_WF_INT8, N.AM_WF_BF16]
PRE = {N.AM_WF_INT4: "gemm_i4", N.AM_WF_INT8: "gemm_i8", N.AM_WF_BF16: "gemm_bf16"}


def weight(n, k, seed, group=128, fmt=N.AM_WF_INT4):
    """A device weight of format fmt repacked from seeded bf16 values, and the oracle's
    dequantized fp32 matrix of the same weight (the build SPEC's quantization)."""
    rng = np.random.default_rng(seed)
    bits = bf16_rne_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    w = bits_f32(bits)
    dw, keep = pack_weight(w, fmt, group, src_bf16_bits=bits)
    if fmt == N.AM_WF_INT4:
        pk, sc = O.quant_int4(w, group)
        w = O.dequant_int4(pk, sc, k, group)
    elif fmt == N.AM_WF_INT8:
        w = O.dequant_int8(*O.quant_int8(w))
    return w, dw, keep[:2]


def int4_weight(n, k, seed, group=128):
    return weight(n, k, seed, group, N.AM_WF_INT4)


def unit(fmt, group=128):
    """the split-K unit along k: the INT4 group, 128 for INT8 and bf16"""
    return group if fmt == N.AM_WF_INT4 else 128


def sample_rows(m):
    rows = sorted({0, 1, m - 1, m // 2, min(m - 1, 127), min(m - 1, 128), min(m - 1, 255), min(m - 1, 300)})
    return [r for r in rows if 0 <= r < m]


def rd(t):
    return O.bf16_to_f32(bits_host(t))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [512, 200, 17])
def test_split_qkv(m, fmt):
    n_q, n_kv, k = 4096, 1024, 4096
    w, dw, keep = weight(n_q + 2 * n_kv, k, seed=201, fmt=fmt)
    x = act_rows(202, m, k)
    xd = bf16_dev(bf16_rne_bits(x))
    outs = [empty((m, n), torch.int16) for n in (n_q, n_kv, n_kv)]
    a = N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_SPLIT, (N.vp * 3)(*[p(o) for o in outs]),
                            (N.i64 * 2)(n_q, n_q + n_kv))
    L.call("am_gfx950_prefill_linear", a, stream())
    assert launched().startswith(PRE[fmt] + "<split,"), launched()
    rows = sample_rows(m)
    ref = rbf(O.linear(np.ascontiguousarray(x[rows]), w))
    got = np.concatenate([rd(o) for o in outs], axis=1)
    for i, r in enumerate(rows):
        close(got[r], ref[i], TOL, f"q|k|v row {r} (m={m})")
        for c0, c1 in ((0, n_q), (n_q, n_q + n_kv), (n_q + n_kv, n_q + 2 * n_kv)):
            close(got[r, c0:c1], ref[i, c0:c1], TOL, f"row {r} cols {c0}:{c1}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [512, 77])
def test_silu_mul_gate_up(m, fmt):
    F, k = 14336, 4096
    w, dw, keep = weight(2 * F, k, seed=211, fmt=fmt)
    x = act_rows(212, m, k)
    xd = bf16_dev(bf16_rne_bits(x))
    out = empty((m, F), torch.int16)
    a = N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_SILU_MUL, (N.vp * 3)(p(out), None, None), (N.i64 * 2)(0, 0))
    L.call("am_gfx950_prefill_linear", a, stream())
    assert launched() == (PRE[fmt] + ("<silu_mul,bn=256,splits=1>" if m >= 256 else "<silu_mul,bn=128,splits=1>")), \
        launched()
    rows = sample_rows(m)
    gu = rbf(O.linear(np.ascontiguousarray(x[rows]), w))
    ref = rbf(O.silu_mul(gu[:, :F], gu[:, F:]))
    got = rd(out)
    for i, r in enumerate(rows):
        close(got[r], ref[i], TOL, f"silu row {r} (m={m})")
        for seg in range(0, F, 2048):
            close(got[r, seg:seg + 2048], ref[i, seg:seg + 2048], 3 * TOL, f"row {r} features {seg}+")


@pytest.mark.parametrize("shape", [(512, 4096, 14336, 128), (200, 4096, 4096, 128), (130, 260, 512, 256),
                                   (33, 130, 128, 128), (512, 16384, 512, 64)])
@pytest.mark.parametrize("fmt", FMTS)
def test_linear_store_and_residual(shape, fmt):
    m, n, k, group = shape
    w, dw, keep = weight(n, k, seed=221 + n, group=group, fmt=fmt)
    x = act_rows(222, m, k)
    res = act_rows(223, m, n)
    xd, rdv = bf16_dev(bf16_rne_bits(x)), bf16_dev(bf16_rne_bits(res))
    out = empty((m, n), torch.int16)
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(out), N.AM_DT_BF16, None, 2), stream())
    assert launched().startswith(PRE[fmt] + "<store,"), launched()
    rows = sample_rows(m)
    ref = O.linear(np.ascontiguousarray(x[rows]), w)
    got = rd(out)
    for i, r in enumerate(rows):
        close(got[r], rbf(ref[i]), TOL, f"store row {r} {shape}")
    # Linear then Add, in place on the residual (out aliases residual)
    L.call("am_gfx950_linear", N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(rdv), N.AM_DT_BF16, p(rdv), 2), stream())
    assert launched().startswith(PRE[fmt] + "<residual,"), launched()
    got = rd(rdv)
    for i, r in enumerate(rows):
        close(got[r], rbf(res[r] + rbf(ref[i])), TOL, f"residual row {r} {shape}")


def workspace(m, n, k, group):
    nbytes = L.am_gfx950_gemm_workspace_bytes(m, n, k, group)
    return nbytes, (torch.zeros(max(nbytes, 16), dtype=torch.uint8, device="cuda") if nbytes else None)


def splits_of(name):
    return int(name.split("splits=")[1].rstrip(">"))


def tickets_zero(ws, tiles):
    return not host(ws)[:4 * tiles].any()


# (m, n, k, group, expected splits for INT4 and INT8, for bf16): the 8B o and down
# shapes (the 128-wide INT4 and INT8 tiles fit two blocks per CU, the bf16 tile one, so
# their launches may hold twice the blocks), ragged tiles, a split count capped by the
# group count, per-element epilogue chunks (n % 8 != 0)
SPLIT_SHAPES = [(512, 4096, 4096, 128, 4, 2), (512, 4096, 14336, 128, 4, 2), (100, 520, 4096, 128, 4, 4),
                (33, 130, 2048, 128, 2, 2), (64, 1000, 8192, 256, 4, 4)]


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
@pytest.mark.parametrize("fmt", FMTS)
def test_split_k_residual(shape, fmt):
    m, n, k, group, want_q, want_bf16 = shape
    want = want_bf16 if fmt == N.AM_WF_BF16 else want_q
    w, dw, keep = weight(n, k, seed=241 + n, group=group, fmt=fmt)
    x = act_rows(242, m, k)
    res = act_rows(243, m, n)
    xd = bf16_dev(bf16_rne_bits(x))
    nbytes, ws = workspace(m, n, k, unit(fmt, group))
    assert nbytes > 0
    rows = sample_rows(m)
    ref = O.linear(np.ascontiguousarray(x[rows]), w)
    outs = []
    for rep in range(2):  # the second call runs on the tickets the first left behind
        rdv = bf16_dev(bf16_rne_bits(res))
        args = N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(rdv), N.AM_DT_BF16, p(rdv), 2)
        args.workspace, args.workspace_bytes = p(ws), nbytes
        L.call("am_gfx950_linear", args, stream())
        assert launched().startswith(PRE[fmt] + "<residual,") and splits_of(launched()) == want, launched()
        got = rd(rdv)
        for i, r in enumerate(rows):
            close(got[r], rbf(res[r] + rbf(ref[i])), TOL, f"split residual row {r} {shape} call {rep}")
        outs.append(bits_host(rdv))
    assert np.array_equal(outs[0], outs[1]), "split-K results differ between calls"
    assert tickets_zero(ws, -(-m // 128) * -(-n // 128)), "tickets not left at zero"
    # the store epilogue on the same workspace
    out = empty((m, n), torch.int16)
    args = N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(out), N.AM_DT_BF16, None, 2)
    args.workspace, args.workspace_bytes = p(ws), nbytes
    L.call("am_gfx950_linear", args, stream())
    assert launched().startswith(PRE[fmt] + "<store,") and splits_of(launched()) == want, launched()
    got = rd(out)
    for i, r in enumerate(rows):
        close(got[r], rbf(ref[i]), TOL, f"split store row {r} {shape}")


def test_split_k_qkv_and_silu_few_rows():
    m, k = 64, 4096
    n_q, n_kv = 4096, 1024
    w, dw, keep = int4_weight(n_q + 2 * n_kv, k, seed=251)
    x = act_rows(252, m, k)
    xd = bf16_dev(bf16_rne_bits(x))
    nbytes, ws = workspace(m, n_q + 2 * n_kv, k, 128)
    outs = [empty((m, n), torch.int16) for n in (n_q, n_kv, n_kv)]
    a = N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_SPLIT, (N.vp * 3)(*[p(o) for o in outs]),
                            (N.i64 * 2)(n_q, n_q + n_kv), p(ws), nbytes)
    L.call("am_gfx950_prefill_linear", a, stream())
    assert launched().startswith("gemm_i4<split,") and splits_of(launched()) > 1, launched()
    rows = sample_rows(m)
    ref = rbf(O.linear(np.ascontiguousarray(x[rows]), w))
    got = np.concatenate([rd(o) for o in outs], axis=1)
    for i, r in enumerate(rows):
        close(got[r], ref[i], TOL, f"split-K q|k|v row {r}")
    F = 2048
    w, dw, keep = int4_weight(2 * F, k, seed=253)
    nbytes, ws = workspace(m, 2 * F, k, 128)
    out = empty((m, F), torch.int16)
    a = N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_SILU_MUL, (N.vp * 3)(p(out), None, None), (N.i64 * 2)(0, 0),
                            p(ws), nbytes)
    L.call("am_gfx950_prefill_linear", a, stream())
    assert launched().startswith("gemm_i4<silu_mul,") and splits_of(launched()) > 1, launched()
    gu = rbf(O.linear(np.ascontiguousarray(x[rows]), w))
    ref = rbf(O.silu_mul(gu[:, :F], gu[:, F:]))
    got = rd(out)
    for i, r in enumerate(rows):
        close(got[r], ref[i], TOL, f"split-K silu row {r}")
    assert tickets_zero(ws, F // 64), "tickets not left at zero"


@pytest.mark.parametrize("fmt", FMTS)
def test_split_k_shapes_share_one_workspace(fmt):
    """A session's prefill runs q|k|v, o, gate|up and down on one workspace: a launch
    with few tiles leaves its partials where a launch with more tiles keeps tickets
    unless the ticket region is the same for every shape.  2048-wide layer at 24 rows:
    q|k|v 24 tiles, gate|up 88 tiles, down 16 tiles, all split."""
    m, H, F, nq, nkv = 24, 2048, 5632, 2048, 512
    shapes = [(nq + 2 * nkv, H), (2 * F, H), (H, F)]
    nbytes = max(L.am_gfx950_gemm_workspace_bytes(m, n, k, 128) for n, k in shapes)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    # the third value keeps the device tensors the weight structs point into alive
    wq, dq, kq = weight(nq + 2 * nkv, H, seed=271, fmt=fmt)
    wg, dg, kg = weight(2 * F, H, seed=272, fmt=fmt)
    wd, dd, kd = weight(H, F, seed=273, fmt=fmt)
    x = act_rows(274, m, H)
    xd = bf16_dev(bf16_rne_bits(x))
    rows = sample_rows(m)
    for rep in range(2):
        outs = [empty((m, n), torch.int16) for n in (nq, nkv, nkv)]
        a = N.PrefillLinearArgs(p(xd), m, dq, N.AM_PREFILL_SPLIT, (N.vp * 3)(*[p(o) for o in outs]),
                                (N.i64 * 2)(nq, nq + nkv), p(ws), nbytes)
        L.call("am_gfx950_prefill_linear", a, stream())
        assert launched().startswith(PRE[fmt] + "<split,") and splits_of(launched()) > 1, launched()
        got = np.concatenate([rd(o) for o in outs], axis=1)
        ref = rbf(O.linear(np.ascontiguousarray(x[rows]), wq))
        for i, r in enumerate(rows):
            close(got[r], ref[i], TOL, f"shared workspace q|k|v row {r} call {rep}")
        act = empty((m, F), torch.int16)
        a = N.PrefillLinearArgs(p(xd), m, dg, N.AM_PREFILL_SILU_MUL, (N.vp * 3)(p(act), None, None),
                                (N.i64 * 2)(0, 0), p(ws), nbytes)
        L.call("am_gfx950_prefill_linear", a, stream())
        assert launched().startswith(PRE[fmt] + "<silu_mul,") and splits_of(launched()) > 1, launched()
        gu = rbf(O.linear(np.ascontiguousarray(x[rows]), wg))
        ref = rbf(O.silu_mul(gu[:, :F], gu[:, F:]))
        got = rd(act)
        for i, r in enumerate(rows):
            close(got[r], ref[i], TOL, f"shared workspace silu row {r} call {rep}")
        a_host = rd(act)
        out = empty((m, H), torch.int16)
        args = N.LinearArgs(p(act), N.AM_DT_BF16, m, dd, p(out), N.AM_DT_BF16, None, 2)
        args.workspace, args.workspace_bytes = p(ws), nbytes
        L.call("am_gfx950_linear", args, stream())
        assert launched().startswith(PRE[fmt] + "<store,") and splits_of(launched()) > 1, launched()
        ref = rbf(O.linear(np.ascontiguousarray(a_host[rows]), wd))
        got = rd(out)
        for i, r in enumerate(rows):
            close(got[r], ref[i], TOL, f"shared workspace down row {r} call {rep}")
    assert tickets_zero(ws, 4096 // 4), "tickets not left at zero"
    del kq, kg, kd


def qkv_rope_run(m, start, hq=16, hkv=4, d=128, H=2048, cap=256, with_ws=True, seed=281, fmt=N.AM_WF_INT4):
    """One AM_PREFILL_QKV_ROPE_KV launch on fresh zeroed cache planes; returns the
    oracle inputs and the device outputs."""
    import ctypes as C
    n = (hq + 2 * hkv) * d
    w, dw, keep = weight(n, H, seed=seed, fmt=fmt)
    x = act_rows(seed + 1, m, H)
    xd = bf16_dev(bf16_rne_bits(x))
    ctab, stab = O.rope_tables(cap, d, 10000.0)
    cd, sd = torch.from_numpy(ctab).cuda(), torch.from_numpy(stab).cuda()
    kc = torch.zeros(hkv * cap * d, dtype=torch.int16, device="cuda")
    vc = torch.zeros(hkv * cap * d, dtype=torch.int16, device="cuda")
    q = empty((m, hq * d), torch.int16)
    startd = torch.tensor([start], dtype=torch.int64, device="cuda")
    errd = torch.zeros(1, dtype=torch.int32, device="cuda")
    nbytes, ws = workspace(m, n, H, 128) if with_ws else (0, None)
    r = N.PrefillRopeKv(p(cd), p(sd), cap, p(startd), p(kc), p(vc), hq, hkv, d, cap, None, p(errd))
    a = N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_QKV_ROPE_KV, (N.vp * 3)(p(q), None, None), (N.i64 * 2)(0, 0),
                            p(ws), nbytes, C.pointer(r))
    L.call("am_gfx950_prefill_linear", a, stream())
    name = launched()
    out = dict(q=rd(q), k=rd(kc).reshape(hkv, cap, d), v=rd(vc).reshape(hkv, cap, d), err=int(host(errd)[0]))
    del keep
    return x, w, ctab, stab, out, name


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m,start", [(200, 37), (24, 100), (1, 255)])
def test_qkv_rope_kv_epilogue(m, start, fmt):
    """q|k|v GEMM with RoPE and the KV cache write in the epilogue, against the
    oracle's Linear -> bf16 -> RoPE -> bf16 (q, k) and Linear -> bf16 (v) at positions
    start + i; cache rows outside [start, start + m) stay untouched.  24 rows split K."""
    hq, hkv, d, cap = 16, 4, 128, 256
    x, w, ctab, stab, out, name = qkv_rope_run(m, start, fmt=fmt)
    assert name.startswith(PRE[fmt] + "<qkv_rope_kv,"), name
    if m == 24:
        assert splits_of(name) > 1, name
    rows = sample_rows(m)
    lin = rbf(O.linear(np.ascontiguousarray(x[rows]), w))
    pos = start + np.asarray(rows, np.int64)
    qref = rbf(O.rope(lin[:, :hq * d], hq, d, pos, ctab, stab))
    kref = rbf(O.rope(lin[:, hq * d:(hq + hkv) * d], hkv, d, pos, ctab, stab))
    vref = lin[:, (hq + hkv) * d:]
    for i, r in enumerate(rows):
        close(out["q"][r], qref[i], TOL, f"q row {r}")
        close(out["k"][:, start + r, :].reshape(-1), kref[i], TOL, f"k row {r}")
        close(out["v"][:, start + r, :].reshape(-1), vref[i], TOL, f"v row {r}")
    for t in ("k", "v"):
        assert not out[t][:, :start].any() and not out[t][:, start + m:].any(), f"{t} rows outside the chunk written"
    assert out["err"] == 0


def test_qkv_rope_kv_rows_past_capacity():
    """Rows whose position reaches the capacity write no cache row and set the flag."""
    cap, m, start = 256, 24, 246
    x, w, ctab, stab, out, name = qkv_rope_run(m, start, with_ws=False)
    assert name.startswith("gemm_i4<qkv_rope_kv,") and splits_of(name) == 1, name
    assert out["err"] == 1
    assert out["k"][:, start:cap].any() and out["v"][:, start:cap].any()
    assert not out["k"][:, :start].any() and not out["v"][:, :start].any()


def test_qkv_rope_kv_bit_identical_to_separate_nodes_long_chunk():
    """The fused epilogue against the nodes it replaces, bit for bit, at the long-context
    chunk: 2048 rows at positions 6144..8191 of the 8B q|k|v shape (16 row tiles, two
    tile bands): split GEMM, then am_gfx950_rope, then am_gfx950_kv_update."""
    import ctypes as C
    m, start, cap, hq, hkv, d, H = 2048, 6144, 8192, 32, 8, 128, 4096
    n = (hq + 2 * hkv) * d
    w, dw, keep = int4_weight(n, H, seed=291)
    xd = bf16_dev(bf16_rne_bits(act_rows(292, m, H)))
    ctab, stab = O.rope_tables(cap, d, 500000.0)
    cd, sd = torch.from_numpy(ctab).cuda(), torch.from_numpy(stab).cuda()
    startd = torch.tensor([start], dtype=torch.int64, device="cuda")
    posd = torch.arange(start, start + m, dtype=torch.int64, device="cuda")
    planes = [torch.zeros(hkv * cap * d, dtype=torch.int16, device="cuda") for _ in range(4)]
    # fused
    qf = empty((m, hq * d), torch.int16)
    r = N.PrefillRopeKv(p(cd), p(sd), cap, p(startd), p(planes[0]), p(planes[1]), hq, hkv, d, cap, None, None)
    L.call("am_gfx950_prefill_linear", N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_QKV_ROPE_KV,
                                                            (N.vp * 3)(p(qf), None, None), (N.i64 * 2)(0, 0), None, 0,
                                                            C.pointer(r)), stream())
    assert launched().startswith("gemm_i4<qkv_rope_kv,"), launched()
    # the three nodes
    q, k, v = empty((m, hq * d), torch.int16), empty((m, hkv * d), torch.int16), empty((m, hkv * d), torch.int16)
    L.call("am_gfx950_prefill_linear", N.PrefillLinearArgs(p(xd), m, dw, N.AM_PREFILL_SPLIT,
                                                            (N.vp * 3)(p(q), p(k), p(v)),
                                                            (N.i64 * 2)(hq * d, (hq + hkv) * d)), stream())
    L.call("am_gfx950_rope", N.RopeArgs(p(q), p(k), p(q), p(k), p(posd), p(cd), p(sd), m, hq, hkv, d, cap,
                                        N.AM_DT_BF16), stream())
    L.call("am_gfx950_kv_update", N.KvUpdateArgs(p(k), p(v), p(planes[2]), p(planes[3]), m, hkv, d, cap, 0,
                                                 p(startd), N.AM_DT_BF16, None, None), stream())
    torch.cuda.synchronize()
    assert torch.equal(qf, q), int((qf != q).sum())
    assert torch.equal(planes[0], planes[2]) and torch.equal(planes[1], planes[3])
    del keep


def test_workspace_too_small_runs_unsplit():
    m, n, k = 512, 4096, 4096
    w, dw, keep = int4_weight(n, k, seed=261)
    x = act_rows(262, m, k)
    xd = bf16_dev(bf16_rne_bits(x))
    ws = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    out = empty((m, n), torch.int16)
    args = N.LinearArgs(p(xd), N.AM_DT_BF16, m, dw, p(out), N.AM_DT_BF16, None, 2)
    args.workspace, args.workspace_bytes = p(ws), 4096
    L.call("am_gfx950_linear", args, stream())
    assert launched() == "gemm_i4<store,bn=128,splits=1>", launched()
    rows = sample_rows(m)
    ref = O.linear(np.ascontiguousarray(x[rows]), w)
    got = rd(out)
    for i, r in enumerate(rows):
        close(got[r], rbf(ref[i]), TOL, f"row {r}")


def test_prefill_linear_rejects_other_formats():
    """fp32 weights have no MFMA prefill kernel: the fused entry point refuses them
    (the plan takes one node per Linear instead)."""
    rng = np.random.default_rng(3)
    dw, keep = pack_weight(rng.standard_normal((256, 512), dtype=np.float32), N.AM_WF_F32, 128)
    x = bf16_dev(bf16_rne_bits(act_rows(4, 64, 512)))
    out = empty((64, 128), torch.int16)
    a = N.PrefillLinearArgs(p(x), 64, dw, N.AM_PREFILL_SILU_MUL, (N.vp * 3)(p(out), None, None), (N.i64 * 2)(0, 0))
    with pytest.raises(N.NativeError) as e:
        L.call("am_gfx950_prefill_linear", a, stream())
    assert e.value.status == "UNIMPLEMENTED"
