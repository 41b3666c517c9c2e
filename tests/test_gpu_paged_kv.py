"""Paged (block) KV cache: am_gfx950_kv_pages on the attention, KV-write and fused
q/k/v kernels, and sessions with kv_block_size > 0 (the Phase-2 direction of the
reference's KV design, kv_cache_design.md sections 6.7 and 10; aethermind_prd.md:437-444).

Oracle: the contiguous-cache path, itself checked against the CPU oracle in
test_gpu_kernels.py / test_gpu_batch.py / test_gpu_model.py.  A paged cache holds the
same rows scattered over blocks named by a scrambled block table, so every result here
must equal the contiguous one bit for bit: attention outputs (decode with and without
splits, prefill with a start offset, batched rows), the rows the KV writers store, and
a whole session's logits and tokens.  Unused blocks hold NaN, so a read through a
wrong table entry shows up.  The pool bookkeeping (exhaustion, reuse after a row is
prefilled again) is checked through a session with a small pool."""

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

L = N.lib()
NAN_BF16 = 0x7FC0


def rand_bits(rng, shape, scale=1.0):
    return O.bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


class Paged:
    """A contiguous cache [B][hkv][cap][d] scattered into a pool of blocks through a
    random block table (spare blocks hold NaN)."""

    def __init__(self, rng, cache, bs, spare=3):
        B, hkv, cap, d = cache.shape
        self.bs, self.per = bs, -(-cap // bs)
        self.nb = B * self.per + spare
        ids = rng.permutation(self.nb)[:B * self.per].astype(np.int32)
        self.table = ids.reshape(B, self.per)
        pool = np.full((self.nb, hkv, bs, d), NAN_BF16, np.uint16)
        for b in range(B):
            for j in range(self.per):
                rows = cache[b, :, j * bs:(j + 1) * bs, :]
                pool[self.table[b, j], :, :rows.shape[1], :] = rows
        self.pool = pool
        self.dtable = dev(self.table)
        self.pages = N.KvPages(p(self.dtable), bs, self.per, self.nb)

    def gather(self, pool_host, B, hkv, cap, d):
        """pool -> contiguous [B][hkv][cap][d]"""
        out = np.zeros((B, hkv, cap, d), np.uint16)
        for b in range(B):
            for j in range(self.per):
                n = min(self.bs, cap - j * self.bs)
                out[b, :, j * self.bs:j * self.bs + n, :] = pool_host[self.table[b, j], :, :n, :]
        return out


def attention(q, kc, vc, B, seq, hq, hkv, d, cap, start, pages=None):
    out = empty((B * seq, hq * d), torch.int16)
    wsb = L.am_gfx950_attention_workspace_bytes(B, seq, hq, hkv, d, cap, 0)
    ws = zeros((max(wsb, 256),), torch.uint8)
    sd = dev(np.asarray(start, np.int64))
    a = N.AttentionArgs(p(q), p(kc), p(vc), p(out), seq, hq, hkv, d, cap, 0, p(sd), B, hkv * cap * d, N.AM_DT_BF16, 0,
                        p(ws), wsb, C.pointer(pages) if pages is not None else None)
    L.call("am_gfx950_attention", C.byref(a), stream())
    torch.cuda.synchronize()
    return bits_host(out)


@pytest.mark.parametrize("bs", [32, 64, 256])
@pytest.mark.parametrize("ctx", [[1], [31], [33], [512], [777], [4097], [5, 300, 1000]])
def test_decode_attention_paged_equals_contiguous(bs, ctx):
    rng = np.random.default_rng(len(ctx) * 1000 + ctx[0] + bs)
    B, hq, hkv, d, cap = len(ctx), 32, 8, 128, 4160
    cache_k = rand_bits(rng, (B, hkv, cap, d))
    cache_v = rand_bits(rng, (B, hkv, cap, d))
    q = bf16_dev(rand_bits(rng, (B, hq * d)))
    start = [c - 1 for c in ctx]
    want = attention(q, bf16_dev(cache_k), bf16_dev(cache_v), B, 1, hq, hkv, d, cap, start)
    pk = Paged(rng, cache_k, bs)
    vpool = np.full_like(pk.pool, NAN_BF16)  # V in the same blocks as K
    for b in range(B):
        for j in range(pk.per):
            rows = cache_v[b, :, j * bs:(j + 1) * bs, :]
            vpool[pk.table[b, j], :, :rows.shape[1], :] = rows
    got = attention(q, bf16_dev(pk.pool), bf16_dev(vpool), B, 1, hq, hkv, d, cap, start, pk.pages)
    assert not np.isnan(O.bf16_to_f32(got)).any()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bs", [32, 128])
def test_prefill_attention_paged_equals_contiguous(bs):
    """chunked prefill: 37 query rows at positions [start, start + 37) of two sequences"""
    rng = np.random.default_rng(bs)
    B, S, hq, hkv, d, cap = 2, 37, 32, 8, 128, 400
    ck, cv = rand_bits(rng, (B, hkv, cap, d)), rand_bits(rng, (B, hkv, cap, d))
    q = bf16_dev(rand_bits(rng, (B * S, hq * d)))
    start = [0, 300]
    want = attention(q, bf16_dev(ck), bf16_dev(cv), B, S, hq, hkv, d, cap, start)
    pk = Paged(rng, ck, bs)
    vpool = np.full_like(pk.pool, NAN_BF16)
    for b in range(B):
        for j in range(pk.per):
            rows = cv[b, :, j * bs:(j + 1) * bs, :]
            vpool[pk.table[b, j], :, :rows.shape[1], :] = rows
    got = attention(q, bf16_dev(pk.pool), bf16_dev(vpool), B, S, hq, hkv, d, cap, start, pk.pages)
    assert np.array_equal(got, want)


def test_kv_update_paged_writes_the_mapped_rows_only():
    rng = np.random.default_rng(3)
    hkv, d, cap, bs, S, start = 8, 128, 300, 64, 70, 100
    cache = np.full((1, hkv, cap, d), 0x3F80, np.uint16)  # 1.0
    pg = Paged(rng, cache, bs)
    pool_k, pool_v = bf16_dev(pg.pool), bf16_dev(pg.pool)
    k, v = rand_bits(rng, (S, hkv * d)), rand_bits(rng, (S, hkv * d))
    kd, vd = bf16_dev(k), bf16_dev(v)  # held: a freed temporary's memory would be reused
    a = N.KvUpdateArgs(p(kd), p(vd), p(pool_k), p(pool_v), S, hkv, d, cap, start, None, N.AM_DT_BF16, None,
                       C.pointer(pg.pages))
    L.call("am_gfx950_kv_update", C.byref(a), stream())
    for pool, src in ((pool_k, k), (pool_v, v)):
        got = pg.gather(bits_host(pool).reshape(pg.pool.shape), 1, hkv, cap, d)[0]
        exp = cache[0].copy()
        exp[:, start:start + S, :] = src.reshape(S, hkv, d).transpose(1, 0, 2)
        assert np.array_equal(got, exp)
        # spare blocks untouched
        used = set(pg.table.reshape(-1).tolist())
        raw = bits_host(pool).reshape(pg.pool.shape)
        for blk in range(pg.nb):
            if blk not in used:
                assert (raw[blk] == NAN_BF16).all()


def test_kv_update_skips_unassigned_blocks():
    """A table entry outside [0, num_blocks) (an unassigned block, -1, or past the pool)
    is never written through: the rows of those positions are skipped, the pages'
    err_flag is set, and every block of the pool other than the mapped ones keeps its
    contents (the reader's clamp would have sent the rows to block 0 or the last
    block)."""
    rng = np.random.default_rng(4)
    hkv, d, cap, bs, S, start = 2, 64, 256, 32, 96, 32
    cache = np.full((1, hkv, cap, d), 0x3F80, np.uint16)
    pg = Paged(rng, cache, bs)
    pg.table[0, 2] = -1  # positions 64..95
    pg.table[0, 3] = pg.nb + 5  # positions 96..127
    pg.dtable = dev(pg.table)
    err = zeros((1,), torch.int32)
    pages = N.KvPages(p(pg.dtable), bs, pg.per, pg.nb, p(err))
    pool_k, pool_v = bf16_dev(pg.pool), bf16_dev(pg.pool)
    k, v = rand_bits(rng, (S, hkv * d)), rand_bits(rng, (S, hkv * d))
    kd, vd = bf16_dev(k), bf16_dev(v)
    a = N.KvUpdateArgs(p(kd), p(vd), p(pool_k), p(pool_v), S, hkv, d, cap, start, None, N.AM_DT_BF16, None,
                       C.pointer(pages))
    L.call("am_gfx950_kv_update", C.byref(a), stream())
    assert int(host(err)[0]) == 1
    for pool, src in ((pool_k, k), (pool_v, v)):
        raw = bits_host(pool).reshape(pg.pool.shape)
        want = pg.pool.copy()
        src3 = src.reshape(S, hkv, d)
        for pos in range(start, start + S):
            j = pos // bs
            if j in (2, 3):
                continue
            want[pg.table[0, j], :, pos % bs, :] = src3[pos - start]
        assert np.array_equal(raw, want)


@pytest.mark.parametrize("rows", [1, 3])
def test_fused_qkv_skips_unassigned_blocks(rows):
    """The fused q/k/v decode epilogue (batch-1 and batched kernels) writes no K/V row
    for a position whose block is unassigned: the pool is left as it was, the err flag
    is set, and q is still produced."""
    rng = np.random.default_rng(11 + rows)
    H, hq, hkv, d, cap, bs = 512, 8, 2, 64, 256, 32
    n = (hq + 2 * hkv) * d
    bits = O.synth_bf16(9, 0x21, n * H).reshape(n, H)
    dw, keep = pack_weight(O.bf16_to_f32(bits).copy(), N.AM_WF_INT4, 128, src_bf16_bits=bits)
    h = bf16_dev(rand_bits(rng, (rows, H)))
    nw = bf16_dev(rand_bits(rng, (H,)))
    pos = np.array([5, 130, 255][:rows], np.int64)
    ct, st = O.rope_tables(cap, d, 10000.0)
    pd, ctd, std_ = dev(pos), dev(ct), dev(st)
    pg = Paged(rng, np.zeros((rows, hkv, cap, d), np.uint16), bs)
    for r in range(rows):
        pg.table[r, pos[r] // bs] = -1
    pg.dtable = dev(pg.table)
    err = zeros((1,), torch.int32)
    pages = N.KvPages(p(pg.dtable), bs, pg.per, pg.nb, p(err))
    pk, pv = bf16_dev(pg.pool), bf16_dev(pg.pool)
    qo = zeros((rows, hq * d), torch.int16)
    a = N.FusedQkvArgs(p(h), p(nw), 1e-5, dw, p(ctd), p(std_), p(pd), p(qo), p(pk), p(pv), hq, hkv, d, cap,
                       N.AM_DT_BF16, rows, 0, C.pointer(pages))
    L.call("am_gfx950_fused_qkv", C.byref(a), stream())
    assert int(host(err)[0]) == 1
    for pool in (pk, pv):
        assert np.array_equal(bits_host(pool).reshape(pg.pool.shape), pg.pool)
    assert np.any(bits_host(qo) != 0)


@pytest.mark.parametrize("rows", [1, 3])
@pytest.mark.parametrize("fmt", [N.AM_WF_INT4, N.AM_WF_BF16])
def test_fused_qkv_paged_equals_contiguous(rows, fmt):
    rng = np.random.default_rng(rows + fmt)
    H, hq, hkv, d, cap, bs = 512, 8, 2, 64, 256, 32
    n = (hq + 2 * hkv) * d
    bits = O.synth_bf16(9, 0x21, n * H).reshape(n, H)
    dw, keep = pack_weight(O.bf16_to_f32(bits).copy(), fmt, 128, src_bf16_bits=bits)
    h = bf16_dev(rand_bits(rng, (rows, H)))
    nw = bf16_dev(rand_bits(rng, (H,)))
    pos = np.array([5, 130, 255][:rows], np.int64)
    ct, st = O.rope_tables(cap, d, 10000.0)
    pd, ctd, std_ = dev(pos), dev(ct), dev(st)

    def run(kc, vc, cbs, pages):
        qo = empty((rows, hq * d), torch.int16)
        a = N.FusedQkvArgs(p(h), p(nw), 1e-5, dw, p(ctd), p(std_), p(pd), p(qo), p(kc), p(vc), hq, hkv, d, cap,
                           N.AM_DT_BF16, rows, cbs, C.pointer(pages) if pages is not None else None)
        L.call("am_gfx950_fused_qkv", C.byref(a), stream())
        torch.cuda.synchronize()
        return bits_host(qo)

    cache = np.zeros((rows, hkv, cap, d), np.uint16)
    kc, vc = bf16_dev(cache), bf16_dev(cache)
    q_want = run(kc, vc, hkv * cap * d, None)
    pg = Paged(rng, cache, bs)
    pk, pv = bf16_dev(pg.pool), bf16_dev(pg.pool)
    q_got = run(pk, pv, 0, pg.pages)
    assert np.array_equal(q_got, q_want)
    for paged, contig in ((pk, kc), (pv, vc)):
        got = pg.gather(bits_host(paged).reshape(pg.pool.shape), rows, hkv, cap, d)
        assert np.array_equal(got, bits_host(contig).reshape(rows, hkv, cap, d))


# ---------------------------------------------------------------- sessions

CFG = dict(O.TINY, act="bf16", ffn=1536, vocab=4096, num_layers=2, max_tokens=160)


def _model(rt, fmt=N.AM_WF_INT4, seed=7):
    c = CFG
    mc = N.ModelConfig(c["num_layers"], c["hidden"], c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["ffn"],
                       c["vocab"], c["rms_eps"], c["rope_theta"], N.AM_DT_BF16, fmt, 128, c["max_tokens"], 16)
    m = N.vp()
    L.call("am_model_create_synthetic", rt, C.byref(mc), seed, C.byref(m))
    return m


def _run(m, opts, prompts, steps):
    s = N.vp()
    L.call("am_session_open", m, C.byref(opts), C.byref(s))
    B = L.am_session_batch(s)
    V = CFG["vocab"]
    lg = np.zeros((B, V), np.float32)
    firsts, logits = [], []
    for r, pr in enumerate(prompts):
        first = N.i64()
        L.call("am_session_prefill_row", s, r, pr.ctypes.data, pr.size, C.byref(first))
        firsts.append(int(first.value))
    L.call("am_session_logits", s, lg.ctypes.data)
    logits.append(lg.copy())
    out = np.zeros((B, steps), np.int64)
    for i in range(steps):
        one = np.zeros((B, 1), np.int64)
        L.call("am_session_decode", s, 1, one.ctypes.data)
        out[:, i] = one[:, 0]
        L.call("am_session_logits", s, lg.ctypes.data)
        logits.append(lg.copy())
    L.am_session_destroy(s)
    return firsts, out, logits


@pytest.mark.parametrize("batch,fused,graph", [(3, 1, 1), (3, 1, 0), (1, 1, 1), (1, 0, 1)])
def test_paged_session_equals_contiguous(batch, fused, graph):
    """prompts of 40 / 5 / 70 tokens, 40 decode steps (crossing block boundaries of
    every row): the paged session's first tokens, decode tokens and every step's logits
    are the contiguous session's, bit for bit"""
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    m = _model(rt)
    prompts = [O.token_ids(7, 20 + r, CFG["vocab"], n) for r, n in enumerate((40, 5, 70))][:batch]
    want = _run(m, N.SessionOptions(fused, graph, batch, 0, 0, 0), prompts, 40)
    got = _run(m, N.SessionOptions(fused, graph, batch, 0, 32, 0), prompts, 40)
    assert got[0] == want[0]
    assert np.array_equal(got[1], want[1])
    for i, (a, b) in enumerate(zip(got[2], want[2])):
        assert np.array_equal(a, b), f"logits differ after step {i}"
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)


def test_paged_pool_exhaustion_and_reuse():
    """two sequences sharing a 6-block pool of 32 positions (192 positions, less than
    2 x 160): growth past the pool is refused before any work is enqueued, and a row
    prefilled again with a shorter prompt returns its blocks"""
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    m = _model(rt)
    s = N.vp()
    L.call("am_session_open", m, C.byref(N.SessionOptions(1, 1, 2, 0, 32, 6)), C.byref(s))
    first = N.i64()
    p0 = O.token_ids(3, 1, CFG["vocab"], 100)  # 4 blocks
    p1 = O.token_ids(3, 2, CFG["vocab"], 30)   # 1 block
    L.call("am_session_prefill_row", s, 0, p0.ctypes.data, p0.size, C.byref(first))
    L.call("am_session_prefill_row", s, 1, p1.ctypes.data, p1.size, C.byref(first))
    out = np.zeros((2, 28), np.int64)
    L.call("am_session_decode", s, 28, out.ctypes.data)  # rows reach 128 (4 blocks) and 58 (2 blocks)
    assert (L.am_session_row_position(s, 0), L.am_session_row_position(s, 1)) == (128, 58)
    with pytest.raises(N.NativeError) as e:
        L.call("am_session_decode", s, 1, out.ctypes.data)  # row 0 needs a 5th block
    assert e.value.status == "RESOURCE_EXHAUSTED"
    assert (L.am_session_row_position(s, 0), L.am_session_row_position(s, 1)) == (128, 58)
    big = O.token_ids(3, 3, CFG["vocab"], 130)
    with pytest.raises(N.NativeError) as e:  # 5 blocks while row 1 holds 2
        L.call("am_session_prefill_row", s, 0, big.ctypes.data, big.size, C.byref(first))
    assert e.value.status == "RESOURCE_EXHAUSTED"
    short = O.token_ids(3, 4, CFG["vocab"], 20)
    L.call("am_session_prefill_row", s, 0, short.ctypes.data, short.size, C.byref(first))  # 1 block
    L.call("am_session_decode", s, 40, np.zeros((2, 40), np.int64).ctypes.data)  # 2 + 4 blocks
    assert (L.am_session_row_position(s, 0), L.am_session_row_position(s, 1)) == (60, 98)
    L.am_session_destroy(s)
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)


def test_paged_session_refuses_what_it_cannot_run():
    rt = N.vp()
    L.call("am_runtime_open", 0, C.byref(rt))
    m = _model(rt)
    s = N.vp()
    for opts, code in ((N.SessionOptions(1, 1, 1, 0, 48, 0), "INVALID_ARGUMENT"),
                       (N.SessionOptions(1, 1, 1, 0, 16, 0), "INVALID_ARGUMENT"),
                       (N.SessionOptions(1, 1, 1, 1, 32, 0), "UNIMPLEMENTED")):
        with pytest.raises(N.NativeError) as e:
            L.call("am_session_open", m, C.byref(opts), C.byref(s))
        assert e.value.status == code
    L.am_model_destroy(m)
    L.am_runtime_destroy(rt)
