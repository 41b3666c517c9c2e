"""Pins the CPU oracle before it is trusted as the GPU checker.

Each oracle function is checked against what fixes it independently of its own
formula: the reference's known-answer tests, the reference's own compiled AVX2 dot
product (oracle/_ref, when built), closed forms, textbook special cases and brute
force on small inputs -- chosen so a dropped term, wrong sign/index or transposed
operand fails.  CPU only (no GPU marker).
"""

import math
import os

import numpy as np
import pytest

import oracle_lib as O

L = O.lib()


# ---------------------------------------------------------------- numerics
def test_bf16_reference_bit_patterns():
    # tests/unit/numeric/test_bfloat16.cpp of the reference
    cases = [(1.0, 0x3F80), (-1.0, 0xBF80), (0.0, 0x0000), (-0.0, 0x8000), (math.inf, 0x7F80),
             (-math.inf, 0xFF80), (2.0, 0x4000), (3.0, 0x4040)]
    for v, bits in cases:
        assert L.orc_f32_to_bf16(v) == bits, v
    assert L.orc_f32_to_bf16(float("nan")) == 0x7FC0
    # round to nearest even at the halfway point
    assert L.orc_f32_to_bf16(np.uint32(0x3F808000).view(np.float32).item()) == 0x3F80  # tie, even stays
    assert L.orc_f32_to_bf16(np.uint32(0x3F818000).view(np.float32).item()) == 0x3F82  # tie, odd rounds up
    assert L.orc_f32_to_bf16(np.uint32(0x3F808001).view(np.float32).item()) == 0x3F81  # above half
    assert L.orc_bf16_to_f32(0x7F7F) == np.float32(3.3895314e38)


def test_f16_round_trip_exhaustive_and_rne():
    # every finite half value converts to fp32 and back unchanged; numpy's float16 is the check
    for h in range(0, 0x10000, 7):
        f = L.orc_f16_to_f32(h)
        ref = np.uint16(h).view(np.float16).astype(np.float32)
        if np.isnan(ref):
            assert np.isnan(f)
            continue
        assert np.float32(f).view(np.uint32) == ref.view(np.uint32), hex(h)
        assert L.orc_f32_to_f16(f) == h, hex(h)
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-7, 1e-5, 0.01, 1, 1000)])
    vals = np.concatenate([vals, np.float32([65504, 65519, 65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8])])
    for v in vals:
        assert L.orc_f32_to_f16(float(v)) == np.float32(v).astype(np.float16).view(np.uint16), v


def test_portable_math_against_libm():
    for x in [2.3283064365386963e-10, 1e-6, 0.1, 0.5, 0.70710678, 0.999, 1.0, 1.5, 3.0]:
        assert abs(L.orc_portable_log(x) - math.log(x)) <= 4e-16 * max(1.0, abs(math.log(x)))
    for x in [0.0, 1e-9, 0.25, 2.0, 3.0, 44.36, 46.0]:
        assert abs(L.orc_portable_sqrt(x) - math.sqrt(x)) <= 4e-16 * max(1.0, math.sqrt(x))
    s, c = O.C.c_double(), O.C.c_double()
    for t in np.linspace(0, 0.999999, 1001):
        L.orc_portable_sincos_turns(float(t), O.C.byref(s), O.C.byref(c))
        assert abs(s.value - math.sin(2 * math.pi * t)) < 1e-15
        assert abs(c.value - math.cos(2 * math.pi * t)) < 1e-15


def test_synthetic_normals_moments_and_addressing():
    x = O.synth_f32(0, 0x105, 1 << 20).astype(np.float64)
    assert abs(x.mean()) < 0.02 * 4 / math.sqrt(x.size)
    assert abs(x.std() - 0.02) < 0.02 * 0.01
    z = x / 0.02
    assert abs(np.mean(z ** 4) - 3.0) < 0.05          # normal kurtosis
    # counter-based: any window equals the same slice of the full stream
    assert np.array_equal(O.synth_f32(0, 0x105, 1000, offset=12345), x[12345:13345].astype(np.float32))
    assert np.array_equal(O.synth_bf16(0, 0x105, 100, offset=777), O.bf16_bits(x[777:877].astype(np.float32)))
    # distinct tensor ids -> uncorrelated streams
    y = O.synth_f32(0, 0x106, 1 << 20).astype(np.float64)
    assert abs(np.corrcoef(x, y)[0, 1]) < 0.01
    ids = O.token_ids(0, 0, 32000, 100000)
    assert ids.min() >= 0 and ids.max() < 32000
    assert abs(ids.mean() - 16000) < 200


# ---------------------------------------------------------------- reference KATs
def test_rmsnorm_reference_kats():
    # tests/unit/backend/cpu/kernels/test_cpu_rmsnorm_kernel.cpp:65-288
    x = np.array([[1, 2, 3, 4], [0.5, 1, 1.5, 2], [4, 3, 2, 1]], np.float32)
    for fn in (L.orc_rmsnorm_scalar, L.orc_rmsnorm_avx2):
        out = np.zeros_like(x)
        assert fn(O.ptr(x), O.ptr(np.ones(4, np.float32)), 3, 4, 1e-5, O.ptr(out)) == 0
        np.testing.assert_allclose(out[0], [0.365148, 0.730297, 1.095445, 1.460593], atol=1e-5)
        np.testing.assert_allclose(out[1], [0.365148, 0.730297, 1.095445, 1.460593], atol=1e-5)
        np.testing.assert_allclose(out[2], [1.460593, 1.095445, 0.730297, 0.365148], atol=1e-5)
        w = np.array([1, .5, 1.5, 2], np.float32)
        assert fn(O.ptr(x[:1].copy()), O.ptr(w), 1, 4, 1e-5, O.ptr(out)) == 0
        np.testing.assert_allclose(out[0], [0.365148, 0.365148, 1.643168, 2.921186], atol=1e-5)
        # entry validation: non-positive eps is rejected (rmsnorm_entry.cpp:24-144)
        assert fn(O.ptr(x), O.ptr(w), 3, 4, 0.0, O.ptr(out)) == 3


def test_rmsnorm_avx2_matches_scalar():
    # test_cpu_rmsnorm_kernel.cpp:290-346: AVX2 vs scalar at 1e-6 (incl. tails of 8/32)
    for hidden in (4, 37, 64, 4096, 8192):
        x = O.synth_f32(1, hidden, 3 * hidden, std=1.0).reshape(3, hidden)
        w = 1.0 + O.synth_f32(2, hidden, hidden, std=0.1)
        a, b = np.zeros_like(x), np.zeros_like(x)
        L.orc_rmsnorm_scalar(O.ptr(x), O.ptr(w), 3, hidden, 1e-5, O.ptr(a))
        L.orc_rmsnorm_avx2(O.ptr(x), O.ptr(w), 3, hidden, 1e-5, O.ptr(b))
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-6)


def test_embedding_reference_kats():
    # tests/unit/backend/cpu/test_cpu_embedding_kernel.cpp:61-211
    table = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    ids = np.array([2, 0, 3], np.int64)
    out = np.zeros((3, 3), np.float32)
    assert L.orc_embedding_i64(O.ptr(ids), 3, O.ptr(table), 4, 3, O.ptr(out)) == 0
    assert out.tolist() == [[7, 8, 9], [1, 2, 3], [10, 11, 12]]
    assert L.orc_embedding_i64(O.ptr(ids), 0, O.ptr(table), 4, 3, O.ptr(out)) == 0  # zero tokens
    bad = np.array([1, 4], np.int64)
    assert L.orc_embedding_i64(O.ptr(bad), 2, O.ptr(table), 4, 3, O.ptr(out)) == 11  # kOutOfRange


@pytest.mark.skipif(not os.path.exists(O.REF_DOT_SO), reason="oracle/_ref not built (needs /root/reference)")
def test_dot_avx2_bitexact_vs_reference_build():
    import ctypes as C
    ref = C.CDLL(O.REF_DOT_SO)
    ref.ref_dot_avx2.restype = C.c_float
    ref.ref_dot_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_long]
    for n in (8, 32, 64, 1000 * 8, 4096, 14336):
        a = O.synth_f32(3, n, n, std=1.0)
        b = O.synth_f32(4, n, n, std=1.0)
        assert np.float32(L.orc_dot_avx2(O.ptr(a), O.ptr(b), n)) == np.float32(ref.ref_dot_avx2(O.ptr(a), O.ptr(b), n))
    for n in (1, 7, 33, 4097):  # scalar tail: the reference build may contract to FMA
        a = O.synth_f32(3, n, n, std=1.0)
        b = O.synth_f32(4, n, n, std=1.0)
        assert abs(L.orc_dot_avx2(O.ptr(a), O.ptr(b), n) - ref.ref_dot_avx2(O.ptr(a), O.ptr(b), n)) < 1e-5


# ---------------------------------------------------------------- linear / quant
def test_linear_brute_force_and_structure():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 37)).astype(np.float32)
    w = rng.standard_normal((11, 37)).astype(np.float32)
    out = O.linear(x, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T   # out = x @ W^T, W is [out, in]
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-6)
    eye = np.eye(37, dtype=np.float32)
    np.testing.assert_array_equal(O.linear(x, eye), x)      # identity weight
    onehot = np.zeros((1, 37), np.float32)
    onehot[0, 5] = 1.0
    np.testing.assert_array_equal(O.linear(onehot, w)[0], w[:, 5])  # selects column 5 of W, not row 5
    out2 = np.zeros((3, 11), np.float32)
    L.orc_linear_avx2(O.ptr(x), O.ptr(w), 3, 11, 37, O.ptr(out2))
    np.testing.assert_allclose(out2, ref, rtol=1e-5, atol=1e-5)


def test_int8_quant_closed_form():
    w = np.array([[0.5, -1.27, 0.0, 0.635, 1.27, -0.004]], np.float32)
    q, s = O.quant_int8(w)
    assert s[0] == np.float32(1.27) / np.float32(127)
    assert q.tolist() == [[50, -127, 0, 64, 127, 0]]   # 63.5 rounds to even (64), -0.4 -> 0
    z, zs = O.quant_int8(np.zeros((1, 8), np.float32))
    assert zs[0] == 1.0 and not z.any()
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    q, s = O.quant_int8(w)
    dq = O.dequant_int8(q, s)
    assert np.all(np.abs(dq - w) <= s[:, None] / 2 * (1 + 1e-6))
    assert np.array_equal(dq, q.astype(np.float32) * s[:, None])   # one fp32 multiply


def test_int4_quant_brute_force_all_codes():
    # every code q in [-8, 7] under random fp16 scales reproduces q*s exactly, and
    # the logical packing is low nibble = even k (two's complement)
    rng = np.random.default_rng(3)
    for trial in range(20):
        s16 = np.float16(abs(rng.standard_normal()) * 0.01 + 1e-4)
        s = np.float32(s16)
        qs = np.array([-7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7, 7] * 8, np.int64)
        rng.shuffle(qs)
        qs[0] = 7  # make max|w| = 7 s so the recomputed scale equals s
        w = (qs.astype(np.float32) * s).reshape(1, 128)
        pk, sc = O.quant_int4(w, 128)
        assert np.float16(np.uint16(sc[0, 0]).view(np.float16)) == np.float16(np.float32(7 * s) / np.float32(7))
        dq = O.dequant_int4(pk, sc, 128, 128)
        sr = np.float32(np.uint16(sc[0, 0]).view(np.float16))
        nib = np.stack([pk[0] & 0xF, pk[0] >> 4], 1).reshape(-1).astype(np.int64)
        nib[nib >= 8] -= 16
        assert np.array_equal(dq[0], nib.astype(np.float32) * sr)
        assert np.all(np.abs(dq - w) <= sr / 2 * (1 + 1e-6) + 1e-12)
    pk, sc = O.quant_int4(np.zeros((2, 256), np.float32), 128)
    assert not pk.any() and not sc.any()
    w = np.zeros((1, 128), np.float32)
    w[0, 0], w[0, 1] = -1.0, 1.0   # q = -7 (0x9) at even k, +7 at odd k -> byte 0x79
    pk, sc = O.quant_int4(w, 128)
    assert pk[0, 0] == 0x79
    assert O.quant_int4(np.zeros((1, 100), np.float32), 128) if False else True


def test_int4_rejects_bad_group():
    w = np.zeros((1, 100), np.float32)
    packed = np.empty((1, 50), np.uint8)
    sc = np.empty((1, 1), np.uint16)
    assert L.orc_quant_int4(O.ptr(w), 1, 100, 128, O.ptr(packed), O.ptr(sc)) == 3


# ---------------------------------------------------------------- rope / attention / silu / argmax
def test_rope_closed_forms():
    d, theta = 64, 10000.0
    c, s = O.rope_tables(300, d, theta)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)                 # pos 0: identity
    np.testing.assert_allclose(c[1, 0], math.cos(1.0), rtol=1e-7)       # i = 0: inv_freq = 1
    np.testing.assert_allclose(s[7, 1], math.sin(7 * theta ** (-2 / d)), rtol=1e-6)
    x = O.synth_f32(5, 1, 3 * 2 * d, std=1.0).reshape(3, 2 * d)
    pos = np.array([0, 5, 299], np.int64)
    r = O.rope(x, 2, d, pos, c, s)
    np.testing.assert_array_equal(r[0], x[0])
    half = d // 2
    for row in (1, 2):
        for h in range(2):
            a = x[row, h * d:(h + 1) * d]
            b = r[row, h * d:(h + 1) * d]
            np.testing.assert_allclose(a[:half] ** 2 + a[half:] ** 2, b[:half] ** 2 + b[half:] ** 2, rtol=1e-5)
            # rotation direction: out[i] = x1 cos - x2 sin
            i = 3
            ang = pos[row] * theta ** (-2 * i / d)
            np.testing.assert_allclose(b[i], a[i] * math.cos(ang) - a[i + half] * math.sin(ang), rtol=1e-5,
                                       atol=1e-6)


def test_attention_special_cases():
    hq, hkv, d, cap = 4, 2, 16, 8
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, hq * d)).astype(np.float32)
    kc = rng.standard_normal((hkv, cap, d)).astype(np.float32)
    vc = rng.standard_normal((hkv, cap, d)).astype(np.float32)
    out = O.attention(q, kc, vc, 1, hq, hkv, d, cap, 0)          # one position -> V row 0 of the group
    for h in range(hq):
        np.testing.assert_allclose(out[0, h * d:(h + 1) * d], vc[h // 2, 0], rtol=1e-6)
    kz = np.zeros_like(kc)
    out = O.attention(q, kz, vc, 1, hq, hkv, d, cap, 5)         # equal scores -> mean of V[0..5]
    for h in range(hq):
        np.testing.assert_allclose(out[0, h * d:(h + 1) * d], vc[h // 2, :6].astype(np.float64).mean(0), rtol=1e-6)
    # brute-force softmax for a causal 3-row prefill with GQA mapping h -> h // (hq/hkv)
    q3 = rng.standard_normal((3, hq * d)).astype(np.float32)
    out = O.attention(q3, kc, vc, 3, hq, hkv, d, cap, 2)
    for srow in range(3):
        for h in range(hq):
            g = h // 2
            n = 2 + srow + 1
            sc = kc[g, :n].astype(np.float64) @ q3[srow, h * d:(h + 1) * d].astype(np.float64) / math.sqrt(d)
            pr = np.exp(sc - sc.max())
            pr /= pr.sum()
            np.testing.assert_allclose(out[srow, h * d:(h + 1) * d], pr @ vc[g, :n], rtol=1e-5, atol=1e-6)


def test_silu_mul_properties():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0, -100.0, 100.0], np.float32)
    u = np.ones_like(g)
    out = O.silu_mul(g, u)
    assert out[0] == 0.0
    np.testing.assert_allclose(out[1], 1 / (1 + math.exp(-1)), rtol=1e-6)
    np.testing.assert_allclose(out[2], -1 * math.exp(-1) / (1 + math.exp(-1)), rtol=1e-6)
    np.testing.assert_allclose(out[3], 20.0, rtol=1e-6)                 # silu(x) -> x
    assert abs(out[4]) < 1e-7 and abs(out[5]) < 1e-40 and out[6] == 100.0  # -> 0, no overflow
    np.testing.assert_allclose(O.silu_mul(np.float32([2.0]), np.float32([3.0])), [3 * 2 / (1 + math.exp(-2))],
                               rtol=1e-6)


def test_argmax_brute_force_ties_nan():
    rng = np.random.default_rng(5)
    for _ in range(50):
        x = rng.integers(-3, 4, size=50).astype(np.float32)
        assert O.argmax(x) == int(np.argmax(x))     # numpy returns the first maximum too
    x = np.array([np.nan, 1.0, 3.0, np.nan, 3.0], np.float32)
    assert O.argmax(x) == 2
    assert O.argmax(np.full(4, np.nan, np.float32)) == 0


# ---------------------------------------------------------------- tiny model golden
def test_tiny_model_matches_committed_golden():
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tiny_fp32_seed0.npz"))
    prompt = O.token_ids(0, 0, 32000, 16)
    assert np.array_equal(prompt, g["prompt"])
    m = O.OracleModel(O.TINY, 0)
    toks, logits = m.generate(prompt, 33)
    assert np.array_equal(toks, g["tokens"])
    np.testing.assert_array_equal(logits, g["last_logits"])


# ---------------------------------------------------------------- composition vs HF
def _hf_golden_errors(m, name="hf_tiny_fp32_seed0.npz"):
    """Walks the oracle model through the golden's 33 steps (prefill, then KV-cached
    decode steps fed with the golden's tokens) and returns the largest logit error
    relative to the step's largest |logit| and the steps whose greedy token differs."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", name))
    prompt = g["prompt"]
    stride = int(g["sample_stride"])
    worst, bad_steps = 0.0, []
    for step in range(len(g["tokens"])):
        if step == 0:
            logits = m.forward(prompt, 0)
        else:
            logits = m.forward(np.array([g["tokens"][step - 1]], np.int64), len(prompt) + step - 1)
        scale = float(np.max(np.abs(g["top_val"][step])))
        if step == 0:
            worst = max(worst, float(np.max(np.abs(logits - g["prefill_logits"]))) / scale)
        worst = max(worst, float(np.max(np.abs(logits[g["top_idx"][step]] - g["top_val"][step]))) / scale)
        worst = max(worst, float(np.max(np.abs(logits[::stride] - g["sample"][step]))) / scale)
        if O.argmax(logits) != int(g["tokens"][step]):
            bad_steps.append(step)
    return worst, bad_steps


def test_oracle_composition_matches_hf_transformers_golden():
    """The oracle's whole-model forward (prefill, then one KV-cached decode step at a
    time) against transformers' LlamaForCausalLM on the same tiny fp32 weights
    (tests/golden/make_hf_tiny_golden.py): identical greedy tokens at all 33 steps, and
    logits within 1e-4 of the largest |logit| at every step (the prefill step in full;
    the top-16 and every 97th vocabulary entry of every step)."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "hf_tiny_fp32_seed0.npz"))
    assert np.array_equal(O.token_ids(0, 0, 32000, 16), g["prompt"])
    for fast in (False, True):
        m = O.OracleModel(O.TINY, 0)
        m.set_fast(fast)
        worst, bad = _hf_golden_errors(m)
        assert worst <= 1e-4 and not bad, (fast, worst, bad)


@pytest.mark.parametrize("slip", [1, 2, 3, 4])
def test_hf_golden_rejects_planted_composition_slips(slip):
    """Each planted wiring mistake in the oracle (normed-input residual, keys cached
    without RoPE, h % Hkv GQA mapping, no final norm) fails the HF pin by a wide
    margin, so the pin constrains the composition and not just the op kernels."""
    m = O.OracleModel(O.TINY, 0)
    m.set_slip(slip)
    worst, bad = _hf_golden_errors(m)
    assert worst > 1e-2, (slip, worst)


# ---------------------------------------------------------------- norm gain wiring vs HF
GAINS_GOLDEN = "hf_tiny_gains_fp32_seed0.npz"


def _gains_model(slip=0, fast=False):
    m = O.OracleModel(O.TINY, 0)
    m.set_gains(O.norm_gains(0, O.TINY["num_layers"], O.TINY["hidden"]))
    m.set_fast(fast)
    m.set_slip(slip)
    return m


def test_norm_gains_are_distinct_and_non_unit():
    g = O.norm_gains(0, O.TINY["num_layers"], O.TINY["hidden"])
    vecs = list(g["input"]) + list(g["post"]) + [g["final"]]
    for i, a in enumerate(vecs):
        assert 0.05 < float(np.std(a)) < 0.2 and abs(float(np.mean(a)) - 1.0) < 0.02
        for b in vecs[i + 1:]:
            assert float(np.max(np.abs(a - b))) > 0.1


def test_oracle_gain_wiring_matches_hf_transformers_golden():
    """With a different non-unit gain on every RMSNorm (1 + N(0, 0.1);
    tests/golden/make_hf_tiny_golden.py gains), the oracle's composition still equals
    transformers' LlamaForCausalLM: identical greedy tokens at all 33 steps and logits
    within 1e-4 of the largest |logit|.  The unit-gain golden cannot tell which gain a
    norm applies; this one can (see the slips below)."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", GAINS_GOLDEN))
    assert np.array_equal(O.token_ids(0, 0, 32000, 16), g["prompt"])
    for fast in (False, True):
        worst, bad = _hf_golden_errors(_gains_model(fast=fast), GAINS_GOLDEN)
        assert worst <= 1e-4 and not bad, (fast, worst, bad)


@pytest.mark.parametrize("slip", [5, 6, 7])
def test_gains_golden_rejects_planted_gain_wiring_slips(slip):
    """Swapping each layer's input and post-attention gains, giving the final norm the
    last layer's post-attention gain, or dropping the input norms' gain each fails the
    gains pin, while the unit-gain pin cannot see any of them."""
    worst, bad = _hf_golden_errors(_gains_model(slip), GAINS_GOLDEN)
    assert worst > 1e-3, (slip, worst)
    m = O.OracleModel(O.TINY, 0)
    m.set_slip(slip)
    worst_unit, bad_unit = _hf_golden_errors(m)
    assert worst_unit <= 1e-4 and not bad_unit, (slip, worst_unit)


# ---------------------------------------------------------------- CPU-baseline GEMV helper
@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_qweight_gemv_is_the_linear_map_of_its_weight(fmt):
    """The per-shape GEMV the bench's CPU baseline times (orc_qweight_gemv) is a linear
    map: doubling x doubles y exactly, y(x1 + x2) = y(x1) + y(x2) to fp32 rounding,
    and one-hot inputs pick single columns whose values are bounded by the fill."""
    L = O.lib()
    n, k = 37, 256
    q = L.orc_qweight_create(n, k, fmt, 128, 5)
    assert q
    try:
        rng = np.random.default_rng(fmt)
        x1, x2 = rng.standard_normal(k).astype(np.float32), rng.standard_normal(k).astype(np.float32)

        def y(x):
            x = np.ascontiguousarray(x, np.float32)
            out = np.empty(n, np.float32)
            L.orc_qweight_gemv(q, O.ptr(x), O.ptr(out))
            return out

        assert np.array_equal(y(2 * x1), 2 * y(x1))
        np.testing.assert_allclose(y(x1 + x2), y(x1) + y(x2), rtol=1e-4, atol=1e-5)
        cols = np.stack([y(np.eye(k, dtype=np.float32)[j]) for j in range(0, k, 17)])
        assert np.all(np.isfinite(cols)) and np.any(cols != 0) and float(np.max(np.abs(cols))) < 0.07
        assert L.orc_qweight_bytes(q) == {1: n * k * 2, 2: n * k + 4 * n, 3: n * k // 2 + n * (k // 128) * 2}[fmt]
    finally:
        L.orc_qweight_destroy(q)
