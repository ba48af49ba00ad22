"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against (a) the known answers in the
reference's own unit tests (tests/golden/reference_known_answers.json),
(b) oracle/_ref/libssref.so, the reference's cpu_neon.c built from its own
source, where that covers it, and (c) closed forms, invariants and
independent float64 brute force chosen so a dropped term, wrong sign or
transposed operand fails.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle
from tests.util import Q4_0, Q8_0, dequant_np, make_blocks, rel_err

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
L = oracle.lib()
REF = oracle.ref()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference tree absent)")


def p(a):
    return oracle._ptr(a)


# ---------------------------------------------------------------- f16
def test_f16_known_answers():
    for h, v, tol in GOLD["f16_to_f32"]["cases"]:
        assert abs(L.orc_f16_to_f32(h) - v) < tol


def test_f16_to_f32_exhaustive_matches_ieee():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], np.float32)])
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- dequant
def test_dequant_known_answers():
    g = GOLD["dequant_f32"]
    out = oracle.dequantize(np.array(g["src"], np.float32), 4, 0)
    assert np.allclose(out, g["out"], atol=g["tol"])
    g = GOLD["dequant_f16"]
    out = oracle.dequantize(np.array(g["src"], np.uint16), 4, 1)
    assert np.allclose(out, g["out"], atol=g["tol"])


def test_q4_0_hand_built_block():
    # d = 1.0; byte j = j | (15 - j) << 4  ->  w[j] = j - 8, w[j + 16] = 7 - j
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    blk[2:] = [j | ((15 - j) << 4) for j in range(16)]
    out = oracle.dequantize(blk, 32, Q4_0)
    assert out[:16].tolist() == [j - 8 for j in range(16)]
    assert out[16:].tolist() == [7 - j for j in range(16)]
    # d = -2.0 (0xC000) and a subnormal d = 2^-24 (0x0001)
    blk[0:2] = np.array([0xC000], np.uint16).view(np.uint8)
    assert oracle.dequantize(blk, 32, Q4_0)[0] == 16.0
    blk[0:2] = np.array([0x0001], np.uint16).view(np.uint8)
    assert oracle.dequantize(blk, 32, Q4_0)[0] == np.float32(-8 * 2.0 ** -24)


def test_q8_0_hand_built_block():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([0x3800], np.uint16).view(np.uint8)   # 0.5
    codes = np.array([127, -127, 0, 1, -1] + list(range(-13, 14)), np.int8)[:32]
    blk[2:] = codes.view(np.uint8)
    assert np.array_equal(oracle.dequantize(blk, 32, Q8_0), codes.astype(np.float32) * 0.5)


def test_matvec_known_answer_orientation():
    """test_tensor_ops.c:66-78 encoded exactly as Q8_0 (d = 1): [[1,2,3],[4,5,6]] @ [1,2,3]."""
    g = GOLD["matvec"]
    rows, cols = 2, 32
    blocks = np.zeros((rows, 34), np.uint8)
    for r in range(rows):
        blocks[r, 0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
        codes = np.zeros(32, np.int8)
        codes[:3] = g["mat"][r]
        blocks[r, 2:] = codes.view(np.uint8)
    x = np.zeros(cols, np.float32)
    x[:3] = g["vec"]
    assert oracle.matvec(blocks.reshape(-1), x, rows, cols, Q8_0).tolist() == g["out"]


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("rows,cols", [(1, 32), (37, 256), (300, 4096)])
def test_matvec_vs_float64_brute_force(qtype, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = make_blocks(qtype, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    want = dequant_np(w, rows, cols, qtype) @ x.astype(np.float64)
    assert rel_err(oracle.matvec(w, x, rows, cols, qtype), want) < 2e-6


@needs_ref
def test_dot_and_matvec_vs_reference_cpu_neon():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    ref = REF.ss_neon_dot(p(a), p(b), 1000)
    assert abs(L.orc_dot(p(a), p(b), 1000) - ref) <= 1e-5 * max(1.0, abs(ref))
    # F32 matvec known answer through the reference's own ss_neon_matvec
    mat = np.array([1, 2, 3, 4, 5, 6], np.float32)
    vec = np.array([1, 2, 3], np.float32)
    out = np.zeros(2, np.float32)
    REF.ss_neon_matvec(p(out), p(mat), p(vec), 2, 3)
    assert out.tolist() == GOLD["matvec"]["out"]


# ---------------------------------------------------------------- norms / activations
def test_rmsnorm_known_answer():
    g = GOLD["rmsnorm"]
    out = oracle.rmsnorm(g["x"], g["w"], g["eps"])
    s = 1.0 / math.sqrt(g["rms_sq"])
    assert abs(out[0] - 1 * s) < g["tol"] and abs(out[1] - 2 * s) < g["tol"]


@needs_ref
@pytest.mark.parametrize("n", [4, 2048, 4096, 8192])
def test_rmsnorm_bit_exact_vs_reference(n):
    rng = np.random.default_rng(n)
    x = (5 * rng.standard_normal(n)).astype(np.float32)
    w = (1 + 0.01 * rng.standard_normal(n)).astype(np.float32)
    ref = np.zeros(n, np.float32)
    REF.ss_neon_rmsnorm(p(ref), p(x), p(w), n, 1e-5)
    assert np.array_equal(oracle.rmsnorm(x, w, 1e-5), ref)


def test_gemma_rmsnorm_known_answer():
    """tensor.c:133-152: x * (1 / sqrt(mean(x^2) + eps)) * (w + 1); w = 0 is
    the plain RMSNorm with unit weights."""
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    s = 1.0 / math.sqrt((1 + 4 + 9 + 16) / 4.0 + 1e-5)
    assert np.allclose(oracle.gemma_rmsnorm(x, np.zeros(4, np.float32), 1e-5), x * s, rtol=1e-6)
    assert np.allclose(oracle.gemma_rmsnorm(x, np.full(4, 0.5, np.float32), 1e-5), 1.5 * x * s, rtol=1e-6)
    assert np.array_equal(oracle.gemma_rmsnorm(x, np.zeros(4, np.float32), 1e-5),
                          oracle.rmsnorm(x, np.ones(4, np.float32), 1e-5))


@needs_ref
@pytest.mark.parametrize("n", [4, 2304, 3584])
def test_gemma_rmsnorm_bit_exact_vs_reference(n):
    rng = np.random.default_rng(n + 1)
    x = (5 * rng.standard_normal(n)).astype(np.float32)
    w = (0.1 * rng.standard_normal(n)).astype(np.float32)
    ref = np.zeros(n, np.float32)
    REF.ss_neon_gemma_rmsnorm(p(ref), p(x), p(w), n, 1e-6)
    assert np.array_equal(oracle.gemma_rmsnorm(x, w, 1e-6), ref)


def test_gelu_closed_form_and_limits():
    """tensor.c:181-190, the tanh form: 0 at 0, odd part x/2, -> x for large
    x and -> 0 for large negative x; GELU(1) = 0.841192 (tanh form)."""
    v = oracle.gelu([0.0, 1.0, -1.0, 10.0, -10.0, 3.0])
    assert v[0] == 0.0
    assert abs(v[1] - 0.8411920) < 1e-6 and abs(v[1] - v[2] - 1.0) < 1e-6   # gelu(x) - gelu(-x) = x
    assert abs(v[3] - 10.0) < 1e-6 and abs(v[4]) < 1e-6
    x = 3.0
    want = 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    assert abs(v[5] - want) < 1e-6


def test_softcap_closed_form():
    """tensor.c:194-200: cap * tanh(x / cap); cap <= 0 leaves x."""
    x = np.array([0.0, 1.0, -1.0, 100.0, -100.0, 2.5], np.float32)
    out = oracle.softcap(x, 5.0)
    assert np.allclose(out, 5.0 * np.tanh(x / 5.0), rtol=1e-6, atol=1e-7)
    assert out[3] <= 5.0 and out[4] >= -5.0 and out[0] == 0.0
    assert np.array_equal(oracle.softcap(x, 0.0), x)


def test_silu_known_answers():
    for g, want in GOLD["silu"]["cases"]:
        assert abs(L.orc_silu_mul(g, 1.0) - want) < GOLD["silu"]["tol"]


@needs_ref
def test_silu_bit_exact_vs_reference():
    rng = np.random.default_rng(1)
    g = (8 * rng.standard_normal(4099)).astype(np.float32)
    ref = g.copy()
    REF.ss_neon_silu(p(ref), ref.size)
    got = np.array([L.orc_silu_mul(float(v), 1.0) for v in g], np.float32)
    assert np.array_equal(got, ref)


def test_softmax_known_answers():
    g = GOLD["softmax_uniform"]
    assert np.allclose(oracle.softmax(g["x"]), g["out"], atol=g["tol"])
    g = GOLD["softmax_sums_to_one"]
    assert abs(float(np.sum(oracle.softmax(g["x"]))) - g["sum"]) < g["tol"]
    x = np.array([1000.0, 999.0, -1e30], np.float32)        # max subtraction keeps it finite
    s = oracle.softmax(x)
    assert np.all(np.isfinite(s)) and abs(s[0] / s[1] - math.e) < 1e-5


def test_argmax_known_answers_and_tie_rule():
    assert oracle.argmax(GOLD["argmax"]["x"]) == GOLD["argmax"]["out"]
    assert oracle.argmax([2.0, 5.0, 5.0, 1.0]) == 1            # first maximum
    assert oracle.argmax([float("nan"), 3.0]) == 0              # starts from x[0]
    assert oracle.argmax([1.0, float("nan"), 3.0]) == 2


# ---------------------------------------------------------------- RoPE
def test_rope_position_zero_is_identity():
    rng = np.random.default_rng(2)
    q = rng.standard_normal(4 * 64).astype(np.float32)
    k = rng.standard_normal(2 * 64).astype(np.float32)
    for neox in (False, True):
        q2, k2 = oracle.rope(q, k, 4, 2, 64, 64, 0, 10000.0, neox)
        assert np.array_equal(q2, q) and np.array_equal(k2, k)


@pytest.mark.parametrize("neox", [False, True])
def test_rope_closed_form_and_norms(neox):
    hd, pos, theta = 64, 37, 10000.0
    rng = np.random.default_rng(4)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal(hd).astype(np.float32)
    q2, _ = oracle.rope(q, k, 1, 1, hd, hd, pos, theta, neox)
    half = hd // 2
    for i in range(half):
        a, b = (i, i + half) if neox else (2 * i, 2 * i + 1)
        ang = pos * theta ** (-(2.0 * i) / hd)
        ca, sa = math.cos(ang), math.sin(ang)
        assert abs(q2[a] - (q[a] * ca - q[b] * sa)) < 2e-5
        assert abs(q2[b] - (q[a] * sa + q[b] * ca)) < 2e-5
        assert abs(math.hypot(q2[a], q2[b]) - math.hypot(q[a], q[b])) < 1e-5


def test_rope_partial_dim_leaves_tail():
    rng = np.random.default_rng(5)
    q = rng.standard_normal(128).astype(np.float32)
    q2, _ = oracle.rope(q, q[:128].copy(), 1, 1, 128, 64, 99, 10000.0, False)
    assert np.array_equal(q2[64:], q[64:]) and not np.array_equal(q2[:64], q[:64])


def test_rope_table_matches_rope():
    rd, npos = 64, 50
    cs = np.zeros(npos * rd, np.float32)
    L.orc_rope_table(p(cs), rd, npos, 10000.0)
    q = np.zeros(rd, np.float32)
    q[0::2] = 1.0
    for pos in (0, 7, 49):
        q2, _ = oracle.rope(q, q.copy(), 1, 1, rd, rd, pos, 10000.0, False)
        assert np.array_equal(q2[0::2], cs[pos * rd:(pos + 1) * rd][0::2])   # cos
        assert np.array_equal(q2[1::2], cs[pos * rd:(pos + 1) * rd][1::2])   # sin


# ---------------------------------------------------------------- KV int8
def test_kv_int8_closed_form():
    rng = np.random.default_rng(6)
    x = (3 * rng.standard_normal(1024)).astype(np.float32)
    q, s = oracle.kv_int8_encode(x)
    amax = np.max(np.abs(x))
    assert s == np.float32(amax) / np.float32(127.0)
    assert q.min() >= -127 and q.max() <= 127 and 127 in np.abs(q)
    assert np.max(np.abs(q.astype(np.float32) * s - x)) <= s / 2 * (1 + 1e-5)
    want = np.round(x.astype(np.float64) * (1.0 / np.float64(np.float32(s)))).astype(np.int8)
    assert np.mean(q == want) > 0.999
    qz, sz = oracle.kv_int8_encode(np.zeros(64, np.float32))
    assert sz == 0.0 and not qz.any()


# ---------------------------------------------------------------- attention
def test_attention_single_position_is_v0():
    rng = np.random.default_rng(7)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal((1, 64)).astype(np.float32)
    v = rng.standard_normal((1, 64)).astype(np.float32)
    assert np.array_equal(oracle.attention_head(q, k, v), v[0])


def test_attention_identical_keys_average_values():
    rng = np.random.default_rng(8)
    q = rng.standard_normal(64).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 64)).astype(np.float32), 10, axis=0)
    v = rng.standard_normal((10, 64)).astype(np.float32)
    assert np.allclose(oracle.attention_head(q, k, v), v.mean(axis=0), atol=1e-6)


def test_attention_vs_float64():
    rng = np.random.default_rng(9)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal((300, 128)).astype(np.float32)
    v = rng.standard_normal((300, 128)).astype(np.float32)
    s = (k.astype(np.float64) @ q) / math.sqrt(128)
    pr = np.exp(s - s.max())
    pr /= pr.sum()
    assert rel_err(oracle.attention_head(q, k, v), pr @ v.astype(np.float64)) < 1e-5


def test_thread_count_does_not_change_results():
    rng = np.random.default_rng(10)
    w = make_blocks(Q4_0, 333, 2048, rng)
    x = rng.standard_normal(2048).astype(np.float32)
    n0 = L.orc_get_threads()
    outs = []
    for n in (1, 3, 8):
        L.orc_set_threads(n)
        outs.append(oracle.matvec(w, x, 333, 2048, Q4_0))
    L.orc_set_threads(n0)
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


# ---------------------------------------------------------------- sampling
# ss_sample (tensor.c:363-451), pinned by closed forms: the xorshift64 stream
# (tensor.c:331-343), greedy and top-k = 1 reducing to the argmax, a
# hand-worked top-p renormalisation, and the uniform-distribution draw.

M64 = (1 << 64) - 1


def xorshift64(s):
    s ^= (s << 13) & M64
    s ^= s >> 7
    s ^= (s << 17) & M64
    return s


def uniform_draw(s):
    return float(np.float32(np.float32(s >> 11) / np.float32(2.0 ** 53)))


def test_sample_rng_stream_closed_form():
    x = np.zeros(16, np.float32)
    st = 0x9E3779B97F4A7C15
    for _ in range(20):
        _, nst, _, r = oracle.sample(x, 1.0, 1.0, 0, st)
        assert nst == xorshift64(st)
        assert r == uniform_draw(nst)
        st = nst


def test_sample_greedy_and_top1_are_argmax():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(500).astype(np.float32)
    x[123] = x[77] = x.max() + 1.0            # a tie: the first index wins
    i, st, _, _ = oracle.sample(x, 0.0, 0.9, 40, 99)
    assert (i, st) == (77, 99)                # T <= 0: argmax, state untouched
    for seed in range(1, 20):
        i, st, _, _ = oracle.sample(x, 0.7, 1.0, 1, seed)
        assert i in (77, 123) and st == xorshift64(seed)


def test_sample_top_p_hand_worked():
    # probabilities 0.5, 0.3, 0.2 (and tiny others): top_p 0.6 keeps 0.5 and
    # 0.3 (the running sum reaches 0.8 at 0.3), renormalised to 0.625, 0.375
    x = np.log(np.array([0.5, 0.3, 0.2], np.float64)).astype(np.float32)
    for seed in range(1, 200):
        i, st, p, r = oracle.sample(x, 1.0, 0.6, 0, seed)
        assert p[2] == 0.0
        assert abs(p[0] - 0.625) < 1e-6 and abs(p[1] - 0.375) < 1e-6
        if abs(r - 0.625) > 1e-5:
            assert i == (0 if r < 0.625 else 1)


def test_sample_top_k_keeps_k_largest():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(300).astype(np.float32)
    _, _, p, _ = oracle.sample(x, 1.0, 1.0, 10, 11)
    kept = set(np.nonzero(p)[0].tolist())
    assert kept == set(np.argsort(-x)[:10].tolist())
    assert abs(float(p.sum(dtype=np.float64)) - 1.0) < 1e-5


def test_sample_uniform_draw_index():
    V = 1000
    x = np.zeros(V, np.float32)
    for seed in range(1, 300):
        i, _, p, r = oracle.sample(x, 1.0, 1.0, 0, seed)
        assert np.all(p == p[0])
        j = int(np.floor(r * V))
        if abs(r * V - round(r * V)) > 1e-3:   # away from a cell boundary
            assert i == j


# ---------------------------------------------------------------- Q4_K
def _q4k_expected(d, dmin, sc, mn, q):
    """The reference's fp32 arithmetic for one super-block (quantize.c:287-307):
    d1 = d * sc, m1 = dmin * m, weight = d1 * q - m1, each rounded to fp32."""
    out = np.zeros(256, np.float32)
    df, mf = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    for k in range(8):
        d1 = np.float32(df * np.float32(sc[k]))
        m1 = np.float32(mf * np.float32(mn[k]))
        for l in range(32):
            out[32 * k + l] = np.float32(np.float32(d1 * np.float32(q[k][l])) - m1)
    return out


@pytest.mark.parametrize("case", range(6))
def test_q4_K_dequant_known_blocks(case):
    """Hand-built super-blocks (packed from chosen scales, mins and nibbles by
    the format definition, tests/util.q4k_pack_scales) dequantise to exactly
    d*sc*q - dmin*m: every scale and min bit position is exercised (values
    0, 63, and patterns whose top two bits differ)."""
    from tests.util import q4k_block
    rng = np.random.default_rng(case)
    scs = [[1] * 8, [63] * 8, [0, 63, 16, 47, 32, 15, 48, 31], list(rng.integers(0, 64, 8)),
           [5, 9, 17, 33, 48, 60, 2, 40], list(rng.integers(0, 64, 8))]
    mns = [[0] * 8, [63] * 8, [63, 0, 47, 16, 31, 48, 15, 32], list(rng.integers(0, 64, 8)),
           [40, 2, 60, 48, 33, 17, 9, 5], list(rng.integers(0, 64, 8))]
    ds = [1.0, 0.5, -0.0078125, 0.0123, -2.0, 6.1e-5]
    dms = [0.0, 0.25, 0.001, -0.5, 0.0625, -3.0e-5]
    q = [[(k * 5 + l) % 16 for l in range(32)] for k in range(8)] if case % 2 == 0 else \
        [list(rng.integers(0, 16, 32)) for _ in range(8)]
    blk = q4k_block(ds[case], dms[case], scs[case], mns[case], q)
    got = oracle.dequantize(blk, 256, 12)
    want = _q4k_expected(ds[case], dms[case], scs[case], mns[case], q)
    assert np.array_equal(got, want)


def test_q4_K_identity_block():
    """d = 1, every scale 1 and min 0: the weights are the nibbles themselves,
    sub-block 2j from the low and 2j+1 from the high nibbles of bytes 32j.."""
    from tests.util import q4k_block
    q = [[(3 * k + l) % 16 for l in range(32)] for k in range(8)]
    blk = q4k_block(1.0, 0.0, [1] * 8, [0] * 8, q)
    got = oracle.dequantize(blk, 256, 12)
    assert np.array_equal(got, np.array(q, np.float32).reshape(-1))
    # the raw bytes: low nibble of byte 16 + l is weight l of sub-block 0
    assert (blk[16] & 15) == q[0][0] and (blk[16] >> 4) == q[1][0]


def test_q4_K_scale_unpack_round_trip():
    from tests.util import q4k_pack_scales, q4k_unpack_scales
    rng = np.random.default_rng(3)
    for _ in range(200):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        s2, m2 = q4k_unpack_scales(q4k_pack_scales(sc, mn))
        assert np.array_equal(s2, sc) and np.array_equal(m2, mn)


@pytest.mark.parametrize("rows,cols", [(3, 256), (37, 1024), (16, 4096)])
def test_q4_K_matvec_fp64(rows, cols):
    from tests.util import Q4_K, dequant_np, make_q4_k
    rng = np.random.default_rng(rows)
    w = make_q4_k(rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = oracle.matvec(w, x, rows, cols, Q4_K)
    want = dequant_np(w, rows, cols, Q4_K) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5
    # the numpy decoder is the oracle's dequantisation, value for value
    deq = oracle.dequantize(w[:144], 256, Q4_K)
    assert np.allclose(deq, dequant_np(w[:144], 1, 256, Q4_K)[0], rtol=1e-6, atol=1e-9)


# ---------------------------------------------------------------- Q2_K, Q3_K, Q5_K, Q6_K
@pytest.mark.parametrize("qtype", [10, 11, 13, 14])
def test_kquant_dequant_matches_independent_numpy(qtype):
    """quantize.c:180-263, 310-383 against the vectorised fp64 numpy reading
    of the GGML layouts in tests/util.py (for Q3_K through the 32-bit-word
    scale unpacking): equal on random super-blocks (every product involved
    is exact in fp32 or rounds once the same way)."""
    from tests.util import KQ_BYTES, dequant_np, make_kq
    rng = np.random.default_rng(qtype)
    rows, cols = 5, 1024
    w = make_kq(qtype, rows, cols, rng)
    want = dequant_np(w, rows, cols, qtype)
    rb = cols // 256 * KQ_BYTES[qtype]
    got = np.stack([oracle.dequantize(w[r * rb:(r + 1) * rb], cols, qtype) for r in range(rows)])
    assert np.max(np.abs(got - want)) <= 1e-7 * np.max(np.abs(want))


def test_q2_K_closed_form():
    """Bits 2j..2j+1 of byte 32h + l for weight 128h + 32j + l; scale byte
    8h + 2j + l/16 = sc | m << 4: every byte 0b11100100 gives q = j."""
    blk = np.zeros(84, np.uint8)
    blk[0:16] = [(s % 16) | (((s * 3) % 16) << 4) for s in range(16)]
    blk[16:80] = 0xE4
    blk[80:82] = np.array([0.5], np.float16).view(np.uint8)
    blk[82:84] = np.array([0.25], np.float16).view(np.uint8)
    got = oracle.dequantize(blk, 256, 10)
    for i in range(256):
        h, j, l = i // 128, (i % 128) // 32, i % 32
        s = 8 * h + 2 * j + l // 16
        assert got[i] == np.float32(0.5 * (s % 16) * j - 0.25 * ((s * 3) % 16)), i


def test_q3_K_closed_form():
    """Zero scale bytes give scale 0 - 32; q = bits 2j..2j+1 (0b11100100: j),
    minus 4 where the hmask bit 4h + j is clear (odd bits set here)."""
    blk = np.zeros(110, np.uint8)
    blk[0:32] = 0xAA                       # bits 1, 3, 5, 7 set
    blk[32:96] = 0xE4
    blk[108:110] = np.array([0.125], np.float16).view(np.uint8)
    got = oracle.dequantize(blk, 256, 11)
    for i in range(256):
        h, j, l = i // 128, (i % 128) // 32, i % 32
        q = j - (0 if (0xAA >> (4 * h + j)) & 1 else 4)
        assert got[i] == np.float32(0.125 * -32 * q), i


def test_q5_K_closed_form():
    """Sub-block k: nibble (low for even k) plus 16 times bit k of qh byte l."""
    from tests.util import q4k_pack_scales
    sc, mn = np.arange(8) * 7 + 1, np.arange(8) * 5
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.25], np.float16).view(np.uint8)
    blk[4:16] = q4k_pack_scales(sc, mn)
    blk[16:48] = 0x55                      # bits 0, 2, 4, 6: even sub-blocks get +16
    blk[48:176] = [(l % 16) | (((l * 3) % 16) << 4) for l in range(32)] * 4
    got = oracle.dequantize(blk, 256, 13)
    for i in range(256):
        k, l = i // 32, i % 32
        q = (l % 16 if k % 2 == 0 else (l * 3) % 16) + (16 if k % 2 == 0 else 0)
        assert got[i] == np.float32(np.float32(0.5 * sc[k]) * q - np.float32(0.25 * mn[k])), i


def test_q6_K_closed_form():
    """Low nibbles 0 and high pairs 0 give q = -32; scale 8h + 2c + l/16."""
    blk = np.zeros(210, np.uint8)
    blk[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    blk[208:210] = np.array([0.5], np.float16).view(np.uint8)
    got = oracle.dequantize(blk, 256, 14)
    for i in range(256):
        h, c, l = i // 128, (i % 128) // 32, i % 32
        assert got[i] == np.float32(0.5 * (8 * h + 2 * c + l // 16 - 8) * -32), i


@pytest.mark.parametrize("qtype", [10, 11, 13, 14])
def test_kquant_matvec_fp64(qtype):
    from tests.util import dequant_np, make_kq
    rng = np.random.default_rng(qtype + 100)
    rows, cols = 16, 2048
    w = make_kq(qtype, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = oracle.matvec(w, x, rows, cols, qtype)
    want = dequant_np(w, rows, cols, qtype) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


# ---------------------------------------------------------------- Q4_1, Q5_0, Q5_1, Q8_1, F16, F32
MORE = [0, 1, 3, 6, 7, 9]


@pytest.mark.parametrize("qtype", MORE)
def test_more_dequant_matches_independent_numpy(qtype):
    """quantize.c:74-176 against the vectorised fp64 numpy reading of the
    GGML layouts in tests/util.py: equal on random blocks (each weight is one
    exact product plus at most one fp32 rounding)."""
    from tests.util import B32_BYTES, dequant_np, make_more
    rng = np.random.default_rng(qtype + 50)
    rows, cols = 5, 256
    w = make_more(qtype, rows, cols, rng)
    want = dequant_np(w, rows, cols, qtype)
    rb = cols // 32 * B32_BYTES[qtype]
    got = np.stack([oracle.dequantize(w[r * rb:(r + 1) * rb], cols, qtype) for r in range(rows)])
    assert np.max(np.abs(got - want)) <= 1e-7 * np.max(np.abs(want))


def _nibble_block():
    return np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)   # weight j: j, weight j+16: 15-j


def test_q4_1_closed_form():
    """d * nibble + m, weight j in the low nibble of byte j, j + 16 in the high."""
    blk = np.zeros(20, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:4] = np.array([-1.25], np.float16).view(np.uint8)
    blk[4:20] = _nibble_block()
    got = oracle.dequantize(blk, 32, 3)
    want = [0.5 * j - 1.25 for j in range(16)] + [0.5 * (15 - j) - 1.25 for j in range(16)]
    assert np.array_equal(got, np.array(want, np.float32))


def test_q5_0_closed_form():
    """(q - 16) * d with q = nibble | bit j of the little-endian qh << 4."""
    qh = 0xF0F0F00F
    blk = np.zeros(22, np.uint8)
    blk[0:2] = np.array([0.25], np.float16).view(np.uint8)
    blk[2:6] = np.array([qh], np.uint32).view(np.uint8)
    blk[6:22] = _nibble_block()
    got = oracle.dequantize(blk, 32, 6)
    nib = list(range(16)) + [15 - j for j in range(16)]
    want = [((nib[j] | (((qh >> j) & 1) << 4)) - 16) * 0.25 for j in range(32)]
    assert np.array_equal(got, np.array(want, np.float32))


def test_q5_1_closed_form():
    """q * d + m; qh 0x0000FFFF lifts the first 16 weights by 16."""
    blk = np.zeros(24, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.75], np.float16).view(np.uint8)
    blk[4:8] = np.array([0x0000FFFF], np.uint32).view(np.uint8)
    blk[8:24] = _nibble_block()
    got = oracle.dequantize(blk, 32, 7)
    want = [(j + 16) * 0.5 + 0.75 for j in range(16)] + [(15 - j) * 0.5 + 0.75 for j in range(16)]
    assert np.array_equal(got, np.array(want, np.float32))


def test_q8_1_closed_form():
    """fp32 d (0.1 has no binary16 form: the whole fp32 word is read) times
    the int8 code; the sum field s is ignored."""
    blk = np.zeros(40, np.uint8)
    blk[0:4] = np.array([0.1], np.float32).view(np.uint8)
    blk[4:8] = np.array([123.0], np.float32).view(np.uint8)
    blk[8:40] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    got = oracle.dequantize(blk, 32, 9)
    assert np.array_equal(got, np.float32(0.1) * (np.arange(32) - 16).astype(np.float32))


def test_f16_f32_rows_are_the_weights():
    """quantize.c:167-172 (F16 widened exactly, subnormals and signed zero
    included) and :391-393 (F32 copied)."""
    h = np.array([0.0, -0.0, 1.0, -2.5, 6.1e-5, 5.96e-8, 65504.0, 0.333], np.float16)
    assert np.array_equal(oracle.dequantize(h.view(np.uint8), h.size, 1), h.astype(np.float32))
    f = np.array([1e-40, -3.25, 7.0, 1e30], np.float32)
    assert np.array_equal(oracle.dequantize(f.view(np.uint8), f.size, 0), f)


@pytest.mark.parametrize("qtype", MORE)
def test_more_matvec_fp64(qtype):
    from tests.util import dequant_np, make_more
    rng = np.random.default_rng(qtype + 150)
    rows, cols = 16, 2048
    w = make_more(qtype, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = oracle.matvec(w, x, rows, cols, qtype)
    want = dequant_np(w, rows, cols, qtype) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
