"""Device sampling (ss_hip_sample_logits, ss_hip_sample) against the oracle's
ss_sample (tensor.c:363-451), through the C-ABI.

Bar: the advanced xorshift64 state is identical (integer work). The sampled
index is identical whenever the uniform draw r lies more than TOL(V) from
every cumulative boundary of the oracle's final distribution (fp64 cumulative
sums of it), TOL(V) = V * 2^-24 being the worst-case error of the
reference's sequential fp32 sums over V terms (softmax, renormalisation and
the cumulative walk). Nearer a boundary, where those fp32 sums decide, the
device index (exact fixed-point sums) must still be consistent with the
oracle's distribution: cdf(index - 1) - TOL <= r < cdf(index) + TOL.
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _tol(V):
    return V * 2.0 ** -24


def _band_distance(p, r):
    """Distance of r from the nearest cumulative boundary that fp32 rounding
    can move: the cumulative sums after positive terms (a run of leading
    zeros sums to exactly 0 on both sides)."""
    cdf = np.cumsum(p.astype(np.float64))
    steps = cdf[p > 0]
    return float(np.min(np.abs(steps - r))) if steps.size else 1.0


def _check_index(got, want, p, r):
    """Identical away from the boundaries, consistent with p near them."""
    cdf = np.cumsum(p.astype(np.float64))
    tol = _tol(p.size)
    if _band_distance(p, r) > tol:
        assert got == want, (got, want, r)
        return 0
    lo = cdf[got - 1] if got > 0 else 0.0
    assert lo - tol <= r < cdf[got] + tol or (got == p.size - 1 and r >= cdf[-1] - tol), (got, want, r)
    return 1


def _device_sample(hip, logits, T, top_p, top_k, rng):
    X = hip.upload(np.ascontiguousarray(logits, np.float32))
    st = C.c_uint64(rng)
    out = C.c_int32(-1)
    rc = hip.L.ss_hip_sample_logits(hip.ctx, X.ptr, logits.size, T, top_p, top_k, C.byref(st), C.byref(out))
    X.free()
    assert rc == 0, hip.err()
    return out.value, st.value


def _logits(kind, V, rng):
    if kind == "normal":
        return (rng.standard_normal(V) * 2.0).astype(np.float32)
    if kind == "peaked":
        x = rng.standard_normal(V).astype(np.float32)
        x[rng.integers(0, V, 3)] += 12.0
        return x
    if kind == "ties":   # few distinct values: ties at every threshold
        return rng.integers(0, 5, V).astype(np.float32)
    if kind == "nan":
        x = rng.standard_normal(V).astype(np.float32)
        x[rng.integers(0, V, 4)] = np.nan
        return x
    raise ValueError(kind)


CASES = [(V, kind) for V in (7, 512, 32000, 128256) for kind in ("normal", "peaked", "ties", "nan")]
PARAMS = [(0.7, 1.0, 0), (1.0, 0.9, 40), (1.3, 0.5, 0), (0.8, 0.999, 1), (1.0, 1.0, 5), (0.6, 0.95, 2)]


@pytest.mark.parametrize("V,kind", CASES)
def test_sample_matches_oracle(hip, V, kind):
    rng = np.random.default_rng(V + len(kind))
    close = 0
    for trial, (T, top_p, top_k) in enumerate(PARAMS * 3):
        x = _logits(kind, V, rng)
        seed = int(rng.integers(1, 2 ** 63))
        want, want_st, p, r = oracle.sample(x, T, top_p, top_k, seed)
        got, got_st = _device_sample(hip, x, T, top_p, top_k, seed)
        assert got_st == want_st, (trial, T, top_p, top_k)
        assert 0 <= got < V
        close += _check_index(got, want, p, r)
    print("draws within the fp32 band of a boundary: %d of %d" % (close, 3 * len(PARAMS)))


def test_sample_top_k_ties_and_greedy(hip):
    # k-th largest value shared by several entries: all of them stay
    x = np.array([1.0, 3.0, 2.0, 3.0, 2.0, 2.0, 0.5], np.float32)
    for seed in range(1, 60):
        want, want_st, p, r = oracle.sample(x, 1.0, 1.0, 3, seed)
        got, got_st = _device_sample(hip, x, 1.0, 1.0, 3, seed)
        assert got_st == want_st
        _check_index(got, want, p, r)
    # temperature <= 0: the first maximum, state untouched
    got, st = _device_sample(hip, x, 0.0, 0.9, 3, 1234)
    assert (got, st) == (1, 1234)


def test_model_sample_matches_oracle(tmp_path):
    """ss_hip_sample over a model's own logits (left in HBM by the prompt)."""
    from phonemap_amd import api
    path = str(tmp_path / "s.gguf")
    spec = api.SynthSpec(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512,
                         vocab=512, context_length=64, seed=5)
    api.write_synthetic_gguf(path, spec)
    with api.Model(path, max_context=64) as m:
        lg, _ = m.eval_prompt(list(range(3, 12)), 0)
        for seed in (1, 2, 3, 99, 12345):
            want, want_st, p, r = oracle.sample(lg, 0.8, 0.9, 40, seed)
            got, got_st = m.sample(0.8, 0.9, 40, seed)
            assert got_st == want_st
            _check_index(got, want, p, r)


STOP_TEXTS = {"<|im_end|>", "<|eot_id|>", "<|end|>", "<|endoftext|>", "<|user|>", "</s>", "<end_of_turn>",
              "<eos>"}   # engine.c stop tokens, as ss_generate checks them


def test_generate_samples_on_device(tmp_path):
    """ss_generate with temperature > 0 samples on the device (the logits stay
    in HBM); the tokens it reports equal a host replay that samples the
    oracle's ss_sample over logits copied back, with the same seed."""
    from phonemap_amd import api
    L = api._lib()
    path = str(tmp_path / "g.gguf")
    spec = api.SynthSpec(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512,
                         vocab=512, context_length=128, seed=9)
    api.write_synthetic_gguf(path, spec)
    T, top_p, top_k, seed, n_max = 0.9, 0.95, 50, 0x4F6CDD1D, 24   # seed: uint32_t (slipstream.h)
    with api.Model(path, max_context=128) as m:
        prm = L.ss_default_params()
        prm.max_tokens, prm.temperature, prm.top_p, prm.top_k, prm.seed = n_max, T, top_p, top_k, seed
        prm.stop_sequence = None
        got = []
        cb = api.TOKEN_CB(lambda text, tid, ud: got.append(int(tid)) is None)
        assert L.ss_generate(m.h, b"the quick brown fox", C.byref(prm), cb, None) == 0
        # host replay through the oracle's sampler
        toks = m.tokenize("the quick brown fox")
        m.reset()
        lg, _ = m.eval_prompt(toks, 0)
        eos, rng, pos, want, why = L.ss_eos_id(m.h), seed, len(toks), [], "max_tokens"
        for _ in range(n_max):
            i, rng, p, r = oracle.sample(lg, T, top_p, top_k, rng)
            if _band_distance(p, r) <= _tol(p.size):
                why = "band"   # within the fp32 band: the continuation may legitimately differ
                break
            if i == eos or m.token_text(i) in STOP_TEXTS:
                why = "stop %d %r" % (i, m.token_text(i))
                break
            want.append(i)
            lg, _ = m.eval_token(i, pos)
            pos += 1
        assert got[:len(want)] == want, (why, got, want)
        assert len(want) >= 8 or why != "band", (why, got, want)
