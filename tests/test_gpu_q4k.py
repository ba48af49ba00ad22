"""Q4_K (256-weight K-quant super-blocks, quantize.c:265-310; the Metal
backend's matvec_q4_K, metal_backend.m:111-154) on the HIP path against the
CPU oracle, through the C-ABI.

* The matvec at the Llama-2-7B decode shapes ([Wq;Wk;Wv] 12288 x 4096, Wo
  4096 x 4096, gate/up 11008 x 4096, down 4096 x 11008, an LM head
  32000 x 4096) and at edge shapes (one super-block, rows not a multiple
  of 16): max |gpu - oracle| / max |oracle| <= 1e-3, and (all but the head)
  per row against the exact fp64 product
  max_i |y_i - e_i| / sum_j |w_ij x_j| <= 1e-6 (tests/util.py
  check_elementwise).
* ss_hip_matvec_q4_k equals ss_hip_matvec(type 12) bit for bit; the fused
  RMSNorm + residual and gate/up + SwiGLU forms hold the same bar.
* Embedding rows dequantise bit-exactly (d*sc and dmin*m exact in fp32, then
  one rounded product and one rounded difference, as quantize.c:300-305).
* Whole models with Q4_K layers, embedding and LM head: greedy tokens equal
  to the oracle's and logits within 1e-3 (fp16 cache; 5e-2 int8) of the
  oracle's at every step, for graph and eager launches (the persistent
  launch falls back to graph) and both cache types; prompts run token by
  token. The fp64 model's distance is printed beside the oracle's
  (OracleBar). One step is listed in KNOWN: at seed 31, position 21, the
  oracle's fp16 cache rounds a value across a binary16 midpoint the other
  way than exact arithmetic does, and its logits leave the fp64 model's by
  1.51e-3. The GPU is 4.7e-6 from the fp64 model there and 1.51e-3 from the
  oracle, so that step holds the oracle at 2e-3 and the fp64 model at 1e-3.
* Streaming mode (layers uploaded per use) gives the resident logits bit
  for bit.
* A shape the Q4_K matvec cannot take (columns not a multiple of 256) is
  refused.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.ref_model import RefModel
from tests.util import OracleBar, Q4_K, check_elementwise, make_q4_k, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
TOL_INT8 = 5e-2


def _case(hip, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = make_q4_k(rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    W, X, Y = hip.packed(w, Q4_K, rows, cols), hip.upload(x), hip.buf(4 * rows)
    return rng, w, x, W, X, Y


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4096, 4096), (11008, 4096), (4096, 11008),
                                       (32000, 4096), (1, 256), (7, 512), (33, 2816), (17, 14336)])
def test_q4k_matvec(hip, rows, cols):
    print("q4k matvec", rows, cols, flush=True)
    _, w, x, W, X, Y = _case(hip, rows, cols, rows + cols)
    assert hip.L.ss_hip_matvec(hip.ctx, Y.ptr, W.ptr, X.ptr, rows, cols, Q4_K, None) == 0, hip.err()
    got = Y.read(np.float32, rows)
    assert np.all(np.isfinite(got))
    want = oracle.matvec(w, x, rows, cols, Q4_K)
    assert rel_err(got, want) <= TOL
    if rows * cols <= 12288 * 4096:   # the fp64 reading of the 32000-row head takes ~25 s
        check_elementwise(got, want, w, x, rows, cols, Q4_K)


def test_q4k_typed_entry_point(hip):
    rows, cols = 300, 4096
    _, w, x, W, X, Y = _case(hip, rows, cols, 5)
    Y2 = hip.buf(4 * rows)
    assert hip.L.ss_hip_matvec(hip.ctx, Y.ptr, W.ptr, X.ptr, rows, cols, Q4_K, None) == 0
    assert hip.L.ss_hip_matvec_q4_k(hip.ctx, Y2.ptr, W.ptr, X.ptr, rows, cols, None) == 0, hip.err()
    assert np.array_equal(Y.read(np.float32, rows), Y2.read(np.float32, rows))


def test_q4k_rejects_partial_super_blocks(hip):
    rows, cols = 16, 288                      # 9 blocks of 32: not whole super-blocks
    Y, W, X = hip.buf(4 * rows), hip.buf(1 << 16), hip.buf(4 * cols)
    assert hip.L.ss_hip_matvec(hip.ctx, Y.ptr, W.ptr, X.ptr, rows, cols, Q4_K, None) == -5
    assert "256" in hip.err()


def test_q4k_fused_norm_residual_and_gate_up(hip):
    rows, cols, eps = 1100, 2048, 1e-5
    rng = np.random.default_rng(11)
    wg, wu = make_q4_k(rows, cols, rng), make_q4_k(rows, cols, rng)
    x = (3.0 * rng.standard_normal(cols)).astype(np.float32)
    nw = (1.0 + 0.01 * rng.standard_normal(cols)).astype(np.float32)
    res = rng.standard_normal(rows).astype(np.float32)
    xn = oracle.rmsnorm(x, nw, eps)
    WG, WU = hip.packed(wg, Q4_K, rows, cols), hip.packed(wu, Q4_K, rows, cols)
    X, NW, Y = hip.upload(x), hip.upload(nw), hip.upload(res)
    assert hip.L.ss_hip_matvec_fused(hip.ctx, Y.ptr, WG.ptr, X.ptr, NW.ptr, C.c_float(eps), 1, rows, cols, Q4_K,
                                     None) == 0, hip.err()
    assert rel_err(Y.read(np.float32, rows), oracle.matvec(wg, xn, rows, cols, Q4_K) + res) <= TOL
    g = oracle.matvec(wg, xn, rows, cols, Q4_K)
    u = oracle.matvec(wu, xn, rows, cols, Q4_K)
    lib = oracle.lib()
    want = np.array([lib.orc_silu_mul(float(a), float(b)) for a, b in zip(g, u)], np.float32)
    O = hip.buf(4 * rows)
    assert hip.L.ss_hip_ffn_gate_up(hip.ctx, O.ptr, WG.ptr, WU.ptr, X.ptr, NW.ptr, C.c_float(eps), rows, cols,
                                    Q4_K, None) == 0, hip.err()
    assert rel_err(O.read(np.float32, rows), want) <= TOL


def test_q4k_embed_row_bit_exact(hip):
    rows, cols = 50, 4096
    rng = np.random.default_rng(9)
    w = make_q4_k(rows, cols, rng)
    bpr = cols // 256 * 144
    T, O = hip.packed(w, Q4_K, rows, cols), hip.buf(4 * cols)
    for tok in (0, 17, 49):
        assert hip.L.ss_hip_embed_row(hip.ctx, O.ptr, T.ptr, Q4_K, rows, cols, tok, None) == 0, hip.err()
        want = oracle.dequantize(w[tok * bpr:(tok + 1) * bpr], cols, Q4_K)
        assert np.array_equal(O.read(np.float32, cols), want)


SPECS = {
    "q4k_gqa": dict(n_layers=3, hidden=1024, n_heads=16, n_kv_heads=4, head_dim=64, ffn=2816, vocab=3000,
                    context_length=256, seed=31, layer_type=Q4_K, embd_type=Q4_K, out_type=Q4_K, scale_mode=1),
    "q4k_tied": dict(n_layers=2, hidden=512, n_heads=8, n_kv_heads=8, head_dim=64, ffn=1536, vocab=700,
                     context_length=256, seed=32, layer_type=Q4_K, embd_type=Q4_K, out_type=-1, scale_mode=1),
}




# Steps at which the oracle's fp16 cache rounds a K/V value across a binary16
# midpoint the other way than exact arithmetic does ((spec, kv, step) ->
# (oracle bar, reason)); every other step holds the oracle bar (OracleBar).
KNOWN = {
    ("q4k_gqa", "f16", 21): (2e-3, "the oracle's fp16 cache leaves the fp64 model by 1.51e-3 at this step"),
}


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("launch", ["graph", "eager", "sweep"])
@pytest.mark.parametrize("spec", sorted(SPECS))
def test_q4k_model_greedy_and_logits(tmp_path, spec, launch, kv):
    kw = SPECS[spec]
    path = str(tmp_path / (spec + ".gguf"))
    api.write_synthetic_gguf(path, api.SynthSpec(**kw))
    print("q4k model", spec, launch, kv, flush=True)
    rng = np.random.default_rng(7)
    prompt = rng.integers(3, kw["vocab"], 12).tolist()
    om = oracle.Model(path, 128, kv)
    rm = RefModel(path, 128, kv)
    tol = TOL if kv == "f16" else TOL_INT8
    bar = OracleBar("q4k %s %s %s" % (spec, launch, kv), tol,
                    {k[2]: v for k, v in KNOWN.items() if k[:2] == (spec, kv)})
    L = api._lib()
    with api.Model(path, max_context=128, kv=kv, launch=launch) as m:
        want = api.LAUNCH["graph"] if launch == "sweep" else api.LAUNCH[launch]
        assert L.ss_hip_model_launch(L.ss_model_hip(m.h)) == want
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        bar.check("prompt", lg, olg, rm.prefill(prompt, 0))
        assert am == oracle.argmax(olg)
        tok, pos, prev = am, len(prompt), olg
        changes = []
        for _ in range(16):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            bar.check(pos, lg, olg, rm.forward(tok, pos))
            assert am == oracle.argmax(olg), pos
            changes.append(rel_err(olg, prev))
            tok, pos, prev = am, pos + 1, olg
        assert np.median(changes) >= 10 * TOL     # the model responds to its input
    om.close()
    bar.report()


def test_q4k_streaming_matches_resident(tmp_path):
    """Streaming mode carries the super-block plane with each layer upload:
    logits bit-identical to the resident model's."""
    kw = SPECS["q4k_gqa"]
    path = str(tmp_path / "q4k_gqa.gguf")
    api.write_synthetic_gguf(path, api.SynthSpec(**kw))
    prompt = np.random.default_rng(5).integers(3, kw["vocab"], 10).tolist()
    runs = []
    for streaming in (False, True):
        print("q4k streaming", streaming, flush=True)
        with api.Model(path, max_context=64, streaming=streaming) as m:
            out = [m.eval_prompt(prompt, 0)]
            tok, pos = out[0][1], len(prompt)
            for _ in range(8):
                lg, am = m.eval_token(tok, pos)
                out.append((lg.copy(), am))
                tok, pos = am, pos + 1
        runs.append(out)
    for i, ((a, ia), (b, ib)) in enumerate(zip(*runs)):
        assert np.array_equal(a, b), i
        assert ia == ib, i
