"""The fp16-MFMA prompt products over every block format (Q4_1, Q5_0, Q5_1,
Q8_1 and the K-quants; Q4_0 and Q8_0 are in test_gpu_kernels.py) against the
oracle's RMSNorm + matvec per token (quantize.c:74-383 dequantisation,
:446-494 matvec): each token's y within max |gpu - oracle| / max |oracle|
<= 1e-3, the accumulating form adding to y. Each block is
sum_g (A_g * sum c x - B_g * sum x) over its 16-weight groups; the shapes
cover a ragged token tile, one token, rows not a multiple of 16 and a
32-weight type whose row ends inside a 4-block tile.

Whole models (Q4_K layers with a Q6_K head as Q4_K_M files have, Q6_K,
Q3_K, Q5_1 with Q4_1 / Q8_1 tables) evaluate a 300-token prompt as products,
against the oracle's token-serial prefill, then decode: logits within 1e-3
(fp16 cache; 5e-2 int8) of the oracle's at every step, with the distance to
the fp64 model of tests/ref_model.py printed beside it (OracleBar; measured
worst against the oracle 2.4e-4).
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.ref_model import RefModel
from tests.util import OracleBar, Q2_K, Q3_K, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_1, make_blocks, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
BLOCK32 = [Q4_1, Q5_0, Q5_1, Q8_1]
KQ = [Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]


def _gemm_check(hip, qtype, rows, cols, T):
    rng = np.random.default_rng(rows + cols + T + qtype)
    w = make_blocks(qtype, rows, cols, rng)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    y0 = rng.standard_normal((T, rows)).astype(np.float32)
    W, X, NW = hip.packed(w, qtype, rows, cols), hip.upload(x), hip.upload(nw)
    Y = hip.upload(y0)
    assert hip.L.ss_hip_gemm(hip.ctx, Y.ptr, W.ptr, X.ptr, NW.ptr, C.c_float(1e-5), 1, rows, cols, T, qtype,
                             None) == 0, hip.err()
    acc = Y.read(np.float32, T * rows).reshape(T, rows)
    assert hip.L.ss_hip_gemm(hip.ctx, Y.ptr, W.ptr, X.ptr, None, C.c_float(1e-5), 0, rows, cols, T, qtype,
                             None) == 0, hip.err()
    plain = Y.read(np.float32, T * rows).reshape(T, rows)
    for t in range(T):
        xn = oracle.rmsnorm(x[t], nw, 1e-5)
        assert rel_err(acc[t] - y0[t], oracle.matvec(w, xn, rows, cols, qtype)) <= TOL, t
        assert rel_err(plain[t], oracle.matvec(w, x[t], rows, cols, qtype)) <= TOL, t
    for b in (W, X, NW, Y):
        b.free()


@pytest.mark.parametrize("qtype", BLOCK32)
@pytest.mark.parametrize("rows,cols,T", [(4096, 4096, 70), (48, 11008, 17), (300, 2080, 1), (33, 96, 9)])
def test_block32_products(hip, qtype, rows, cols, T):
    print("products", qtype, rows, cols, T, flush=True)
    _gemm_check(hip, qtype, rows, cols, T)


@pytest.mark.parametrize("qtype", KQ)
@pytest.mark.parametrize("rows,cols,T", [(4096, 4096, 70), (48, 11008, 17), (300, 2048, 1), (33, 256, 9)])
def test_kquant_products(hip, qtype, rows, cols, T):
    print("products", qtype, rows, cols, T, flush=True)
    _gemm_check(hip, qtype, rows, cols, T)


def test_products_refuse_float_and_partial_super_blocks(hip):
    W, X, Y = hip.buf(1 << 20), hip.buf(1 << 16), hip.buf(1 << 16)
    for qtype, cols in [(0, 256), (1, 256), (Q4_K, 288)]:
        assert hip.L.ss_hip_gemm(hip.ctx, Y.ptr, W.ptr, X.ptr, None, C.c_float(1e-5), 0, 16, cols, 4, qtype,
                                 None) != 0


BASE = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=4, head_dim=64, ffn=2816, vocab=900,
            context_length=512, scale_mode=1)
SPECS = {
    "q4_k_q6_k_head": dict(BASE, layer_type=Q4_K, embd_type=Q4_K, out_type=Q6_K, seed=81),
    "q6_k": dict(BASE, layer_type=Q6_K, embd_type=Q6_K, out_type=Q6_K, seed=82),
    "q3_k": dict(BASE, layer_type=Q3_K, embd_type=Q4_K, out_type=Q6_K, seed=83),
    "q5_1_q4_1": dict(BASE, layer_type=Q5_1, embd_type=Q4_1, out_type=Q8_1, seed=84),
}

# Steps at which the oracle's fp16 cache rounds a K/V value across a binary16
# midpoint the other way than exact arithmetic does ((spec, kv, step) ->
# (oracle bar, reason)); every other step holds the oracle bar (OracleBar).
KNOWN = {}


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("spec", sorted(SPECS))
def test_long_prompt_as_products(tmp_path, spec, kv):
    """A 300-token prompt in one chunk of products (fp16 cache), or token by
    token (int8 cache, where the products do not run), then decode steps."""
    print("products model", spec, kv, flush=True)
    path = str(tmp_path / (spec + ".gguf"))
    api.write_synthetic_gguf(path, api.SynthSpec(**SPECS[spec]))
    prompt = np.random.default_rng(9).integers(3, 900, 300).tolist()
    om = oracle.Model(path, 400, kv)
    rm = RefModel(path, 400, kv)
    tol = TOL if kv == "f16" else 5e-2
    bar = OracleBar("products %s %s" % (spec, kv), tol,
                    {k[2]: v for k, v in KNOWN.items() if k[:2] == (spec, kv)})
    with api.Model(path, max_context=400, kv=kv) as m:
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        bar.check("prompt", lg, olg, rm.prefill(prompt, 0))
        assert am == oracle.argmax(olg)
        tok, pos = am, len(prompt)
        for _ in range(6):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            bar.check(pos, lg, olg, rm.forward(tok, pos))
            assert am == oracle.argmax(olg), pos
            tok, pos = am, pos + 1
    om.close()
    bar.report()
