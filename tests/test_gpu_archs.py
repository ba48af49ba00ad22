"""Parity of the architecture branches beyond the plain llama block on the
GPU: fused attn_qkv and ffn_up (layer_scheduler.c:337-347,518-524), q/k/v
biases in F32 and F16 (:367-402) and NeoX RoPE (qwen2, :144-149), through
the public C API against the CPU oracle on the same synthetic files.

The HIP path runs these models on the llama kernels: the engine splits fused
tensors into row views, uploads the biases as one fp32 vector per layer (added
in the QKV epilogue, or before RoPE in the prompt path), and puts Wq/Wk rows
(and q/k biases, and injected K rows) of NeoX models in the per-head order in
which NeoX pairs are adjacent. Bar, as for the llama models: identical greedy
tokens, logits within 1e-3 (5e-2 with the int8 cache).
"""
import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.test_gpu_model import GQA8, TINY, TINY_Q8, TOL, TOL_INT8, _model_file
from tests.util import rel_err

pytestmark = pytest.mark.gpu

QWEN = dict(GQA8, arch=1, qkv_bias=1, seed=31)                                    # NeoX, F32 biases
QWEN_F16_FUSED = dict(TINY, arch=1, qkv_bias=2, fused_qkv=1, fused_up=1, seed=32)  # NeoX, F16 biases, fused
LLAMA_FUSED = dict(TINY_Q8, fused_qkv=1, fused_up=1, seed=33)                     # GPT-J, fused, Q8_0
QWEN_NOBIAS = dict(TINY, arch=1, seed=34)                                          # NeoX only
SPECS = {"qwen": QWEN, "qwen_f16_fused": QWEN_F16_FUSED, "llama_fused": LLAMA_FUSED,
         "qwen_nobias": QWEN_NOBIAS}


def _decode(m, om, tok, pos, steps, tol):
    for _ in range(steps):
        lg, am = m.eval_token(tok, pos)
        olg = om.forward(tok, pos)
        assert rel_err(lg, olg) <= tol, pos
        assert am == oracle.argmax(olg), pos
        tok, pos = am, pos + 1


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("launch", ["graph", "eager"])
@pytest.mark.parametrize("spec", ["qwen", "qwen_f16_fused", "llama_fused"])
def test_variants_greedy_and_logits(spec, launch, kv):
    kw = SPECS[spec]
    path = _model_file(spec, **kw)
    print("arch", spec, launch, kv, flush=True)
    rng = np.random.default_rng(5)
    prompt = rng.integers(3, kw["vocab"], 12).tolist()
    tol = TOL if kv == "f16" else TOL_INT8
    om = oracle.Model(path, 128, kv)
    with api.Model(path, max_context=128, kv=kv, launch=launch) as m:
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        assert rel_err(lg, olg) <= tol
        assert am == oracle.argmax(olg)
        _decode(m, om, am, len(prompt), 24, tol)
    om.close()


@pytest.mark.parametrize("spec", ["qwen", "qwen_f16_fused", "llama_fused"])
def test_variants_prompt_products(spec):
    """A 600-token prompt as products (512 + 88), a 30-token continuation,
    then decode steps over the cache the products wrote."""
    kw = SPECS[spec]
    path = _model_file(spec, **kw)
    print("arch prompt", spec, flush=True)
    rng = np.random.default_rng(9)
    p1 = rng.integers(3, kw["vocab"], 600).tolist()
    p2 = rng.integers(3, kw["vocab"], 30).tolist()
    om = oracle.Model(path, 1024, "f16")
    with api.Model(path, max_context=1024) as m:
        lg, am = m.eval_prompt(p1, 0)
        olg = om.prefill(p1, 0)
        assert rel_err(lg, olg) <= TOL
        assert am == oracle.argmax(olg)
        lg, am = m.eval_prompt(p2, len(p1))
        olg = om.prefill(p2, len(p1))
        assert rel_err(lg, olg) <= TOL
        assert am == oracle.argmax(olg)
        _decode(m, om, am, len(p1) + len(p2), 12, TOL)
    om.close()


def test_neox_under_the_persistent_launch_and_biases_refused():
    path = _model_file("qwen_nobias", **QWEN_NOBIAS)
    print("arch sweep", flush=True)
    prompt = [5, 9, 300, 17, 4, 88, 23, 61, 2, 7]
    om = oracle.Model(path, 128, "f16")
    with api.Model(path, max_context=128, launch="sweep") as m:
        L = api._lib()
        assert L.ss_hip_model_launch(L.ss_model_hip(m.h)) == api.LAUNCH["sweep"]
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        assert rel_err(lg, olg) <= TOL and am == oracle.argmax(olg)
        _decode(m, om, am, len(prompt), 16, TOL)
    om.close()
    with pytest.raises(api.SlipStreamError):
        api.Model(_model_file("qwen", **QWEN), max_context=128, launch="sweep")


def test_neox_kv_injection_matches_oracle():
    """K/V written in the reference's [pos][kv_dim] order reach a NeoX model
    in its head order."""
    path = _model_file("qwen", **QWEN)
    rng = np.random.default_rng(13)
    n_pre, kvdim = 100, QWEN["n_kv_heads"] * QWEN["head_dim"]
    om = oracle.Model(path, 256, "f16")
    with api.Model(path, max_context=256) as m:
        m.reset()
        for layer in range(QWEN["n_layers"]):
            k = rng.standard_normal((n_pre, kvdim)).astype(np.float16).view(np.uint16)
            v = rng.standard_normal((n_pre, kvdim)).astype(np.float16).view(np.uint16)
            m.kv_write(layer, 0, k, v)
            for p in range(n_pre):
                om.kv_write(layer, p, k[p], v[p])
        _decode(m, om, 17, n_pre, 12, TOL)
    om.close()


@pytest.mark.parametrize("spec", ["qwen", "qwen_f16_fused"])
def test_variants_streaming_matches_resident(spec):
    kw = SPECS[spec]
    path = _model_file(spec, **kw)
    prompt = np.random.default_rng(3).integers(3, kw["vocab"], 20).tolist()
    out = []
    for streaming in (False, True):
        with api.Model(path, max_context=128, streaming=streaming) as m:
            lg, am = m.eval_prompt(prompt, 0)
            seq = [lg]
            tok, pos = am, len(prompt)
            for _ in range(8):
                lg, tok = m.eval_token(tok, pos)
                seq.append(lg)
                pos += 1
            out.append(np.stack(seq))
    assert np.array_equal(out[0], out[1])


def test_general_alignment_is_honoured():
    """A file whose data is 4096-byte aligned (general.alignment) holds the
    same weights as the 32-byte aligned one and gives identical logits."""
    paths = [_model_file("align%d" % a, **dict(TINY, seed=35, alignment=a)) for a in (32, 4096)]
    prompt = [3, 14, 15, 92, 65, 35, 89, 79, 32, 38]
    out = []
    for path in paths:
        with api.Model(path, max_context=64) as m:
            lg, am = m.eval_prompt(prompt, 0)
            seq = [lg]
            tok, pos = am, len(prompt)
            for _ in range(6):
                lg, tok = m.eval_token(tok, pos)
                seq.append(lg)
                pos += 1
            out.append(np.stack(seq))
    assert np.array_equal(out[0], out[1])
