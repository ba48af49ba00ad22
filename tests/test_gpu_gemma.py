"""The Gemma branches and softcaps on the HIP path against the CPU oracle,
through the public API (ss_model_load_ex on synthetic GGUFs):

* "gemma" files: (1 + w) RMSNorms (tensor.c:133-152), the sqrt(d) embedding
  scale (layer_scheduler.c:597-602), GeGLU (:529-531, tensor.c:181-190) and
  the 1/sqrt(d) logit scale (:667-672);
* "gemma2" files: the same plus post-attention and post-FFN norms
  (:474-481, 553-560), with attention and final logit softcaps (:446-448,
  674-676);
* a llama file with softcaps (the reference applies them for any
  architecture that sets the keys);
* head_dim 256 (every Gemma release) with 1, 2 and 8 query heads per KV
  head, including a context long enough for the split merge by the last
  split.

Bar: greedy tokens equal to the oracle's at every step; logits within 1e-3
(fp16 cache) or 5e-2 (int8) of the oracle's at every step, with the distance
to the fp64 model of tests/ref_model.py printed beside it (OracleBar;
measured worst against the oracle 2.4e-5 with the fp16 cache). With the fp16
cache the 9-token prompts run as MFMA products (GeGLU epilogue, post norms
over rows, softcapped flash attention at head_dim 64 and 256); the int8
cache runs them token by token. The persistent launch falls back to graph
launches.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.ref_model import RefModel
from tests.util import OracleBar, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
TOL_INT8 = 5e-2

BASE = dict(n_layers=2, hidden=512, n_heads=8, n_kv_heads=4, head_dim=64, ffn=1024, vocab=600,
            context_length=256, embd_type=8, out_type=-1, scale_mode=1)
SPECS = {
    "gemma": dict(BASE, arch=2, seed=41),
    "gemma2_softcap": dict(BASE, arch=3, attn_softcap=1.5, final_softcap=0.4, seed=42),
    "llama_softcap": dict(BASE, arch=0, n_kv_heads=2, out_type=8, attn_softcap=1.0, final_softcap=3.0, seed=43),
    "gemma_hd256_mha": dict(BASE, arch=2, n_heads=4, n_kv_heads=4, head_dim=256, seed=44),
    "gemma2_hd256_g2": dict(BASE, arch=3, n_heads=4, n_kv_heads=2, head_dim=256, attn_softcap=2.0,
                            final_softcap=0.5, seed=45),
    "gemma_hd256_g8": dict(BASE, arch=2, n_heads=8, n_kv_heads=1, head_dim=256, seed=46),
    "gemma2_hd256_g4": dict(BASE, arch=3, n_heads=8, n_kv_heads=2, head_dim=256, seed=47),
}


def _file(tmp_path, name):
    path = str(tmp_path / (name + ".gguf"))
    api.write_synthetic_gguf(path, api.SynthSpec(**SPECS[name]))
    return path


# Steps at which the oracle's fp16 cache rounds a K/V value across a binary16
# midpoint the other way than exact arithmetic does ((spec, kv, step) ->
# (oracle bar, reason)); every other step holds the oracle bar (OracleBar).
KNOWN = {}


def _run(path, kv, launch, prompt, steps, max_ctx=128, spec=""):
    om = oracle.Model(path, max_ctx, kv)
    rm = RefModel(path, max_ctx, kv)
    tol = TOL if kv == "f16" else TOL_INT8
    bar = OracleBar("gemma %s %s %s" % (spec, launch, kv), tol,
                    {k[2]: v for k, v in KNOWN.items() if k[:2] == (spec, kv)})
    L = api._lib()
    changes = []
    with api.Model(path, max_context=max_ctx, kv=kv, launch=launch) as m:
        want = api.LAUNCH["eager"] if launch == "eager" else api.LAUNCH["graph"]
        assert L.ss_hip_model_launch(L.ss_model_hip(m.h)) == want
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        bar.check("prompt", lg, olg, rm.prefill(prompt, 0))
        assert am == oracle.argmax(olg)
        tok, pos, prev = am, len(prompt), olg
        for _ in range(steps):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            bar.check(pos, lg, olg, rm.forward(tok, pos))
            assert am == oracle.argmax(olg), pos
            changes.append(rel_err(olg, prev))
            tok, pos, prev = am, pos + 1, olg
    om.close()
    bar.report()
    return changes


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("launch", ["graph", "eager", "sweep"])
@pytest.mark.parametrize("spec", sorted(SPECS))
def test_greedy_and_logits(tmp_path, spec, launch, kv):
    print("gemma model", spec, launch, kv, flush=True)
    path = _file(tmp_path, spec)
    prompt = np.random.default_rng(7).integers(3, SPECS[spec]["vocab"], 9).tolist()
    changes = _run(path, kv, launch, prompt, 12, spec=spec)
    assert np.median(changes) >= 10 * TOL     # the model responds to its input


@pytest.mark.parametrize("spec", ["gemma_hd256_mha", "gemma2_hd256_g2", "gemma2_softcap"])
def test_long_context_split_merge(tmp_path, spec):
    """A 1024-position context gives more than 8 attention splits per KV head
    (16 at head_dim 256, group 1), so the last split of each KV head merges;
    K/V injected to 600 positions, then decode steps against the oracle."""
    path = _file(tmp_path, spec)
    print("gemma long context", spec, flush=True)
    kw = SPECS[spec]
    n_pre, ctx = 600, 1024
    kvdim = kw["n_kv_heads"] * kw["head_dim"]
    rng = np.random.default_rng(600)
    om = oracle.Model(path, ctx, "f16")
    with api.Model(path, max_context=ctx, kv="f16") as m:
        for layer in range(kw["n_layers"]):
            k = (0.5 * rng.standard_normal((n_pre, kvdim))).astype(np.float16).view(np.uint16)
            v = rng.standard_normal((n_pre, kvdim)).astype(np.float16).view(np.uint16)
            m.kv_write(layer, 0, k, v)
            for p in range(n_pre):
                om.kv_write(layer, p, k[p], v[p])
        tok, pos = 11, n_pre
        for _ in range(6):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            assert rel_err(lg, olg) <= TOL, pos
            assert am == oracle.argmax(olg), pos
            tok, pos = am, pos + 1
    om.close()


def test_streaming_matches_resident(tmp_path):
    """Post norms and the Gemma scales in streaming mode: logits bit-identical
    to the resident model's."""
    path = _file(tmp_path, "gemma2_hd256_g4")
    prompt = np.random.default_rng(5).integers(3, 600, 8).tolist()
    runs = []
    for streaming in (False, True):
        print("gemma streaming", streaming, flush=True)
        with api.Model(path, max_context=64, streaming=streaming) as m:
            out = [m.eval_prompt(prompt, 0)]
            tok, pos = out[0][1], len(prompt)
            for _ in range(6):
                lg, am = m.eval_token(tok, pos)
                out.append((lg.copy(), am))
                tok, pos = am, pos + 1
        runs.append(out)
    for i, ((a, ia), (b, ib)) in enumerate(zip(*runs)):
        assert np.array_equal(a, b), i
        assert ia == ib, i


@pytest.mark.parametrize("spec", ["gemma2_softcap", "gemma_hd256_g8"])
def test_embed_matches_oracle(tmp_path, spec):
    """ss_embed (layer_scheduler.c:805-911): the (1 + w) final norm on every
    token, mean pool, L2 normalise."""
    path = _file(tmp_path, spec)
    toks = [5, 77, 300, 12, 9, 41, 133]
    om = oracle.Model(path, 64)
    want = om.embed(toks)
    om.close()
    L = api._lib()
    t = np.array(toks, np.int32)
    got = np.zeros(SPECS[spec]["hidden"], np.float32)
    with api.Model(path, max_context=64) as m:
        assert L.ss_hip_embed(L.ss_model_hip(m.h), t.ctypes.data_as(C.POINTER(C.c_int32)), t.size,
                              got.ctypes.data_as(C.POINTER(C.c_float))) == 0, L.ss_hip_last_error()
    assert abs(np.linalg.norm(got) - 1.0) < 1e-4
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("spec", ["gemma2_hd256_g4", "gemma2_softcap", "gemma_hd256_g8"])
def test_long_prompt_as_products(tmp_path, spec):
    """A 300-token prompt through the Gemma prompt products (fp16 cache),
    against the oracle's token-serial prefill, then decode steps."""
    path = _file(tmp_path, spec)
    print("gemma long prompt", spec, flush=True)
    prompt = np.random.default_rng(12).integers(3, SPECS[spec]["vocab"], 300).tolist()
    om = oracle.Model(path, 400, "f16")
    rm = RefModel(path, 400, "f16")
    bar = OracleBar("gemma long prompt %s" % spec, TOL,
                    {k[2]: v for k, v in KNOWN.items() if k[:2] == (spec + " long", "f16")})
    with api.Model(path, max_context=400) as m:
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
