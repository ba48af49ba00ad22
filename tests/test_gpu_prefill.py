"""Prompts as matrix products: with an fp16 cache, ss_eval_prompt runs a
prompt of 8 or more tokens through each layer as MFMA products over chunks of
up to 512 tokens (ss_scheduler_prefill, layer_scheduler.c:681-803, evaluates
a prompt layer by layer with one matvec per token and matrix).

Bar, as for decode: last-token logits within max |gpu - oracle| / max |oracle|
<= 1e-3 of the CPU oracle, identical argmax, and identical greedy tokens for
the decode steps that read the cache the prompt wrote.
"""
import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.test_gpu_model import GQA8, TINY, TINY_Q8, TOL, _model_file
from tests.conftest import sweep_optin
from tests.util import rel_err

pytestmark = pytest.mark.gpu
SPECS = {"tiny": TINY, "tiny_q8": TINY_Q8, "gqa8": GQA8}


def _decode_against(m, om, tok, pos, steps):
    for _ in range(steps):
        lg, am = m.eval_token(tok, pos)
        olg = om.forward(tok, pos)
        assert rel_err(lg, olg) <= TOL, pos
        assert am == oracle.argmax(olg), pos
        tok, pos = am, pos + 1


@pytest.mark.parametrize("launch", ["graph", "sweep"])
@pytest.mark.parametrize("spec", ["tiny", "tiny_q8", "gqa8"])
def test_batched_prompt_matches_oracle(spec, launch):
    """A 600-token prompt (two chunks: 512 + 88), then a 30-token prompt that
    continues it at position 600, then decode steps."""
    if launch == "sweep":
        sweep_optin(spec == "gqa8")
    kw = SPECS[spec]
    path = _model_file(spec, **kw)
    print("prefill", spec, launch, flush=True)
    rng = np.random.default_rng(21)
    p1 = rng.integers(3, kw["vocab"], 600).tolist()
    p2 = rng.integers(3, kw["vocab"], 30).tolist()
    om = oracle.Model(path, 1024, "f16")
    with api.Model(path, max_context=1024, launch=launch) as m:
        lg, am = m.eval_prompt(p1, 0)
        olg = om.prefill(p1, 0)
        assert rel_err(lg, olg) <= TOL
        assert am == oracle.argmax(olg) == int(np.argmax(lg))
        lg, am = m.eval_prompt(p2, len(p1))
        olg = om.prefill(p2, len(p1))
        assert rel_err(lg, olg) <= TOL
        assert am == oracle.argmax(olg)
        _decode_against(m, om, am, len(p1) + len(p2), 12)
    om.close()


@pytest.mark.parametrize("n", [1, 7, 8, 63, 64, 65])
def test_batched_prompt_sizes(n):
    """Chunk edges of the 64-token product tile, and the threshold: every
    size forced through the products (threshold 1) against the oracle."""
    path = _model_file("gqa8", **GQA8)
    rng = np.random.default_rng(100 + n)
    prompt = rng.integers(3, GQA8["vocab"], n).tolist()
    om = oracle.Model(path, 256, "f16")
    with api.Model(path, max_context=256) as m:
        m.set_prompt_batch(1)
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        assert rel_err(lg, olg) <= TOL
        assert am == oracle.argmax(olg)
        _decode_against(m, om, am, n, 6)
    om.close()


def test_batched_equals_token_by_token():
    """The same prompt through the products and token by token: the same
    greedy continuation, logits within the decode tolerance of each other."""
    path = _model_file("gqa8", **GQA8)
    rng = np.random.default_rng(5)
    prompt = rng.integers(3, GQA8["vocab"], 100).tolist()
    out = {}
    for batch in (0, -1):
        with api.Model(path, max_context=256) as m:
            m.set_prompt_batch(batch)
            lg, am = m.eval_prompt(prompt, 0)
            out[batch] = (lg, am, m.decode_greedy(20))
    (lb, ab, tb), (lt, at, tt) = out[0], out[-1]
    assert rel_err(lb, lt) <= TOL
    assert ab == at and tb == tt


@pytest.mark.parametrize("mode", ["products", "token_by_token", "int8"])
def test_embed_prompt_matches_oracle(mode):
    """ss_embed (ss_scheduler_embed, layer_scheduler.c:805-911): every
    token's final hidden state through the output norm, mean-pooled, L2
    normalised; a text of a few hundred tokens through the products, token
    by token, and with the int8 cache."""
    import ctypes as C
    path = _model_file("gqa8", **GQA8)
    text = " ".join("word%d, and the PhoneMap index %d;" % (i, i * 7) for i in range(30))
    kv = "int8" if mode == "int8" else "f16"
    L = api._lib()
    libc = C.CDLL(None)
    libc.free.argtypes = [C.c_void_p]
    with api.Model(path, max_context=1024, kv=kv) as m:
        if mode == "token_by_token":
            m.set_prompt_batch(-1)
        toks = m.tokenize(text)
        assert 100 <= len(toks) <= 1024
        out = C.POINTER(C.c_float)()
        dim = C.c_uint32(0)
        assert L.ss_embed(m.h, text.encode(), C.byref(out), C.byref(dim)) == 0
        got = np.ctypeslib.as_array(out, (dim.value,)).copy()
        libc.free(C.cast(out, C.c_void_p))
    om = oracle.Model(path, 1024, kv)
    want = om.embed(toks)
    om.close()
    assert abs(np.linalg.norm(got) - 1.0) < 1e-5
    assert rel_err(got, want) <= (TOL if kv == "f16" else 5e-2)


# Two layers at the Llama-2-70B layer shape (d 8192, 64 query heads and 8 KV
# heads of dim 128, FFN 28672), all Q4_0, with a small vocabulary so that the
# oracle's prompt takes seconds.
W70 = dict(n_layers=2, hidden=8192, n_heads=64, n_kv_heads=8, head_dim=128, ffn=28672, vocab=512,
           context_length=1024, seed=71, scale_mode=1)
# ss_hip_gemm_launch_counts slots: 2 * epilogue (store, add, SwiGLU) + rows per wave - 1
ADD_RG2 = 3


def _gemm_counts():
    import ctypes as C
    L = api._lib()
    out = (C.c_int64 * 6)()
    assert L.ss_hip_gemm_launch_counts(out, 6) == 0
    return list(out)


@pytest.mark.timeout(600)
def test_prompt_at_70b_layer_width():
    """A 600-token prompt (chunks of 512 and 88 tokens) through two layers of
    the 70B shape, then 8 greedy steps: every logit vector within 1e-3 of the
    oracle's prefill / forward (layer_scheduler.c:681-803, :571-679), the
    argmax equal, and the model responding to its input (the step-to-step
    guard of the full-shape tests). At d = 8192 and 512 tokens the Wo and
    down products run with two row groups per wave (k_gemm_h EPI_ADD, RG 2),
    which no smaller shape selects; the launch counters show that they ran."""
    from tests.test_gpu_fullshape import Trace
    path = _model_file("w70", **W70)
    rng = np.random.default_rng(700)
    prompt = rng.integers(3, W70["vocab"], 600).tolist()
    ctx = len(prompt) + 9
    print("prefill w70 600 tokens", flush=True)
    om = oracle.Model(path, ctx, "f16")
    tr = Trace("w70")
    with api.Model(path, max_context=ctx) as m:
        before = _gemm_counts()
        lg, am = m.eval_prompt(prompt, 0)
        after = _gemm_counts()
        olg = om.prefill(prompt, 0)
        tr.step(-1, lg, am, olg)
        tok, pos = am, len(prompt)
        for i in range(8):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            tr.step(i, lg, am, olg)
            tok, pos = am, pos + 1
    om.close()
    tr.done()
    ran = after[ADD_RG2] - before[ADD_RG2]
    print("k_gemm_h EPI_ADD RG=2 launches during the prompt:", ran, flush=True)
    assert ran >= 2 * W70["n_layers"], (before, after)
