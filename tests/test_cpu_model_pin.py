"""Pins the oracle's whole-model functions (orc_prefill, orc_forward,
orc_embed) against tests/ref_model.py, an fp64 numpy restatement written
from SlipStream/src/core/layer_scheduler.c:291-911 over the independent
Python GGUF parser: the two share no code, so a mistake in the oracle's
wiring (a norm weight on the wrong matvec, a wrong KV head for a query head,
a rope pair mix-up, a fused tensor split at the wrong row, a bias on the
wrong projection, a Gemma branch missing or misplaced) shows as an O(1)
difference.

Bars (measured worst cases in brackets): the int8 cache rounds K/V to one
of 255 levels per (layer, position), coarse enough that fp32 and fp64 land
on the same codes, and logits agree to 2e-5 of max|logit| [1.4e-6]. The
fp16 cache rounds each K/V element to binary16, and an element within fp32
rounding of a binary16 rounding boundary goes the other way in fp64 (a
one-ulp, 2^-11 relative, step): those steps move the logits by up to
~1e-4, so the fp16 bar is 5e-4 [1.6e-4]. The argmax must match at every
step.

Self-check: mis-wired copies of the fp64 model (query heads mapped to the
wrong KV head, attention and FFN norm weights swapped, no RoPE on K) must
miss the oracle by more than 20 times the looser bar; they miss it by
4.7e-2 to 1.8.
"""
import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.ref_model import RefModel

BAR = {"f16": 5e-4, "int8": 2e-5}


def _spec(**kw):
    s = dict(n_layers=2, hidden=256, n_heads=8, n_kv_heads=2, head_dim=32, ffn=512, vocab=400,
             context_length=128, seed=21, layer_type=2, embd_type=8, out_type=8, scale_mode=1)
    s.update(kw)
    return api.SynthSpec(**s)


VARIANTS = {
    "llama_gqa": {},
    "tied_q8": dict(layer_type=8, embd_type=8, out_type=-1, seed=22),
    "legacy_scales": dict(scale_mode=0, seed=23),
    "fused_qkv_up": dict(fused_qkv=1, fused_up=1, seed=24),
    "qwen2_f32_bias": dict(arch=1, qkv_bias=1, seed=25),
    "qwen2_f16_bias_fused": dict(arch=1, qkv_bias=2, fused_qkv=1, seed=26),
    "mha_hd64": dict(n_heads=4, n_kv_heads=4, head_dim=64, seed=27),
    "q4_k": dict(layer_type=12, embd_type=12, out_type=12, seed=28),
    "q2_k_q6_head": dict(layer_type=10, embd_type=10, out_type=14, seed=34),
    "q3_k_q5_head": dict(layer_type=11, embd_type=13, out_type=13, seed=35),
    "q5_k": dict(layer_type=13, embd_type=14, out_type=-1, seed=36),
    "q6_k": dict(layer_type=14, embd_type=14, out_type=14, seed=37),
    # the other 32-weight block types and float matrices (quantize.c:74-176)
    "q4_1_q8_1_head": dict(layer_type=3, embd_type=3, out_type=9, seed=38),
    "q5_0_f16_head": dict(layer_type=6, embd_type=6, out_type=1, seed=39),
    "q5_1_tied": dict(layer_type=7, embd_type=7, out_type=-1, seed=40),
    "f16": dict(layer_type=1, embd_type=1, out_type=1, seed=41),
    "f32_q8_1": dict(layer_type=0, embd_type=9, out_type=0, seed=42),
    # tokenizer shorter than the tables: the vocabulary is clamped to it
    "padded_tied": dict(embd_type=2, out_type=-1, vocab_tokens=360, seed=29),
    "padded_out": dict(vocab_tokens=370, seed=30),
    # Gemma: (1 + w) norms, sqrt(d) embedding, GeGLU, 1/sqrt(d) logits, tied head
    "gemma": dict(arch=2, embd_type=8, out_type=-1, seed=31),
    # Gemma 2: post norms, and softcaps small enough to bend the scores and logits
    "gemma2_softcap": dict(arch=3, embd_type=8, out_type=-1, attn_softcap=1.5, final_softcap=0.4, seed=32),
    # the softcaps apply to any architecture that sets the keys
    "llama_softcap": dict(attn_softcap=1.0, final_softcap=3.0, seed=33),
}


def _err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def _run(path, kv, ref):
    """Prompt, then 6 greedy steps; returns the worst error and whether every
    argmax matched."""
    om = oracle.Model(path, 64, kv)
    rng = np.random.default_rng(3)
    prompt = rng.integers(3, ref.vocab, 9).tolist()
    worst, same = 0.0, True
    olg = om.prefill(prompt, 0)
    rlg = ref.prefill(prompt, 0)
    worst = max(worst, _err(olg, rlg))
    same &= oracle.argmax(olg) == int(np.argmax(rlg))
    tok, pos = oracle.argmax(olg), len(prompt)
    for _ in range(6):
        olg = om.forward(tok, pos)
        rlg = ref.forward(tok, pos)
        worst = max(worst, _err(olg, rlg))
        same &= oracle.argmax(olg) == int(np.argmax(rlg))
        tok, pos = oracle.argmax(olg), pos + 1
    om.close()
    return worst, same


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_oracle_forward_and_prefill_match_fp64_restatement(tmp_path, name, kv):
    path = str(tmp_path / (name + ".gguf"))
    api.write_synthetic_gguf(path, _spec(**VARIANTS[name]))
    ref = RefModel(path, 64, kv)
    worst, same = _run(path, kv, ref)
    assert worst <= BAR[kv], worst
    assert same


@pytest.mark.parametrize("name", ["padded_tied", "padded_out"])
def test_vocab_clamped_to_the_tokenizer(tmp_path, name):
    """layer_scheduler.c:186-197: the vocabulary is the tokenizer's size when
    the embedding/output tables have more rows; logits cover it only."""
    path = str(tmp_path / (name + ".gguf"))
    api.write_synthetic_gguf(path, _spec(**VARIANTS[name]))
    ref = RefModel(path, 64)
    assert ref.vocab == VARIANTS[name]["vocab_tokens"] < ref.embd.shape[0] == 400
    om = oracle.Model(path, 64)
    assert om.forward(5, 0).shape == (ref.vocab,)
    om.close()


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("name", ["llama_gqa", "qwen2_f16_bias_fused", "gemma2_softcap"])
def test_oracle_embed_matches_fp64_restatement(tmp_path, name, kv):
    path = str(tmp_path / (name + ".gguf"))
    api.write_synthetic_gguf(path, _spec(**VARIANTS[name]))
    ref = RefModel(path, 64, kv)
    toks = [5, 77, 300, 12, 9, 41, 133]
    om = oracle.Model(path, 64, kv)
    got = om.embed(toks)
    om.close()
    want = ref.embed(toks)
    assert abs(np.linalg.norm(got) - 1.0) < 1e-5
    assert _err(got, want) <= BAR[kv]


def test_fp64_restatement_detects_miswiring(tmp_path):
    """The comparison above discriminates: mis-wired copies of the fp64 model
    disagree with the oracle far beyond the bar."""
    path = str(tmp_path / "m.gguf")
    api.write_synthetic_gguf(path, _spec())
    ref = RefModel(path, 64, "f16")

    class WrongKvHead(RefModel):
        def layer(self, l, x, pos):
            # query head h reads KV head (h + 1) % KVH instead of h / (H / KVH)
            ly = self.layers[l]
            wk, wv = ly["wk"], ly["wv"]
            hd = self.hd
            perm = np.concatenate([np.arange(((k + 1) % self.KVH) * hd, ((k + 1) % self.KVH + 1) * hd)
                                   for k in range(self.KVH)])
            ly2 = dict(ly, wk=wk[perm], wv=wv[perm])
            self.layers[l] = ly2
            try:
                return RefModel.layer(self, l, x, pos)
            finally:
                self.layers[l] = ly

    class SwappedNorms(RefModel):
        def layer(self, l, x, pos):
            ly = self.layers[l]
            self.layers[l] = dict(ly, attn_norm=ly["ffn_norm"], ffn_norm=ly["attn_norm"])
            try:
                return RefModel.layer(self, l, x, pos)
            finally:
                self.layers[l] = ly

    class NoRopeOnK(RefModel):
        def rope(self, v, n_heads, pos):
            return v if n_heads == self.KVH else RefModel.rope(self, v, n_heads, pos)

    good, _ = _run(path, "f16", ref)
    assert good <= BAR["f16"]
    for cls in (WrongKvHead, SwappedNorms, NoRopeOnK):
        bad, _ = _run(path, "f16", cls(path, 64, "f16"))
        assert bad > 20 * BAR["f16"], (cls.__name__, bad)


def test_fp64_restatement_detects_gemma_miswiring(tmp_path):
    """The Gemma branches are each visible: dropping any one of them from
    the fp64 model (SiLU for GeGLU, no post norms, no softcaps, w for 1 + w)
    misses the oracle by far more than the bar."""
    path = str(tmp_path / "g.gguf")
    api.write_synthetic_gguf(path, _spec(**VARIANTS["gemma2_softcap"]))

    class SiluNotGelu(RefModel):
        def ffn_act(self, gt, up):
            return up * (gt / (1.0 + np.exp(-gt)))

    class NoPostNorms(RefModel):
        def layer(self, l, x, pos):
            ly = self.layers[l]
            self.layers[l] = dict(ly, post_attn=None, post_ffn=None)
            try:
                return RefModel.layer(self, l, x, pos)
            finally:
                self.layers[l] = ly

    class NoSoftcaps(RefModel):
        def softcap(self, x, cap):
            return x

    class PlainNorms(RefModel):
        def rmsnorm(self, x, w, gemma=None):
            return RefModel.rmsnorm(self, x, w, gemma=False)

    good, _ = _run(path, "f16", RefModel(path, 64, "f16"))
    assert good <= BAR["f16"]
    for cls in (SiluNotGelu, NoPostNorms, NoSoftcaps, PlainNorms):
        bad, _ = _run(path, "f16", cls(path, 64, "f16"))
        assert bad > 20 * BAR["f16"], (cls.__name__, bad)


@pytest.mark.parametrize("kv", ["f16", "int8"])
@pytest.mark.parametrize("name", ["llama_gqa", "tied_q8", "fused_qkv_up", "qwen2_f16_bias_fused", "gemma2_softcap"])
def test_batched_prefill_is_bit_identical_to_token_serial(tmp_path, name, kv):
    """orc_prefill runs each layer's tokens together (rows dequantised once);
    orc_prefill_serial is the reference's token-by-token loop
    (layer_scheduler.c:721-755). Logits, the cache they leave and the decode
    steps after them agree bit for bit."""
    path = str(tmp_path / (name + ".gguf"))
    api.write_synthetic_gguf(path, _spec(**VARIANTS[name]))
    rng = np.random.default_rng(5)
    prompt = rng.integers(3, 400, 23).tolist()
    runs = []
    for serial in (False, True):
        om = oracle.Model(path, 64, kv)
        first = om.prefill_serial(prompt[:17], 0) if serial else om.prefill(prompt[:17], 0)
        second = om.prefill_serial(prompt[17:], 17) if serial else om.prefill(prompt[17:], 17)
        steps = [om.forward(t, 23 + i).copy() for i, t in enumerate([7, 99, 250])]
        runs.append([first, second] + steps)
        om.close()
    for a, b in zip(*runs):
        assert np.array_equal(a, b)
