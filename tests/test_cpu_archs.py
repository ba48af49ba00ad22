"""CPU pins of the architecture branches beyond the plain llama block.

The reference takes them by tensor name or by architecture string
(SlipStream/src/core/layer_scheduler.c): fused attn_qkv (:337-347), fused
ffn_up = [gate; up] (:518-524), q/k/v biases in F32 or F16 (:367-402 with
safe_load_f32 :284-289), and NeoX RoPE pairs for qwen/falcon/phi/deepseek
(:144-149, tensor.c:223-248). The oracle restates each; these tests pin that
restatement (and the synthetic writer's variants) without a GPU:

* NeoX RoPE equals the GPT-J branch applied to each head in the order where
  unit 2i holds i and unit 2i+1 holds i + rope_dim/2: the identity the HIP
  path is built on (it runs NeoX models as GPT-J ones with Wq/Wk rows in that
  order).
* A fused file holds byte-for-byte the parts of the plain file with the same
  seed, and the oracle's fused branch gives bit-identical logits.
* A bias of zero changes nothing (x + 0 = x); an F16 bias equals the F32 bias
  of its widened values; a qwen2 file and a llama file with the same weights
  agree at position 0 (RoPE is the identity there) and differ after it.
"""
import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.test_cpu_host import BLOCK, parse_gguf, tiny_spec


def neox_perm(n_units, hd, rope_dim):
    """Source index of each unit in the NeoX-as-adjacent-pairs head order."""
    half = rope_dim // 2
    u = np.arange(n_units)
    h, p = u // hd, u % hd
    src = np.where(p < 2 * half, np.where(p & 1, p // 2 + half, p // 2), p)
    return h * hd + src


@pytest.mark.parametrize("hd,rope_dim", [(16, 16), (64, 64), (64, 32), (128, 128)])
@pytest.mark.parametrize("pos", [0, 1, 7, 300, 4095])
def test_neox_rope_is_gptj_rope_of_reordered_heads(hd, rope_dim, pos):
    rng = np.random.default_rng(pos + hd)
    H, KVH, theta = 4, 2, 1e6
    q = rng.standard_normal(H * hd).astype(np.float32)
    k = rng.standard_normal(KVH * hd).astype(np.float32)
    qn, kn = oracle.rope(q, k, H, KVH, hd, rope_dim, pos, theta, neox=True)
    pq, pk = neox_perm(H * hd, hd, rope_dim), neox_perm(KVH * hd, hd, rope_dim)
    qg, kg = oracle.rope(q[pq], k[pk], H, KVH, hd, rope_dim, pos, theta, neox=False)
    assert np.array_equal(qn[pq], qg) and np.array_equal(kn[pk], kg)
    # attention scores only see q.k within a head: the order changes none of them
    for h in range(H):
        kv = h // (H // KVH)
        a = np.dot(qn[h * hd:(h + 1) * hd].astype(np.float64), kn[kv * hd:(kv + 1) * hd])
        b = np.dot(qg[h * hd:(h + 1) * hd].astype(np.float64), kg[kv * hd:(kv + 1) * hd])
        assert a == pytest.approx(b, rel=1e-12)
    if pos == 0:
        assert np.array_equal(qn, q) and np.array_equal(kn, k)


def _tensors(path):
    _, meta, tensors, data, raw = parse_gguf(path)
    out = {}
    for name, dims, t, off in tensors:
        per, nb = BLOCK[t]
        n = int(np.prod(dims))
        out[name] = (dims, t, raw[data + off:data + off + n // per * nb])
    return meta, out, data, raw


def _trace(path, steps=3, prompt=(5, 17, 42, 7, 299)):
    m = oracle.Model(path, 64)
    try:
        logits = [m.prefill(list(prompt))]
        pos = len(prompt)
        for _ in range(steps):
            logits.append(m.forward(oracle.argmax(logits[-1]), pos))
            pos += 1
        return np.stack(logits)
    finally:
        m.close()


@pytest.mark.parametrize("arch", [0, 1])
@pytest.mark.parametrize("fq,fu", [(1, 0), (0, 1), (1, 1)])
def test_fused_files_hold_the_plain_weights_and_give_the_same_logits(tmp_path, arch, fq, fu):
    plain, fused = str(tmp_path / "p.gguf"), str(tmp_path / "f.gguf")
    api.write_synthetic_gguf(plain, tiny_spec(arch=arch))
    api.write_synthetic_gguf(fused, tiny_spec(arch=arch, fused_qkv=fq, fused_up=fu))
    mp, tp, _, _ = _tensors(plain)
    mf, tf, _, _ = _tensors(fused)
    assert mf["general.architecture"] == ("qwen2" if arch else "llama")
    for l in range(2):
        b = "blk.%d." % l
        if fq:
            dims, t, data = tf[b + "attn_qkv.weight"]
            assert dims == [64, 64 + 2 * 32] and not any(b + n in tf for n in ("attn_q.weight", "attn_k.weight"))
            assert data == tp[b + "attn_q.weight"][2] + tp[b + "attn_k.weight"][2] + tp[b + "attn_v.weight"][2]
        if fu:
            dims, t, data = tf[b + "ffn_up.weight"]
            assert dims == [64, 2 * 96] and b + "ffn_gate.weight" not in tf
            assert data == tp[b + "ffn_gate.weight"][2] + tp[b + "ffn_up.weight"][2]
    for name in tf:
        if name in tp and not (fu and name.endswith("ffn_up.weight")):
            assert tf[name][2] == tp[name][2], name
    assert np.array_equal(_trace(plain), _trace(fused))


def _patch(path, out, name, values):
    meta, t, data, raw = _tensors(path)
    _, _, tensors, _, _ = parse_gguf(path)
    off = [o for n, _, _, o in tensors if n == name][0]
    b = bytearray(raw)
    v = np.ascontiguousarray(values).tobytes()
    b[data + off:data + off + len(v)] = v
    open(out, "wb").write(bytes(b))


def test_qkv_bias_zero_is_no_bias_and_f16_is_widened_f32(tmp_path):
    plain, f32, f16 = (str(tmp_path / n) for n in ("p.gguf", "b32.gguf", "b16.gguf"))
    api.write_synthetic_gguf(plain, tiny_spec(arch=1))
    api.write_synthetic_gguf(f32, tiny_spec(arch=1, qkv_bias=1))
    api.write_synthetic_gguf(f16, tiny_spec(arch=1, qkv_bias=2))
    _, tp, _, _ = _tensors(plain)
    _, t32, _, _ = _tensors(f32)
    _, t16, _, _ = _tensors(f16)
    for name in tp:
        assert t32[name][2] == tp[name][2] and t16[name][2] == tp[name][2], name
    sizes = {"attn_q.bias": 64, "attn_k.bias": 32, "attn_v.bias": 32}
    zero, wide = str(tmp_path / "z.gguf"), str(tmp_path / "w.gguf")
    open(zero, "wb").write(open(f32, "rb").read())
    open(wide, "wb").write(open(f32, "rb").read())
    for l in range(2):
        for sfx, n in sizes.items():
            name = "blk.%d.%s" % (l, sfx)
            assert t32[name][0] == [n] and t32[name][1] == 0 and t16[name][1] == 1
            v32 = np.frombuffer(t32[name][2], np.float32)
            v16 = np.frombuffer(t16[name][2], np.float16)
            assert 0.03 < v32.std() < 0.3
            assert np.array_equal(v32.astype(np.float16), v16)   # the same draws, rounded to binary16
            _patch(zero, zero, name, np.zeros(n, np.float32))
            _patch(wide, wide, name, v16.astype(np.float32))
    base = _trace(plain)
    assert np.array_equal(_trace(zero), base)
    assert not np.allclose(_trace(f32), base, rtol=1e-3, atol=1e-4)
    assert np.array_equal(_trace(f16), _trace(wide))


def test_qwen2_and_llama_agree_at_position_zero_only(tmp_path):
    llama, qwen = str(tmp_path / "l.gguf"), str(tmp_path / "q.gguf")
    api.write_synthetic_gguf(llama, tiny_spec(arch=0))
    api.write_synthetic_gguf(qwen, tiny_spec(arch=1))
    _, tl, _, _ = _tensors(llama)
    _, tq, _, _ = _tensors(qwen)
    assert all(tq[n][2] == tl[n][2] for n in tl)
    ml, mq = oracle.Model(llama, 16), oracle.Model(qwen, 16)
    try:
        assert np.array_equal(ml.forward(11, 0), mq.forward(11, 0))
        assert not np.allclose(ml.forward(12, 1), mq.forward(12, 1), rtol=1e-3, atol=1e-4)
    finally:
        ml.close()
        mq.close()


def test_gemma_files_hold_the_llama_matrices(tmp_path):
    """arch 3 ("gemma2") changes no matrix of the llama file with the same
    seed; its norm weights are the llama ones minus one (the format's 1 + w),
    and it adds the two post norms per layer and the softcap keys."""
    plain, gem = str(tmp_path / "p.gguf"), str(tmp_path / "g.gguf")
    api.write_synthetic_gguf(plain, tiny_spec())
    api.write_synthetic_gguf(gem, tiny_spec(arch=3, attn_softcap=50.0, final_softcap=30.0))
    mp, tp, _, _ = _tensors(plain)
    mg, tg, _, _ = _tensors(gem)
    assert mg["general.architecture"] == "gemma2"
    assert mg["gemma2.attn_logit_softcapping"] == 50.0 and mg["gemma2.final_logit_softcapping"] == 30.0
    for name, (dims, t, data) in tp.items():
        if name.endswith("norm.weight"):
            lw = np.frombuffer(data, np.float32)
            gw = np.frombuffer(tg[name][2], np.float32)
            assert np.max(np.abs((gw + np.float32(1)) - lw)) <= 2.4e-7, name
        else:
            assert tg[name][2] == data, name
    for l in range(2):
        for n in ("post_attention_norm.weight", "post_ffw_norm.weight"):
            dims, t, data = tg["blk.%d.%s" % (l, n)]
            w = np.frombuffer(data, np.float32)
            assert t == 0 and dims == [64] and abs(float(np.mean(w))) < 0.01 and 0 < np.std(w) < 0.02


def test_huge_softcaps_change_nothing_and_small_ones_do(tmp_path):
    """cap * tanh(x / cap) -> x as cap grows: llama logits with caps of 1e6
    equal the uncapped ones to fp32 rounding; caps of the scores' size move
    them (tensor.c:194-200 applied at layer_scheduler.c:446-448, 674-676)."""
    paths = {}
    for name, kw in (("none", {}), ("huge", dict(attn_softcap=1e6, final_softcap=1e6)),
                     ("small", dict(attn_softcap=0.5, final_softcap=0.5))):
        paths[name] = str(tmp_path / (name + ".gguf"))
        api.write_synthetic_gguf(paths[name], tiny_spec(**kw))
    base, huge, small = (_trace(paths[n]) for n in ("none", "huge", "small"))
    assert np.max(np.abs(huge - base)) <= 1e-5 * np.max(np.abs(base))
    assert np.max(np.abs(small)) <= 0.5
    assert np.max(np.abs(small - base)) > 0.1 * np.max(np.abs(base))
