"""An fp64 numpy restatement of the reference's model functions, written from
SlipStream/src/core/layer_scheduler.c (not from the oracle's C), over GGUF
files read by the independent Python parser of tests/test_cpu_host.py and
dequantised by tests/util.dequant_np.

It pins the oracle's whole-model functions: orc_forward
(ss_scheduler_forward, layer_scheduler.c:571-679, with process_layer
:291-567), orc_prefill (ss_scheduler_prefill :681-803) and orc_embed
(ss_scheduler_embed :805-911), with the Gemma branches: the (1 + w) norm
(tensor.c:133-152), the sqrt(d) embedding and 1/sqrt(d) logit scales
(:597-602, 667-672), GeGLU (:529-531, tensor.c:181-190), the post norms
(:474-481, 553-560) and the softcaps (:446-448, 674-676, tensor.c:194-200). Everything is computed in fp64 apart from the
two KV cache encodings, which round as the reference stores: binary16 for
the fp16 cache, and the absmax int8 codes of kv_turboquant_encode
(:101-118, one scale per (layer, position) over all KV heads) for the int8
cache. Structural mistakes (a norm weight on the wrong matvec, a wrong
kv_head = h / heads_per_kv, a transposed matrix, a rope pair mix-up) change
the logits at O(1); fp32 rounding changes them at ~1e-6.

Test infrastructure only.
"""
import numpy as np

from tests.test_cpu_host import parse_gguf
from tests.util import B32_BYTES, KQ_BYTES, dequant_np

NEOX_ARCHS = ("qwen", "falcon", "phi", "deepseek")       # layer_scheduler.c:144-149


def _vector(raw, data, dims, ttype, off):
    n = int(np.prod(dims))
    o = data + off
    if ttype == 0:
        return np.frombuffer(raw, np.float32, n, o).astype(np.float64)
    if ttype == 1:
        return np.frombuffer(raw, np.float16, n, o).astype(np.float64)
    raise ValueError("vector type %d" % ttype)


def _matrix(raw, data, dims, ttype, off):
    cols, rows = int(dims[0]), int(dims[1])
    if ttype in (0, 1):
        return _vector(raw, data, dims, ttype, off).reshape(rows, cols)
    nbytes = rows * cols // 256 * KQ_BYTES[ttype] if ttype in KQ_BYTES else rows * (cols // 32) * B32_BYTES[ttype]
    blocks = np.frombuffer(raw, np.uint8, nbytes, data + off)
    return dequant_np(blocks, rows, cols, ttype)


class RefModel:
    def __init__(self, path, max_seq, kv="f16"):
        _, meta, tensors, data, raw = parse_gguf(path)
        arch = meta["general.architecture"]
        self.neox = any(s in arch for s in NEOX_ARCHS)
        self.gemma = "gemma" in arch                                   # :152-155
        g = lambda k, dflt=None: meta.get("%s.%s" % (arch, k), dflt)
        self.attn_softcap = float(g("attn_logit_softcapping", 0.0))
        self.final_softcap = float(g("final_logit_softcapping", 0.0))
        self.L = int(g("block_count"))
        self.d = int(g("embedding_length"))
        self.H = int(g("attention.head_count"))
        self.KVH = int(g("attention.head_count_kv", 0)) or self.H
        self.ffn = int(g("feed_forward_length"))
        self.eps = float(g("attention.layer_norm_rms_epsilon", 1e-5))
        self.theta = float(g("rope.freq_base", 10000.0))
        info = {name: (dims, t, off) for name, dims, t, off in tensors}
        self.info = info
        self._raw, self._data = raw, data
        # head_dim: key_length, else attn_q rows / H, else fused rows / (H + 2 KVH) (:154-177)
        hd = int(g("attention.key_length", 0))
        if not hd:
            if "blk.0.attn_q.weight" in info:
                hd = int(info["blk.0.attn_q.weight"][0][1]) // self.H
            elif "blk.0.attn_qkv.weight" in info:
                hd = int(info["blk.0.attn_qkv.weight"][0][1]) // (self.H + 2 * self.KVH)
            else:
                hd = self.d // self.H
        self.hd = hd
        self.rope_dim = int(g("rope.dimension_count", 0)) or hd
        # vocab from the tokens array, clamped to the embedding/output rows (:186-197)
        vocab = len(meta["tokenizer.ggml.tokens"]) if "tokenizer.ggml.tokens" in meta else int(
            g("vocab_size", 0))
        for name in ("output.weight", "token_embd.weight"):
            if name in info and len(info[name][0]) == 2:
                vocab = min(vocab, int(info[name][0][1]))
        self.vocab = vocab
        self.max_seq = max_seq
        self.kv = kv
        self.embd = self._mat("token_embd.weight")
        self.out_norm = self._vec("output_norm.weight") if "output_norm.weight" in info else None
        self.out = self._mat("output.weight") if "output.weight" in info else self.embd   # tied (:653-657)
        qd, kvd = self.H * hd, self.KVH * hd
        self.layers = []
        for l in range(self.L):
            p = "blk.%d." % l
            ly = {"attn_norm": self._vec(p + "attn_norm.weight"), "wo": self._mat(p + "attn_output.weight"),
                  "ffn_norm": self._vec(p + "ffn_norm.weight"), "wd": self._mat(p + "ffn_down.weight")}
            if p + "attn_qkv.weight" in info:        # [q; k; v] rows (:337-347)
                w = self._mat(p + "attn_qkv.weight")
                ly["wq"], ly["wk"], ly["wv"] = w[:qd], w[qd:qd + kvd], w[qd + kvd:qd + 2 * kvd]
            else:
                ly["wq"], ly["wk"], ly["wv"] = (self._mat(p + n) for n in
                                                ("attn_q.weight", "attn_k.weight", "attn_v.weight"))
            if p + "ffn_gate.weight" in info:
                ly["wg"], ly["wu"] = self._mat(p + "ffn_gate.weight"), self._mat(p + "ffn_up.weight")
            else:                                      # fused [gate; up] (:518-524)
                w = self._mat(p + "ffn_up.weight")
                ly["wg"], ly["wu"] = w[:self.ffn], w[self.ffn:2 * self.ffn]
            for b in ("q", "k", "v"):                  # biases (:367-402); attn_qkv.bias is never applied
                n = p + "attn_%s.bias" % b
                ly["b" + b] = self._vec(n) if n in info else None
            for k, n in (("post_attn", "post_attention_norm.weight"), ("post_ffn", "post_ffw_norm.weight")):
                ly[k] = self._vec(p + n) if p + n in info else None
            self.layers.append(ly)
        self.reset()

    def _mat(self, name):
        dims, t, off = self.info[name]
        return _matrix(self._raw, self._data, dims, t, off)

    def _vec(self, name):
        dims, t, off = self.info[name]
        return _vector(self._raw, self._data, dims, t, off)

    def reset(self):
        kvd = self.KVH * self.hd
        self.kc = np.zeros((self.L, self.max_seq, kvd))
        self.vc = np.zeros((self.L, self.max_seq, kvd))

    # ---- pieces, each restating one reference function ----
    def rmsnorm(self, x, w, gemma=None):              # tensor.c:114-152
        gemma = self.gemma if gemma is None else gemma
        return x / np.sqrt(np.mean(x * x) + self.eps) * (w + 1.0 if gemma else w)

    def ffn_act(self, gt, up):
        if self.gemma:                                # :529-531, tensor.c:181-190
            return up * 0.5 * gt * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (gt + 0.044715 * gt ** 3)))
        return up * (gt / (1.0 + np.exp(-gt)))        # :533-549

    def softcap(self, x, cap):                        # tensor.c:194-200
        return cap * np.tanh(x / cap) if cap > 0 else x

    def rope(self, v, n_heads, pos):                  # tensor.c:220-275
        v = v.reshape(n_heads, self.hd).copy()
        rd = self.rope_dim
        i = np.arange(0, rd, 2)
        ang = pos * (1.0 / self.theta ** (i / rd))
        c, s = np.cos(ang), np.sin(ang)
        if self.neox:
            a, b = v[:, :rd // 2].copy(), v[:, rd // 2:rd].copy()
            v[:, :rd // 2] = a * c - b * s
            v[:, rd // 2:rd] = a * s + b * c
        else:
            a, b = v[:, 0:rd:2].copy(), v[:, 1:rd:2].copy()
            v[:, 0:rd:2] = a * c - b * s
            v[:, 1:rd:2] = a * s + b * c
        return v.reshape(-1)

    def kv_encode(self, x):
        """What the cache returns for x: binary16, or kv_turboquant_encode
        (:101-118) then decode (:120-125)."""
        if self.kv == "f16":
            return x.astype(np.float16).astype(np.float64)
        s = np.max(np.abs(x)) / 127.0
        if s == 0:
            return np.zeros_like(x)
        t = x / s
        q = np.sign(t) * np.floor(np.abs(t) + 0.5)        # roundf: halves away from zero
        return np.clip(q, -128, 127) * s

    def layer(self, l, x, pos):                       # process_layer, :291-567 (llama branch)
        ly = self.layers[l]
        h = self.rmsnorm(x, ly["attn_norm"])
        q, k, v = ly["wq"] @ h, ly["wk"] @ h, ly["wv"] @ h
        if ly["bq"] is not None:
            q = q + ly["bq"]
        if ly["bk"] is not None:
            k = k + ly["bk"]
        if ly["bv"] is not None:
            v = v + ly["bv"]
        q = self.rope(q, self.H, pos)
        k = self.rope(k, self.KVH, pos)
        self.kc[l, pos] = self.kv_encode(k)
        self.vc[l, pos] = self.kv_encode(v)
        n = pos + 1
        hd, G = self.hd, self.H // self.KVH
        att = np.zeros(self.H * hd)
        for hh in range(self.H):                      # :424-468
            kvh = hh // G
            K = self.kc[l, :n, kvh * hd:(kvh + 1) * hd]
            V = self.vc[l, :n, kvh * hd:(kvh + 1) * hd]
            sc = self.softcap(K @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd), self.attn_softcap)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            att[hh * hd:(hh + 1) * hd] = p @ V
        o = ly["wo"] @ att                            # :471-484
        if ly["post_attn"] is not None:
            o = self.rmsnorm(o, ly["post_attn"], gemma=True)
        x = x + o
        h = self.rmsnorm(x, ly["ffn_norm"])
        o = ly["wd"] @ self.ffn_act(ly["wg"] @ h, ly["wu"] @ h)   # :552-566
        if ly["post_ffn"] is not None:
            o = self.rmsnorm(o, ly["post_ffn"], gemma=True)
        return x + o

    def head(self, x):                                # :634-676
        if self.out_norm is not None:
            x = self.rmsnorm(x, self.out_norm)
        self.hidden = x
        y = self.out[:self.vocab] @ x
        if self.gemma:
            y = y / np.sqrt(self.d)
        return self.softcap(y, self.final_softcap)

    def embed_row(self, token):                       # :578-602
        x = self.embd[token].copy()
        return x * np.sqrt(self.d) if self.gemma else x

    def forward(self, token, pos):                    # ss_scheduler_forward, :571-679
        x = self.embed_row(token)
        for l in range(self.L):
            x = self.layer(l, x, pos)
        return self.head(x)

    def prefill(self, tokens, start_pos):             # ss_scheduler_prefill, :681-803 (layer-major)
        xs = [self.embed_row(t) for t in tokens]
        for l in range(self.L):
            xs = [self.layer(l, x, start_pos + i) for i, x in enumerate(xs)]
        return self.head(xs[-1])

    def embed(self, tokens):                          # ss_scheduler_embed, :805-911
        xs = [self.embed_row(t) for t in tokens]
        for l in range(self.L):
            xs = [self.layer(l, x, i) for i, x in enumerate(xs)]
        if self.out_norm is not None:
            xs = [self.rmsnorm(x, self.out_norm) for x in xs]
        e = np.mean(xs, axis=0)
        return e / (np.sqrt(np.sum(e * e)) + 1e-12)
