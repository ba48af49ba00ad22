"""Host-side (no GPU) checks of the native library: exported C-ABI, the GGUF
writer/reader pair, the synthetic-model generator and the tokenizer.

The GGUF format is restated independently here in Python (gguf_loader.c:210-485
reads the same layout) so that neither C reader is checked only against itself.
"""
import ctypes as C
import hashlib
import os
import re
import struct

import numpy as np
import pytest

import oracle
from phonemap_amd import api

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "phonemap_amd", "libslipstream_hip.so")


def _lib():
    return C.CDLL(LIB_PATH)


# --------------------------------------------------------------------- ABI

def _declared_functions(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = set()
    for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(ss_\w+)\s*\(", text, flags=re.M):
        if not text[:m.start()].rstrip().endswith("typedef"):
            names.add(m.group(1))
    return names


@pytest.mark.parametrize("header,count", [("slipstream.h", 36), ("ss_hip.h", 55), ("ss_synth.h", 2)])
def test_library_exports_every_declared_function(header, count):
    names = _declared_functions(header)
    assert len(names) == count, sorted(names)
    lib = _lib()
    missing = sorted(n for n in names if not hasattr(lib, n))
    assert not missing, missing


def test_cpu_and_metal_backends_fail_loudly(tmp_path):
    path = str(tmp_path / "m.gguf")
    api.write_synthetic_gguf(path, tiny_spec())
    L = api._lib()
    for backend in (api.SS_BACKEND_CPU, api.SS_BACKEND_METAL):
        cfg = L.ss_default_config()
        cfg.backend = backend
        assert not L.ss_model_load(path.encode(), C.byref(cfg))
        assert L.ss_last_error() == -7   # SS_ERROR_BACKEND


def test_sample_greedy_and_argmax_tie_rule():
    L = api._lib()
    x = np.array([0.5, 3.0, -1.0, 3.0, 2.0], dtype=np.float32)
    p = x.ctypes.data_as(C.POINTER(C.c_float))
    assert L.ss_argmax(p, 5) == 1                                  # first maximum (tensor.c:318-328)
    rng = C.c_uint64(42)
    assert L.ss_sample(p, 5, C.c_float(0.0), C.c_float(1.0), 0, C.byref(rng)) == 1   # T <= 0: greedy


def test_sample_top_k_one_is_argmax():
    L = api._lib()
    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    p = x.ctypes.data_as(C.POINTER(C.c_float))
    rng = C.c_uint64(7)
    for _ in range(5):
        assert L.ss_sample(p, 1000, C.c_float(0.8), C.c_float(1.0), 1, C.byref(rng)) == int(np.argmax(x))


# -------------------------------------------------------------- GGUF model

def tiny_spec(**kw):
    s = dict(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, ffn=96, vocab=300,
             context_length=128, rope_theta=10000.0, rms_eps=1e-5, layer_type=2, embd_type=8,
             out_type=-1, seed=5, scale_sigma=0.0, norm_sigma=0.0, with_vocab=1, n_threads=0)
    s.update(kw)
    return api.SynthSpec(**s)


GGUF_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
               11: "<q", 12: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34)}


def parse_gguf(path):
    """Independent GGUF v2/v3 reader: metadata dict, tensor infos, data offset."""
    b = open(path, "rb").read()
    o = 0

    def rd(fmt):
        nonlocal o
        v = struct.unpack_from(fmt, b, o)
        o += struct.calcsize(fmt)
        return v[0]

    def rstr():
        nonlocal o
        n = rd("<Q")
        s = b[o:o + n].decode()
        o += n
        return s

    def rval(t):
        if t == 8:
            return rstr()
        if t == 9:
            et, n = rd("<I"), rd("<Q")
            return [rval(et) for _ in range(n)]
        return rd(GGUF_SCALAR[t])

    assert b[:4] == b"GGUF"
    o = 4
    version = rd("<I")
    n_t, n_kv = rd("<Q"), rd("<Q")
    meta = {}
    for _ in range(n_kv):
        k = rstr()
        meta[k] = rval(rd("<I"))
    tensors = []
    for _ in range(n_t):
        name = rstr()
        nd = rd("<I")
        dims = [rd("<Q") for _ in range(nd)]
        t = rd("<I")
        off = rd("<Q")
        tensors.append((name, dims, t, off))
    a = meta.get("general.alignment", 32)          # the GGUF format's data alignment
    data = (o + a - 1) & ~(a - 1)
    return version, meta, tensors, data, b


class GTensor(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("type", C.c_int32), ("offset", C.c_uint64), ("size_bytes", C.c_uint64),
                ("layer_index", C.c_int32)]


class GFile(C.Structure):
    _fields_ = [("fd", C.c_int), ("file_size", C.c_uint64), ("base", C.c_void_p),
                ("data_offset", C.c_uint64), ("version", C.c_uint32), ("n_tensors", C.c_uint64),
                ("n_kv", C.c_uint64), ("tensors", C.POINTER(GTensor)), ("layers", C.c_void_p),
                ("num_layers", C.c_uint32), ("arch", C.c_char * 64), ("hidden_size", C.c_uint32),
                ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32), ("vocab_size", C.c_uint32),
                ("context_length", C.c_uint32), ("intermediate_size", C.c_uint32),
                ("head_dim", C.c_uint32), ("rope_dim", C.c_uint32), ("rope_theta", C.c_float),
                ("rms_norm_eps", C.c_float), ("attn_logit_softcapping", C.c_float),
                ("final_logit_softcapping", C.c_float), ("vocab", C.POINTER(C.c_char_p)),
                ("vocab_scores", C.POINTER(C.c_float)), ("merges", C.POINTER(C.c_char_p)),
                ("n_merges", C.c_uint32)]


def gguf_open(path):
    lib = _lib()
    lib.ss_gguf_open.restype = C.POINTER(GFile)
    lib.ss_gguf_open.argtypes = [C.c_char_p]
    lib.ss_gguf_close.argtypes = [C.POINTER(GFile)]
    lib.ss_gguf_tensor_data.restype = C.c_void_p
    lib.ss_gguf_tensor_data.argtypes = [C.POINTER(GFile), C.POINTER(GTensor)]
    lib.ss_gguf_find.restype = C.POINTER(GTensor)
    lib.ss_gguf_find.argtypes = [C.POINTER(GFile), C.c_char_p]
    lib.ss_gguf_find_in_layer.restype = C.POINTER(GTensor)
    lib.ss_gguf_find_in_layer.argtypes = [C.POINTER(GFile), C.c_uint32, C.c_char_p]
    lib.ss_gguf_error.restype = C.c_char_p
    f = lib.ss_gguf_open(path.encode())
    return lib, f


@pytest.mark.parametrize("alignment", [0, 64, 4096])
@pytest.mark.parametrize("out_type", [-1, 8])
def test_synthetic_gguf_round_trip(tmp_path, out_type, alignment):
    """Writer and reader agree, for the reference's 32-byte alignment and for
    general.alignment values the reference would misread (gguf_loader.c:426)."""
    path = str(tmp_path / "m.gguf")
    spec = tiny_spec(out_type=out_type, alignment=alignment)
    api.write_synthetic_gguf(path, spec)
    version, meta, tensors, data_off, raw = parse_gguf(path)
    assert version in (2, 3)
    a = alignment or 32
    assert meta["general.alignment"] == a and data_off % a == 0
    assert all(off % a == 0 for _, _, _, off in tensors)
    assert meta["general.architecture"] == "llama"
    assert meta["llama.embedding_length"] == 64
    assert meta["llama.block_count"] == 2
    assert meta["llama.attention.head_count"] == 4
    assert meta["llama.attention.head_count_kv"] == 2
    assert meta["llama.feed_forward_length"] == 96
    assert len(meta["tokenizer.ggml.tokens"]) == 300
    names = [t[0] for t in tensors]
    assert ("output.weight" in names) == (out_type >= 0)
    per_layer = {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate",
                 "ffn_up", "ffn_down"}
    for l in range(2):
        assert {n.split(".")[2] for n in names if n.startswith("blk.%d." % l)} == per_layer

    lib, f = gguf_open(path)
    assert f, lib.ss_gguf_error()
    try:
        g = f.contents
        assert g.arch.decode() == "llama"
        assert (g.hidden_size, g.num_heads, g.num_kv_heads, g.vocab_size, g.context_length,
                g.intermediate_size, g.num_layers) == (64, 4, 2, 300, 128, 96, 2)
        # head_dim comes from attention.key_length when present, else later from attn_q rows / heads
        assert g.head_dim == meta.get("llama.attention.key_length", 0)
        assert g.rope_theta == pytest.approx(10000.0)
        assert g.rms_norm_eps == pytest.approx(1e-5)
        assert g.n_tensors == len(tensors)
        assert g.data_offset == data_off
        for i in range(g.n_tensors):
            t = g.tensors[i]
            name, dims, typ, off = tensors[i]
            assert t.name.decode() == name and t.type == typ
            assert list(t.dims[:t.n_dims]) == dims
            n = int(np.prod(dims))
            be, bb = BLOCK[typ]
            assert t.size_bytes == n // be * bb
            p = lib.ss_gguf_tensor_data(f, C.byref(t))
            got = C.string_at(p, t.size_bytes)
            assert got == raw[data_off + off: data_off + off + t.size_bytes], name
            assert t.layer_index == (int(name.split(".")[1]) if name.startswith("blk.") else -1)
        q = lib.ss_gguf_find_in_layer(f, 1, b"attn_k.weight")
        assert q and q.contents.name.decode() == "blk.1.attn_k.weight"
        assert not lib.ss_gguf_find(f, b"no.such.tensor")
        vocab = [g.vocab[i].decode() for i in range(g.vocab_size)]
        assert vocab == meta["tokenizer.ggml.tokens"]
    finally:
        lib.ss_gguf_close(f)


def test_gguf_reader_rejects_bad_files(tmp_path):
    lib = _lib()
    lib.ss_gguf_open.restype = C.c_void_p
    lib.ss_gguf_error.restype = C.c_char_p
    assert not lib.ss_gguf_open(str(tmp_path / "missing.gguf").encode())
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 60)
    assert not lib.ss_gguf_open(str(bad).encode())
    trunc = tmp_path / "trunc.gguf"
    path = str(tmp_path / "m.gguf")
    api.write_synthetic_gguf(path, tiny_spec())
    trunc.write_bytes(open(path, "rb").read()[:200])
    assert not lib.ss_gguf_open(str(trunc).encode())


def test_synthetic_gguf_independent_of_thread_count(tmp_path):
    digests = []
    for n in (1, 3, 8):
        path = str(tmp_path / ("m%d.gguf" % n))
        api.write_synthetic_gguf(path, tiny_spec(n_threads=n, hidden=128, ffn=256, vocab=512))
        digests.append(hashlib.sha256(open(path, "rb").read()).hexdigest())
    assert len(set(digests)) == 1


def test_synthetic_weights_follow_spec(tmp_path):
    path = str(tmp_path / "m.gguf")
    api.write_synthetic_gguf(path, tiny_spec(layer_type=2, embd_type=8, out_type=8, hidden=128,
                                             ffn=256, vocab=512))
    _, meta, tensors, off, raw = parse_gguf(path)
    info = {t[0]: t for t in tensors}
    name, dims, typ, o = info["blk.0.ffn_gate.weight"]
    n = dims[0] * dims[1] // 32
    blk = np.frombuffer(raw, np.uint8, n * 18, off + o).reshape(n, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    assert (d >= 0).all() and 0.005 < float(d.mean()) < 0.05      # |N(0, 0.02)|
    nib = np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4]).ravel()
    assert set(np.unique(nib)) == set(range(16))
    name, dims, typ, o = info["output.weight"]
    n = dims[0] * dims[1] // 32
    blk8 = np.frombuffer(raw, np.uint8, n * 34, off + o).reshape(n, 34)
    q8 = blk8[:, 2:].view(np.int8)
    assert q8.min() >= -127 and q8.max() == 127
    d8 = blk8[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    assert (d8 >= 0).all() and 0.005 / 16 < float(d8.mean()) < 0.05 / 16   # |N(0, 0.02 / 16)|
    # equal weight spread for both types: sigma * std(nibble - 8) vs sigma / 16 * std(code)
    w4 = d[:, None] * (np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4], axis=1).astype(np.float32) - 8)
    w8 = d8[:, None] * q8.astype(np.float32)
    assert 0.8 < float(w8.std()) / float(w4.std()) < 1.25
    name, dims, typ, o = info["blk.1.attn_norm.weight"]
    w = np.frombuffer(raw, np.float32, dims[0], off + o)
    assert abs(float(w.mean()) - 1.0) < 0.01 and 0.003 < float(w.std()) < 0.03


# --------------------------------------------------------------- tokenizer

TEXTS = ["Hello world", "The quick brown fox jumps over the lazy dog.", "  leading spaces",
         "tabs\tand\nnewlines", "numbers 12345 and 3.14", "unicode café naïve 日本語 🙂", "", "a",
         "<s> special </s> tokens", "repeated repeated repeated words words"]


def _ref_tokenizer():
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref (reference tokenizer build) not present")
    return r


def _vocab_arrays(vocab, scores):
    arr = (C.c_char_p * len(vocab))(*[v.encode() for v in vocab])
    sc = np.asarray(scores, dtype=np.float32)
    return arr, sc


def _encode_both(vocab, scores, merges, arch, texts):
    r = _ref_tokenizer()
    lib = _lib()
    va, sc = _vocab_arrays(vocab, scores)
    ma = (C.c_char_p * max(1, len(merges)))(*[m.encode() for m in merges]) if merges else None
    scp = sc.ctypes.data_as(C.POINTER(C.c_float))
    lib.ss_tok_create.restype = C.c_void_p
    lib.ss_tok_create.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.c_uint32, C.c_void_p, C.c_uint32,
                                  C.c_char_p]
    lib.ss_tok_encode.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_int32), C.c_int32]
    lib.ss_tok_free.argtypes = [C.c_void_p]
    r.ss_tokenizer_create.restype = C.c_void_p
    r.ss_tokenizer_create.argtypes = lib.ss_tok_create.argtypes
    r.ss_tokenizer_encode.argtypes = lib.ss_tok_encode.argtypes
    r.ss_tokenizer_free.argtypes = [C.c_void_p]
    a = lib.ss_tok_create(va, scp, len(vocab), ma, len(merges), arch.encode())
    b = r.ss_tokenizer_create(va, scp, len(vocab), ma, len(merges), arch.encode())
    out = []
    try:
        for t in texts:
            ba = (C.c_int32 * 4096)()
            bb = (C.c_int32 * 4096)()
            na = lib.ss_tok_encode(a, t.encode(), ba, 4096)
            nb = r.ss_tokenizer_encode(b, t.encode(), bb, 4096)
            out.append((t, list(ba[:na]), list(bb[:nb])))
    finally:
        lib.ss_tok_free(a)
        r.ss_tokenizer_free(b)
    return out


def test_tokenizer_sentencepiece_matches_reference(tmp_path):
    path = str(tmp_path / "m.gguf")
    api.write_synthetic_gguf(path, tiny_spec(vocab=2000))
    _, meta, _, _, _ = parse_gguf(path)
    vocab = meta["tokenizer.ggml.tokens"]
    scores = meta.get("tokenizer.ggml.scores", [0.0] * len(vocab))
    for t, mine, ref in _encode_both(vocab, scores, [], "llama", TEXTS):
        assert mine == ref, t


def test_tokenizer_bpe_matches_reference():
    # GPT-2 style byte-level vocabulary with a few merges ("Ġ" marks a space)
    base = [chr(c) for c in range(33, 127)] + ["Ġ"]
    merges = ["h e", "l l", "o Ġ", "he ll", "Ġ w", "Ġw o", "r l", "rl d", "t h", "th e"]
    vocab = ["<unk>", "<s>", "</s>"] + base + [m.replace(" ", "") for m in merges]
    scores = [0.0] * len(vocab)
    texts = ["hello world", "the the", "hell", "world hello", "abc xyz"]
    for t, mine, ref in _encode_both(vocab, scores, merges, "llama3", texts):
        assert mine == ref, t


def test_host_sample_equals_oracle():
    """The engine's host ss_sample (slipstream.h) and the oracle's restatement
    of tensor.c:363-451 agree exactly (index and RNG state) on seeded cases."""
    import oracle
    L = api._lib()
    rng = np.random.default_rng(17)
    for trial in range(60):
        V = int(rng.choice([5, 64, 1000, 32000]))
        x = (rng.standard_normal(V) * rng.uniform(0.5, 4.0)).astype(np.float32)
        T = float(rng.choice([0.0, 0.5, 1.0, 1.5]))
        top_p = float(rng.choice([0.0, 0.5, 0.9, 1.0]))
        top_k = int(rng.choice([0, 1, 10, V]))
        seed = int(rng.integers(1, 2 ** 63))
        want, want_st, _, _ = oracle.sample(x, T, top_p, top_k, seed)
        st = C.c_uint64(seed)
        got = L.ss_sample(x.ctypes.data_as(C.POINTER(C.c_float)), V, C.c_float(T), C.c_float(top_p), top_k,
                          C.byref(st))
        assert (got, st.value) == (want, want_st), trial


def _gguf_bytes(kvs):
    """A GGUF v3 file with the given metadata and no tensors."""
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    out = b"GGUF" + struct.pack("<IQQ", 3, 0, len(kvs))
    for k, (vt, v) in kvs.items():
        out += s(k) + struct.pack("<I", vt)
        if vt == 8:
            out += s(v)
        elif vt == 9:
            et, items = v
            out += struct.pack("<IQ", et, len(items))
            for it in items:
                out += s(it) if et == 8 else struct.pack(GGUF_SCALAR[et], it)
        else:
            out += struct.pack(GGUF_SCALAR[vt], v)
    return out + b"\0" * ((-len(out)) % 32)


@pytest.mark.parametrize("n_scores", [3, 5, 7])
def test_gguf_scores_used_only_when_they_match_the_vocab(tmp_path, n_scores):
    """tokenizer.ggml.scores shorter or longer than tokenizer.ggml.tokens is
    dropped (merges then rank by string length) instead of being read past
    its end."""
    path = str(tmp_path / "v.gguf")
    toks = ["<unk>", "<s>", "</s>", "a", "b"]
    open(path, "wb").write(_gguf_bytes({"general.architecture": (8, "llama"),
                                        "tokenizer.ggml.tokens": (9, (8, toks)),
                                        "tokenizer.ggml.scores": (9, (6, [0.5] * n_scores))}))
    lib, f = gguf_open(path)
    assert f, lib.ss_gguf_error()
    assert f.contents.vocab_size == 5
    assert bool(f.contents.vocab_scores) == (n_scores == 5)
    lib.ss_gguf_close(f)
