"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of
oracle/_ref/libssref.so built from the reference's own sources.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product never imports it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libssref.so")

KV_INT8, KV_F16 = 0, 1   # oracle enum order (ss_oracle.h)

_o = None
_r = None

_fp = C.POINTER(C.c_float)
_vp = C.c_void_p
_i32 = C.c_int32


def _ptr(a):
    return a.ctypes.data_as(_vp)


def lib():
    global _o
    if _o is not None:
        return _o
    if not os.path.exists(ORACLE_SO):
        raise RuntimeError("oracle not built: make -C oracle")
    L = C.CDLL(ORACLE_SO)
    protos = {
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_dequantize": (None, [_vp, _vp, _i32, _i32]),
        "orc_dot": (C.c_float, [_vp, _vp, _i32]),
        "orc_dequant_matvec": (None, [_vp, _vp, _vp, _i32, _i32, _i32]),
        "orc_rmsnorm": (None, [_vp, _vp, _vp, _i32, C.c_float]),
        "orc_softmax": (None, [_vp, _i32]),
        "orc_silu_mul": (C.c_float, [C.c_float, C.c_float]),
        "orc_gemma_rmsnorm": (None, [_vp, _vp, _vp, _i32, C.c_float]),
        "orc_gelu": (C.c_float, [C.c_float]),
        "orc_softcap": (None, [_vp, _i32, C.c_float]),
        "orc_rope": (None, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, C.c_float, _i32]),
        "orc_rope_table": (None, [_vp, _i32, _i32, C.c_float]),
        "orc_argmax": (_i32, [_vp, _i32]),
        "orc_sample": (_i32, [_vp, _i32, C.c_float, C.c_float, _i32, C.POINTER(C.c_uint64), _vp, _vp]),
        "orc_kv_int8_encode": (None, [_vp, _vp, _vp, _i32]),
        "orc_attention_head": (None, [_vp, _vp, _vp, _vp, _i32, _i32, _i32]),
        "orc_set_threads": (None, [_i32]),
        "orc_get_threads": (_i32, []),
        "orc_model_open": (_vp, [C.c_char_p, _i32, _i32]),
        "orc_model_close": (None, [_vp]),
        "orc_model_dims": (None, [_vp, _vp]),
        "orc_model_eps": (C.c_float, [_vp]),
        "orc_model_theta": (C.c_float, [_vp]),
        "orc_forward": (_fp, [_vp, _i32, _i32]),
        "orc_prefill": (_fp, [_vp, _vp, _i32, _i32]),
        "orc_prefill_serial": (_fp, [_vp, _vp, _i32, _i32]),
        "orc_embed": (_i32, [_vp, _vp, _i32, _vp]),
        "orc_reset": (None, [_vp]),
        "orc_kv_write": (_i32, [_vp, _i32, _i32, _vp, _vp]),
        "orc_hidden": (_fp, [_vp]),
    }
    for n, (res, args) in protos.items():
        f = getattr(L, n)
        f.restype = res
        f.argtypes = args
    _o = L
    return L


def ref():
    """The reference's cpu_neon.c + tokenizer.c, or None when not built."""
    global _r
    if _r is not None:
        return _r
    if not os.path.exists(REF_SO):
        return None
    L = C.CDLL(REF_SO)
    L.ss_neon_dot.restype = C.c_float
    L.ss_neon_dot.argtypes = [_vp, _vp, _i32]
    L.ss_neon_rmsnorm.restype = None
    L.ss_neon_rmsnorm.argtypes = [_vp, _vp, _vp, _i32, C.c_float]
    L.ss_neon_gemma_rmsnorm.restype = None
    L.ss_neon_gemma_rmsnorm.argtypes = [_vp, _vp, _vp, _i32, C.c_float]
    L.ss_neon_silu.restype = None
    L.ss_neon_silu.argtypes = [_vp, _i32]
    L.ss_neon_matvec.restype = None
    L.ss_neon_matvec.argtypes = [_vp, _vp, _vp, _i32, _i32]
    L.ss_tokenizer_create.restype = _vp
    L.ss_tokenizer_create.argtypes = [_vp, _vp, C.c_uint32, _vp, C.c_uint32, C.c_char_p]
    L.ss_tokenizer_encode.restype = _i32
    L.ss_tokenizer_encode.argtypes = [_vp, C.c_char_p, _vp, _i32]
    L.ss_tokenizer_decode.restype = C.c_char_p
    L.ss_tokenizer_decode.argtypes = [_vp, _i32]
    L.ss_tokenizer_free.restype = None
    L.ss_tokenizer_free.argtypes = [_vp]
    _r = L
    return L


# ---- numpy conveniences ----
def matvec(w_bytes, x, rows, cols, qtype):
    y = np.zeros(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w_bytes, np.uint8)
    lib().orc_dequant_matvec(_ptr(y), _ptr(w), _ptr(x), rows, cols, qtype)
    return y


def dequantize(src_bytes, n, qtype):
    out = np.zeros(n, np.float32)
    s = np.ascontiguousarray(src_bytes)
    lib().orc_dequantize(_ptr(s), _ptr(out), n, qtype)
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib().orc_rmsnorm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
    return out


def gemma_rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib().orc_gemma_rmsnorm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
    return out


def gelu(x):
    f = lib().orc_gelu
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)


def softcap(x, cap):
    x = np.array(x, np.float32)
    lib().orc_softcap(_ptr(x), x.size, cap)
    return x


def rope(q, k, n_heads, n_kv_heads, head_dim, rope_dim, pos, theta, neox=False):
    q = np.array(q, np.float32)
    k = np.array(k, np.float32)
    lib().orc_rope(_ptr(q), _ptr(k), n_heads, n_kv_heads, head_dim, rope_dim, pos, theta, int(neox))
    return q, k


def kv_int8_encode(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.int8)
    s = np.zeros(1, np.float32)
    lib().orc_kv_int8_encode(_ptr(x), _ptr(q), _ptr(s), x.size)
    return q, float(s[0])


def attention_head(q, keys, values):
    """keys/values: [seq, head_dim] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.zeros(q.size, np.float32)
    lib().orc_attention_head(_ptr(out), _ptr(q), _ptr(keys), _ptr(values), q.size, keys.shape[0], q.size)
    return out


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().orc_argmax(_ptr(x), x.size))


def sample(logits, temperature, top_p, top_k, rng):
    """ss_sample (tensor.c:363-451): returns (index, new rng state, final
    probabilities, uniform draw)."""
    x = np.ascontiguousarray(logits, np.float32)
    st = C.c_uint64(rng)
    probs = np.zeros(x.size, np.float32)
    r = np.zeros(1, np.float32)
    i = lib().orc_sample(_ptr(x), x.size, temperature, top_p, top_k, C.byref(st), _ptr(probs), _ptr(r))
    return int(i), int(st.value), probs, float(r[0])


def softmax(x):
    x = np.array(x, np.float32)
    lib().orc_softmax(_ptr(x), x.size)
    return x


class Model:
    """The oracle's scheduler over a GGUF file."""

    def __init__(self, path, max_seq, kv="f16"):
        L = lib()
        mode = KV_F16 if kv == "f16" else KV_INT8
        self.h = L.orc_model_open(path.encode(), max_seq, mode)
        if not self.h:
            raise RuntimeError("oracle could not open %s" % path)
        d = np.zeros(8, np.int32)
        L.orc_model_dims(self.h, _ptr(d))
        (self.n_layers, self.d, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn,
         self.vocab, self.max_seq) = [int(v) for v in d]

    def close(self):
        if self.h:
            lib().orc_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, token, pos):
        p = lib().orc_forward(self.h, token, pos)
        if not p:
            raise RuntimeError("oracle forward failed")
        return np.ctypeslib.as_array(p, (self.vocab,)).copy()

    def prefill(self, tokens, start_pos=0):
        t = np.ascontiguousarray(tokens, np.int32)
        p = lib().orc_prefill(self.h, _ptr(t), t.size, start_pos)
        if not p:
            raise RuntimeError("oracle prefill failed")
        return np.ctypeslib.as_array(p, (self.vocab,)).copy()

    def prefill_serial(self, tokens, start_pos=0):
        t = np.ascontiguousarray(tokens, np.int32)
        p = lib().orc_prefill_serial(self.h, _ptr(t), t.size, start_pos)
        if not p:
            raise RuntimeError("oracle prefill failed")
        return np.ctypeslib.as_array(p, (self.vocab,)).copy()

    def embed(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(self.d, np.float32)
        if lib().orc_embed(self.h, _ptr(t), t.size, _ptr(out)) != 0:
            raise RuntimeError("oracle embed failed")
        return out

    def reset(self):
        lib().orc_reset(self.h)

    def kv_write(self, layer, pos, k_f16, v_f16):
        k = np.ascontiguousarray(k_f16, np.uint16)
        v = np.ascontiguousarray(v_f16, np.uint16)
        if lib().orc_kv_write(self.h, layer, pos, _ptr(k), _ptr(v)) != 0:
            raise RuntimeError("oracle kv_write failed")

    def kv_write_rows(self, layer, pos0, k_f16, v_f16):
        """Rows pos0 .. pos0 + n - 1 of one layer from [n][kv_dim] binary16 arrays."""
        k = np.ascontiguousarray(k_f16, np.uint16)
        v = np.ascontiguousarray(v_f16, np.uint16)
        kvd = k.shape[1]
        for i in range(k.shape[0]):
            if lib().orc_kv_write(self.h, layer, pos0 + i, _ptr(k[i]), _ptr(v[i])) != 0:
                raise RuntimeError("oracle kv_write failed")

    def greedy(self, prompt, n_steps):
        """Prefill then n_steps greedy tokens; returns (first, [tokens])."""
        logits = self.prefill(prompt, 0)
        tok = argmax(logits)
        first = tok
        out = []
        pos = len(prompt)
        for _ in range(n_steps):
            tok = argmax(self.forward(tok, pos))
            out.append(tok)
            pos += 1
        return first, out
