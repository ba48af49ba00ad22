"""Python mirror of the SlipStream C API over the MI355X-native library.

The library (libslipstream_hip.so, built in-tree by phonemap_amd.build) holds
the HIP kernels, the C-ABI of include/ss_hip.h and the C engine behind
include/slipstream.h. This module only binds it with ctypes; loading fails
loudly when the library is missing - there is no fallback path.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libslipstream_hip.so")

# ggml types (src/core/gguf_loader.h:41-55 of the reference)
F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
KV_F16, KV_INT8 = 0, 1
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34}

_lib = None

_vp, _i32, _u64, _f32, _sz = C.c_void_p, C.c_int32, C.c_uint64, C.c_float, C.c_size_t
_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)
_u16p = C.POINTER(C.c_uint16)
_dp = C.POINTER(C.c_double)

# name: (restype, argtypes)
_PROTOS = {
    # include/ss_hip.h
    "ss_hip_init": (_vp, [_i32]),
    "ss_hip_free": (None, [_vp]),
    "ss_hip_last_error": (C.c_char_p, []),
    "ss_hip_device_count": (_i32, []),
    "ss_hip_device_name": (_i32, [_i32, C.c_char_p, _i32]),
    "ss_hip_stream": (_vp, [_vp]),
    "ss_hip_sync": (_i32, [_vp]),
    "ss_hip_malloc": (_vp, [_vp, _sz]),
    "ss_hip_mfree": (_i32, [_vp, _vp]),
    "ss_hip_memcpy_h2d": (_i32, [_vp, _vp, _vp, _sz]),
    "ss_hip_memcpy_d2h": (_i32, [_vp, _vp, _vp, _sz]),
    "ss_hip_packed_bytes": (_sz, [_i32, _i32, _i32]),
    "ss_hip_pack_matrix": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32]),
    "ss_hip_matvec": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "ss_hip_gemm": (_i32, [_vp, _vp, _vp, _vp, _vp, _f32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ss_hip_matvec_q4_0": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "ss_hip_matvec_q8_0": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "ss_hip_matvec_q4_k": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "ss_hip_matvec_fused": (_i32, [_vp, _vp, _vp, _vp, _vp, _f32, _i32, _i32, _i32, _i32, _vp]),
    "ss_hip_ffn_gate_up": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _f32, _i32, _i32, _i32, _vp]),
    "ss_hip_rmsnorm": (_i32, [_vp, _vp, _vp, _vp, _i32, _f32, _vp]),
    "ss_hip_rope": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp]),
    "ss_hip_kv_append": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ss_hip_attention": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ss_hip_attention_rows": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ss_hip_attention_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                        _vp]),
    "ss_hip_swiglu": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp]),
    "ss_hip_argmax": (_i32, [_vp, _vp, _vp, _i32, _vp]),
    "ss_hip_sample_logits": (_i32, [_vp, _vp, _i32, _f32, _f32, _i32, C.POINTER(_u64), _ip]),
    "ss_hip_sample": (_i32, [_vp, _f32, _f32, _i32, C.POINTER(_u64), _ip]),
    "ss_hip_embed_row": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "ss_hip_matvec_host": (_i32, [_vp, _fp, _vp, _fp, _i32, _i32, _i32]),
    "ss_hip_should_use_gpu": (_i32, [_i32, _i32]),
    "ss_hip_model_create": (_vp, [_vp, _vp]),
    "ss_hip_model_free": (None, [_vp]),
    "ss_hip_eval_token": (_i32, [_vp, _i32, _i32, _fp, _ip]),
    "ss_hip_eval_prompt": (_i32, [_vp, _ip, _i32, _i32, _fp, _ip]),
    "ss_hip_decode_greedy": (_i32, [_vp, _i32, _ip]),
    "ss_hip_set_prompt_batch": (_i32, [_vp, _i32]),
    "ss_hip_embed": (_i32, [_vp, _ip, _i32, _fp]),
    "ss_hip_kv_reset": (_i32, [_vp]),
    "ss_hip_kv_write": (_i32, [_vp, _i32, _i32, _i32, _u16p, _u16p]),
    "ss_hip_hidden": (_i32, [_vp, _fp]),
    "ss_hip_set_cancel_flag": (None, [_vp, _ip]),
    "ss_hip_model_bytes": (_u64, [_vp]),
    "ss_hip_model_host_bytes": (_u64, [_vp]),
    "ss_hip_model_launch": (_i32, [_vp]),
    "ss_hip_trace_enable": (_i32, [_vp, _i32]),
    "ss_hip_trace_read": (C.c_int64, [_vp, C.POINTER(C.c_uint64), _sz]),
    "ss_hip_profile_begin": (_i32, [_vp]),
    "ss_hip_profile_end": (_i32, [_vp, _dp, _i32]),
}


class SlipStreamError(RuntimeError):
    pass


def lib():
    """Load the native library; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise SlipStreamError("native library %s is missing: run python -m phonemap_amd.build" % LIB_PATH)
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _PROTOS.items():
        f = getattr(L, name, None)
        if f is None:
            continue
        f.restype = res
        f.argtypes = args
    _extra_protos(L)
    _lib = L
    return L


def _extra_protos(L):
    try:
        from . import api
        api.bind(L)
    except ImportError:
        pass


def check(rc, what="call"):
    if rc != 0:
        msg = lib().ss_hip_last_error()
        raise SlipStreamError("%s failed (%d): %s" % (what, rc, msg.decode() if msg else ""))
    return rc
