"""ctypes mirror of include/slipstream.h and include/ss_synth.h."""
import ctypes as C

import numpy as np

_i32, _u32, _u64, _f32 = C.c_int32, C.c_uint32, C.c_uint64, C.c_float
_vp = C.c_void_p
_ip = C.POINTER(C.c_int32)
_fp = C.POINTER(C.c_float)
_u16p = C.POINTER(C.c_uint16)

SS_BACKEND_AUTO, SS_BACKEND_CPU, SS_BACKEND_METAL, SS_BACKEND_HIP = 0, 1, 2, 3
SS_KV_F16, SS_KV_INT8 = 0, 1
LAUNCH = {"eager": 0, "graph": 1, "sweep": 2}   # SS_LAUNCH_*
ERRORS = {0: "SS_OK", -1: "SS_ERROR_FILE_NOT_FOUND", -2: "SS_ERROR_INVALID_MODEL",
          -3: "SS_ERROR_OUT_OF_MEMORY", -4: "SS_ERROR_MMAP_FAILED", -5: "SS_ERROR_INVALID_PARAMS",
          -6: "SS_ERROR_CANCELLED", -7: "SS_ERROR_BACKEND", -8: "SS_ERROR_TOKENIZER", -99: "SS_ERROR_UNKNOWN"}


class ModelConfig(C.Structure):       # slipstream.h:87-94
    _fields_ = [("backend", _i32), ("n_threads", _u32), ("max_memory", _u64), ("use_mmap", C.c_bool),
                ("prefetch", C.c_bool), ("context_size", _u32)]


class GenerateParams(C.Structure):    # slipstream.h:98-106
    _fields_ = [("max_tokens", _u32), ("temperature", _f32), ("top_p", _f32), ("top_k", _u32),
                ("repeat_penalty", _f32), ("seed", _u32), ("stop_sequence", C.c_char_p)]


class ModelExt(C.Structure):
    _fields_ = [("kv_type", _i32), ("device", _i32), ("max_context", _u32), ("streaming", _u32),
                ("launch", _u32)]


class ModelInfo(C.Structure):         # slipstream.h:65-79
    _fields_ = [("model_name", C.c_char * 256), ("architecture", C.c_char * 64), ("chat_format", C.c_char * 64),
                ("num_layers", _u32), ("hidden_size", _u32), ("num_heads", _u32), ("num_kv_heads", _u32),
                ("vocab_size", _u32), ("context_length", _u32), ("intermediate_size", _u32),
                ("quant_type", _i32), ("file_size", _u64), ("per_layer_size", _u64)]


class DeviceInfo(C.Structure):        # slipstream.h:274-284
    _fields_ = [("device_model", C.c_char * 64), ("chip_name", C.c_char * 64), ("cpu_core_count", _u32),
                ("perf_core_count", _u32), ("efficiency_core_count", _u32), ("gpu_core_count", _u32),
                ("total_memory", _u64), ("available_memory", _u64), ("thermal_state", _i32)]


class SynthSpec(C.Structure):         # ss_synth.h
    _fields_ = [("n_layers", _i32), ("hidden", _i32), ("n_heads", _i32), ("n_kv_heads", _i32),
                ("head_dim", _i32), ("ffn", _i32), ("vocab", _i32), ("context_length", _i32),
                ("rope_theta", _f32), ("rms_eps", _f32), ("layer_type", _i32), ("embd_type", _i32),
                ("out_type", _i32), ("seed", _u64), ("scale_sigma", _f32), ("norm_sigma", _f32),
                ("with_vocab", _i32), ("n_threads", _i32), ("arch", _i32), ("fused_qkv", _i32),
                ("fused_up", _i32), ("qkv_bias", _i32), ("alignment", _i32), ("scale_mode", _i32),
                ("vocab_tokens", _i32), ("attn_softcap", _f32), ("final_softcap", _f32)]

    def __init__(self, **kw):
        d = dict(rope_theta=10000.0, rms_eps=1e-5, layer_type=2, embd_type=2, out_type=2, seed=0,
                 scale_sigma=0.02, norm_sigma=0.01, with_vocab=1, n_threads=0, context_length=2048)
        d.update(kw)
        super().__init__(**d)


TOKEN_CB = C.CFUNCTYPE(C.c_bool, C.c_char_p, C.c_uint32, C.c_void_p)
PROGRESS_CB = C.CFUNCTYPE(None, C.c_uint32, C.c_uint32, C.c_char_p, C.c_void_p)

PROTOS = {
    "ss_default_config": (ModelConfig, []),
    "ss_default_params": (GenerateParams, []),
    "ss_default_ext": (ModelExt, []),
    "ss_model_load": (_vp, [C.c_char_p, C.POINTER(ModelConfig)]),
    "ss_model_load_ex": (_vp, [C.c_char_p, C.POINTER(ModelConfig), C.POINTER(ModelExt)]),
    "ss_model_get_info": (_i32, [_vp, C.POINTER(ModelInfo)]),
    "ss_model_free": (None, [_vp]),
    "ss_set_throttle": (None, [_vp, _u32]),
    "ss_get_memory_usage": (_u64, []),
    "ss_get_last_profile_path": (C.c_char_p, []),
    "ss_set_profile_output_dir": (None, [C.c_char_p]),
    "ss_generate": (_i32, [_vp, C.c_char_p, C.POINTER(GenerateParams), TOKEN_CB, _vp]),
    "ss_embed": (_i32, [_vp, C.c_char_p, C.POINTER(_fp), C.POINTER(_u32)]),
    "ss_cancel": (None, [_vp]),
    "ss_set_progress_callback": (None, [_vp, PROGRESS_CB, _vp]),
    "ss_last_error": (_i32, []),
    "ss_error_string": (C.c_char_p, [_i32]),
    "ss_version": (C.c_char_p, []),
    "ss_estimate_memory": (_i32, [C.c_char_p, _u32, C.POINTER(_u64)]),
    "ss_get_device_info": (_i32, [C.POINTER(DeviceInfo)]),
    "ss_get_cpu_usage": (C.c_double, []),
    "ss_tokenize": (_i32, [_vp, C.c_char_p, _ip, _i32]),
    "ss_token_text": (C.c_char_p, [_vp, _i32]),
    "ss_bos_id": (_i32, [_vp]),
    "ss_eos_id": (_i32, [_vp]),
    "ss_n_vocab": (_i32, [_vp]),
    "ss_n_ctx": (_i32, [_vp]),
    "ss_n_embd": (_i32, [_vp]),
    "ss_reset": (_i32, [_vp]),
    "ss_eval_token": (_i32, [_vp, _i32, _i32, _fp, _ip]),
    "ss_eval_prompt": (_i32, [_vp, _ip, _i32, _i32, _fp, _ip]),
    "ss_decode_greedy": (_i32, [_vp, _i32, _ip]),
    "ss_kv_write": (_i32, [_vp, _i32, _i32, _i32, _u16p, _u16p]),
    "ss_model_hip": (_vp, [_vp]),
    "ss_argmax": (_i32, [_fp, _i32]),
    "ss_sample": (_i32, [_fp, _i32, _f32, _f32, _i32, C.POINTER(_u64)]),
    "ss_synth_gguf_write": (_i32, [C.c_char_p, C.POINTER(SynthSpec)]),
    "ss_synth_vocab_string": (C.c_char_p, [_i32, _i32, C.c_char_p, _i32]),
}


def bind(L):
    for name, (res, args) in PROTOS.items():
        f = getattr(L, name, None)
        if f is None:
            continue
        f.restype = res
        f.argtypes = args


def _lib():
    from . import lib
    return lib()


class SlipStreamError(RuntimeError):
    pass


def _check(rc, what):
    if rc != 0:
        from . import lib
        msg = lib().ss_hip_last_error()
        raise SlipStreamError("%s: %s (%s)" % (what, ERRORS.get(rc, rc), msg.decode() if msg else ""))


def write_synthetic_gguf(path, spec):
    rc = _lib().ss_synth_gguf_write(path.encode(), C.byref(spec))
    if rc != 0:
        raise SlipStreamError("ss_synth_gguf_write(%s) failed: %d" % (path, rc))


def _ptr(a, t):
    return a.ctypes.data_as(t)


class Model:
    """A loaded model on the HIP backend (ss_model_load_ex)."""

    def __init__(self, path, max_context=0, kv="f16", device=0, launch="graph", backend=SS_BACKEND_HIP,
                 streaming=False):
        L = _lib()
        cfg = L.ss_default_config()
        cfg.backend = backend
        ext = L.ss_default_ext()
        ext.kv_type = SS_KV_F16 if kv == "f16" else SS_KV_INT8
        ext.device = device
        ext.max_context = max_context
        ext.launch = LAUNCH[launch]
        ext.streaming = 1 if streaming else 0
        self.h = L.ss_model_load_ex(path.encode(), C.byref(cfg), C.byref(ext))
        if not self.h:
            raise SlipStreamError("ss_model_load_ex(%s) failed: %s" % (path, ERRORS.get(L.ss_last_error())))
        self.vocab = L.ss_n_vocab(self.h)
        self.n_ctx = L.ss_n_ctx(self.h)
        self.n_embd = L.ss_n_embd(self.h)

    def close(self):
        if getattr(self, "h", None):
            _lib().ss_model_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        _check(_lib().ss_reset(self.h), "ss_reset")

    def eval_token(self, token, pos, want_logits=True):
        am = C.c_int32(-1)
        lg = np.zeros(self.vocab, np.float32) if want_logits else None
        rc = _lib().ss_eval_token(self.h, token, pos, _ptr(lg, _fp) if want_logits else None, C.byref(am))
        _check(rc, "ss_eval_token")
        return (lg, am.value) if want_logits else am.value

    def eval_prompt(self, tokens, start_pos=0, want_logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        am = C.c_int32(-1)
        lg = np.zeros(self.vocab, np.float32) if want_logits else None
        rc = _lib().ss_eval_prompt(self.h, _ptr(t, _ip), t.size, start_pos,
                                   _ptr(lg, _fp) if want_logits else None, C.byref(am))
        _check(rc, "ss_eval_prompt")
        return (lg, am.value) if want_logits else am.value

    def set_prompt_batch(self, min_tokens):
        """Shortest prompt evaluated as matrix products (0: default, < 0: never)."""
        L = _lib()
        _check(L.ss_hip_set_prompt_batch(L.ss_model_hip(self.h), min_tokens), "ss_hip_set_prompt_batch")

    def sample(self, temperature, top_p, top_k, rng):
        """ss_sample over the last evaluated token's logits, on the device:
        returns (token, advanced rng state)."""
        L = _lib()
        st = C.c_uint64(rng)
        tok = C.c_int32(-1)
        _check(L.ss_hip_sample(L.ss_model_hip(self.h), temperature, top_p, top_k, C.byref(st), C.byref(tok)),
               "ss_hip_sample")
        return tok.value, st.value

    def decode_greedy(self, n_steps):
        out = np.zeros(max(n_steps, 1), np.int32)
        _check(_lib().ss_decode_greedy(self.h, n_steps, _ptr(out, _ip)), "ss_decode_greedy")
        return out[:n_steps].tolist()

    def greedy(self, prompt, n_steps):
        """Prefill then n_steps greedy tokens; returns (first, [tokens])."""
        self.reset()
        first = self.eval_prompt(prompt, 0, want_logits=False)
        return first, self.decode_greedy(n_steps)

    def kv_write(self, layer, pos0, k_f16, v_f16):
        k = np.ascontiguousarray(k_f16, np.uint16)
        v = np.ascontiguousarray(v_f16, np.uint16)
        n_pos = k.shape[0] if k.ndim > 1 else 1
        _check(_lib().ss_kv_write(self.h, layer, pos0, n_pos, _ptr(k, _u16p), _ptr(v, _u16p)), "ss_kv_write")

    def tokenize(self, text, max_tokens=4096):
        out = np.zeros(max_tokens, np.int32)
        n = _lib().ss_tokenize(self.h, text.encode(), _ptr(out, _ip), max_tokens)
        return out[:n].tolist()

    def token_text(self, tid):
        s = _lib().ss_token_text(self.h, tid)
        return s.decode("utf-8", "replace") if s is not None else ""
