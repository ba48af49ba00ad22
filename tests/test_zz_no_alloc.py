"""ss_hip_attention_noalloc (no device allocation: split partials and
counters in a fixed per-GPU scratch array) against ss_hip_attention (its
scratch allocated by the library) through the C-ABI: two calls in a row, the
second with a smaller input, each bit-identical to the allocating entry
point (the same kernels with the same split count) and within 1e-3 of an
fp64 numpy attention (layer_scheduler.c:415-468). A shape that needs more
scratch than the array holds is refused with SS_ERROR_INVALID_PARAMS before
any launch."""
import numpy as np
import pytest

from tests.util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _ref(q, kc, vc, H, KVH, hd, seq, ks=None, vs=None):
    G = H // KVH
    out = np.zeros(H * hd)
    for h in range(H):
        g = h // G
        K = kc[g, :seq].astype(np.float64)
        V = vc[g, :seq].astype(np.float64)
        if ks is not None:
            K = K * ks[:seq, None]
            V = V * vs[:seq, None]
        s = K @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


def _case(hip, kv_type, H, KVH, hd, seq, max_seq, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(H * hd).astype(np.float32)
    if kv_type == 0:
        kc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float16)
        vc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float16)
        ks = vs = None
    else:
        kc = rng.integers(-127, 128, (KVH, max_seq, hd)).astype(np.int8)
        vc = rng.integers(-127, 128, (KVH, max_seq, hd)).astype(np.int8)
        ks = (rng.random(max_seq) * 0.03).astype(np.float32)
        vs = (rng.random(max_seq) * 0.03).astype(np.float32)
    bufs = [hip.upload(a) for a in (q, kc, vc)]
    KS = hip.upload(ks) if ks is not None else None
    VS = hip.upload(vs) if vs is not None else None
    outs = []
    for fn in (hip.L.ss_hip_attention_noalloc, hip.L.ss_hip_attention):
        O = hip.buf(4 * H * hd)
        rc = fn(hip.ctx, O.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, KS.ptr if KS else None,
                VS.ptr if VS else None, H, KVH, hd, max_seq, seq, kv_type, None)
        assert rc == 0, hip.err()
        outs.append(O.read(np.float32, H * hd))
    assert np.array_equal(outs[0], outs[1])
    assert rel_err(outs[0], _ref(q, kc, vc, H, KVH, hd, seq, ks, vs)) <= TOL


@pytest.mark.parametrize("kv_type", [0, 1])
def test_noalloc_attention_matches_allocating_entry_point(hip, kv_type):
    print("noalloc attention kv_type", kv_type, "large then small", flush=True)
    _case(hip, kv_type, 32, 8, 128, 4100, 4224, 1)     # 8B shape, context 4100
    _case(hip, kv_type, 8, 2, 64, 77, 512, 2)          # smaller: fewer heads, shorter context


def test_noalloc_attention_refuses_oversized_scratch(hip):
    H, KVH, hd, max_seq = 32768, 4096, 128, 64
    small = hip.buf(4096)
    rc = hip.L.ss_hip_attention_noalloc(hip.ctx, small.ptr, small.ptr, small.ptr, small.ptr, None, None, H, KVH,
                                        hd, max_seq, 8, 0, None)
    assert rc == -5
    assert "scratch" in hip.err()
