"""Causal attention of prompt rows on MFMA (ss_hip_attention_rows) against
the CPU oracle: token t of a chunk starting at position pos0 attends to
positions 0..pos0+t (layer_scheduler.c:415-468 per token of
ss_scheduler_prefill, :681-803), for every token and head; head_dim 64, 128
and 256 (Gemma).

Bar: max |gpu - oracle| / max |oracle| <= 1e-3 over all rows (the kernel
keeps q and P to 2^-22 through two fp16 parts each; the oracle sums in fp32
position by position). Shapes: head_dim 64 and 128, 1, 2, 4 and 8 query
heads per KV head, token counts that leave ragged 64-row tiles and 64-key
blocks, a chunk that continues an earlier one (pos0 > 0), a single token,
and the 7B prompt chunk (512 tokens, 32 heads). Cache rows past the chunk
hold NaN: a read of them would show in the output.
"""
import numpy as np
import pytest

import oracle
from tests.util import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _ref(q, kc, vc, H, KVH, hd, pos0, n):
    G = H // KVH
    out = np.zeros((n, H * hd), np.float32)
    for t in range(n):
        ctx = pos0 + t + 1
        for h in range(H):
            g = h // G
            out[t, h * hd:(h + 1) * hd] = oracle.attention_head(
                q[t, h * hd:(h + 1) * hd], kc[g, :ctx].astype(np.float32), vc[g, :ctx].astype(np.float32))
    return out


def _run(hip, H, KVH, hd, pos0, n, max_seq, seed, qscale=1.0):
    rng = np.random.default_rng(seed)
    q = (qscale * rng.standard_normal((n, H * hd))).astype(np.float32)
    kc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float16)
    vc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float16)
    kc[:, pos0 + n:] = np.nan
    vc[:, pos0 + n:] = np.nan
    Q, KC, VC, O = hip.upload(q), hip.upload(kc), hip.upload(vc), hip.buf(4 * n * H * hd)
    rc = hip.L.ss_hip_attention_rows(hip.ctx, O.ptr, Q.ptr, KC.ptr, VC.ptr, H, KVH, hd, max_seq, pos0, n, None)
    assert rc == 0, hip.err()
    got = O.read(np.float32, n * H * hd).reshape(n, H * hd)
    for b in (Q, KC, VC, O):
        b.free()
    return got, q, kc, vc


@pytest.mark.parametrize("H,KVH,hd,pos0,n,max_seq", [
    (4, 4, 64, 0, 70, 128),        # group 1, ragged tile and block
    (8, 4, 64, 5, 33, 64),         # group 2
    (8, 2, 128, 60, 20, 96),       # group 4, continues a chunk
    (16, 2, 64, 100, 13, 128),     # group 8
    (8, 1, 128, 0, 1, 8),          # one token
    (4, 2, 128, 200, 129, 400),    # more rows than one workgroup holds
    (8, 4, 256, 0, 70, 128),       # head_dim 256 (Gemma): 32-key blocks
    (8, 1, 256, 30, 33, 96),       # head_dim 256, group 8
])
def test_rows_match_oracle(hip, H, KVH, hd, pos0, n, max_seq):
    print("attention rows", H, KVH, hd, pos0, n, flush=True)
    got, q, kc, vc = _run(hip, H, KVH, hd, pos0, n, max_seq, seed=n + pos0)
    assert np.all(np.isfinite(got))
    assert rel_err(got, _ref(q, kc, vc, H, KVH, hd, pos0, n)) <= TOL


def test_rows_7b_chunk(hip):
    """The 7B prompt chunk (32 heads, head_dim 128, 512 tokens); the oracle
    checks every 8th token (all heads)."""
    H, KVH, hd, n = 32, 32, 128, 512
    print("attention rows 7b", flush=True)
    got, q, kc, vc = _run(hip, H, KVH, hd, 0, n, 640, seed=7)
    assert np.all(np.isfinite(got))
    rows = np.arange(0, n, 8)
    want = np.stack([_ref(q[t:t + 1], kc[:, :t + 1], vc[:, :t + 1], H, KVH, hd, t, 1)[0] for t in rows])
    assert rel_err(got[rows], want) <= TOL


def test_rows_sharp_and_small_queries(hip):
    """q scaled by 40 (near one-hot softmax rows) and by 1e-30 (the per-row
    power-of-two scale keeps the fp16 parts normal; the rows become means)."""
    H, KVH, hd, n = 4, 2, 128, 40
    for qs in (40.0, 1e-30):
        print("attention rows qscale", qs, flush=True)
        got, q, kc, vc = _run(hip, H, KVH, hd, 3, n, 64, seed=11, qscale=qs)
        assert np.all(np.isfinite(got))
        assert rel_err(got, _ref(q, kc, vc, H, KVH, hd, 3, n)) <= TOL


def test_rows_reject_bad_shapes(hip):
    Q = hip.buf(4 * 4 * 64)
    KC = hip.buf(2 * 4 * 64 * 8)
    for H, KVH, hd, max_seq, pos0, n in [(4, 4, 96, 8, 0, 1),    # head_dim 96
                                          (4, 4, 64, 8, 4, 5),    # past max_seq
                                          (6, 4, 64, 8, 0, 1),    # heads not a multiple
                                          (4, 4, 64, 8, 0, 0)]:   # no tokens
        assert hip.L.ss_hip_attention_rows(hip.ctx, Q.ptr, Q.ptr, KC.ptr, KC.ptr, H, KVH, hd, max_seq, pos0, n,
                                           None) != 0
