"""Shared helpers: seeded GGUF-layout block generators and a device buffer
wrapper over the library's own ss_hip_malloc/memcpy."""
import ctypes as C

import numpy as np

Q4_0, Q8_0, Q4_K = 2, 8, 12
Q2_K, Q3_K, Q5_K, Q6_K = 10, 11, 13, 14
F32, F16, Q4_1, Q5_0, Q5_1, Q8_1 = 0, 1, 3, 6, 7, 9
KQ_BYTES = {Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}   # per 256 weights
# per 32 weights (GGML block sizes; float matrices counted in 32-weight pieces)
B32_BYTES = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q8_1: 40, F16: 64, F32: 128}


def _vp(a):
    return a.ctypes.data_as(C.c_void_p)


def f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def make_q4_0(rows, cols, rng, sigma=0.02):
    """GGUF Q4_0 blocks: fp16 d = |N(0, sigma)|, 16 bytes of uniform nibbles."""
    nb = rows * (cols // 32)
    blk = np.zeros((nb, 18), np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, sigma, nb)))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blk.reshape(-1)


def make_q8_0(rows, cols, rng, sigma=0.02):
    """GGUF Q8_0 blocks: fp16 d = |N(0, sigma)|, int8 codes uniform in [-127, 127]."""
    nb = rows * (cols // 32)
    blk = np.zeros((nb, 34), np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, sigma, nb)))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return blk.reshape(-1)


def q4k_pack_scales(sc, mn):
    """The 12-byte scale array of a Q4_K super-block from eight 6-bit scales
    and mins, laid out as the GGML K-quant format defines it: bytes 0-3 hold
    scales 0-3 in their low 6 bits and the top 2 bits of scales 4-7 above
    them; bytes 4-7 the same for the mins; bytes 8-11 hold scale 4+i in the
    low nibble and min 4+i in the high nibble (their low 4 bits)."""
    b = np.zeros(12, np.uint8)
    for i in range(4):
        b[i] = (sc[i] & 63) | ((sc[4 + i] >> 4) << 6)
        b[4 + i] = (mn[i] & 63) | ((mn[4 + i] >> 4) << 6)
        b[8 + i] = (sc[4 + i] & 15) | ((mn[4 + i] & 15) << 4)
    return b


def q4k_block(d, dmin, sc, mn, q):
    """One 144-byte Q4_K super-block: fp16 d and dmin, 8 scales and mins
    (0..63), q[8][32] nibbles: sub-block 2j in the low and 2j+1 in the high
    nibbles of bytes 32j..32j+31."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([d], np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], np.float16).view(np.uint8)
    blk[4:16] = q4k_pack_scales(sc, mn)
    q = np.asarray(q, np.uint8)
    for j in range(4):
        blk[16 + 32 * j:16 + 32 * j + 32] = (q[2 * j] & 15) | ((q[2 * j + 1] & 15) << 4)
    return blk


def make_q4_k(rows, cols, rng, sigma=0.02):
    """GGUF Q4_K super-blocks: d, dmin = fp16(N(0, sigma / 32)), random 6-bit
    scales and mins, uniform nibbles."""
    nsb = rows * (cols // 256)
    out = np.zeros((nsb, 144), np.uint8)
    d = f16_bits(rng.normal(0.0, sigma / 32, nsb))
    dm = f16_bits(rng.normal(0.0, sigma / 32, nsb))
    out[:, 0:2] = d.view(np.uint8).reshape(nsb, 2)
    out[:, 2:4] = dm.view(np.uint8).reshape(nsb, 2)
    sc = rng.integers(0, 64, (nsb, 8))
    mn = rng.integers(0, 64, (nsb, 8))
    for i in range(nsb):
        out[i, 4:16] = q4k_pack_scales(sc[i], mn[i])
    out[:, 16:] = rng.integers(0, 256, (nsb, 128), dtype=np.uint8)
    return out.reshape(-1)


def _f16_into(out, lo, vals):
    out[:, lo:lo + 2] = f16_bits(vals).view(np.uint8).reshape(-1, 2)


def make_kq(qtype, rows, cols, rng, sigma=0.02):
    """GGUF Q2_K / Q3_K / Q5_K / Q6_K super-blocks with every code and scale
    field uniformly random, d (and dmin) = fp16(N(0, s)) with s chosen so that
    the weights spread about sigma."""
    nsb = rows * (cols // 256)
    nbytes = KQ_BYTES[qtype]
    out = rng.integers(0, 256, (nsb, nbytes), dtype=np.uint8)
    if qtype == Q2_K:     # w = d*sc*q - dmin*m, sc, m < 16, q < 4
        _f16_into(out, 80, rng.normal(0.0, sigma / 18.7, nsb))
        _f16_into(out, 82, rng.normal(0.0, sigma / 18.7, nsb))
    elif qtype == Q3_K:   # w = d*(s - 32)*q, q in [-4, 3]
        _f16_into(out, 108, rng.normal(0.0, sigma / 43.3, nsb))
    elif qtype == Q5_K:   # w = d*sc*q - dmin*m, sc, m < 64, q < 32
        _f16_into(out, 0, rng.normal(0.0, sigma / 660.0, nsb))
        _f16_into(out, 2, rng.normal(0.0, sigma / 660.0, nsb))
    elif qtype == Q6_K:   # w = d*sc*q, sc int8, q in [-32, 31]
        _f16_into(out, 208, rng.normal(0.0, sigma / 1366.0, nsb))
    else:
        raise ValueError(qtype)
    return out.reshape(-1)


def make_more(qtype, rows, cols, rng, sigma=0.02):
    """F32 / F16 matrices (weights N(0, 4.6 sigma), the spread of make_q4_0's)
    and GGUF Q4_1 / Q5_0 / Q5_1 / Q8_1 blocks: random codes and high bits,
    d = |N(0, s)| (fp32 for Q8_1), m = -(centre code) d + noise."""
    if qtype in (F32, F16):
        w = rng.normal(0.0, 4.6 * sigma, rows * cols)
        return (w.astype(np.float32) if qtype == F32 else w.astype(np.float16)).view(np.uint8)
    nb = rows * (cols // 32)
    out = rng.integers(0, 256, (nb, B32_BYTES[qtype]), dtype=np.uint8)
    if qtype == Q8_1:
        d = np.abs(rng.normal(0.0, sigma / 16.0, nb)).astype(np.float32)
        out[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
        out[:, 4:8] = rng.normal(0.0, 1.0, nb).astype(np.float32).view(np.uint8).reshape(nb, 4)   # s, unused
        out[:, 8:40] = rng.integers(-127, 128, (nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
        return out.reshape(-1)
    centre, rms = {Q4_1: (7.5, 4.6), Q5_0: (0.0, 9.25), Q5_1: (15.5, 9.2)}[qtype]
    d = np.abs(rng.normal(0.0, 4.6 * sigma / rms, nb))
    _f16_into(out, 0, d)
    if qtype != Q5_0:
        _f16_into(out, 2, -centre * d + rng.normal(0.0, 0.5 * sigma, nb))
    return out.reshape(-1)


def make_blocks(qtype, rows, cols, rng, sigma=0.02):
    if qtype in B32_BYTES and qtype not in (Q4_0, Q8_0):
        return make_more(qtype, rows, cols, rng, sigma)
    if qtype == Q4_K:
        return make_q4_k(rows, cols, rng, sigma)
    if qtype in (Q2_K, Q3_K, Q5_K, Q6_K):
        return make_kq(qtype, rows, cols, rng, sigma)
    return make_q4_0(rows, cols, rng, sigma) if qtype == Q4_0 else make_q8_0(rows, cols, rng, sigma)


def q4k_unpack_scales(b):
    """Inverse of q4k_pack_scales (per the format definition): (sc[8], mn[8])."""
    b = np.asarray(b, np.int64)
    sc = np.zeros(8, np.int64)
    mn = np.zeros(8, np.int64)
    for i in range(4):
        sc[i] = b[i] & 63
        mn[i] = b[4 + i] & 63
        sc[4 + i] = (b[8 + i] & 15) | ((b[i] >> 6) << 4)
        mn[4 + i] = (b[8 + i] >> 4) | ((b[4 + i] >> 6) << 4)
    return sc, mn


def dequant_np(blocks, rows, cols, qtype):
    """Independent numpy dequantisation (GGML block spec), fp64."""
    nb = cols // 32
    if qtype == Q4_0:
        b = blocks.reshape(rows * nb, 18)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
        q = b[:, 2:]
        lo = (q & 0xF).astype(np.int64) - 8
        hi = (q >> 4).astype(np.int64) - 8
        w = np.concatenate([lo, hi], axis=1) * d[:, None]
    elif qtype == Q8_0:
        b = blocks.reshape(rows * nb, 34)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
        w = b[:, 2:].view(np.int8).astype(np.float64) * d[:, None]
    elif qtype in (Q2_K, Q3_K, Q5_K, Q6_K):
        w = _dequant_kq(blocks, rows, cols, qtype)
    elif qtype in (F32, F16, Q4_1, Q5_0, Q5_1, Q8_1):
        w = _dequant_more(blocks, rows, cols, qtype)
    else:   # Q4_K super-blocks of 256
        nsb = rows * (cols // 256)
        b = blocks.reshape(nsb, 144)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
        dm = b[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1)
        w = np.zeros((nsb, 256))
        for i in range(nsb):
            sc, mn = q4k_unpack_scales(b[i, 4:16])
            q = b[i, 16:].astype(np.int64)
            for k in range(8):
                nib = (q[32 * (k // 2):32 * (k // 2) + 32] >> (4 * (k % 2))) & 15
                w[i, 32 * k:32 * k + 32] = d[i] * sc[k] * nib - dm[i] * mn[k]
    return w.reshape(rows, cols)


def _dequant_more(blocks, rows, cols, qtype):
    """F32 / F16 and Q4_1 / Q5_0 / Q5_1 / Q8_1 in fp64 from the GGML block
    layouts: Q4_1 = d, m, 16 nibble bytes (weight j low, j + 16 high), d q + m;
    Q5_0 = d, qh, nibbles, (q - 16) d; Q5_1 = d, m, qh, nibbles, d q + m, with
    bit j of the little-endian qh as bit 4 of weight j; Q8_1 = fp32 d, fp32 s,
    32 int8, d q."""
    raw = np.ascontiguousarray(blocks, np.uint8)
    if qtype == F32:
        return raw.view(np.float32).astype(np.float64).reshape(rows, cols)
    if qtype == F16:
        return raw.view(np.float16).astype(np.float64).reshape(rows, cols)
    b = raw.reshape(rows * (cols // 32), B32_BYTES[qtype])
    if qtype == Q8_1:
        d = b[:, 0:4].copy().view(np.float32).astype(np.float64).reshape(-1)
        return (b[:, 8:].view(np.int8).astype(np.float64) * d[:, None]).reshape(rows, cols)
    d = _f16_col(b, 0)
    m = _f16_col(b, 2) if qtype != Q5_0 else 0.0
    qs = b[:, {Q4_1: 4, Q5_0: 6, Q5_1: 8}[qtype]:].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=1)
    if qtype != Q4_1:
        o = 2 if qtype == Q5_0 else 4
        qh = b[:, o:o + 4].copy().view(np.uint32).astype(np.int64).reshape(-1)
        q = q | (((qh[:, None] >> np.arange(32)[None, :]) & 1) << 4)
    w = (q - 16) * d[:, None] if qtype == Q5_0 else q * d[:, None] + m[:, None]
    return w.reshape(rows, cols)


def _f16_col(b, lo):
    return b[:, lo:lo + 2].copy().view(np.float16).astype(np.float64).reshape(-1)


def _dequant_kq(blocks, rows, cols, qtype):
    """Q2_K / Q3_K / Q5_K / Q6_K in fp64, vectorised over the 256 weights of a
    super-block from the GGML block layouts (weight index i = 128h + 32j + l
    for the 2-bit-plane formats and Q6_K; sub-block i // 32 for Q5_K)."""
    nsb = rows * (cols // 256)
    b = blocks.reshape(nsb, KQ_BYTES[qtype]).astype(np.int64)
    i = np.arange(256)
    h, j, l = i // 128, (i % 128) // 32, i % 32
    if qtype == Q2_K:
        q = (b[:, 16 + 32 * h + l] >> (2 * j)) & 3
        sb = b[:, 8 * h + 2 * j + l // 16]
        return (_f16_col(b.astype(np.uint8), 80)[:, None] * (sb & 15) * q
                - _f16_col(b.astype(np.uint8), 82)[:, None] * (sb >> 4))
    if qtype == Q3_K:
        # the 16 6-bit scales from the 12 packed bytes, as 32-bit words
        w32 = b[:, 96:108].astype(np.uint8).copy().view("<u4").astype(np.int64)
        a0, a1, t = w32[:, 0], w32[:, 1], w32[:, 2]
        m2, m1 = 0x0F0F0F0F, 0x03030303
        aux = np.stack([(a0 & m2) | (((t >> 0) & m1) << 4), (a1 & m2) | (((t >> 2) & m1) << 4),
                        ((a0 >> 4) & m2) | (((t >> 4) & m1) << 4), ((a1 >> 4) & m2) | (((t >> 6) & m1) << 4)],
                       axis=1).astype("<u4")
        scales = aux.view(np.uint8).astype(np.int64).reshape(nsb, 16)
        hbit = (b[:, l] >> (4 * h + j)) & 1
        q = ((b[:, 32 + 32 * h + l] >> (2 * j)) & 3) - np.where(hbit == 1, 0, 4)
        return _f16_col(b.astype(np.uint8), 108)[:, None] * (scales[:, 8 * h + 2 * j + l // 16] - 32) * q
    if qtype == Q5_K:
        k = i // 32
        sc = np.zeros((nsb, 8), np.int64)
        mn = np.zeros((nsb, 8), np.int64)
        for s in range(nsb):
            sc[s], mn[s] = q4k_unpack_scales(b[s, 4:16])
        byte = b[:, 48 + 32 * (k // 2) + l]
        q = np.where(k % 2 == 1, byte >> 4, byte & 15) + 16 * ((b[:, 16 + l] >> k) & 1)
        return (_f16_col(b.astype(np.uint8), 0)[:, None] * sc[:, k] * q
                - _f16_col(b.astype(np.uint8), 2)[:, None] * mn[:, k])
    # Q6_K
    lb = b[:, 64 * h + 32 * (j & 1) + l]
    lo = np.where(j < 2, lb & 15, lb >> 4)
    q = (lo | (((b[:, 128 + 32 * h + l] >> (2 * j)) & 3) << 4)) - 32
    sc = b[:, 192:208].astype(np.uint8).view(np.int8).astype(np.int64)
    return _f16_col(b.astype(np.uint8), 208)[:, None] * sc[:, 8 * h + 2 * j + l // 16] * q


def rel_err(got, want):
    """max |got - want| / max |want|: error relative to the output's scale."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.max(np.abs(want))
    return float(np.max(np.abs(got - want)) / (scale if scale > 0 else 1.0))


def elem_rel_err(got, want, floor=1e-6):
    """max_i |got_i - want_i| / max(|want_i|, floor * max |want|): every
    element's error relative to its own size, small elements measured
    against floor times the largest."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.max(np.abs(want))
    den = np.maximum(np.abs(want), floor * (scale if scale > 0 else 1.0))
    return float(np.max(np.abs(got - want) / den))


def check_elementwise(got, oracle_y, blocks, x, rows, cols, qtype, comp_tol=1e-6):
    """Per-row error of a matvec result against the exact product e (fp64
    over dequant_np's weights), relative to what fp32 summation of that row
    can be held to: max_i |y_i - e_i| / sum_j |w_ij x_j| <= comp_tol. fp32
    sums (the oracle's) reach 5e-8 to 7e-8 here; a 1% error in the scale of
    one 16-weight group of one row gives 5e-7 to 5e-5. The elementwise form
    max_i |y_i - e_i| / max(|e_i|, 1e-6 max|e|) is printed for the result
    and for the oracle: near-zero outputs put both at fp32 cancellation
    noise (up to ~7e-2), so it is reported, not asserted, for these formats."""
    w = dequant_np(blocks, rows, cols, qtype)
    xd = np.asarray(x, np.float64)
    exact = w @ xd
    mag = np.maximum(np.abs(w) @ np.abs(xd), 1e-300)
    c_got = float(np.max(np.abs(np.asarray(got, np.float64) - exact) / mag))
    c_orc = float(np.max(np.abs(np.asarray(oracle_y, np.float64) - exact) / mag))
    print("per-row vs exact: hip %.3g, oracle %.3g; elementwise: hip %.3g, oracle %.3g" %
          (c_got, c_orc, elem_rel_err(got, exact), elem_rel_err(oracle_y, exact)), flush=True)
    assert c_got <= comp_tol, (c_got, c_orc)


class Buf:
    def __init__(self, dev, nbytes):
        self.dev = dev
        self.nbytes = nbytes
        self.ptr = dev.L.ss_hip_malloc(dev.ctx, nbytes)
        if not self.ptr:
            raise RuntimeError("ss_hip_malloc failed")

    def write(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        rc = self.dev.L.ss_hip_memcpy_h2d(self.dev.ctx, self.ptr, _vp(arr), arr.nbytes)
        assert rc == 0, self.dev.err()
        return self

    def read(self, dtype, count):
        out = np.zeros(count, dtype)
        assert out.nbytes <= self.nbytes
        rc = self.dev.L.ss_hip_memcpy_d2h(self.dev.ctx, _vp(out), self.ptr, out.nbytes)
        assert rc == 0, self.dev.err()
        return out

    def free(self):
        if self.ptr:
            self.dev.L.ss_hip_mfree(self.dev.ctx, self.ptr)
            self.ptr = None


class Dev:
    def __init__(self, L, ctx):
        self.L = L
        self.ctx = ctx

    def err(self):
        m = self.L.ss_hip_last_error()
        return m.decode() if m else ""

    def buf(self, nbytes):
        return Buf(self, int(nbytes))

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        return self.buf(max(arr.nbytes, 4)).write(arr)

    def packed(self, blocks, qtype, rows, cols):
        nbytes = self.L.ss_hip_packed_bytes(qtype, rows, cols)
        b = self.buf(nbytes)
        rc = self.L.ss_hip_pack_matrix(self.ctx, b.ptr, _vp(np.ascontiguousarray(blocks)), qtype, rows, cols)
        assert rc == 0, self.err()
        return b

    def sync(self):
        assert self.L.ss_hip_sync(self.ctx) == 0, self.err()


class OracleBar:
    """Logits held against the oracle at every step:
    max |gpu - oracle| / max |oracle| <= tol. The fp64 model's distance
    (tests/ref_model.py) is computed beside it and printed with the worst
    figures by report(); it is not an alternative to the oracle bar.

    known maps (tag, step) to (bar, reason) for a step at which the oracle's
    own fp16 cache is known to round a K/V value across a binary16 midpoint
    the other way than exact arithmetic does: the oracle's logits then leave
    the fp64 model's, and the GPU's leave the oracle's, by about the same
    measured amount. There the oracle bar is that stated figure, and the GPU
    must also be within tol of the fp64 model."""

    def __init__(self, name, tol, known=None):
        self.name, self.tol, self.known = name, tol, dict(known or {})
        self.worst = self.worst_ref = 0.0

    def check(self, key, lg, olg, ref):
        e = rel_err(lg, olg)
        r = rel_err(lg, ref)
        self.worst, self.worst_ref = max(self.worst, e), max(self.worst_ref, r)
        if key in self.known:
            bar, why = self.known[key]
            assert e <= bar and r <= self.tol, (self.name, key, e, r, why)
        else:
            assert e <= self.tol, (self.name, key, "oracle", e, "fp64 model", r)
        return e

    def report(self):
        print("%s: worst vs oracle %.2e, vs fp64 model %.2e (bar %.0e)"
              % (self.name, self.worst, self.worst_ref, self.tol), flush=True)
