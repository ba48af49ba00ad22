"""Shared helpers: seeded GGUF-layout block generators and a device buffer
wrapper over the library's own ss_hip_malloc/memcpy."""
import ctypes as C

import numpy as np

Q4_0, Q8_0 = 2, 8


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


def make_blocks(qtype, rows, cols, rng, sigma=0.02):
    return make_q4_0(rows, cols, rng, sigma) if qtype == Q4_0 else make_q8_0(rows, cols, rng, sigma)


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
    else:
        b = blocks.reshape(rows * nb, 34)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
        w = b[:, 2:].view(np.int8).astype(np.float64) * d[:, None]
    return w.reshape(rows, cols)


def rel_err(got, want):
    """max |got - want| / max |want|: error relative to the output's scale."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.max(np.abs(want))
    return float(np.max(np.abs(got - want)) / (scale if scale > 0 else 1.0))


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
