"""The per-matvec backend plug from a C caller: tests/c/plug_snippet.c is
the INTEGRATION.md snippet inside a copy of ss_matmul_dispatch
(layer_scheduler.c:248-279), built with gcc against include/ss_hip.h and
linked with the library. Its GPU results must match the oracle's matvec
(quantize.c:446-494), and a shape the plug rejects must reach the CPU
branch (ss_hip_matvec_host returns false, the Metal calls' convention).
Batched dispatches (ss_hip_begin_batch / ss_hip_end_batch) hold the same
bar, each with its own vector."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from tests.util import F32, Q4_0, Q4_K, Q8_0, make_blocks, rel_err

pytestmark = pytest.mark.gpu
EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "plug_snippet")


def _run(tmp_path, w, x, rows, cols, qtype, *extra):
    wp, xp, yp = (str(tmp_path / n) for n in ("w.bin", "x.bin", "y.bin"))
    np.ascontiguousarray(w).tofile(wp)
    np.ascontiguousarray(x, np.float32).tofile(xp)
    r = subprocess.run([EXE, wp, xp, yp, str(rows), str(cols), str(qtype), *extra], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stderr)
    return int(r.stdout.split()[-1]), np.fromfile(yp, np.float32)


@pytest.mark.parametrize("qtype,rows,cols", [(Q4_0, 512, 4096), (Q8_0, 1000, 2048), (Q4_0, 33, 96),
                                             (Q4_K, 700, 4096), (Q4_K, 33, 256), (F32, 300, 1024)])
def test_plug_snippet_matches_oracle(tmp_path, qtype, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = make_blocks(qtype, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    fallbacks, y = _run(tmp_path, w, x, rows, cols, qtype)
    assert fallbacks == 0
    assert rel_err(y, oracle.matvec(w, x, rows, cols, qtype)) <= 1e-3


@pytest.mark.parametrize("qtype,cols", [(Q4_0, 40), (Q4_K, 288)])
def test_plug_snippet_rejected_shape_falls_back(tmp_path, qtype, cols):
    # not a whole number of blocks (32 weights) or super-blocks (256): the plug says false
    rows = 64
    fallbacks, y = _run(tmp_path, np.zeros(rows * 10 * 18, np.uint8), np.ones(cols, np.float32), rows, cols, qtype)
    assert fallbacks == 2
    assert np.all(y == -1.0)


@pytest.mark.parametrize("qtype,rows,cols", [(Q4_0, 512, 4096), (Q8_0, 300, 2048), (Q4_K, 200, 1024)])
def test_plug_batch_defers_outputs(tmp_path, qtype, rows, cols):
    """ss_hip_begin_batch / ss_hip_end_batch (ss_metal_begin_batch /
    ss_metal_end_batch, metal_backend.m:307-330): 17 dispatches inside one
    batch, dispatch i reading (i + 1) x. The first 16 are deferred and land
    in their own host arrays at ss_hip_end_batch (each call its own vector);
    the 17th finds the batch full, gets false and runs on the CPU branch."""
    rng = np.random.default_rng(rows * 3 + cols)
    w = make_blocks(qtype, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    fallbacks, y = _run(tmp_path, w, x, rows, cols, qtype, "batch")
    assert fallbacks == 1
    y = y.reshape(17, rows)
    for i in range(16):
        want = oracle.matvec(w, ((i + 1) * x).astype(np.float32), rows, cols, qtype)
        assert rel_err(y[i], want) <= 1e-3, i
    assert np.all(y[16] == -1.0)
