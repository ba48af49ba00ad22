"""Greedy decode parity at the benchmark model shapes: the HIP token loop
(public C API) against the CPU oracle on the benchmark's own synthetic GGUF
files, step by step.

* TinyLlama-1.1B shape, all Q4_0: 32-token prompt, 128 greedy steps.
* Llama-2-7B shape, Q4_0 layers with Q8_0 embedding/output: 512-token
  prompt (the GPU evaluates it as MFMA products), 128 greedy steps.
* Llama-3-8B shape, all Q8_0, vocab 128256: KV cache of every layer filled
  with fp16 N(0, 1) at positions 0..4095 through ss_kv_write, then 128
  greedy steps from position 4096.
* Llama-2-70B shape, all Q4_0 (39 GB): KV filled to 1024 positions, then 16
  greedy steps, resident in HBM; and the same in streaming mode (layers
  uploaded per use from pinned host memory), whose logits must equal the
  resident run's bit for bit.

At every step: the GPU's argmax equals the oracle's (both then continue
from that token, so the two greedy sequences are identical), and
max |gpu - oracle| / max |oracle| <= 1e-3 over the logits (fp32 accumulation
on both sides; reference loop layer_scheduler.c:571-679, engine.c:235-290).

The synthetic weights use signed block scales with weight spread
1/sqrt(cols) (ss_synth.h scale_mode 1), so these models respond to their
input: each test also checks that consecutive steps' oracle logits differ
by at least ten times the tolerance, so that a GPU path ignoring its input
could not pass.
"""
import os
import sys

import numpy as np
import pytest

import oracle
from phonemap_amd import api
from tests.util import rel_err

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
import bench  # noqa: E402  (the benchmark's model shapes and files)

pytestmark = pytest.mark.gpu
TOL = 1e-3
TMP = os.environ.get("SS_TEST_TMP", "/tmp")


def _floor_rel(got, want):
    """max_i |got_i - want_i| / max(|want_i|, 1e-6 max|want|): reported, not
    held (an element near zero carries the rounding of its whole sum)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.maximum(np.abs(want), 1e-6 * np.max(np.abs(want)))
    return float(np.max(np.abs(got - want) / den))


class Trace:
    def __init__(self, name):
        self.name, self.worst, self.worst_floor, self.sens = name, 0.0, 0.0, []
        self.prev = None

    def step(self, i, lg, am, olg):
        e = rel_err(lg, olg)
        self.worst = max(self.worst, e)
        self.worst_floor = max(self.worst_floor, _floor_rel(lg, olg))
        oam = oracle.argmax(olg)
        top = np.sort(olg)[::-1]
        assert e <= TOL, (self.name, i, e)
        assert am == oam, (self.name, i, am, oam, "oracle top-2 gap %.3e" % (top[0] - top[1]))
        if self.prev is not None:
            self.sens.append(rel_err(olg, self.prev))
        self.prev = olg

    def done(self):
        med = float(np.median(self.sens)) if self.sens else 0.0
        print("%s: worst rel err %.2e (elementwise with floor %.2e), step-to-step change median %.2e"
              % (self.name, self.worst, self.worst_floor, med), flush=True)
        assert med >= 10 * TOL, (self.name, med)


def _kv_fill(models, spec, n, seed):
    kvd = spec["n_kv_heads"] * spec["head_dim"]
    rng = np.random.default_rng(seed)
    for layer in range(spec["n_layers"]):
        k = rng.standard_normal((n, kvd), np.float32).astype(np.float16).view(np.uint16)
        v = rng.standard_normal((n, kvd), np.float32).astype(np.float16).view(np.uint16)
        for m in models:
            if isinstance(m, oracle.Model):
                m.kv_write_rows(layer, 0, k, v)
            else:
                m.kv_write(layer, 0, k, v)


def _prompt_run(name, prompt_len, steps):
    spec = bench.CONFIGS[name]["spec"]
    path = bench.model_file(name, TMP)
    rng = np.random.default_rng(2024)
    prompt = rng.integers(3, spec["vocab"], prompt_len).tolist()
    ctx = prompt_len + steps + 1
    print("model", name, "prompt", prompt_len, "steps", steps, flush=True)
    om = oracle.Model(path, ctx, "f16")
    tr = Trace(name)
    with api.Model(path, max_context=ctx) as m:
        lg, am = m.eval_prompt(prompt, 0)
        olg = om.prefill(prompt, 0)
        tr.step(-1, lg, am, olg)
        tok, pos = am, prompt_len
        for i in range(steps):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            tr.step(i, lg, am, olg)
            tok, pos = am, pos + 1
    om.close()
    tr.done()


@pytest.mark.timeout(600)
def test_tinyllama_shape_prompt32_128_steps():
    _prompt_run("tinyllama", 32, 128)


@pytest.mark.timeout(900)
def test_llama2_7b_shape_prompt512_128_steps():
    _prompt_run("llama2-7b", 512, 128)


@pytest.mark.timeout(900)
def test_llama3_8b_shape_kv4096_128_steps():
    name = "llama3-8b"
    spec = bench.CONFIGS[name]["spec"]
    path = bench.model_file(name, TMP)
    n_pre, steps = 4096, 128
    ctx = n_pre + steps + 1
    print("model", name, "kv", n_pre, "steps", steps, flush=True)
    om = oracle.Model(path, ctx, "f16")
    tr = Trace(name)
    with api.Model(path, max_context=ctx) as m:
        m.reset()
        _kv_fill([m, om], spec, n_pre, 4096)
        tok, pos = 11, n_pre
        for i in range(steps):
            lg, am = m.eval_token(tok, pos)
            olg = om.forward(tok, pos)
            tr.step(i, lg, am, olg)
            tok, pos = am, pos + 1
    om.close()
    tr.done()


@pytest.mark.timeout(1200)
def test_llama2_70b_shape_resident_and_streaming():
    name = "llama2-70b"
    spec = bench.CONFIGS[name]["spec"]
    path = bench.model_file(name, TMP)
    n_pre, steps = 1024, 16
    ctx = n_pre + steps + 1
    runs = []
    for streaming in (False, True):
        print("model", name, "streaming" if streaming else "resident", "kv", n_pre, "steps", steps, flush=True)
        out = []
        with api.Model(path, max_context=ctx, streaming=streaming) as m:
            m.reset()
            _kv_fill([m], spec, n_pre, 70)
            tok, pos = 11, n_pre
            for i in range(steps):
                lg, am = m.eval_token(tok, pos)
                out.append((lg, am))
                tok, pos = am, pos + 1
        runs.append(out)
    for i, ((a, ia), (b, ib)) in enumerate(zip(*runs)):
        assert np.array_equal(a, b), i
        assert ia == ib, i
    print("oracle", name, flush=True)
    om = oracle.Model(path, ctx, "f16")
    _kv_fill([om], spec, n_pre, 70)
    tr = Trace(name)
    tok, pos = 11, n_pre
    for i, (lg, am) in enumerate(runs[0]):
        olg = om.forward(tok, pos)
        tr.step(i, lg, am, olg)
        tok, pos = am, pos + 1
    om.close()
    tr.done()
