"""Batch-1 decode benchmark of the SlipStream token loop on one MI355X.

Default workload: Llama-2-7B-shape decoder with random-init weights (32
layers, d 4096, 32 heads = 32 KV heads of dim 128, FFN 11008, vocab 32000),
Q4_0 layer matrices with Q8_0 token_embd/output, a 512-token random prompt,
then greedy decode at batch 1 with an fp16 KV cache. A "step" is one decode
token: embedding, 32 layers, output norm, LM head, argmax.

Prints one JSON line. `value` is decode tokens/s over exactly --steps decode
steps (after --warmup untimed ones), with the weights resident in HBM. The
roofline object is for the dominant kernel class: the matvec of the layer
quantisation type (per-kernel launches, the default) or the whole-token
kernel (--launch sweep, one persistent launch per token). It is measured
with HIP events in a profiled eager replay of further decode steps: the
matvec and attention kernels are launched with hipExtLaunchKernelGGL, whose
start/stop events the dispatch itself records when the kernel begins and
ends (kernel execution time, as a kernel trace reports it); other launches
are bracketed by events on the model stream. cpu_baseline is the CPU oracle (the
reference path restated in C) on the same GGUF, timed on this host on a
bounded sample.

Other workloads (--config): tinyllama (22 layers, all Q4_0, 32-token
prompt, 128 steps); llama3-8b (all Q8_0, vocab 128256, KV cache pre-filled
to 4096 positions with fp16 N(0, 1) through ss_kv_write, 128 steps);
llama2-70b (80 layers, all Q4_0, 1024-token prompt, 64 steps) resident in
HBM, and llama2-70b-stream, the same model in streaming mode (layers
uploaded per use from pinned host memory; the extra "link" object relates
the host-to-device bytes per token to a pinned hipMemcpyAsync measured in
the same run); matvec-q4_0-4096 (the standalone 4096 x 4096 Q4_0 matvec
over rotating weight copies larger than the 256 MB last-level cache).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

METRIC = "batch-1 decode tokens/sec (7B Q4_0); matvec achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    "llama2-7b": dict(spec=dict(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=32, head_dim=128,
                                ffn=11008, vocab=32000, context_length=4096, layer_type=2, embd_type=8,
                                out_type=8, seed=7, scale_mode=1), prompt=512, steps=256,
                      name="llama2-7b-shape, Q4_0 layers + Q8_0 token_embd/output"),
    "tinyllama": dict(spec=dict(n_layers=22, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=64,
                                ffn=5632, vocab=32000, context_length=2048, layer_type=2, embd_type=2,
                                out_type=2, seed=1001, scale_mode=1), prompt=32, steps=128,
                      name="tinyllama-1.1b-shape, all Q4_0"),
    "llama3-8b": dict(spec=dict(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128,
                                ffn=14336, vocab=128256, context_length=8192, rope_theta=500000.0,
                                layer_type=8, embd_type=8, out_type=8, seed=8, scale_mode=1), prompt=0, kv_fill=4096,
                      steps=128, name="llama3-8b-shape, all Q8_0"),
    "llama2-70b": dict(spec=dict(n_layers=80, hidden=8192, n_heads=64, n_kv_heads=8, head_dim=128,
                                 ffn=28672, vocab=32000, context_length=4096, layer_type=2, embd_type=2,
                                 out_type=2, seed=70, scale_mode=1), prompt=1024, steps=64,
                       name="llama2-70b-shape, all Q4_0, resident in HBM"),
    "llama2-70b-stream": dict(model="llama2-70b", streaming=True, prompt=1024, steps=64, profile_steps=2,
                              name="llama2-70b-shape, all Q4_0, streaming mode (layers uploaded per use "
                                   "from pinned host memory)"),
}
for _c in CONFIGS.values():       # a streaming config shares its model's file and shape
    if "model" in _c:
        _c["spec"] = CONFIGS[_c["model"]]["spec"]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_file(name, model_dir="/tmp"):
    """The synthetic GGUF of config `name` (written once; the name carries the
    seed and the scale mode, so a file of another spec is never reused)."""
    from phonemap_amd import api
    spec = CONFIGS[name]["spec"]
    path = os.path.join(model_dir, "ss_bench_%s_s%d_m%d.gguf" % (name, spec["seed"], spec.get("scale_mode", 0)))
    if not os.path.exists(path):
        t = time.perf_counter()
        api.write_synthetic_gguf(path + ".part", api.SynthSpec(**spec))
        os.replace(path + ".part", path)
        log("wrote %s (%.2f GB) in %.1f s" % (path, os.path.getsize(path) / 1e9, time.perf_counter() - t))
    return path


def token_bytes(spec, ctx):
    """Algorithmic HBM bytes of one decode token at context length ctx."""
    L, d, H, KVH, hd, F, V = (spec[k] for k in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                                 "head_dim", "ffn", "vocab"))
    bpw = {2: 18 / 32, 8: 34 / 32}
    lt = bpw[spec["layer_type"]]
    layer_w = (H * hd * d + 2 * KVH * hd * d + d * H * hd + 3 * F * d) * lt
    head = V * d * bpw[spec["out_type"] if spec["out_type"] >= 0 else spec["embd_type"]]
    kv_read = 2 * L * ctx * KVH * hd * 2
    kv_write = 2 * L * KVH * hd * 2
    norms = (2 * L + 1) * d * 4
    embd_row = d * bpw[spec["embd_type"]]
    return L * layer_w + head + kv_read + kv_write + norms + embd_row


def cpu_baseline(path, spec, prompt_len, budget_s=15.0, max_steps=160):
    """The oracle (reference CPU path restated in C) on the same file: KV for
    positions 0..prompt_len-1 pre-filled with fp16 values, then decode steps
    at positions prompt_len.. until the time budget is spent."""
    import oracle
    om = oracle.Model(path, prompt_len + max_steps + 1, "f16")
    rng = np.random.default_rng(0)
    kvdim = spec["n_kv_heads"] * spec["head_dim"]
    for layer in range(spec["n_layers"]):
        k = rng.standard_normal((prompt_len, kvdim)).astype(np.float16).view(np.uint16)
        for p in range(prompt_len):
            om.kv_write(layer, p, k[p], k[p])
    tok = 11
    om.forward(tok, prompt_len)   # untimed: pages the weights in
    t0 = time.perf_counter()
    n = 0
    while n < max_steps and (time.perf_counter() - t0) < budget_s:
        tok = oracle.argmax(om.forward(tok, prompt_len + 1 + n))
        n += 1
    dt = time.perf_counter() - t0
    threads = oracle.lib().orc_get_threads()
    om.close()
    return {"value": n / dt, "unit": "tok/s", "cores": int(threads), "kind": "port",
            "cpu": host_cpu(),
            "sample": "%d decode steps at context %d (KV pre-filled), same GGUF, %d threads, %.1f s"
                      % (n, prompt_len + 1, threads, dt)}


def host_cpu():
    """The host CPU model and the CPUs this process may use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return "%s, %d CPUs in the affinity mask of %d online" % (model, len(os.sched_getaffinity(0)),
                                                             os.cpu_count() or 0)


def copy_calibration(mib):
    """20 device-to-device copies of mib MiB (torch is only the allocator here)."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty(n, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t) / 20
    log("copy %d MiB: %.1f us, %.0f GB/s read+write" % (mib, dt * 1e6, 2 * n / dt / 1e9))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="llama2-7b", choices=sorted(CONFIGS) + ["matvec-q4_0-4096"])
    ap.add_argument("--kv", default="f16", choices=["f16", "int8"])
    ap.add_argument("--model-dir", default=os.environ.get("SS_BENCH_DIR", "/tmp"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--launch", default="graph", choices=["graph", "sweep", "eager"],
                    help="per-kernel launches replayed from a HIP graph (default), one persistent "
                         "launch per token, or per-kernel launches issued eagerly")
    ap.add_argument("--profile-steps", type=int, default=None)
    ap.add_argument("--prompt-len", type=int, default=None,
                    help="override the prompt length (counter runs use a short prompt)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 20 device-to-device copies of MIB MiB (the known-size kernel that "
                         "scales the FETCH_SIZE/WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (--gpus %d requested)"
              % args.gpus, file=sys.stderr)
        sys.exit(2)

    if args.config == "matvec-q4_0-4096":
        bench_matvec(args)
        return
    from phonemap_amd import api
    cfg = CONFIGS[args.config]
    spec = cfg["spec"]
    steps = args.steps if args.steps is not None else cfg["steps"]
    warm = args.warmup
    prompt_len = args.prompt_len if args.prompt_len is not None else cfg["prompt"]
    kv_fill = cfg.get("kv_fill", 0)
    streaming = cfg.get("streaming", False)
    prof_steps = args.profile_steps if args.profile_steps is not None else cfg.get("profile_steps", 16)
    path = model_file(cfg.get("model", args.config), args.model_dir)
    max_ctx = prompt_len + kv_fill + 1 + warm + steps + prof_steps + 2
    t = time.perf_counter()
    m = api.Model(path, max_context=max_ctx, kv=args.kv, launch=args.launch, streaming=streaming)
    log("loaded in %.1f s" % (time.perf_counter() - t))
    L = api._lib()
    rng = np.random.default_rng(1234)
    prompt = rng.integers(3, spec["vocab"], prompt_len).tolist()

    m.reset()
    prefill_s = None
    if kv_fill:
        # KV cache pre-filled with fp16 N(0, 1) through ss_kv_write, then one
        # token at position kv_fill starts the greedy continuation
        kvdim = spec["n_kv_heads"] * spec["head_dim"]
        krng = np.random.default_rng(4096)
        t = time.perf_counter()
        for layer in range(spec["n_layers"]):
            k = krng.standard_normal((kv_fill, kvdim), np.float32).astype(np.float16).view(np.uint16)
            v = krng.standard_normal((kv_fill, kvdim), np.float32).astype(np.float16).view(np.uint16)
            m.kv_write(layer, 0, k, v)
        log("KV pre-filled to %d positions in %.1f s" % (kv_fill, time.perf_counter() - t))
        m.eval_token(11, kv_fill, want_logits=False)
        prompt_len = kv_fill + 1
    else:
        t = time.perf_counter()
        m.eval_prompt(prompt, 0, want_logits=False)
        prefill_s = time.perf_counter() - t
        log("prefill %d tokens: %.3f s" % (prompt_len, prefill_s))
    if warm:
        m.decode_greedy(warm)
    t0 = time.perf_counter()
    toks = m.decode_greedy(steps)       # returns after a stream synchronise
    dt = time.perf_counter() - t0
    tps = steps / dt
    log("decode %d steps: %.3f s, %.1f tok/s" % (steps, dt, tps))

    # profiled replay (eager launches bracketed by HIP events on the model stream)
    roof = None
    try:
        roof = profile_classes(m, prof_steps)
        roof["timed_as"] = "eager replay; start/stop events recorded by each kernel's dispatch" 
        if args.config == "llama2-7b" and args.kv == "f16" and args.prompt_len is None:
            roof["traffic"], roof["traffic_from"] = measured_traffic(roof["kernel_id"])
    except Exception as e:   # profiling is optional for the headline number
        log("profiling failed: %s" % e)

    avg_ctx = prompt_len + warm + (steps + 1) / 2.0
    tb = token_bytes(spec, avg_ctx)
    out = {
        "metric": METRIC, "value": round(tps, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": warm, "ms_per_step": round(1000.0 * dt / steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "%s, %d-token random prompt, then %d greedy decode steps at batch 1, %s KV"
                               % (cfg["name"], prompt_len, steps, args.kv),
                   "global_batch": 1, "seq_len": prompt_len + warm + steps, "parallelism": "none",
                   "prefill_tok_s": round(prompt_len / prefill_s, 2) if prefill_s else None,
                   "kv_prefilled": kv_fill,
                   "token_bytes_GB": round(tb / 1e9, 4),
                   "sweep_GBs": round(tb * tps / 1e9, 1),
                   "sweep_frac": round(tb * tps / 1e9 / HBM_PEAK_GBS, 4),
                   "first_tokens": toks[:8]},
        "roofline": roof,
        "cpu_baseline": None,
    }
    if kv_fill:
        out["config"]["workload"] = ("%s, KV cache pre-filled to %d positions (fp16 N(0,1)), then %d greedy "
                                     "decode steps at batch 1, %s KV" % (cfg["name"], kv_fill, steps, args.kv))
    if streaming:
        hb = L.ss_hip_model_host_bytes(L.ss_model_hip(m.h))
        m.close()
        try:
            peak = pinned_h2d_gbs()
        except Exception as e:
            log("%s" % e)
            peak = float("nan")
        ach = hb * tps / 1e9
        out["link"] = {"bound": "host-to-device copy", "h2d_bytes_per_token": int(hb),
                       "achieved": round(ach, 2), "peak": round(peak, 2), "unit": "GB/s",
                       "frac": round(ach / peak, 4),
                       "peak_is": "pinned hipMemcpyAsync of 1 GiB x 4, measured in this run"}
    m.close()
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(path, spec, prompt_len)
        except Exception as e:
            log("cpu baseline failed: %s" % e)
    print(json.dumps(out), flush=True)


PINNED_COPY = """
import time, torch
n = 1 << 30
h = torch.empty(n, dtype=torch.uint8, pin_memory=True)
h.fill_(1)
d = torch.empty(n, dtype=torch.uint8, device="cuda")
best = 0.0
for _ in range(3):
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(4):
        d.copy_(h, non_blocking=True)
    torch.cuda.synchronize()
    best = max(best, 4 * n / (time.perf_counter() - t) / 1e9)
print(best)
"""


def pinned_h2d_gbs():
    """Host-to-device rate of a pinned 1 GiB buffer (best of three 4-copy
    runs), measured in a child process (torch is only the allocator there)."""
    import subprocess
    r = subprocess.run([sys.executable, "-c", PINNED_COPY], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise RuntimeError("pinned copy measurement failed: " + r.stderr[-300:])
    return float(r.stdout.strip().split()[-1])


def bench_matvec(args):
    """C1: y = W x for one 4096 x 4096 Q4_0 matrix (d = fp16(|N(0, 0.02)|),
    uniform random nibbles), x ~ N(0, 1), fp32 accumulation. Each timed
    launch reads the next of 40 packed copies (378 MB, more than the 256 MB
    last-level cache), so every launch streams its weights from HBM. The
    launches are timed with HIP events on the context's stream."""
    import ctypes as C
    import torch
    import oracle
    from phonemap_amd import lib
    L = lib()
    rows = cols = 4096
    ncopy, iters = 40, args.steps if args.steps is not None else 400
    rng = np.random.default_rng(0)
    nb = rows * cols // 32
    blocks = np.zeros((nb, 18), np.uint8)
    blocks[:, :2] = np.abs(rng.standard_normal(nb) * 0.02).astype(np.float16).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    ctx = L.ss_hip_init(0)
    if not ctx:
        raise SystemExit("ss_hip_init failed")
    pb = L.ss_hip_packed_bytes(2, rows, cols)
    ws = []
    for _ in range(ncopy):
        w = L.ss_hip_malloc(ctx, pb)
        if not w or L.ss_hip_pack_matrix(ctx, w, blocks.ctypes.data_as(C.c_void_p), 2, rows, cols) != 0:
            raise SystemExit("pack failed")
        ws.append(w)
    xd, yd = L.ss_hip_malloc(ctx, 4 * cols), L.ss_hip_malloc(ctx, 4 * rows)
    L.ss_hip_memcpy_h2d(ctx, xd, x.ctypes.data_as(C.c_void_p), 4 * cols)
    stream = torch.cuda.ExternalStream(L.ss_hip_stream(ctx))
    for i in range(2 * ncopy):
        L.ss_hip_matvec(ctx, yd, ws[i % ncopy], xd, rows, cols, 2, None)
    L.ss_hip_sync(ctx)
    y = np.zeros(rows, np.float32)
    L.ss_hip_memcpy_d2h(ctx, y.ctypes.data_as(C.c_void_p), yd, 4 * rows)
    ref = oracle.matvec(blocks.reshape(-1), x, rows, cols, 2)
    err = float(np.max(np.abs(y - ref)) / np.max(np.abs(ref)))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(iters):
        L.ss_hip_matvec(ctx, yd, ws[i % ncopy], xd, rows, cols, 2, None)
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / iters
    alg = nb * 18 + 4 * cols + 4 * rows
    gbs = alg / (us * 1e-6) / 1e9
    # CPU: the oracle's row-chunked GEMV (quantize.c:446-494) on the same matrix
    t = time.perf_counter()
    n = 0
    while time.perf_counter() - t < 10.0:
        oracle.matvec(blocks.reshape(-1), x, rows, cols, 2)
        n += 1
    cpu_s = (time.perf_counter() - t) / n
    threads = oracle.lib().orc_get_threads()
    for w in ws:
        L.ss_hip_mfree(ctx, w)
    L.ss_hip_mfree(ctx, xd)
    L.ss_hip_mfree(ctx, yd)
    L.ss_hip_free(ctx)
    print(json.dumps({
        "metric": "Q4_0 matvec 4096x4096 achieved HBM GB/s", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": iters, "warmup": 2 * ncopy, "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "standalone Q4_0 matvec 4096x4096, batch 1, %d rotating weight copies" % ncopy,
                   "max_rel_err_vs_oracle": err},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "k_gemv Q4_0",
                     "avg_us": round(us, 3), "bytes_per_launch": alg},
        "cpu_baseline": {"value": round(alg / cpu_s / 1e9, 2), "unit": "GB/s", "cores": int(threads),
                         "cpu": host_cpu(),
                         "kind": "port", "sample": "%d oracle GEMVs of the same matrix in %.1f s" % (n, n * cpu_s)},
    }), flush=True)


TRAFFIC_FILES = {"sweep": "traffic_llama2-7b_sweep.md", "q4_0": "traffic_llama2-7b_q4_0_matvec.md"}


def kernel_source_hash():
    """sha256 (first 16 hex digits) of the HIP sources and headers of the
    library (phonemap_amd/csrc/*.hip, *.h, sorted by name): the kernels a
    counter profile was measured on."""
    import hashlib
    h = hashlib.sha256()
    d = os.path.join(ROOT, "phonemap_amd", "csrc")
    for name in sorted(os.listdir(d)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            h.update(open(os.path.join(d, name), "rb").read())
    return h.hexdigest()[:16]


def measured_traffic(kernel_id):
    """HBM bytes per launch of the dominant kernel from the committed
    FETCH_SIZE/WRITE_SIZE counter runs (scaled by a copy kernel of known
    size), and the profile it came from; None when there is no profile or
    it was measured on other library sources than these."""
    if kernel_id not in TRAFFIC_FILES:
        return None, None
    path = os.path.join(ROOT, "profiles", TRAFFIC_FILES[kernel_id])
    fields = {}
    try:
        for line in open(path):
            k, sep, v = line.partition(":")
            if sep and k in ("traffic_bytes_per_launch", "source_hash"):
                fields[k] = v.strip()
    except OSError:
        return None, None
    name = "profiles/" + TRAFFIC_FILES[kernel_id]
    if fields.get("source_hash") != kernel_source_hash():
        return None, name + " (measured on other library sources: not used)"
    if "traffic_bytes_per_launch" not in fields:
        return None, None
    return int(fields["traffic_bytes_per_launch"]), name + " (source_hash %s)" % fields["source_hash"]


def profile_classes(m, n_steps):
    """Per-kernel-class device time over n_steps decode steps."""
    import ctypes as C
    from phonemap_amd import lib
    from phonemap_amd.api import SlipStreamError
    L = lib()
    hm = L.ss_model_hip(m.h)
    if not hm:
        raise SlipStreamError("no HIP model handle")
    if L.ss_hip_profile_begin(hm) != 0:
        raise SlipStreamError("profile_begin failed")
    m.decode_greedy(n_steps)
    out = np.zeros(15, np.float64)
    if L.ss_hip_profile_end(hm, out.ctypes.data_as(C.POINTER(C.c_double)), 15) != 0:
        err = L.ss_hip_last_error()
        raise SlipStreamError("profile_end failed: %s" % (err.decode() if err else "?"))
    if out[13] > 0:      # persistent launches: the whole token is the kernel
        ms, cnt, byt = out[12], out[13], out[14]
        kernel, kid = "k_sweep (whole token: embedding, all layers, LM head, argmax)", "sweep"
    elif out[0] >= out[3]:
        ms, cnt, byt = out[0], out[1], out[2]
        kernel, kid = "k_gemv Q4_0 (all epilogues)", "q4_0"
    else:
        ms, cnt, byt = out[3], out[4], out[5]
        kernel, kid = "k_gemv Q8_0 (all epilogues)", "q8_0"
    if cnt <= 0:
        raise SlipStreamError("no launches of the dominant kernel recorded")
    avg_s = ms / 1e3 / cnt
    ach = byt / cnt / avg_s / 1e9
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": kernel, "kernel_id": kid, "launches": int(cnt),
            "avg_us": round(avg_s * 1e6, 3), "bytes_per_launch": round(byt / cnt, 1),
            "classes_ms": {"q4_0_matvec": round(out[0], 3), "q8_0_matvec": round(out[3], 3),
                           "attention": round(out[6], 3), "other": round(out[9], 3),
                           "sweep": round(out[12], 3)},
            "profiled_steps": n_steps}


if __name__ == "__main__":
    main()
