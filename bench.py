"""Batch-1 decode benchmark of the SlipStream token loop on one MI355X.

Default workload: Llama-2-7B-shape decoder with random-init weights (32
layers, d 4096, 32 heads = 32 KV heads of dim 128, FFN 11008, vocab 32000),
Q4_0 layer matrices with Q8_0 token_embd/output, a 512-token random prompt,
then greedy decode at batch 1 with an fp16 KV cache. A "step" is one decode
token: embedding, 32 layers, output norm, LM head, argmax.

Prints one JSON line. `value` is decode tokens/s over exactly --steps decode
steps (after --warmup untimed ones), with the weights resident in HBM. The
roofline object is for the dominant kernel: with the default launch mode
(one persistent launch per token) that is the whole-token kernel, whose
algorithmic bytes are every weight byte of the token once plus the KV cache
read; with per-kernel launches it is the Q4_0 matvec class. It is measured
with HIP events on the model stream around each launch in a profiled replay
of further decode steps. cpu_baseline is the CPU oracle (the reference path
restated in C) on the same GGUF, timed on this host on a bounded sample.
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
                                out_type=8, seed=7), prompt=512, steps=256,
                      name="llama2-7b-shape, Q4_0 layers + Q8_0 token_embd/output"),
    "tinyllama": dict(spec=dict(n_layers=22, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=64,
                                ffn=5632, vocab=32000, context_length=2048, layer_type=2, embd_type=2,
                                out_type=2, seed=1001), prompt=32, steps=128,
                      name="tinyllama-1.1b-shape, all Q4_0"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


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
            "sample": "%d decode steps at context %d (KV pre-filled), same GGUF, %d threads, %.1f s"
                      % (n, prompt_len + 1, threads, dt)}


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
    ap.add_argument("--config", default="llama2-7b", choices=sorted(CONFIGS))
    ap.add_argument("--kv", default="f16", choices=["f16", "int8"])
    ap.add_argument("--model-dir", default=os.environ.get("SS_BENCH_DIR", "/tmp"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--launch", default="graph", choices=["graph", "sweep", "eager"],
                    help="per-kernel launches replayed from a HIP graph (default), one persistent "
                         "launch per token, or per-kernel launches issued eagerly")
    ap.add_argument("--profile-steps", type=int, default=16)
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

    from phonemap_amd import api
    cfg = CONFIGS[args.config]
    spec = cfg["spec"]
    steps = args.steps if args.steps is not None else cfg["steps"]
    warm = args.warmup
    prompt_len = args.prompt_len if args.prompt_len is not None else cfg["prompt"]
    path = os.path.join(args.model_dir, "ss_bench_%s_s%d.gguf" % (args.config, spec["seed"]))
    if not os.path.exists(path):
        t = time.perf_counter()
        api.write_synthetic_gguf(path + ".part", api.SynthSpec(**spec))
        os.replace(path + ".part", path)
        log("wrote %s (%.2f GB) in %.1f s" % (path, os.path.getsize(path) / 1e9, time.perf_counter() - t))
    max_ctx = prompt_len + warm + steps + args.profile_steps + 2
    t = time.perf_counter()
    m = api.Model(path, max_context=max_ctx, kv=args.kv, launch=args.launch)
    log("loaded in %.1f s" % (time.perf_counter() - t))
    L = api._lib()
    rng = np.random.default_rng(1234)
    prompt = rng.integers(3, spec["vocab"], prompt_len).tolist()

    m.reset()
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
        roof = profile_classes(m, args.profile_steps)
        if args.config == "llama2-7b" and args.kv == "f16" and args.prompt_len is None:
            roof["traffic"] = measured_traffic(roof["kernel_id"])   # counter runs of this workload
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
                   "prefill_tok_s": round(prompt_len / prefill_s, 2),
                   "token_bytes_GB": round(tb / 1e9, 4),
                   "sweep_GBs": round(tb * tps / 1e9, 1),
                   "sweep_frac": round(tb * tps / 1e9 / HBM_PEAK_GBS, 4),
                   "first_tokens": toks[:8]},
        "roofline": roof,
        "cpu_baseline": None,
    }
    m.close()
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(path, spec, prompt_len)
        except Exception as e:
            log("cpu baseline failed: %s" % e)
    print(json.dumps(out), flush=True)


TRAFFIC_FILES = {"sweep": "traffic_llama2-7b_sweep.md", "q4_0": "traffic_llama2-7b_q4_0_matvec.md"}


def measured_traffic(kernel_id):
    """HBM bytes per launch of the dominant kernel from the committed
    FETCH_SIZE/WRITE_SIZE counter runs (scaled by a copy kernel of known
    size), or None."""
    path = os.path.join(ROOT, "profiles", TRAFFIC_FILES[kernel_id])
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


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
        raise SlipStreamError("profile_end failed")
    if out[13] > 0:      # persistent launches: the whole token is the kernel
        ms, cnt, byt = out[12], out[13], out[14]
        kernel, kid = "k_sweep (whole token: embedding, all layers, LM head, argmax)", "sweep"
    else:
        ms, cnt, byt = out[0], out[1], out[2]
        kernel, kid = "k_gemv Q4_0 (all epilogues)", "q4_0"
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
