#!/usr/bin/env python3
"""Benchmark: accepted tok/s of greedy prompt-lookup decoding on one MI355X.

Workload (the configuration the headline metric is quoted on): a
Mistral-7B-shaped decoder (32 layers, hidden 4096, FFN 14336, 32 q-heads /
8 kv-heads, head_dim 128, vocab 32000), random-init N(0, 0.02) weights,
symmetric int4 RTN at group 32 with f16 scales in the .raimodel layout; a
4096-token copy-heavy synthetic prompt; prompt lookup with n-gram 3, k = 8,
greedy acceptance; 256 generated tokens at batch 1.

A "step" is one decoded token; `value` = generated tokens / decode seconds
(prefill timed separately, weights and prompt resident in HBM before the
timed region).  The JSON line also carries:
  roofline      the W4A8 verify GEMV (M = 9 tokens, 14336x4096, the largest
                per-layer matrix) timed with HIP events on its own stream:
                algorithmic bytes per launch / average launch time vs 8 TB/s;
  cpu_baseline  the CPU oracle (a C++ restatement of the reference's AVX2
                path) timed on a bounded sample on this host.

`--gpus N` with N > 1 is refused: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_algorithmic_bytes(n: int, k: int, m: int, gs: int) -> int:
    # Packed nibbles + f16 (scale, zero) per group + f32 activations in/out
    # (the reference gemm-bench weight bytes, bin/gemm_bench.rs:73, plus I/O).
    return n * k // 2 + n * (-(-k // gs)) * 4 + m * k * 4 + m * n * 4


# Weight copies the GEMV timer rotates over: together well past the MI355X's
# 256 MB last-level cache, so every timed launch streams its weights from HBM
# as it does inside a model step (one copy would be served from that cache).
ROTATE_BYTES = 640e6


def measure_gemv(rai, n, k, m, gs, iters=50):
    from rai_amd.workload import gemv_operands
    nib, params, x = gemv_operands(n, k, m, gs, seed=n + k + m)
    copies = max(1, int(-(-ROTATE_BYTES // (nib.nbytes + params.nbytes))))
    ms = rai.w4a8_time(nib, params, x, n, k, m, gs, iters=iters, copies=copies)
    b = gemv_algorithmic_bytes(n, k, m, gs)
    return ms, b / (ms * 1e-3) / 1e9, b


COPY_BYTES = 256 << 20  # the plain device copy whose counters calibrate the traffic pass


def roofline_only(gs: int) -> int:
    """The roofline GEMV launches (rotating weight copies) and one plain
    device-to-device copy of COPY_BYTES: the program the counter passes
    profile."""
    import rai_amd
    import torch
    from rai_amd.workload import MISTRAL_7B
    n, k = MISTRAL_7B["intermediate_size"], MISTRAL_7B["hidden_size"]
    measure_gemv(rai_amd, n, k, 9, gs, iters=20)
    a = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    return 0


def _counter_pass(counter: str, gs: int, tmp: str):
    """Run `bench.py --roofline-only` under one rocprofv3 counter pass; return
    {kernel name: [per-dispatch values]}."""
    import csv
    import subprocess
    out = os.path.join(tmp, counter)
    cmd = ["timeout", "-s", "KILL", "150", "rocprofv3", "--pmc", counter, "-f", "csv", "-d", out, "-o", "c",
           "--", sys.executable, os.path.abspath(__file__), "--roofline-only"]
    r = subprocess.run(cmd, cwd=tmp, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"rocprofv3 --pmc {counter} exited {r.returncode}: {r.stderr[-400:]}")
    vals = {}
    for root, _, files in os.walk(out):
        for f in files:
            if f.endswith("counter_collection.csv"):
                for row in csv.DictReader(open(os.path.join(root, f))):
                    if row["Counter_Name"] == counter:
                        vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return vals


def measure_traffic(gs: int):
    """HBM bytes per launch of the roofline GEMV from FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch), each scaled by what the counter reads for the plain
    copy of COPY_BYTES (read and written once).  None when rocprofv3 is
    absent."""
    import shutil
    import tempfile
    if not shutil.which("rocprofv3"):
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        res = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            vals = _counter_pass(counter, gs, tmp)
            gemv = [v for name, vs in vals.items() if "k_gemv" in name for v in vs]
            copy = [v for name, vs in vals.items() if "copy" in name.lower() or "elementwise" in name for v in vs]
            if not gemv or not copy:
                raise RuntimeError(f"{counter}: kernels not found in {list(vals)}")
            factor = (COPY_BYTES / 1024.0) / max(copy)
            res[counter] = (float(np.median(gemv)) * 1024.0 * factor, factor)
    return res


def cpu_baseline(img: bytes, cfg: dict, seconds: float, prompt_len: int, threads: int):
    """Oracle (C++ restatement of the reference AVX2 path) on a bounded sample:
    same model, a short copy-heavy prompt, greedy lookup steps for ~`seconds`."""
    from oracle import ora
    from rai_amd.workload import copy_heavy_prompt
    ora.set_threads(threads)
    m = ora.Model(img, 0)
    prompt = copy_heavy_prompt(prompt_len, cfg["vocab_size"], seed=11).astype(np.int32)
    dec = ora.LookupDecoder(m, prompt_len + 512)
    pos = dec.prefill(prompt)
    ctx = prompt.tolist()
    produced = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        toks, met = dec.step(pos, ctx, 8, 3, 3)
        ctx += toks
        pos += met.produced
        produced += met.produced
    dt = time.perf_counter() - t0
    return produced / dt, produced, dt


def forced_verify_steps(dec, context, pos: int, cfg, n_steps: int):
    """Decoder steps whose draft is forced: before each step the context's
    last three tokens are overwritten with an earlier 3-gram, so the n-gram
    search returns a full k = 8 draft and the step runs the 9-token verify
    forward, lm_head and argmax, greedy acceptance and the KV rollback.  Only
    the timing is meaningful (the token stream is not the model's own)."""
    ctx = list(context)
    times, drafted, accepted = [], 0, 0
    for i in range(n_steps):
        src = 64 + 53 * i
        ctx[-3:] = ctx[src:src + 3]
        t0 = time.perf_counter()
        toks, met = dec.step(pos, ctx, cfg)
        times.append(time.perf_counter() - t0)
        drafted += met.drafted
        accepted += met.accepted
        ctx += toks
        pos += met.produced
    return times, drafted, accepted


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="tokens to generate (timed)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode tokens before timing")
    ap.add_argument("--workload", choices=["mistral7b", "tinyllama"], default="mistral7b")
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--roofline-only", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.roofline_only:
        return roofline_only(32)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1"}))
        return 2

    import rai_amd
    from rai_amd.workload import MISTRAL_7B, TINYLLAMA, copy_heavy_prompt

    shape = dict(MISTRAL_7B if args.workload == "mistral7b" else TINYLLAMA)
    prompt_len = args.prompt or (4096 if args.workload == "mistral7b" else 2048)
    max_ctx = 8192 if args.workload == "mistral7b" else 4096
    gs = 32
    name, cus = rai_amd.device_info()
    log(f"device {name}, {cus} CUs; workload {args.workload}")

    t0 = time.perf_counter()
    img = rai_amd.synth_model(shape["hidden_size"], shape["num_layers"], shape["num_heads"],
                              shape["num_kv_heads"], shape["head_dim"], shape["intermediate_size"],
                              shape["vocab_size"], max_ctx, group_size=gs, seed=1234)
    log(f"synthetic model {len(img) / 1e9:.2f} GB in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    model = rai_amd.RaiModel.from_bytes(img, max_groups=1024)
    log(f"upload {time.perf_counter() - t0:.1f}s; weight bytes/step {model.weight_bytes() / 1e9:.3f} GB")

    prompt = copy_heavy_prompt(prompt_len, shape["vocab_size"], seed=2026)
    cfg = rai_amd.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3, temperature=0.0)
    dec = rai_amd.LookupDecoder(model, max_ctx)
    # Warm-up run (untimed): prefill + a few tokens, then the timed run on a
    # fresh decoder state (same prompt, so the same token stream).
    if args.warmup > 0:
        _, wst = dec.generate(prompt[:512], args.warmup, cfg)
        log(f"warm-up: {wst['generated']} tokens")
    dec = rai_amd.LookupDecoder(model, max_ctx)
    toks, st = dec.generate(prompt, args.steps, cfg)
    decode_s = st["decode_seconds"]
    gen = st["generated"]
    value = gen / decode_s
    log(f"prefill {prompt_len - 1} tokens in {st['prefill_seconds']:.2f}s; decode {gen} tokens in "
        f"{decode_s:.3f}s over {st['steps']} steps ({st['steps_with_draft']} drafted, "
        f"{st['accepted']}/{st['drafted']} draft tokens accepted)")

    # The synthetic workload's model is random, so its own continuations
    # rarely repeat a prompt span and few steps draft.  Time the verify step
    # itself on forced drafts at the same context length.
    vt, vdrafted, vaccepted = forced_verify_steps(dec, list(prompt) + list(toks),
                                                  prompt_len - 1 + len(toks), cfg, 33)
    verify_step_ms = 1e3 * float(np.mean(vt[1:]))
    log(f"forced-draft verify steps: {verify_step_ms:.3f} ms/step ({vdrafted} drafted, "
        f"{vaccepted} accepted over {len(vt)} steps)")

    # Verify-GEMV roofline: the dominant W4A8 matrix at the verify batch size.
    n, k = shape["intermediate_size"], shape["hidden_size"]
    vms, vgbs, vbytes = measure_gemv(rai_amd, n, k, 9, gs)
    dms, dgbs, _ = measure_gemv(rai_amd, n, k, 1, gs)
    log(f"verify GEMV {n}x{k} M=9: {vms * 1e3:.1f} us, {vgbs:.0f} GB/s; M=1: {dms * 1e3:.1f} us, "
        f"{dgbs:.0f} GB/s")

    traffic = None
    if not args.no_traffic:
        try:
            t = measure_traffic(gs)
            if t is not None:
                traffic = round(t["FETCH_SIZE"][0] + t["WRITE_SIZE"][0])
                log(f"verify GEMV HBM traffic {traffic / 1e6:.2f} MB/launch (fetch {t['FETCH_SIZE'][0] / 1e6:.2f} "
                    f"MB x{t['FETCH_SIZE'][1]:.3f}, write {t['WRITE_SIZE'][0] / 1e6:.2f} MB "
                    f"x{t['WRITE_SIZE'][1]:.3f}) vs {vbytes / 1e6:.2f} MB algorithmic")
        except Exception as e:  # the counter passes are a report, not the run
            log(f"traffic passes failed: {e}")

    cpu = None
    if not args.no_cpu:
        threads = os.cpu_count() or 1
        try:
            import psutil
            threads = len(psutil.Process().cpu_affinity()) or threads
        except Exception:
            pass
        threads = min(threads, 16)
        cv, cprod, cdt = cpu_baseline(img, shape, args.cpu_seconds, 64, threads)
        cpu = {"value": round(cv, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": (f"CPU oracle (C++ AVX2 restatement of the reference path), same "
                          f"{args.workload} model, 64-token copy-heavy prompt (prefill excluded), "
                          f"greedy lookup n=3 k=8, {cprod} tokens in {cdt:.1f}s")}
        log(f"cpu baseline {cv:.3f} tok/s on {threads} threads")
    del img

    line = {
        "metric": "accepted tok/s, 7B W4A8 + prompt-lookup; W4A8 GEMV % of HBM peak",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": gen,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * decode_s / max(gen, 1), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8 (int32 accumulate, f32 epilogue)",
        "data": "synthetic (random-init N(0,0.02) weights, copy-heavy random-id prompt)",
        "config": {
            "workload": (f"{args.workload}-shaped W4A8 g32, {prompt_len}-token copy-heavy prompt, "
                         f"prompt-lookup n=3 k=8 greedy, {args.steps} tokens, batch 1"),
            "prefill_seconds": round(st["prefill_seconds"], 4),
            "decode_steps": st["steps"],
            "steps_with_draft": st["steps_with_draft"],
            "draft_tokens": st["drafted"],
            "accepted_draft_tokens": st["accepted"],
            "acceptance_rate": round(st["accepted"] / st["drafted"], 4) if st["drafted"] else None,
            "tokens_per_step": round(gen / max(st["steps"], 1), 4),
            "verify_step_ms": round(verify_step_ms, 4),
            "verify_step_note": (f"{len(vt) - 1} timed steps with a forced k=8 draft "
                                 f"({vdrafted} drafted, {vaccepted} accepted): 9-token verify "
                                 f"forward + lm_head + argmax + acceptance + KV rollback"),
            "verify_gemv_us": round(vms * 1e3, 2),
            "decode_gemv_us": round(dms * 1e3, 2),
            "decode_gemv_gbs": round(dgbs, 1),
        },
        "roofline": {"bound": "hbm", "achieved": round(vgbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(vgbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": f"w4a8 GEMV {n}x{k} g{gs} M=9", "bytes_per_launch": vbytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
