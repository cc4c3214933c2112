#!/usr/bin/env python3
"""Benchmark: accepted tok/s of greedy prompt-lookup decoding on one MI355X.

Workload (the configuration the headline metric is quoted on): a
Mistral-7B-shaped decoder (32 layers, hidden 4096, FFN 14336, 32 q-heads /
8 kv-heads, head_dim 128, vocab 32000), random-init N(0, 0.02) weights,
symmetric int4 RTN at group 32 with f16 scales in the .raimodel layout; a
4096-token copy-heavy synthetic prompt; prompt lookup with n-gram 3, k = 8,
greedy acceptance; 256 generated tokens at batch 1.

The prompt.  A random-init model's own continuation never repeats a span of
a random-id prompt, so on such a prompt no 3-gram draft fires and the run is
plain decoding.  The bench therefore decodes the copy-heavy prompt greedily
once (the plain-decode figure), and splices that 256-token continuation,
preceded by the prompt's last three tokens, into the middle of the prompt as
an earlier span: the workload prompt still has 4096 tokens, ends like the
original, and quotes text the model goes on to produce, as the prompts
prompt lookup is meant for do.  Acceptance is whatever the model's greedy
tokens give; token identity with plain greedy decoding of the same prompt is
checked.

A step is one 256-token generation from the prefilled prompt (the KV cache
is rolled back to the prompt before each one; prefill is timed once,
separately).  `value` = generated tokens / seconds over the timed steps, with
the model and the prompt resident in HBM.  The JSON line also carries:
  roofline      the in-model verify GEMV (gate|up, 28672x4096, M = 9 tokens)
                timed with HIP events on its own stream: algorithmic bytes per
                launch / average launch time, against 8 TB/s; `traffic` from
                two rocprofv3 counter passes;
  cpu_baseline  the CPU oracle (a C++ restatement of the reference's AVX2
                path) stepping the same decoder state (its KV cache copied
                from the GPU's after the prefill) at the same context length,
                at the reference's default thread count; config.cpu_* has the
                all-cores figure and the host CPU.

The line also carries, measured in the same run: plain greedy decoding,
an exact-sampling generation (temperature 0.7, the decoder's StdRng), the
forced k = 8 verify step, the 4095-token prefill, every W4A8 shape of the
model step at 1 and 9 tokens, the prefill GEMM at M = 512 (the matrix-core
kernel; its integer-op rate against the 5 POPS int8 dense peak and its f32
epilogue rate against the VALU peak), and the other configurations:
  config 1  TinyLlama-1.1B shape, 128-token uniform prompt, greedy decode of
            128 tokens without speculation (tok/s, GB/s, HBM fraction, CPU);
  config 2  the same model, 2048-token copy-heavy prompt, prompt lookup n=3
            k=8 greedy, 256 tokens (acceptance, tokens/step, steps drafted,
            tok/s, token identity, CPU);
  config 3  the W4A8 sweep: M in {1, 5, 9, 17} on the four sweep shapes
            (µs, GB/s, HBM fraction) and M = 512 (integer-op rate against the
            int8 peak, epilogue rate against the VALU peak);
  config 5  the OLMoE-1B-7B-shaped MoE decoder, 2048-token copy-heavy prompt,
            128 tokens (grouped-expert GEMVs on the device; tok/s, plain
            decode HBM fraction, token identity, CPU).

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
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA
# f32 VALU lane operations per second at MI355X's published FP32 vector peak
# (157.3 TFLOP/s, 78.6 T fused multiply-adds): 256 CUs x 128 lanes x 2.4 GHz.
# Independent v_fmac_f32 measured on the device sustain 51.6 T/s (eight waves
# per SIMD), above the 64-lane-per-CU figure once used here.
VALU_PEAK_GOPS = 256 * 128 * 2.4


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


def roofline_shape():
    from rai_amd.workload import MISTRAL_7B
    return 2 * MISTRAL_7B["intermediate_size"], MISTRAL_7B["hidden_size"], 9


def roofline_only(gs: int) -> int:
    """The roofline GEMV launches (rotating weight copies) and one plain
    device-to-device copy of COPY_BYTES: the program the counter passes
    profile."""
    import rai_amd
    import torch
    n, k, m = roofline_shape()
    measure_gemv(rai_amd, n, k, m, gs, iters=20)
    a = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    return 0


def profile_workload(which: str) -> int:
    """One workload on its own, for a kernel trace or a counter pass:
    prefill   - Mistral-7B shape, a 4096-token copy-heavy prompt prefilled twice;
    greedy    - Mistral-7B, 2 x 64 greedy lookup tokens (n=3, k=8) after a
                4096-token prefill, then 12 verify steps with 8 forced drafts;
    sampled   - the same at temperature 0.7 (seed 42);
    olmoe     - OLMoE-1B-7B shape, 2048-token prompt, as greedy;
    tinyllama - TinyLlama-1.1B shape, 2048-token prompt, as greedy;
    gemm512   - the prefill GEMM alone: 28672 x 4096 W4A8 g32 at M = 512;
    gemv9     - the five verify-step GEMV shapes alone at M = 9.
    Step graphs are off so the trace shows every kernel launch."""
    import rai_amd
    from rai_amd.workload import MISTRAL_7B, OLMOE, TINYLLAMA, copy_heavy_prompt
    if which == "gemm512":
        n, k, _ = roofline_shape()
        ms, _, _ = measure_gemv(rai_amd, n, k, 512, 32, iters=20)
        log(f"{n}x{k} M=512: {ms * 1e3:.1f} us")
        return 0
    if which == "gemv9":
        h, f, v = MISTRAL_7B["hidden_size"], MISTRAL_7B["intermediate_size"], MISTRAL_7B["vocab_size"]
        qkv = (MISTRAL_7B["num_heads"] + 2 * MISTRAL_7B["num_kv_heads"]) * MISTRAL_7B["head_dim"]
        for n, k in ((qkv, h), (h, h), (2 * f, h), (h, f), (v, h)):
            ms, gbs, _ = measure_gemv(rai_amd, n, k, 9, 32, iters=20)
            log(f"{n}x{k} M=9: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
        return 0
    os.environ["RAI_STEP_GRAPHS"] = "0"
    s = OLMOE if which == "olmoe" else TINYLLAMA if which == "tinyllama" else MISTRAL_7B
    ctx, plen = (4096, 2048) if which in ("olmoe", "tinyllama") else (8192, 4096)
    img = rai_amd.synth_model(s["hidden_size"], s["num_layers"], s["num_heads"], s["num_kv_heads"], s["head_dim"],
                              s["intermediate_size"], s["vocab_size"], ctx, group_size=32,
                              num_experts=s.get("num_experts", 0), experts_per_token=s.get("experts_per_token", 0),
                              seed=77 if which == "olmoe" else 1234)
    model = rai_amd.RaiModel.from_bytes(img, max_groups=1024)
    del img
    dec = rai_amd.LookupDecoder(model, ctx)
    prompt = copy_heavy_prompt(plen, s["vocab_size"], seed=55)
    for _ in range(2 if which == "prefill" else 1):
        dec.kv_cache.truncate(0)
        t0 = time.perf_counter()
        pos = dec.prefill(prompt)
        rai_amd.lib().rai_device_synchronize()
        log(f"prefill {pos} tokens: {time.perf_counter() - t0:.3f}s")
    if which == "prefill":
        return 0
    t = 0.7 if which == "sampled" else 0.0
    cfg = rai_amd.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3, temperature=t)
    dec.seed(42)
    for _ in range(2):
        dec.kv_cache.truncate(pos)
        _, st = dec.decode(prompt, pos, 64, cfg)
    log(f"{which} decode: {st}")
    dec.kv_cache.truncate(pos)
    vt, _ = forced_verify_steps(dec, list(prompt), pos, cfg, 12)
    log(f"verify ms {[round(x * 1e3, 2) for x in vt]}")
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
            gemv = [v for name, vs in vals.items() if "k_gemv" in name or "k_w4a8" in name for v in vs]
            copy = [v for name, vs in vals.items() if "copy" in name.lower() or "elementwise" in name for v in vs]
            if not gemv or not copy:
                raise RuntimeError(f"{counter}: kernels not found in {list(vals)}")
            factor = (COPY_BYTES / 1024.0) / max(copy)
            res[counter] = (float(np.median(gemv)) * 1024.0 * factor, factor)
    return res


def olmoe_line(args) -> dict:
    """Config 5: OLMoE-1B-7B-shaped MoE decoder (16 layers, hidden 2048, 64
    experts top-8, expert FFN 1024, 16 heads of 128, vocab 50304), random-init
    W4A8 g32, a 2048-token copy-heavy prompt, prompt lookup n=3 k=8 greedy,
    128 generated tokens."""
    import rai_amd
    from rai_amd.workload import OLMOE, copy_heavy_prompt
    s = OLMOE
    t0 = time.perf_counter()
    img = rai_amd.synth_model(s["hidden_size"], s["num_layers"], s["num_heads"], s["num_kv_heads"], s["head_dim"],
                              s["intermediate_size"], s["vocab_size"], 4096, group_size=32,
                              num_experts=s["num_experts"], experts_per_token=s["experts_per_token"], seed=77)
    model = rai_amd.RaiModel.from_bytes(img, max_groups=1024)
    log(f"olmoe: synthetic model and upload in {time.perf_counter() - t0:.1f}s")
    cfg = rai_amd.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3, temperature=0.0)
    dec = rai_amd.LookupDecoder(model, 4096)
    prompt = copy_heavy_prompt(2048, s["vocab_size"], seed=55)
    t0 = time.perf_counter()
    pos = dec.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    ntok = 128
    dec.kv_cache.truncate(pos)
    dec.decode(prompt, pos, ntok, cfg)  # warm-up (step graphs)
    rai_amd.lib().rai_device_synchronize()
    runs = max(2, args.steps // 4)
    t0 = time.perf_counter()
    for _ in range(runs):
        dec.kv_cache.truncate(pos)
        toks, st = dec.decode(prompt, pos, ntok, cfg)
    rai_amd.lib().rai_device_synchronize()
    el = time.perf_counter() - t0
    tok_s = runs * st["generated"] / el
    dec.kv_cache.truncate(pos)
    greedy = dec.greedy_decode(prompt, pos, len(toks))  # the last lookup step may overshoot ntok
    # Plain greedy decoding from the same state: its rate gives the decode
    # step's HBM fraction (active weights + the mean context's K and V).
    t0 = time.perf_counter()
    for _ in range(runs):
        dec.kv_cache.truncate(pos)
        dec.greedy_decode(prompt, pos, ntok)
    plain_tok_s = runs * ntok / (time.perf_counter() - t0)
    wb = model.weight_bytes()
    kvpp = s["num_layers"] * 2 * s["num_kv_heads"] * s["head_dim"] * 4
    step_bytes = wb + kvpp * (pos + 1 + (ntok - 1) / 2.0)
    plain_gbs = step_bytes * plain_tok_s / 1e9
    dec.kv_cache.truncate(pos)
    vt, _ = forced_verify_steps(dec, list(prompt), pos, cfg, 18)
    vms = 1e3 * float(np.mean(vt[2:]))
    ref_threads, _ = reference_threads()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(img, s, dec, prompt, pos, toks, args.cpu_seconds / 2, ref_threads)
    log(f"olmoe: {tok_s:.1f} tok/s ({st['steps_with_draft']} steps drafted), plain decode {plain_tok_s:.1f} tok/s "
        f"({plain_gbs / HBM_PEAK_GBS:.3f} of HBM), identical to greedy: {greedy == toks}, verify step {vms:.3f} ms, "
        f"prefill {prefill_s:.2f}s" + (f", cpu {cpu[0]:.2f} tok/s" if cpu else ""))
    return {"workload": "olmoe-1b-7b-shaped W4A8 g32, 64 experts top-8, 2048-token copy-heavy prompt, "
                        "prompt-lookup n=3 k=8 greedy, 128 tokens, batch 1",
            "value_tok_s": round(tok_s, 2), "generations": runs,
            "steps_with_draft": st["steps_with_draft"], "draft_tokens": st["drafted"],
            "accepted_draft_tokens": st["accepted"],
            "acceptance_rate": round(st["accepted"] / st["drafted"], 4) if st["drafted"] else None,
            "verify_step_ms": round(vms, 4), "prefill_seconds": round(prefill_s, 4),
            "token_identical_to_greedy": greedy == toks,
            "plain_decode_tok_s": round(plain_tok_s, 2),
            "plain_decode_bytes_per_token": int(step_bytes), "plain_decode_gbs": round(plain_gbs, 1),
            "plain_decode_hbm_frac": round(plain_gbs / HBM_PEAK_GBS, 4),
            "decode_weight_bytes_per_token": wb,
            "decode_weight_gbs": round(wb * st["generated"] / (el / runs) / 1e9, 1),
            "cpu_baseline": cpu_entry(cpu, ref_threads, f"greedy lookup n=3 k=8 from the GPU's state after the "
                                                        f"{pos}-token prefill") if cpu else None}


def attention_kernels(rai, shape, pos: int, cap: int) -> dict:
    """The step's attention launches (scores, softmax, PV) for one decode
    token and a nine-token verify batch at position `pos`, each timed over
    back-to-back launches between two HIP events, rotating over enough K/V
    caches that K and V stream from HBM.  Algorithmic bytes: scores read K (n x hd x 4 per kv
    head) and q and write the score rows; the softmax reads and writes the
    score rows; PV reads V (n x hd x 4 per kv head) and the probability rows
    and writes the head outputs."""
    nh, nkv, hd = shape["num_heads"], shape["num_kv_heads"], shape["head_dim"]
    kv_bytes = 2 * nkv * cap * hd * 4
    copies = max(2, int(ROTATE_BYTES // kv_bytes) + 1)
    out = {"positions": pos + 1, "kv_cache_positions": cap}
    for m in (1, 9):
        sc, sm, pv = attention_time_median(rai, nh, nkv, hd, cap, pos, m, copies)
        n = pos + m
        rows = sum(pos + t + 1 for t in range(m)) * nh * 4  # score / probability row bytes
        b_sc = nkv * n * hd * 4 + m * nh * hd * 4 + rows
        b_sm = 2 * rows
        b_pv = nkv * n * hd * 4 + rows + m * nh * hd * 4
        ent = {}
        for nm, ms, b in (("scores", sc, b_sc), ("softmax", sm, b_sm), ("pv", pv, b_pv)):
            gbs = b / (ms * 1e-3) / 1e9
            ent[nm] = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                       "bytes": b}
        out[f"m{m}"] = ent
    return out


def attention_time_median(rai, nh, nkv, hd, cap, pos, m, copies, reps: int = 3):
    runs = [rai.attention_time(nh, nkv, hd, cap, pos, m, copies=copies, iters=20) for _ in range(reps)]
    return tuple(float(np.median([r[k] for r in runs])) for k in range(3))


def splice_prompt(base: np.ndarray, cont) -> np.ndarray:
    """The base prompt with (its last three tokens + `cont`) written over the
    positions starting at a quarter of its length; same length, same end."""
    n = len(base)
    span = np.concatenate([base[-3:], np.asarray(cont, np.uint32)])
    at = n // 4
    out = np.concatenate([base[:at], span, base[at + len(span):]]).astype(np.uint32)
    assert len(out) == n and np.array_equal(out[-3:], base[-3:])
    return out


def host_cpu() -> tuple[str, int]:
    name = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except Exception:
        n = os.cpu_count() or 1
    return name, n


def cpu_baseline(img, shape, dec, context, pos, gpu_tokens, seconds: float, threads: int, lookup: bool = True):
    """The oracle's greedy lookup steps (n=3, k=8), or with lookup=False its
    plain decode_one steps, from the GPU decoder's state after the prefill
    (every layer's K/V rows copied over), at the workload's context length,
    for about `seconds`.  Returns (tok/s, tokens, seconds, matches):
    `matches` is whether the oracle's tokens equal the GPU's."""
    from oracle import ora
    ora.set_threads(threads)
    om = ora.Model(img, 0)
    od = ora.LookupDecoder(om, len(context) + 512)
    L, nkv, hd = shape["num_layers"], shape["num_kv_heads"], shape["head_dim"]
    for layer in range(L):
        for which in (0, 1):
            od.import_kv(layer, which, dec.kv_cache.export(layer, which, pos, nkv, hd))
    ctx = list(context)
    produced = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds and produced < len(gpu_tokens):
        if lookup:
            toks, met = od.step(pos, ctx, 8, 3, 3)
            n = met.produced
        else:
            toks, n = [od.decode_one(pos, ctx[-1])], 1
        ctx += toks
        pos += n
        produced += n
    dt = time.perf_counter() - t0
    got = ctx[len(context):]
    matches = got == list(gpu_tokens[:len(got)])
    return produced / dt, produced, dt, matches


def reference_threads() -> tuple[int, int]:
    """(the reference's default thread count, the one-GPU share of the host):
    configure_thread_pool (gemm.rs:1746-1761) uses max(cpus/2 + 1, 2)."""
    _, ncpu = host_cpu()
    share = min(ncpu, 16)
    return max(share // 2 + 1, 2), share


def cpu_entry(res, threads: int, what: str) -> dict:
    cv, cprod, cdt, cmatch = res
    return {"value": round(cv, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle, {threads} threads: {what}; {cprod} tokens in {cdt:.1f}s",
            "tokens_equal_gpu": cmatch}


def config3_sweep(rai) -> dict:
    """Config 3: the isolated W4A8 sweep on the four sweep shapes (int4 g32,
    f16 scales; N(0, 1) activations quantized per group).  M in {1, 5, 9, 17}:
    HBM-bound, µs / GB/s / fraction of 8 TB/s with the weights streamed from
    HBM (rotating copies).  M = 512: the matrix-core GEMM, its integer-op rate
    against the 5 POPS int8 dense peak and its epilogue's f32 operation rate
    (11 ordered operations per row, token and group) against the VALU peak."""
    from rai_amd.workload import GEMV_SHAPES, gemv_operands
    out = {}
    for n, k in GEMV_SHAPES:
        nib, params, x = gemv_operands(n, k, 512, 32, seed=n + k)
        copies = max(1, int(-(-ROTATE_BYTES // (nib.nbytes + params.nbytes))))
        t = rai.GemvTimer(nib, params, n, k, 32, copies)
        ent = {}
        for m in (1, 5, 9, 17):
            ms = float(np.median([t.time(x[:m], m, iters=30) for _ in range(3)]))
            b = gemv_algorithmic_bytes(n, k, m, 32)
            gbs = b / (ms * 1e-3) / 1e9
            ent[f"m{m}"] = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        ms = t.time(x, 512, iters=10)
        tops = 2.0 * n * k * 512 / (ms * 1e-3) / 1e12
        valu = 11.0 * n * (k // 32) * 512 / (ms * 1e-3) / 1e9
        ent["m512"] = {"us": round(ms * 1e3, 1), "int_tops": round(tops, 1),
                       "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                       "epilogue_valu_frac": round(valu / VALU_PEAK_GOPS, 4)}
        out[f"{n}x{k}"] = ent
        del t
    log("config 3: " + "; ".join(f"{sh} " + ", ".join(f"{m} {v.get('frac', v.get('frac_of_int8_peak'))}"
                                                       for m, v in e.items()) for sh, e in out.items()))
    return out


def tinyllama_configs(args) -> tuple[dict, dict]:
    """Configs 1 and 2 on the TinyLlama-1.1B shape (22 layers, hidden 2048,
    FFN 5632, 32 q-heads / 4 kv-heads of 64, vocab 32000), random-init W4A8
    g32.  Config 1: a 128-token uniform-random prompt, greedy decoding of 128
    tokens, speculation off.  Config 2: a 2048-token copy-heavy prompt,
    prompt lookup n=3 k=8 greedy, 256 tokens.  Each with the CPU oracle on the
    same decoder state (KV copied from the GPU) and token identity."""
    import rai_amd
    from rai_amd.workload import TINYLLAMA, copy_heavy_prompt, uniform_prompt
    s = TINYLLAMA
    max_ctx = 4096
    t0 = time.perf_counter()
    img = rai_amd.synth_model(s["hidden_size"], s["num_layers"], s["num_heads"], s["num_kv_heads"], s["head_dim"],
                              s["intermediate_size"], s["vocab_size"], max_ctx, group_size=32, seed=2025)
    model = rai_amd.RaiModel.from_bytes(img, max_groups=1024)
    log(f"tinyllama: synthetic model and upload in {time.perf_counter() - t0:.1f}s")
    wb = model.weight_bytes()
    kvpp = s["num_layers"] * 2 * s["num_kv_heads"] * s["head_dim"] * 4
    ref_threads, _ = reference_threads()
    runs = 5

    # Config 1.
    p1 = uniform_prompt(128, s["vocab_size"], seed=128)
    dec = rai_amd.LookupDecoder(model, max_ctx)
    t0 = time.perf_counter()
    pos = dec.prefill(p1)
    prefill1 = time.perf_counter() - t0
    n1 = 128
    dec.greedy_decode(p1, pos, n1)  # warm-up (step graphs)
    rai_amd.lib().rai_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(runs):
        dec.kv_cache.truncate(pos)
        toks1 = dec.greedy_decode(p1, pos, n1)
    el = time.perf_counter() - t0
    tok_s1 = runs * n1 / el
    step_bytes = wb + kvpp * (pos + 1 + (n1 - 1) / 2.0)  # weights + the mean context's K and V
    gbs1 = step_bytes * tok_s1 / 1e9
    c1 = cpu_baseline(img, s, dec, p1, pos, toks1, args.cpu_seconds / 2, ref_threads, lookup=False)
    log(f"config 1: {tok_s1:.1f} tok/s, {gbs1:.0f} GB/s ({gbs1 / HBM_PEAK_GBS:.3f} of HBM); cpu {c1[0]:.2f} tok/s "
        f"(tokens equal: {c1[3]})")
    cfg1 = {"workload": "tinyllama-1.1b-shaped W4A8 g32, 128-token uniform prompt, greedy decode of 128 tokens, "
                        "speculation off, batch 1",
            "value_tok_s": round(tok_s1, 2), "generations": runs, "prefill_seconds": round(prefill1, 4),
            "bytes_per_token": int(step_bytes), "gbs": round(gbs1, 1), "hbm_frac": round(gbs1 / HBM_PEAK_GBS, 4),
            "cpu_baseline": cpu_entry(c1, ref_threads, f"plain greedy decode_one from the GPU's state after the "
                                                       f"{pos}-token prefill")}
    del dec

    # Config 2.
    p2 = copy_heavy_prompt(2048, s["vocab_size"], seed=2048)
    dec = rai_amd.LookupDecoder(model, max_ctx)
    t0 = time.perf_counter()
    pos = dec.prefill(p2)
    prefill2 = time.perf_counter() - t0
    cfg = rai_amd.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3, temperature=0.0)
    n2 = 256
    dec.decode(p2, pos, n2, cfg)  # warm-up
    rai_amd.lib().rai_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(runs):
        dec.kv_cache.truncate(pos)
        toks2, st = dec.decode(p2, pos, n2, cfg)
    el = time.perf_counter() - t0
    tok_s2 = runs * st["generated"] / el
    dec.kv_cache.truncate(pos)
    greedy2 = dec.greedy_decode(p2, pos, len(toks2))
    c2 = cpu_baseline(img, s, dec, p2, pos, toks2, args.cpu_seconds / 2, ref_threads)
    log(f"config 2: {tok_s2:.1f} tok/s, {st['accepted']}/{st['drafted']} accepted, {st['steps_with_draft']}/"
        f"{st['steps']} steps drafted; identical to greedy: {greedy2 == toks2}; cpu {c2[0]:.2f} tok/s")
    cfg2 = {"workload": "tinyllama-1.1b-shaped W4A8 g32, 2048-token copy-heavy prompt, prompt-lookup n=3 k=8 "
                        "greedy, 256 tokens, batch 1",
            "value_tok_s": round(tok_s2, 2), "generations": runs, "prefill_seconds": round(prefill2, 4),
            "decoder_steps": st["steps"], "steps_with_draft": st["steps_with_draft"],
            "pct_steps_drafted": round(100.0 * st["steps_with_draft"] / max(st["steps"], 1), 2),
            "draft_tokens": st["drafted"], "accepted_draft_tokens": st["accepted"],
            "acceptance_rate": round(st["accepted"] / st["drafted"], 4) if st["drafted"] else None,
            "tokens_per_step": round(st["generated"] / max(st["steps"], 1), 4),
            "token_identical_to_greedy": greedy2 == toks2,
            "cpu_baseline": cpu_entry(c2, ref_threads, f"greedy lookup n=3 k=8 from the GPU's state after the "
                                                       f"{pos}-token prefill")}
    return cfg1, cfg2


def forced_verify_steps(dec, context, pos: int, cfg, n_steps: int):
    """Decoder steps whose draft is forced: before each step the context's
    last three tokens are overwritten with an earlier 3-gram, so the n-gram
    search returns a full k = 8 draft and the step runs the 9-token verify
    forward, lm_head and argmax, greedy acceptance and the KV rollback."""
    ctx = list(context)
    times, drafted = [], 0
    for i in range(n_steps):
        src = 64 + 53 * i
        ctx[-3:] = ctx[src:src + 3]
        t0 = time.perf_counter()
        toks, met = dec.step(pos, ctx, cfg)
        times.append(time.perf_counter() - t0)
        drafted += met.drafted
        ctx += toks
        pos += met.produced
    return times, drafted


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="timed 256-token generations")
    ap.add_argument("--warmup", type=int, default=2, help="untimed generations before timing")
    ap.add_argument("--tokens", type=int, default=256, help="tokens per generation")
    ap.add_argument("--workload", choices=["mistral7b", "tinyllama"], default="mistral7b")
    ap.add_argument("--prompt", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--no-olmoe", action="store_true", help="skip the config-5 (OLMoE) measurement")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations' figures (configs 1, 2, 3 and 5)")
    ap.add_argument("--roofline-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--profile", choices=["prefill", "greedy", "sampled", "olmoe", "tinyllama", "gemm512", "gemv9"],
                    help="run one workload alone (for rocprofv3) and print no JSON line")
    args = ap.parse_args()
    if args.roofline_only:
        return roofline_only(32)
    if args.profile:
        return profile_workload(args.profile)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1"}))
        return 2

    import rai_amd
    from rai_amd.workload import MISTRAL_7B, TINYLLAMA, copy_heavy_prompt

    shape = dict(MISTRAL_7B if args.workload == "mistral7b" else TINYLLAMA)
    prompt_len = args.prompt or (4096 if args.workload == "mistral7b" else 2048)
    max_ctx = 8192 if args.workload == "mistral7b" else 4096
    gs, ntok = 32, args.tokens
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

    cfg = rai_amd.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3, temperature=0.0)
    dec = rai_amd.LookupDecoder(model, max_ctx)
    base = copy_heavy_prompt(prompt_len, shape["vocab_size"], seed=2026)
    cont, st0 = dec.generate(base, ntok, cfg)
    plain_tok_s = st0["generated"] / st0["decode_seconds"]
    log(f"base prompt: prefill {st0['prefill_seconds']:.2f}s, plain decode {st0['generated']} tokens "
        f"at {plain_tok_s:.1f} tok/s ({st0['steps_with_draft']} steps drafted)")

    prompt = splice_prompt(base, cont)
    t0 = time.perf_counter()
    pos = dec.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    log(f"workload prompt: prefill {pos} tokens in {prefill_s:.2f}s")

    for _ in range(args.warmup):
        dec.kv_cache.truncate(pos)
        dec.decode(prompt, pos, ntok, cfg)
    rai_amd.lib().rai_device_synchronize()
    t0 = time.perf_counter()
    runs = []
    for _ in range(args.steps):
        dec.kv_cache.truncate(pos)
        runs.append(dec.decode(prompt, pos, ntok, cfg))
    rai_amd.lib().rai_device_synchronize()
    elapsed = time.perf_counter() - t0
    toks, st = runs[-1]
    gen = sum(r[1]["generated"] for r in runs)
    value = gen / elapsed
    same_runs = all(r[0] == toks for r in runs)
    log(f"timed: {args.steps} generations, {gen} tokens in {elapsed:.3f}s = {value:.1f} tok/s; "
        f"{st['steps']} decoder steps per generation ({st['steps_with_draft']} drafted, "
        f"{st['accepted']}/{st['drafted']} draft tokens accepted)")

    greedy = rai_amd.LookupDecoder(model, max_ctx).greedy_generate(prompt, len(toks))
    identical = greedy == toks and same_runs
    log(f"token identity with plain greedy decoding: {identical}")

    # Exact sampling (temperature 0.7, the decoder's StdRng): same prompt.
    scfg = rai_amd.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3, temperature=0.7)
    dec.seed(42)
    dec.kv_cache.truncate(pos)
    dec.decode(prompt, pos, 32, scfg)
    rai_amd.lib().rai_device_synchronize()
    t0 = time.perf_counter()
    sruns = 3
    for _ in range(sruns):
        dec.kv_cache.truncate(pos)
        stoks, sst = dec.decode(prompt, pos, ntok, scfg)
    rai_amd.lib().rai_device_synchronize()
    sampled_tok_s = sruns * sst["generated"] / (time.perf_counter() - t0)
    log(f"exact sampling (T=0.7): {sampled_tok_s:.1f} tok/s, {sst['accepted']}/{sst['drafted']} accepted")

    # Verify-step time on forced drafts at the same context (graphs warm).
    dec.kv_cache.truncate(pos)
    vt, vdrafted = forced_verify_steps(dec, list(prompt), pos, cfg, 34)
    verify_step_ms = 1e3 * float(np.mean(vt[2:]))
    log(f"forced-draft verify steps: {verify_step_ms:.3f} ms/step")

    # Every W4A8 shape of the model step at the verify (9) and decode (1) sizes.
    H, F, V = shape["hidden_size"], shape["intermediate_size"], shape["vocab_size"]
    qd, kvd = shape["num_heads"] * shape["head_dim"], shape["num_kv_heads"] * shape["head_dim"]
    shapes = {"qkv": (qd + 2 * kvd, H), "o_proj": (H, qd), "gate_up": (2 * F, H), "down": (H, F),
              "lm_head": (V, H)}
    kern = {}
    for nm, (n, k) in shapes.items():
        for m in (9, 1):
            ms, gbs, _ = measure_gemv(rai_amd, n, k, m, gs)
            kern[f"{nm}_{n}x{k}_m{m}"] = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                                          "frac": round(gbs / HBM_PEAK_GBS, 4)}
    log("GEMVs: " + ", ".join(f"{k} {v['us']}us {v['frac']:.3f}" for k, v in kern.items()))
    attn = attention_kernels(rai_amd, shape, len(prompt) - 1, max_ctx)
    log("attention: " + ", ".join(f"{k} {v}" for k, v in attn.items() if isinstance(v, dict)))
    # The prefill GEMM (matrix cores) at M = 512 on gate|up.
    pn, pk, pm = 2 * F, H, 512
    pms, _, _ = measure_gemv(rai_amd, pn, pk, pm, gs, iters=20)
    p_tops = 2.0 * pn * pk * pm / (pms * 1e-3) / 1e12
    p_valu = 11.0 * pn * (pk // gs) * pm / (pms * 1e-3) / 1e9
    prefill_gemm = {"shape": f"{pn}x{pk} M={pm}", "us": round(pms * 1e3, 1), "int_tops": round(p_tops, 1),
                    "frac_of_int8_peak": round(p_tops / INT8_PEAK_TOPS, 4),
                    "epilogue_valu_frac": round(p_valu / VALU_PEAK_GOPS, 4),
                    "note": "11 ordered f32 VALU operations per (row, token, group) bound this kernel; the matrix "
                            "cores compute the exact integer sums"}
    log(f"prefill GEMM {pn}x{pk} M={pm}: {pms * 1e3:.1f} us, {p_tops:.1f} int TOPS, epilogue at "
        f"{p_valu / VALU_PEAK_GOPS:.2f} of the VALU peak")
    rn, rk, rm = roofline_shape()
    # The median of five 20-launch averages: the launch pattern of the
    # `--roofline-only` program whose kernel trace is the rocprof summary.
    reps = sorted(measure_gemv(rai_amd, rn, rk, rm, gs, iters=20) for _ in range(5))
    vms, vgbs, vbytes = reps[len(reps) // 2]
    log(f"roofline GEMV {rn}x{rk} M={rm}: {vms * 1e3:.2f} us, {vgbs:.0f} GB/s")

    traffic = None
    if not args.no_traffic:
        try:
            t = measure_traffic(gs)
            if t is not None:
                traffic = round(t["FETCH_SIZE"][0] + t["WRITE_SIZE"][0])
                log(f"roofline GEMV HBM traffic {traffic / 1e6:.2f} MB/launch (fetch x{t['FETCH_SIZE'][1]:.3f}, "
                    f"write x{t['WRITE_SIZE'][1]:.3f}) vs {vbytes / 1e6:.2f} MB algorithmic")
        except Exception as e:  # the counter passes are a report, not the run
            log(f"traffic passes failed: {e}")

    cpu, cpu_all, cpu_name = None, None, None
    if not args.no_cpu:
        cpu_name, _ = host_cpu()
        ref_threads, share = reference_threads()
        res = {}
        for th in (ref_threads, share):
            res[th] = cpu_baseline(img, shape, dec, prompt, pos, toks, args.cpu_seconds, th)
            log(f"cpu baseline {res[th][0]:.3f} tok/s on {th} threads ({res[th][1]} tokens, "
                f"tokens equal the GPU's: {res[th][3]})")
        cv, cprod, cdt, cmatch = res[ref_threads]
        cpu = {"value": round(cv, 3), "unit": "tok/s", "cores": ref_threads, "kind": "port",
               "sample": (f"CPU oracle (C++ AVX2 restatement of the reference path) on {cpu_name}, "
                          f"{ref_threads} threads (the reference default max(cpus/2+1, 2) for a "
                          f"{share}-CPU share): greedy lookup n=3 k=8 from the same decoder state "
                          f"(KV copied from the GPU after the {pos}-token prefill), {cprod} tokens in "
                          f"{cdt:.1f}s, tokens equal to the GPU's: {cmatch}")}
        cpu_all = {"value": round(res[share][0], 3), "threads": share, "tokens_equal_gpu": res[share][3]}
    del img
    del dec, model
    cfg1 = cfg2 = cfg3 = cfg5 = None
    if not args.no_configs:
        # Secondary figures: a failure is reported, and does not fail the line.
        try:
            cfg3 = config3_sweep(rai_amd)
        except Exception as e:
            log(f"config 3 measurement failed: {e}")
        try:
            cfg1, cfg2 = tinyllama_configs(args)
        except Exception as e:
            log(f"configs 1 and 2 measurement failed: {e}")
    if not args.no_olmoe and not args.no_configs:
        try:
            cfg5 = olmoe_line(args)
        except Exception as e:
            log(f"config 5 measurement failed: {e}")

    line = {
        "metric": "accepted tok/s, 7B W4A8 + prompt-lookup; W4A8 GEMV % of HBM peak",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8 (int32 accumulate, f32 epilogue)",
        "data": "synthetic (random-init N(0,0.02) weights; copy-heavy random-id prompt quoting the model's "
                "own greedy continuation)",
        "config": {
            "workload": (f"{args.workload}-shaped W4A8 g32, {prompt_len}-token copy-heavy prompt, prompt-lookup "
                         f"n=3 k=8 greedy, {ntok} tokens per step, batch 1"),
            "tokens_per_generation": st["generated"],
            "decoder_steps_per_generation": st["steps"],
            "steps_with_draft": st["steps_with_draft"],
            "draft_tokens": st["drafted"],
            "accepted_draft_tokens": st["accepted"],
            "acceptance_rate": round(st["accepted"] / st["drafted"], 4) if st["drafted"] else None,
            "tokens_per_step": round(st["generated"] / max(st["steps"], 1), 4),
            "token_identical_to_greedy": identical,
            "prefill_seconds": round(prefill_s, 4),
            "plain_decode_tok_s": round(plain_tok_s, 2),
            "sampled_t0.7_tok_s": round(sampled_tok_s, 2),
            "acceptance_note": ("random-init weights: the model's greedy continuation is a chaotic function of "
                                "the whole context and never repeats a prompt span, so drafts are rarely "
                                "accepted and the step is plain decoding plus the occasional failed verify"),
            "prefill_gemm_m512": prefill_gemm,
            "config1_tinyllama_greedy": cfg1,
            "config2_tinyllama_lookup": cfg2,
            "config3_w4a8_sweep": cfg3,
            "config5_olmoe": cfg5,
            "verify_step_ms": round(verify_step_ms, 4),
            "verify_step_note": (f"{len(vt) - 2} timed decoder steps with a forced k=8 draft ({vdrafted} drafted "
                                 f"over {len(vt)}): 9-token verify forward + lm_head + argmax + acceptance + "
                                 f"KV rollback"),
            "gemv_kernels": kern,
            "attention_kernels": attn,
            "cpu_host": cpu_name,
            "cpu_all_cores": cpu_all,
        },
        "roofline": {"bound": "hbm", "achieved": round(vgbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(vgbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": f"w4a8 GEMV gate|up {rn}x{rk} g{gs} M={rm}", "bytes_per_launch": vbytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
