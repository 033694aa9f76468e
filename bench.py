"""Benchmark: causal attention fwd+bwd on one MI355X (BASELINE.json metric).

A step is one fused forward (wha_attn_fwd: online softmax, the T x T score
matrix is never materialised; writes O and the row log-sum-exp) plus one fused
backward (wha_attn_bwd: P recomputed on chip from the saved LSE) over the whole
headline batch -- 768-dim config: B=8 sequences, H=12 heads, T=1024,
head_dim 64, fp32 -- with Q, K, V, dO drawn from the seeded generator (seed 42)
and already resident in HBM.  Outputs and the backward workspace are
preallocated, so the timed region holds only kernel launches.

Before any timed region the step is repeated for at least --settle seconds
(after the --warmup steps) so the GPU clocks have ramped; the line states that
time as warmup_s.  The headline `value` and `ms_per_step` come from exactly
--steps un-instrumented steps between two synchronisations.  Per-kernel
durations (kernel_ms, roofline) come from a separate region of the same
--steps steps with HIP events the library records on the launch stream around
each kernel.

Beside the headline the same JSON line carries:
  kept_scores  the training pair that keeps the forward's scores for the
               backward (wha_attn_fwd_keep / wha_attn_bwd_kept), same batch;
  configs      GPU-only results for every other BASELINE config (168-dim,
               384-dim, 4096 preset: both pairs; 768 decode: HBM GB/s);
  parity       max-abs / relative-L2 of the headline outputs against the CPU
               f32 oracle run as the CPU baseline (same seeded inputs);
  cpu_baseline the reference-order f32 oracle, one thread per sequence.

    python bench.py [--steps K] [--warmup W] [--config 768|384|168|4096|decode|wave|wavedecode|layer|probs]
                    [--kept] [--no-suite] [--no-cpu-baseline]

--config other than 768 prints that workload's line alone (used to profile one
workload).  --kept makes the kept-scores pair the one a single-config line
times.  --config wave measures the wave (harmonic coherence) attention layer
the reference trains with; --config layer the dot-product attention layer with
its c_attn / c_proj projections (ComputeBackend::attention) forward and
backward; --config probs the exact-contract backward (att given).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix peak
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E

CONFIGS = {
    "168": dict(name="168-dim research config", B=4, H=4, T=256, D=42),
    "384": dict(name="384-dim grammar config", B=16, H=8, T=512, D=48),
    "768": dict(name="768-dim production config", B=8, H=12, T=1024, D=64),
    "4096": dict(name="4096-dim preset", B=4, H=32, T=2048, D=128),
    "decode": dict(name="768-dim decode (serve tier)", B=64, H=12, T=8192, D=64),
    "wave": dict(name="768-dim wave attention (harmonic coherence, content 16), full fwd+bwd", B=8, H=12,
                 T=1024, D=64, C=16),
    "wavedecode": dict(name="768-dim wave-attention KV-cache decode (serve tier), 64 sequences x 8192 cached",
                       B=64, H=12, T=8192, D=64, C=16),
    "layer": dict(name="768-dim ComputeBackend::attention layer (c_attn, causal core, c_proj), fwd+bwd",
                  B=8, H=12, T=1024, D=64),
    "probs": dict(name="768-dim core, backward from the given att (the exact attention_backward contract)",
                  B=8, H=12, T=1024, D=64),
}

METRIC = "causal attn fwd+bwd tokens/s & TFLOP/s (% fp32 MFMA peak), 768-dim seq1024"
ATTN_KERNELS = ("attn_fwd", "attn_bwd_delta", "attn_bwd_dq", "attn_bwd_dkv")


def credited_flops(B, H, T, D):
    P = T * (T + 1) // 2
    return {"attn_fwd": 4 * B * H * D * P,            # Q K^T and P V
            "attn_bwd_dkv": 6 * B * H * D * P,        # dP = dO V^T, dV = P^T dO, dK = dS^T Q
            "attn_bwd_dq": 2 * B * H * D * P,         # dQ = dS K
            "attn_bwd_delta": 0,
            "total": 12 * B * H * D * P}


def settle(step, args, torch, min_s=None):
    """--warmup untimed steps, then more steps until at least min_s seconds
    (default --settle) have passed since the first, so that the GPU clocks
    have ramped before a timed region.  Returns (seconds, steps)."""
    min_s = args.settle if min_s is None else min_s
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    for _ in range(args.warmup):
        step()
        n += 1
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < min_s:
        for _ in range(4):
            step()
        n += 4
        torch.cuda.synchronize()
    return time.perf_counter() - t0, n


def timed_kernels(step, steps, names, pkg, torch):
    """Run `steps` steps with the library's HIP events around each kernel;
    returns {name: {"avg_ms", "launches"}} and the wall time per step (ms)."""
    torch.cuda.synchronize()
    pkg.timing_reset()
    pkg.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    pkg.timing_enable(False)
    kern = {}
    for name in names:
        ms, n = pkg.timing_read(name)
        kern[name] = {"avg_ms": ms / max(n, 1), "total_ms": ms / steps, "launches": n}
    pkg.timing_reset()
    return kern, wall


def timed_plain(step, steps, torch):
    """Exactly `steps` un-instrumented steps between two synchronisations (ms per step)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def cpu_baseline(cfg, seed=42, max_threads=None, min_seconds=10.0):
    """Reference-order f32 oracle (test infrastructure, the CPU baseline only):
    forward core + backward from att, one thread per sequence as the reference's
    training loop runs one thread per batch element.  The sample (one sequence
    per thread) is repeated until at least min_seconds of CPU work have run.
    Returns (baseline dict, (out, dq, dk, dv) of the sample in [n][H][T][D])."""
    import oracle
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    nthreads = min(B, ncpu, max_threads or 16)
    nseq = nthreads  # one sequence per thread: a bounded sample of the same workload
    q, k, v, do = oracle.synth_inputs(nseq, H, T, D, seed=seed)
    qs, ks, vs, dos = (oracle.bhtd_to_seq(a) for a in (q, k, v, do))
    reps = 0
    t0 = time.perf_counter()
    while True:
        outs = oracle.batch_fwd_bwd_f32_threaded(qs, ks, vs, dos, H, nthreads=nthreads)
        reps += 1
        if time.perf_counter() - t0 >= min_seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    flops = credited_flops(nseq, H, T, D)["total"]
    # one sequence on one thread (attention_cpu itself is single-threaded)
    t1 = time.perf_counter()
    oracle.batch_fwd_bwd_f32_threaded(qs[:1], ks[:1], vs[:1], dos[:1], H, nthreads=1)
    one = time.perf_counter() - t1
    base = {"value": nseq * T / dt, "unit": "tokens/s", "cores": nthreads, "kind": "port",
            "sample": f"{nseq} of the {B} sequences ({nseq}x{T} tokens, {H} heads, D={D}), fwd+bwd, "
                      f"one thread per sequence, repeated {reps}x; host has {ncpu} cores",
            "seconds_per_rep": dt, "tflops": flops / dt / 1e12, "nproc": ncpu,
            "one_thread_seconds_per_sequence": one}
    return base, tuple(oracle.seq_to_bhtd(a, H) for a in outs)


def parity_of(got, want):
    """max-abs and relative-L2 error of device outputs against CPU arrays."""
    import numpy as np
    res = {}
    for name, g, w in zip(("O", "dQ", "dK", "dV"), got, want):
        g = g[:w.shape[0]].detach().cpu().numpy().astype(np.float64)
        w = w.astype(np.float64)
        res[name] = {"max_abs": float(np.abs(g - w).max()),
                     "rel_l2": float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))}
    return res


def attn_pair(args, cfg, pkg, torch, keep, inputs=None, settle_s=None):
    """Times one pair (keep=False: wha_attn_fwd + wha_attn_bwd; keep=True:
    wha_attn_fwd_keep + wha_attn_bwd_kept) on one config.  Returns the result
    dict and the outputs (o, dq, dk, dv) of the last step."""
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    dev = torch.device("cuda:0")
    if inputs is None:
        inputs = tuple(torch.from_numpy(a).to(dev) for a in pkg.synth_inputs(B, H, T, D, seed=42))
    tq, tk, tv, tdo = inputs
    o = torch.empty_like(tq)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    dq, dk, dv = (torch.empty_like(tq) for _ in range(3))
    # pointers and layouts bound once, so a step is two C calls
    plan = pkg.AttnPlan(tq, tk, tv, o, lse, tdo, dq, dk, dv, keep_scores=keep)

    def step():
        plan.fwd()
        plan.bwd()

    warm_s, warm_n = settle(step, args, torch, settle_s)
    kern, ms_events = timed_kernels(step, args.steps, ATTN_KERNELS, pkg, torch)
    ms = timed_plain(step, args.steps, torch)
    flops = credited_flops(B, H, T, D)
    if kern["attn_bwd_dq"]["launches"] == 0:  # small problems: one backward kernel forms dK, dV and dQ
        flops["attn_bwd_dkv"] += flops["attn_bwd_dq"]
        flops["attn_bwd_dq"] = 0
    dom = max(("attn_fwd", "attn_bwd_dq", "attn_bwd_dkv"), key=lambda n: kern[n]["avg_ms"])
    achieved = flops[dom] / (kern[dom]["avg_ms"] * 1e-3) / 1e12
    variant = "kept" if plan.keeps_scores else "recompute"
    res = {
        "pair": ("wha_attn_fwd_keep + wha_attn_bwd_kept" if plan.keeps_scores
                 else "wha_attn_fwd + wha_attn_bwd"),
        "backward": "scores kept by the forward" if plan.keeps_scores else "P recomputed from the saved LSE",
        "ms_per_step": ms, "tokens_per_s": B * T / (ms * 1e-3),
        "tflops": flops["total"] / (ms * 1e-3) / 1e12,
        "pct_fp32_mfma_peak": 100.0 * flops["total"] / (ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
        "kernel_ms": {n: round(kern[n]["avg_ms"], 5) for n in kern},
        "ms_per_step_with_events": ms_events,
        "warmup_s": round(warm_s, 3), "warmup_steps": warm_n,
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": achieved, "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP32_MFMA_PEAK_TFLOPS,
                     **traffic_fields(f"{dom}[{variant}]", cfg),
                     "algorithmic_flops_per_launch": flops[dom], "avg_launch_ms": kern[dom]["avg_ms"]},
    }
    return res, (o, dq, dk, dv), plan


def step_medians(plan, steps, torch):
    """Per-step forward and backward durations (events on the launch stream), medians in ms."""
    stream = torch.cuda.current_stream()
    evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(steps)]
    torch.cuda.synchronize()
    for e0, e1, e2 in evs:
        e0.record(stream)
        plan.fwd()
        e1.record(stream)
        plan.bwd()
        e2.record(stream)
    torch.cuda.synchronize()

    def median(xs):
        xs = sorted(xs)
        return xs[len(xs) // 2] if len(xs) % 2 else 0.5 * (xs[len(xs) // 2 - 1] + xs[len(xs) // 2])

    return median(e0.elapsed_time(e1) for e0, e1, _ in evs), median(e1.elapsed_time(e2) for _, e1, e2 in evs)


def run_attention(args, cfg, pkg, torch):
    """The headline line: the recompute pair (north-star design) on `cfg`, the
    kept pair beside it; with the suite, every other BASELINE config."""
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    dev = torch.device("cuda:0")
    inputs = tuple(torch.from_numpy(a).to(dev) for a in pkg.synth_inputs(B, H, T, D, seed=42))
    head, outs, plan = attn_pair(args, cfg, pkg, torch, keep=args.kept, inputs=inputs)
    fwd_med, bwd_med = step_medians(plan, args.steps, torch)
    ms = head["ms_per_step"]
    k = head["kernel_ms"]
    res = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded xorshift64 + Box-Muller, seed 42)",
        "config": {"workload": cfg["name"], "batch": B, "heads": H, "seq_len": T, "head_dim": D,
                   "layout": "[B,H,T,D] contiguous", "causal": True, "parallelism": "none (1 GPU)",
                   "pair": head["pair"], "backward": head["backward"]},
        "tflops": head["tflops"],
        "pct_fp32_mfma_peak": head["pct_fp32_mfma_peak"],
        "warmup_s": head["warmup_s"], "warmup_steps": head["warmup_steps"],
        "kernel_ms": k,
        "fwd_ms": k["attn_fwd"], "bwd_ms": k["attn_bwd_delta"] + k["attn_bwd_dq"] + k["attn_bwd_dkv"],
        "ms_per_step_with_events": head["ms_per_step_with_events"],
        "fwd_ms_median": fwd_med, "bwd_ms_median": bwd_med,
        "roofline": head["roofline"],
    }
    del plan
    if not args.kept:
        kept, kouts, _ = attn_pair(args, cfg, pkg, torch, keep=True, inputs=inputs, settle_s=min(0.5, args.settle))
        res["kept_scores"] = {n: kept[n] for n in ("pair", "ms_per_step", "tokens_per_s", "tflops",
                                                   "pct_fp32_mfma_peak", "kernel_ms", "roofline")}
        res["_outs_kept"] = kouts
    res["_outs"] = outs
    if args.suite and cfg is CONFIGS["768"]:
        res["configs"] = {}
        for key in ("168", "384", "4096"):
            c = CONFIGS[key]
            sub = {"workload": c["name"], "B": c["B"], "H": c["H"], "T": c["T"], "D": c["D"]}
            for keep in (False, True):
                if keep and pkg.attn_scores_bytes(pkg.layout_bhtd(c["B"], c["H"], c["T"], c["D"])) == 0:
                    sub["kept"] = "same kernels as the recompute pair (this head dim keeps no scores)"
                    continue
                r, _, p = attn_pair(args, c, pkg, torch, keep=keep, settle_s=min(0.5, args.settle))
                sub["kept" if keep else "recompute"] = {
                    n: r[n] for n in ("ms_per_step", "tokens_per_s", "tflops", "pct_fp32_mfma_peak",
                                      "kernel_ms", "roofline")}
                del p
            res["configs"][key] = sub
            torch.cuda.empty_cache()
        res["configs"]["decode"] = run_decode(args, CONFIGS["decode"], pkg, torch, sub=True)
        torch.cuda.empty_cache()
        res["configs"]["probs"] = run_probs(args, CONFIGS["probs"], pkg, torch, sub=True)
        torch.cuda.empty_cache()
    return res


def hbm_read_ceiling(torch, gib=4):
    """Read-only stream rate (GB/s): a calibration kernel (wave-engine_amd/
    libwha_hbm_probe.so: 16-byte loads grid-stride, U of them in flight per
    thread, one float written per thread) over a `gib` GiB buffer, timed with
    HIP events over 10 launches on the launch stream.  The best of a sweep of
    one or two concurrent streams, unrolls (4, 8, 16), plain or non-temporal
    loads, and grids of 4 to 64 blocks per CU is the practical ceiling for
    kernels that only read, such as the decode split kernel.  A device copy (torch copy_, read + write
    bytes) of the same buffer is timed beside it."""
    probe = ctypes.CDLL(str(ROOT / "wave-engine_amd" / "libwha_hbm_probe.so"))
    probe.whp_read_stream_v.restype = ctypes.c_int
    probe.whp_read_stream_v.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    x = torch.ones(gib * (1 << 28), dtype=torch.float32, device="cuda:0")
    out = torch.empty(16384 * 256, dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    n = 10

    def timed(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e-3

    best = (0.0, None)
    for streams in (1, 2):
        for unroll in (4, 8, 16):
            for nt in (0, 1):
                for blocks in (1024, 2048, 4096, 8192, 16384):
                    def run():
                        rc = probe.whp_read_stream_v(x.data_ptr(), x.numel() // 4, out.data_ptr(), blocks, unroll,
                                                     nt, streams, st)
                        if rc:
                            raise RuntimeError(f"whp_read_stream_v failed ({rc})")

                    gbs = x.numel() * 4 / timed(run) / 1e9
                    if gbs > best[0]:
                        best = (gbs, {"streams": streams, "unroll": unroll, "nontemporal": bool(nt),
                                      "blocks": blocks})
    y = torch.empty_like(x)
    copy_gbs = 2 * x.numel() * 4 / timed(lambda: y.copy_(x)) / 1e9
    del x, y, out
    torch.cuda.empty_cache()
    return {"gbs": best[0], **best[1], "buffer_gib": gib, "timing": "hip events, 10 launches",
            "copy_gbs": copy_gbs}


def run_decode(args, cfg, pkg, torch, sub=False):
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    dev = torch.device("cuda:0")
    import numpy as np
    g = pkg.SynthStream(42)
    sd = 1.0 / np.sqrt(D)
    q = torch.from_numpy(g.normal(B * H * D, sd).reshape(B, H, D)).to(dev)
    kc = torch.from_numpy(g.normal(B * H * T * D, sd).reshape(B, H, T, D)).to(dev)
    vc = torch.from_numpy(g.normal(B * H * T * D, sd).reshape(B, H, T, D)).to(dev)
    ws = torch.empty(int(pkg.lib().wha_decode_workspace_size(ctypes.byref(pkg.layout_of(kc)))) // 4 + 64,
                     device=dev)

    def step():
        pkg.decode_fwd(q, kc, vc, workspace=ws)

    warm_s, warm_n = settle(step, args, torch, min(0.5, args.settle) if sub else None)
    kern, _ = timed_kernels(step, args.steps, ("decode_split", "decode_merge"), pkg, torch)
    ms = timed_plain(step, args.steps, torch)
    bytes_kv = 2 * B * H * T * D * 4
    split = kern["decode_split"]["avg_ms"]
    achieved = bytes_kv / (split * 1e-3) / 1e9
    res = {"metric": "decode HBM GB/s (K+V bytes / time), 768-dim decode Tkv 8192",
           "value": bytes_kv / (ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms,
           "config": {"workload": cfg["name"], "batch": B, "heads": H, "kv_len": T, "head_dim": D},
           "kernel_ms": {n: round(kern[n]["avg_ms"], 5) for n in kern},
           "warmup_s": round(warm_s, 3),
           "roofline": {"kernel": "decode_split", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                        **traffic_fields("decode_split", cfg), "algorithmic_bytes_per_launch": bytes_kv,
                        "avg_launch_ms": split}}
    del q, kc, vc, ws
    torch.cuda.empty_cache()
    res["hbm_read_ceiling"] = hbm_read_ceiling(torch)
    res["frac_of_read_ceiling"] = achieved / res["hbm_read_ceiling"]["gbs"]
    if sub:
        return res
    res.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic"})
    return res


def run_probs(args, cfg, pkg, torch, sub=False):
    """Fused forward plus the exact-contract backward (wha_attn_bwd_from_probs:
    att [B,H,T,T] read as given, never recomputed).  att is built once, outside
    the timed region, from the forward's LSE (wha_attn_probs_rows, 256 rows per
    call).  The backward's Delta and dK/dV passes each stream the causal half
    of att (4 B per causal pair); dK/dV also writes the dS tiles, which the dQ
    pass reads back.  The roofline is reported against HBM with algorithmic
    bytes per launch = those streams plus the [T][D] operands each kernel reads
    and writes."""
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    dev = torch.device("cuda:0")
    q, k, v, do = (torch.from_numpy(a).to(dev) for a in pkg.synth_inputs(B, H, T, D, seed=42))
    o, lse = pkg.attn_fwd(q, k, v)
    att = torch.cat([pkg.attn_probs_rows(q, k, lse, range(r, min(T, r + 256))) for r in range(0, T, 256)], dim=2)
    att = att.contiguous()
    ws = torch.empty(int(pkg.lib().wha_attn_bwd_from_probs_workspace_size(ctypes.byref(pkg.layout_of(q)))) // 4 + 64,
                     device=dev)
    lse_o = torch.empty_like(lse)

    def step():
        pkg.attn_fwd(q, k, v, out=o, lse=lse_o)
        pkg.attn_bwd_from_probs(do, q, k, v, att, workspace=ws)

    warm_s, _ = settle(step, args, torch, min(0.5, args.settle) if sub else None)
    names = ("attn_fwd", "attn_bwd_probs_delta", "attn_bwd_probs_dq", "attn_bwd_probs_dkv")
    pkg.timing_reset()
    pkg.timing_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    pkg.timing_enable(False)
    kern = {n: pkg.timing_read(n) for n in names}
    pkg.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    avg = {n: kern[n][0] / max(kern[n][1], 1) for n in names}
    P = B * H * (T * (T + 1) // 2)
    rows = B * H * T * D * 4
    nkt = (T + 63) // 64
    ds = B * H * (nkt * 64 * nkt - 32 * nkt * (nkt - 1)) * 64 * 4     # dS tiles: causal 64-key column blocks
    alg = {"attn_bwd_probs_delta": 4 * P + 2 * rows + B * H * T * 4,      # att, V, dO; Delta out
           "attn_bwd_probs_dkv": 4 * P + 5 * rows + B * H * T * 4 + ds,   # att, Q, V, dO, Delta; dK, dV, dS out
           "attn_bwd_probs_dq": ds + 2 * rows}                            # dS, K; dQ out
    dom = max(alg, key=lambda n: avg[n])
    achieved = alg[dom] / (avg[dom] * 1e-3) / 1e9
    flops = credited_flops(B, H, T, D)["total"]
    del q, k, v, do, o, lse, att, ws, lse_o
    torch.cuda.empty_cache()
    if sub:
        return {"workload": cfg["name"], "pair": "wha_attn_fwd + wha_attn_bwd_from_probs (att given)",
                "ms_per_step": ms, "tokens_per_s": B * T / (ms * 1e-3), "tflops": flops / (ms * 1e-3) / 1e12,
                "kernel_ms": {n: round(avg[n], 5) for n in names},
                "bwd_ms": sum(avg[n] for n in names[1:]),
                "roofline": {"kernel": dom, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, **traffic_fields(dom, cfg),
                             "algorithmic_bytes_per_launch": alg[dom], "avg_launch_ms": avg[dom]}}
    return {"metric": "causal attn fwd + exact-contract bwd (att given) tokens/s, 768-dim seq1024",
            "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "warmup_s": round(warm_s, 3), "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded xorshift64 + Box-Muller, seed 42)",
            "config": {"workload": cfg["name"], "batch": B, "heads": H, "seq_len": T, "head_dim": D,
                       "parallelism": "none (1 GPU)"},
            "tflops": flops / (ms * 1e-3) / 1e12,
            "kernel_ms": {n: round(avg[n], 5) for n in names},
            "bwd_ms": sum(avg[n] for n in names[1:]),
            "roofline": {"kernel": dom, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, **traffic_fields(dom, cfg), "algorithmic_bytes_per_launch": alg[dom],
                         "avg_launch_ms": avg[dom]}}


def wave_admitted_pairs(bucket, torch):
    """(admitted, causal) pair counts of the wave mask over bucket [B,H,T]
    (int32, device): key k <= q is admitted when its bucket is within one of
    the query's mod 8, or k = q - 1 (src/common/attn.rs:189-224)."""
    bk = bucket.long()
    T = bk.shape[-1]
    cum = torch.nn.functional.one_hot(bk, 8).cumsum(dim=2)          # keys k <= q per bucket
    near = sum(cum.gather(3, ((bk + d) % 8).unsqueeze(-1)).squeeze(-1) for d in (-1, 0, 1))
    prev_far = (((bk[..., :-1] - bk[..., 1:] + 1) & 7) > 2)          # k = q-1 outside the bucket window
    admitted = int(near.sum().item()) + int(prev_far.sum().item())
    return admitted, bk.shape[0] * bk.shape[1] * (T * (T + 1) // 2)


def wave_sparse_executed_pairs(bucket, torch):
    """Pairs the bucket-sparse kernels execute: per (b,h), positions sorted by
    bucket (stable) in 16-row chunks; a (query chunk, key chunk) block runs when
    some bucket of one is within one of some bucket of the other and the key
    chunk's first position is not after the query chunk's last (the schedule
    of wave-engine_amd/csrc/wave_sparse.hip), 256 pairs per block."""
    bk = bucket.long().reshape(-1, bucket.shape[-1])
    N, T = bk.shape
    NC = (T + 15) // 16
    vals, pos = torch.sort(bk, dim=1, stable=True)
    pad = NC * 16 - T
    valid = torch.ones_like(vals, dtype=torch.bool)
    if pad:
        vals = torch.nn.functional.pad(vals, (0, pad))
        pos = torch.nn.functional.pad(pos, (0, pad))
        valid = torch.nn.functional.pad(valid, (0, pad))
    vals, pos, valid = (a.reshape(N, NC, 16) for a in (vals, pos, valid))
    sets = (torch.nn.functional.one_hot(vals, 8) * valid.unsqueeze(-1)).amax(dim=2).float()   # [N, NC, 8]
    near = ((sets + sets.roll(1, dims=-1) + sets.roll(-1, dims=-1)) > 0).float()
    bucket_live = torch.bmm(near, sets.transpose(1, 2)) > 0                                   # [N, qc, kc]
    big = torch.iinfo(torch.int64).max
    pmin = torch.where(valid, pos, torch.full_like(pos, big)).amin(dim=2)
    pmax = torch.where(valid, pos, torch.full_like(pos, -1)).amax(dim=2)
    causal = pmin.unsqueeze(1) <= pmax.unsqueeze(2)                                            # [N, qc, kc]
    return 256 * int((bucket_live & causal).sum().item())


def wave_credited_flops(B, H, T, D, C, admitted=None):
    """FLOPs of one wave-attention layer step (wave_attention_forward +
    wave_attention_backward_full).  The core terms are credited for the pairs
    the bucket mask admits (`admitted`; every causal pair if None) with the
    (2 + C)-wide feature dot product, not its 32-wide zero padding; the
    kernels execute every causal pair of a computed tile."""
    E, M, F = H * D, B * T, 2 + C
    P = B * H * (T * (T + 1) // 2) if admitted is None else admitted
    proj = 2 * M * E * H * F          # phase + content projections
    vproj = 2 * M * E * D             # per-head value projections
    outp = 2 * M * E * E
    return {"wave_fwd": 2 * P * (F + D),
            "wave_bwd_dkv": 2 * P * (F + 2 * D + F),   # S, dP, dV, dF_k
            "wave_bwd_dq": 2 * P * F,                  # dF_q = dS F_k
            "linear_fwd": proj + vproj + outp,
            "linear_bwd": 2 * (proj + vproj + outp),   # input and weight gradients
            "total": 2 * P * (F + D) + 2 * P * (3 * F + 2 * D) + 3 * (proj + vproj + outp)}


def run_wave(args, cfg, pkg, torch):
    import numpy as np
    B, H, T, D, C = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["C"]
    E = H * D
    dev = torch.device("cuda:0")
    g = pkg.SynthStream(42)
    t = lambda n, sd, *shape: torch.from_numpy(g.normal(n, sd).reshape(*shape)).to(dev)
    x = t(B * T * E, 1.0, B, T, E)
    W = pkg.WaveAttnWeights(t(H, 1.0, H), t(H * (2 + C) * E, 1 / np.sqrt(E), H, 2 + C, E),
                            t(H * (2 + C), 0.1, H, 2 + C), t(H * D * D, 1 / np.sqrt(D), H, D, D), t(H * D, 0.1, H, D),
                            t(E * E, 1 / np.sqrt(E), E, E), t(E, 0.1, E))
    dy = t(B * T * E, 1.0 / np.sqrt(B * T), B, T, E)
    shape = pkg.WaveShape(B, T, E, H, C)
    ws = torch.empty(pkg.wave_bwd_workspace_bytes(shape) // 4 + 64, dtype=torch.float32, device=dev)
    out = torch.empty_like(x)

    def step():
        _, _, cache = pkg.wave_attention_forward(W, x, out=out)
        pkg.wave_attention_backward_full(W, cache, dy, workspace=ws)

    pkg.wave_set_bucket_sparse({"auto": "auto", "sparse": True, "dense": False}[args.wave_family])
    warm_s, _ = settle(step, args, torch)
    names = ("wave_feat", "wave_sort", "wave_gather", "wave_fwd", "wave_bwd_delta", "wave_bwd_dkv", "wave_bwd_dq",
             "wave_feat_bwd", "wave_harmonic", "linear_fwd", "linear_bwd_dx", "linear_bwd_dw")
    pkg.timing_reset()
    pkg.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    pkg.timing_enable(False)
    kern = {}
    for name in names:
        ms, n = pkg.timing_read(name)
        kern[name] = {"total_ms": ms / args.steps, "avg_ms": ms / max(n, 1), "launches": n}
    pkg.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) / args.steps * 1e3
    _, _, cache = pkg.wave_attention_forward(W, x, out=out)
    admitted, causal = wave_admitted_pairs(cache.bucket, torch)
    fl = wave_credited_flops(B, H, T, D, C, admitted)
    sparse = args.wave_family == "sparse" or (args.wave_family == "auto" and T >= 1024)
    executed = wave_sparse_executed_pairs(cache.bucket, torch) if sparse else causal
    fl_exec = wave_credited_flops(B, H, T, D, C, executed)
    dom = max(("wave_fwd", "wave_bwd_dkv", "wave_bwd_dq"), key=lambda n: kern[n]["avg_ms"])
    achieved = fl[dom] / (kern[dom]["avg_ms"] * 1e-3) / 1e12
    return {
        "metric": "wave attention layer fwd+bwd tokens/s & TFLOP/s, 768-dim seq1024",
        "value": B * T / (ms_per_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "warmup_s": round(warm_s, 3), "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded xorshift64 + Box-Muller, seed 42), random-init weights",
        "config": {"workload": cfg["name"], "batch": B, "heads": H, "seq_len": T, "head_dim": D,
                   "content_dim": C, "parallelism": "none (1 GPU)"},
        "tflops": fl["total"] / (ms_per_step * 1e-3) / 1e12,
        "mask_fraction": admitted / causal,
        "kernels": ("bucket-sparse (positions sorted by bucket, 16 x 16 blocks the mask can admit)" if sparse
                    else "all causal pairs, mask per score"),
        "executed_over_admitted": executed / admitted,
        "credit": "core FLOPs over the admitted (bucket-mask) pairs only",
        "kernel_ms_per_step": {n: round(kern[n]["total_ms"], 5) for n in names},
        "ms_per_step_with_events": wall / args.steps * 1e3,
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": achieved, "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP32_MFMA_PEAK_TFLOPS,
                     **traffic_fields(dom, cfg), "algorithmic_flops_per_launch": fl[dom],
                     "executed_pair_flops_per_launch": fl_exec[dom],
                     "avg_launch_ms": kern[dom]["avg_ms"]},
    }


def run_wave_decode(args, cfg, pkg, torch):
    """One forward_one attention step (projections, split-K decode over the
    cache, merge + append, out_proj) for B sequences with L cached positions
    each; the counts are reset before every step, so each step redoes the same
    work at length L (the append rewrites position L)."""
    import numpy as np
    B, H, L, D, C = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["C"]
    E = H * D
    dev = torch.device("cuda:0")
    g = pkg.SynthStream(42)
    t = lambda n, sd, *shape: torch.from_numpy(g.normal(n, sd).reshape(*shape)).to(dev)
    W = pkg.WaveAttnWeights(t(H, 1.0, H), t(H * (2 + C) * E, 1 / np.sqrt(E), H, 2 + C, E),
                            t(H * (2 + C), 0.1, H, 2 + C), t(H * D * D, 1 / np.sqrt(D), H, D, D), t(H * D, 0.1, H, D),
                            t(E * E, 1 / np.sqrt(E), E, E), t(E, 0.1, E))
    cache = pkg.WaveKvCache(B, H, D, L + 1, dev)
    for b0 in range(0, B, 16):  # prefill the prompts in groups of 16 sequences
        pkg.prefill_attention(W, t(16 * L * E, 1.0, 16, L, E), cache, first_seq=b0)
    torch.cuda.synchronize()
    xn = t(B * E, 1.0, B, E)
    shape = pkg.WaveShape(B, 1, E, H, C)
    ws = torch.empty(pkg.wave_kv_decode_workspace_bytes(shape, cache.capacity) // 4 + 64, dtype=torch.float32,
                     device=dev)

    def step():
        cache.lengths = [L] * B
        return pkg.forward_one_attention(W, xn, cache, workspace=ws)

    warm_s, _ = settle(step, args, torch)
    pkg.timing_reset()
    pkg.timing_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    pkg.timing_enable(False)
    kern = {}
    for name in ("linear_fwd", "wave_kv_query", "wave_kv_split", "wave_kv_merge"):
        ms, n = pkg.timing_read(name)
        kern[name] = {"total_ms": ms / args.steps, "avg_ms": ms / max(n, 1)}
    pkg.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    # algorithmic bytes of the split kernel: cos/sin and bucket of every cached
    # position, plus the value rows of the positions the mask admits
    bk = cache.bucket[:, :, :L]
    qb = cache.bucket[:, :, L:L + 1]
    near = ((bk - qb + 1) & 7) <= 2
    near[:, :, L - 1] = True
    n_valid = int(near.sum().item())
    alg_bytes = B * H * L * 12 + n_valid * D * 4
    achieved = alg_bytes / (kern["wave_kv_split"]["avg_ms"] * 1e-3) / 1e9
    return {"metric": "wave-attention KV-cache decode tokens/s (one new token per sequence), 768-dim, 8192 cached",
            "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "warmup_s": round(warm_s, 3),
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic prompts (seeded), random-init weights",
            "config": {"workload": cfg["name"], "batch": B, "heads": H, "cached": L, "head_dim": D,
                       "content_dim": C},
            "kernel_ms_per_step": {n: round(kern[n]["total_ms"], 5) for n in kern},
            "mask_fraction": n_valid / (B * H * L),
            "roofline": {"kernel": "wave_kv_split", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                         **traffic_fields("wave_kv_split", cfg), "algorithmic_bytes_per_launch": alg_bytes,
                         "avg_launch_ms": kern["wave_kv_split"]["avg_ms"]}}


def layer_flops(B, H, T, D):
    """ComputeBackend::attention forward + backward: c_attn [3E][E] and c_proj [E][E]
    GEMMs over the B*T rows (forward, input gradient, weight gradient), plus the
    core's credited 12*B*H*D*P."""
    E, M = H * D, B * T
    return {"linear_fwd": 2 * M * E * 4 * E, "linear_bwd_dx": 2 * M * E * 4 * E, "linear_bwd_dw": 2 * M * E * 4 * E,
            "core": credited_flops(B, H, T, D)["total"],
            "total": 3 * 2 * M * E * 4 * E + credited_flops(B, H, T, D)["total"]}


def run_layer(args, cfg, pkg, torch):
    """One step = attention_cpu's layer (compute.rs:357-414) forward and its backward
    for the whole batch: qkv = c_attn(x), the fused core on strided views of qkv,
    out = c_proj(o); then d_o = c_proj^T dy, dW/db of c_proj, the core backward into
    a [B*T][3E] gradient, dx = c_attn^T d_qkv and dW/db of c_attn."""
    import numpy as np
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    E, M = H * D, B * T
    dev = torch.device("cuda:0")
    g = pkg.SynthStream(42)
    t = lambda n, sd, *shape: torch.from_numpy(g.normal(n, sd).reshape(*shape)).to(dev)
    x = t(M * E, 1.0, M, E)
    wa, ba = t(3 * E * E, 1 / np.sqrt(E), 3 * E, E), t(3 * E, 0.1, 3 * E)
    wp, bp = t(E * E, 1 / np.sqrt(E), E, E), t(E, 0.1, E)
    dy = t(M * E, 1 / np.sqrt(M), M, E)
    qkv = torch.empty(M, 3 * E, device=dev)
    obuf = torch.empty(M, 3 * E, device=dev)   # o and d_o share q's [B][T][3E] strides
    dobuf = torch.empty(M, 3 * E, device=dev)
    d_qkv = torch.empty(M, 3 * E, device=dev)
    out = torch.empty(M, E, device=dev)
    dx = torch.empty(M, E, device=dev)
    lse = torch.empty(B, H, T, device=dev)
    heads = lambda buf, c: buf.view(B, T, 3 * E)[:, :, c * E:(c + 1) * E].view(B, T, H, D).permute(0, 2, 1, 3)
    q, k, v = heads(qkv, 0), heads(qkv, 1), heads(qkv, 2)
    o4, do4 = heads(obuf, 0), heads(dobuf, 0)
    dq4, dk4, dv4 = heads(d_qkv, 0), heads(d_qkv, 1), heads(d_qkv, 2)
    L = pkg.layout_of(q)
    wsa = torch.empty(pkg.attn_bwd_workspace_bytes(L) // 4 + 64, device=dev)
    sc = None if args.recompute else pkg.attn_scores_buffer(L, dev)  # the core keeps its scores
    wsl = torch.empty(max(int(pkg.lib().wha_linear_bwd_dw_workspace_size(M, n, E)) for n in (E, 3 * E)) // 4 + 64,
                      device=dev)

    def step():
        pkg.linear_fwd(x, wa, ba, out=qkv)
        pkg.attn_fwd(q, k, v, out=o4, lse=lse, scores=sc)
        pkg.linear_fwd(obuf[:, :E], wp, bp, out=out)
        pkg.linear_bwd_dx(dy, wp, out=dobuf[:, :E])
        pkg.linear_bwd_dw(dy, obuf[:, :E], workspace=wsl)
        pkg.attn_bwd(q, k, v, o4, do4, lse, workspace=wsa, dq=dq4, dk=dk4, dv=dv4, scores=sc)
        pkg.linear_bwd_dx(d_qkv, wa, out=dx)
        pkg.linear_bwd_dw(d_qkv, x, workspace=wsl)

    warm_s, _ = settle(step, args, torch)
    names = ("linear_fwd", "linear_bwd_dx", "linear_bwd_dw", "attn_fwd", "attn_bwd_delta",
             "attn_bwd_dkv", "attn_bwd_dq")
    pkg.timing_reset()
    pkg.timing_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    pkg.timing_enable(False)
    kern = {}
    for name in names:
        ms, n = pkg.timing_read(name)
        kern[name] = {"total_ms": ms / args.steps, "avg_ms": ms / max(n, 1), "launches": n}
    pkg.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) / args.steps * 1e3
    fl = layer_flops(B, H, T, D)
    # dominant kernel family by time; its credited FLOPs per step over its time per step
    dom = max(("linear_fwd", "linear_bwd_dx", "linear_bwd_dw"), key=lambda n: kern[n]["total_ms"])
    achieved = fl[dom] / (kern[dom]["total_ms"] * 1e-3) / 1e12
    return {
        "metric": "attention layer (c_attn + causal core + c_proj) fwd+bwd tokens/s & TFLOP/s, 768-dim seq1024",
        "value": M / (ms_per_step * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_s": round(warm_s, 3), "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded xorshift64 + Box-Muller, seed 42)",
        "config": {"workload": cfg["name"], "batch": B, "heads": H, "seq_len": T, "head_dim": D,
                   "parallelism": "none (1 GPU)"},
        "tflops": fl["total"] / (ms_per_step * 1e-3) / 1e12,
        "pct_fp32_mfma_peak": 100.0 * fl["total"] / (ms_per_step * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
        "kernel_ms_per_step": {n: round(kern[n]["total_ms"], 5) for n in names},
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": achieved, "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP32_MFMA_PEAK_TFLOPS, "traffic": None,
                     "algorithmic_flops_per_step": fl[dom], "ms_per_step": kern[dom]["total_ms"],
                     "launches_per_step": kern[dom]["launches"] / args.steps},
    }


def layer_cpu_baseline(cfg, seed=42, max_threads=None):
    """Reference-order f32 oracle of the same layer step, one thread per sequence
    (the reference's B concurrent callers), on a bounded sample of sequences."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    import oracle
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    E = H * D
    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    nthreads = min(B, ncpu, max_threads or 16)
    rng = oracle.Xorshift64(seed)
    x = rng.normal(nthreads * T * E, 1.0).reshape(nthreads, T, E)
    wa, ba = rng.normal(3 * E * E, 1 / np.sqrt(E)).reshape(3 * E, E), rng.normal(3 * E, 0.1)
    wp, bp = rng.normal(E * E, 1 / np.sqrt(E)).reshape(E, E), rng.normal(E, 0.1)
    dy = rng.normal(nthreads * T * E, 1 / np.sqrt(B * T)).reshape(nthreads, T, E)

    def one(i):
        qkv = oracle.linear(x[i], wa, ba)
        q, k, v = qkv[:, :E], qkv[:, E:2 * E], qkv[:, 2 * E:]
        o, att = oracle.core_fwd(q, k, v, H, "f32", want_att=True)
        oracle.linear(o, wp, bp)
        d_o = oracle.linear_backward_dx(dy[i], wp)
        oracle.outer_product_accum(dy[i], o, True)
        dq, dk, dv = oracle.attention_backward(d_o, q, k, v, att, H, "f32")
        d_qkv = np.concatenate([dq, dk, dv], axis=1)
        oracle.linear_backward_dx(d_qkv, wa)
        oracle.outer_product_accum(d_qkv, x[i], True)

    t0 = time.perf_counter()
    with ThreadPoolExecutor(nthreads) as ex:
        list(ex.map(one, range(nthreads)))
    dt = time.perf_counter() - t0
    return {"value": nthreads * T / dt, "unit": "tokens/s", "cores": nthreads, "kind": "port",
            "sample": f"{nthreads} of the {B} sequences ({nthreads}x{T} tokens): c_attn, core, c_proj forward and "
                      f"their backward, one thread per sequence, run once", "seconds": dt, "nproc": ncpu}


def wave_cpu_baseline(cfg, seed=42, max_threads=None, min_seconds=10.0):
    """Reference-order f32 oracle of wave_attention_forward + backward_full, one
    thread per sequence on a bounded sample, repeated to at least min_seconds."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    import oracle
    B, H, T, D, C = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["C"]
    E = H * D
    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    nthreads = min(B, ncpu, max_threads or 16)
    rng = oracle.Xorshift64(seed)
    x = rng.normal(nthreads * T * E, 1.0).reshape(nthreads, T, E)
    w = dict(hraw=rng.normal(H, 1.0), proj_w=rng.normal(H * (2 + C) * E, 1 / np.sqrt(E)).reshape(H, 2 + C, E),
             proj_b=rng.normal(H * (2 + C), 0.1).reshape(H, 2 + C),
             v_w=rng.normal(H * D * D, 1 / np.sqrt(D)).reshape(H, D, D), v_b=rng.normal(H * D, 0.1).reshape(H, D),
             out_w=rng.normal(E * E, 1 / np.sqrt(E)).reshape(E, E), out_b=rng.normal(E, 0.1))
    dy = rng.normal(nthreads * T * E, 1.0 / np.sqrt(B * T)).reshape(nthreads, T, E)

    def one(i):
        oracle.wave_fwd(x[i], w, "f32")
        oracle.wave_bwd(x[i], w, dy[i], "f32")

    reps = 0
    t0 = time.perf_counter()
    with ThreadPoolExecutor(nthreads) as ex:
        while True:
            list(ex.map(one, range(nthreads)))
            reps += 1
            if time.perf_counter() - t0 >= min_seconds:
                break
    dt = (time.perf_counter() - t0) / reps
    return {"value": nthreads * T / dt, "unit": "tokens/s", "cores": nthreads, "kind": "port",
            "sample": f"{nthreads} of the {B} sequences ({nthreads}x{T} tokens), wave_attention_forward + "
                      f"wave_attention_backward_full, one thread per sequence, repeated {reps}x",
            "seconds_per_rep": dt}


def traffic_fields(kernel, cfg):
    """The roofline's traffic entry and, when it is measured, where it comes from."""
    t = load_traffic(kernel, cfg)
    return {"traffic": t, "traffic_source": "profiles/traffic.json" if t is not None else None}


def load_traffic(kernel, cfg):
    """HBM bytes per launch of `kernel` on this workload, from the rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE summary committed under profiles/ (null if absent)."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        table = json.loads(p.read_text())
        return table.get(f"{kernel}@{cfg['B']}x{cfg['H']}x{cfg['T']}x{cfg['D']}")
    except (ValueError, OSError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--settle", type=float, default=2.0,
                    help="seconds the step is repeated (after --warmup steps) before the first timed region")
    ap.add_argument("--config", default="768", choices=sorted(CONFIGS))
    ap.add_argument("--wave-family", default="auto", choices=("auto", "sparse", "dense"),
                    help="wave attention kernels (--config wave): the library's default (bucket-sparse from "
                         "T = 1024), bucket-sparse, or all causal pairs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-suite", dest="suite", action="store_false",
                    help="768 only: leave out the other BASELINE configs")
    ap.add_argument("--kept", action="store_true",
                    help="time the kept-scores pair (wha_attn_fwd_keep + wha_attn_bwd_kept) as the line's "
                         "main pair instead of the recompute pair")
    ap.add_argument("--recompute", action="store_true",
                    help="--config layer: the core runs the recompute pair instead of keeping its scores")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="first run a plain device copy (y = 2*x, torch elementwise kernel) of this many "
                         "MiB five times, as the known-size reference for rocprofv3 byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the (b,h) units shard across GPUs with no "
              "exchange, so run one process per GPU on its share of the batch. --gpus must be 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    cfg = CONFIGS[args.config]
    if args.copy_mb:
        n = args.copy_mb * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.float32, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(5):
            torch.mul(x, 2.0, out=y)
        torch.cuda.synchronize()
        del x, y
    if args.config == "decode":
        res = run_decode(args, cfg, pkg, torch)
    elif args.config == "wave":
        res = run_wave(args, cfg, pkg, torch)
    elif args.config == "wavedecode":
        res = run_wave_decode(args, cfg, pkg, torch)
    elif args.config == "layer":
        res = run_layer(args, cfg, pkg, torch)
    elif args.config == "probs":
        res = run_probs(args, cfg, pkg, torch)
    else:
        res = run_attention(args, cfg, pkg, torch)
    outs = res.pop("_outs", None)
    outs_kept = res.pop("_outs_kept", None)
    if args.config in ("decode", "wavedecode", "probs"):
        res["cpu_baseline"] = None
    elif not args.no_cpu_baseline:
        if args.config == "wave":
            res["cpu_baseline"] = wave_cpu_baseline(cfg)
        elif args.config == "layer":
            res["cpu_baseline"] = layer_cpu_baseline(cfg)
        else:
            res["cpu_baseline"], cpu_outs = cpu_baseline(cfg)
            # the same seeded inputs on both sides: the GPU outputs of the timed
            # steps against the CPU f32 oracle's (the parity bar is 1e-4 max-abs,
            # 1e-5 relative L2)
            res["parity"] = {"vs": f"CPU f32 oracle, the {cpu_outs[0].shape[0]} sequences of the CPU sample",
                             "pair": parity_of(outs, cpu_outs)}
            if outs_kept is not None:
                res["parity"]["kept_scores"] = parity_of(outs_kept, cpu_outs)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
