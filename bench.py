#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X: Mixtral-8x7B-shape layer, prefill batch.

Workload: hidden 4096, 8 experts, top-2 (softmax, renormalised), SwiGLU
intermediate 14336, bf16 weights N(0,0.02), activations N(0,1), router logits
x @ gate_w with gate_w N(0,0.02); 8192 tokens (default).  One step = one full
layer forward (router -> align -> gate/up+SiLU -> down -> combine) through the
single C-ABI entry point, inputs resident in HBM.

Prints ONE JSON line.  Besides the contract fields it carries:
  roofline      the dominant kernel (grouped gate/up GEMM + SiLU): algorithmic
                FLOPs per launch / its mean duration from HIP events on the
                launch stream, against the bf16 dense MFMA peak
  cpu_baseline  the CPU oracle (fp32 PyTorch restatement of the layer) on a
                bounded token sample, timed on this host
  layer / decode / kernels_ms   whole-layer TFLOP/s, the 64-token decode batch
                (HBM-bound) and the per-kernel breakdown
  suite         the other workloads, warm and cache-cold: tiny fp32, DeepSeek-V2-Lite
                (4096 and 768 tokens, zipf + uniform twin, and routed by the DeepSeek-V3
                gate), the DeepSeek-V3 gate alone, the Qwen3 local share at 1..2048 tokens,
                fp8 Mixtral (W8A8 and W8A16)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0
FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
METRIC = "MoE-layer tokens/s + TFLOP/s (% MFMA peak) on 1 MI355X; vs host-CPU ref"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 10: the chip's clock settles over the first ~8 prefill layers (kernel traces: the first gate/up
    # launches run 3.0-3.5 ms, then 2.7)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--decode-tokens", type=int, default=64)
    ap.add_argument("--cpu-tokens", type=int, default=8192, help="token sample for the CPU baseline (0 = skip)")
    ap.add_argument("--cpu-runs", type=int, default=3)
    ap.add_argument("--no-suite", action="store_true",
                    help="skip the other workloads (tiny fp32 layer, DeepSeek-V2-Lite, Qwen3-30B-A3B local share, "
                         "fp8 Mixtral)")
    ap.add_argument("--profile-case", default=None,
                    metavar="NAME:T[:uniform][:w8a8|:w8a16] | prologue:T:H:E[:f32] | copy",
                    help="profiling driver: 12 cache-flushed fused-layer calls of one workload (names as in "
                         "easyinfra_amd.workloads.SHAPES); prints no JSON line")
    ap.add_argument("--traffic-run", action="store_true",
                    help="counter-collection driver: a 1 GiB device copy (known bytes, calibrates FETCH_SIZE/"
                         "WRITE_SIZE) followed by two fused prefill layers and two 64-token decode layers; prints "
                         "no JSON line")
    ap.add_argument("--trace-summary", default=None, metavar="KERNEL_TRACE_CSV",
                    help="summarise a rocprofv3 kernel trace (its *_kernel_trace.csv): per kernel, the launch "
                         "count, the mean over all launches and over the last --trace-last launches; prints a "
                         "markdown table, no JSON line, and touches no GPU")
    ap.add_argument("--trace-last", type=int, default=20,
                    help="launches per kernel in the steady-state mean of --trace-summary (the bench's --steps)")
    ap.add_argument("--counter-summary", nargs="+", default=None, metavar="COUNTER_CSV",
                    help="summarise rocprofv3 --pmc runs (their *_counter_collection.csv, one per pass) of the same "
                         "program: per kernel, the mean of every counter over its launches, with the clock "
                         "(GRBM_GUI_ACTIVE / 8 XCDs / duration), MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / "
                         "cycles) and FETCH_SIZE / WRITE_SIZE in MB scaled by --fetch-scale / --write-scale; prints a "
                         "markdown table, no JSON line, and touches no GPU")
    ap.add_argument("--fetch-scale", type=float, default=2.0,
                    help="bytes per FETCH_SIZE KiB unit / 1024 (the counter read for a copy of known size)")
    ap.add_argument("--write-scale", type=float, default=1.0, help="likewise for WRITE_SIZE")
    ap.add_argument("--kernel-filter", default="eimoe::", help="kernels whose name contains this (summaries)")
    return ap.parse_args()


def counter_summary(paths, fetch_scale, write_scale, name_filter):
    """Per-kernel means of rocprofv3 counter passes (one CSV per pass; each dispatch's counters
    summed over the instances the CSV lists)."""
    import csv
    sums = {}      # kernel -> counter -> [total, launches]
    durs = {}      # kernel -> [total ns, launches] of the pass that had GRBM_GUI_ACTIVE (else the first)
    for path in paths:
        per = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                k = (int(r["Dispatch_Id"]), r["Kernel_Name"])
                e = per.setdefault(k, {"_dur": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
                e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for (_, name), e in per.items():
            if name_filter not in name:
                continue
            ks = sums.setdefault(_kernel_short_name(name), {})
            for c, v in e.items():
                if c == "_dur":
                    continue
                t = ks.setdefault(c, [0.0, 0])
                t[0] += v
                t[1] += 1
            if "GRBM_GUI_ACTIVE" in e or _kernel_short_name(name) not in durs:
                d = durs.setdefault(_kernel_short_name(name), [0.0, 0, "GRBM_GUI_ACTIVE" in e])
                if "GRBM_GUI_ACTIVE" in e and not d[2]:
                    d[:] = [0.0, 0, True]
                d[0] += e["_dur"]
                d[1] += 1
    counters = sorted({c for ks in sums.values() for c in ks})
    extra = []
    if "GRBM_GUI_ACTIVE" in counters:
        extra.append("clock (GHz)")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in counters and "GRBM_GUI_ACTIVE" in counters:
        extra.append("MFMA busy")
    if "FETCH_SIZE" in counters:
        extra.append("FETCH (MB)")
    if "WRITE_SIZE" in counters:
        extra.append("WRITE (MB)")
    print("| kernel | launches | mean under counters (us) | " + " | ".join(extra + counters) + " |")
    print("|---|---:|---:|" + "---:|" * (len(extra) + len(counters)))
    for name in sorted(sums, key=lambda n: -durs.get(n, [0, 1])[0]):
        ks = sums[name]
        mean = {c: v[0] / v[1] for c, v in ks.items()}
        d = durs.get(name, [0.0, 1])
        dur_ns = d[0] / max(d[1], 1)
        cells = []
        if "clock (GHz)" in extra:
            cells.append(f"{mean.get('GRBM_GUI_ACTIVE', 0) / 8 / dur_ns:.2f}" if dur_ns else "")
        if "MFMA busy" in extra:
            cyc = mean.get("GRBM_GUI_ACTIVE", 0) / 8
            cells.append(f"{100 * mean.get('SQ_VALU_MFMA_BUSY_CYCLES', 0) / 1024 / cyc:.1f} %" if cyc else "")
        if "FETCH (MB)" in extra:
            cells.append(f"{mean.get('FETCH_SIZE', 0) * 1024 * fetch_scale / 1e6:.1f}")
        if "WRITE (MB)" in extra:
            cells.append(f"{mean.get('WRITE_SIZE', 0) * 1024 * write_scale / 1e6:.1f}")
        cells += [f"{mean[c]:.4g}" if c in mean else "" for c in counters]
        short = name if len(name) <= 100 else name[:97] + "..."
        print(f"| `{short}` | {d[1]} | {dur_ns / 1e3:.1f} | " + " | ".join(cells) + " |")


def _kernel_short_name(name):
    """A kernel's name without its parameter list (template arguments kept)."""
    name = name[5:] if name.startswith("void ") else name
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and not name.startswith("(anonymous", i):
            return name[:i]
    return name


def trace_summary(path, last):
    """Per-kernel launch statistics of a rocprofv3 kernel trace, in dispatch order: the bench's
    roofline kernel is launched 2 * (warmup + steps) times (layer calls, then stage calls), and its
    HIP-event mean covers the last `steps` of them, which the last-N column reproduces."""
    import csv
    by = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            by.setdefault(r["Kernel_Name"], []).append((int(r["Dispatch_Id"]), d))
    rows = []
    total = sum(d for v in by.values() for _, d in v)
    for name, v in by.items():
        v.sort()
        ds = [d for _, d in v]
        tail = ds[-last:]
        rows.append((sum(ds), name, len(ds), sum(ds) / len(ds) / 1e3, sum(tail) / len(tail) / 1e3, len(tail)))
    rows.sort(reverse=True)
    print(f"| kernel | calls | mean, all calls (us) | mean, last N calls (us) | N | share |")
    print("|---|---:|---:|---:|---:|---:|")
    for tot, name, n, avg, avg_tail, nt in rows:
        short = _kernel_short_name(name)
        short = short if len(short) <= 100 else short[:97] + "..."
        print(f"| `{short}` | {n} | {avg:.1f} | {avg_tail:.1f} | {nt} | {100.0 * tot / total:.2f}% |")


def timed(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def stage_times(inp, steps, warmup, torch, ops):
    """Same kernels as the fused entry point (same tiles, the layer's K split of the down
    projection, fp32 partial planes), launched one by one with HIP events between them on the
    launch stream; returns mean ms per stage and the down projection's K split."""
    s = inp.shape
    T, H = inp.x.shape
    n_local = inp.w_gate_up.shape[0]
    A = T * s.top_k
    ks = ops.fused_moe_down_split(T, H, s.inter, s.n_experts, s.top_k, n_local, 0, inp.x.dtype,
                                  1 if s.renormalize else 0)
    names = ["router", "align", "gate_up_silu", "down", "combine"]
    sums = [0.0] * len(names)

    def once(evs):
        evs[0].record()
        ids, w = ops.router_topk(inp.logits, s.top_k, s.renormalize)
        evs[1].record()
        al = ops.align(ids, n_local, 0)
        evs[2].record()
        h = ops.gemm_gate_up_silu(inp.x, inp.w_gate_up, al["offsets"], A, a_rows=al["sorted_tok"])
        evs[3].record()
        y = ops.gemm_down(h, inp.w_down, al["offsets"], A, out_dtype=torch.float32, k_split=ks)
        evs[4].record()
        ops.combine(y, al["pos"], w, out_dtype=torch.bfloat16)
        evs[5].record()

    evs = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
    for _ in range(warmup):
        once(evs)
    torch.cuda.synchronize()
    for _ in range(steps):
        once(evs)
        torch.cuda.synchronize()
        for i in range(len(names)):
            sums[i] += evs[i].elapsed_time(evs[i + 1])
    return {n: v / steps for n, v in zip(names, sums)}, ks


def cpu_baseline(inp, n_tokens, runs, torch):
    import oracle
    s = inp.shape
    n_tokens = min(n_tokens, inp.x.shape[0])
    threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    x = inp.x[:n_tokens].cpu()
    logits = inp.logits[:n_tokens].cpu()
    wgu = inp.w_gate_up.cpu().float()        # upcast from bf16 exactly, outside the timing
    wd = inp.w_down.cpu().float()
    fwd = lambda: oracle.moe_forward(x, logits, s.top_k, wgu, wd, s.renormalize)
    fwd()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fwd()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": n_tokens / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"first {n_tokens} of the {inp.x.shape[0]} prefill tokens, fp32 PyTorch oracle, "
                      f"median of {runs} runs after 1 warm-up ({t:.2f} s each); cpu: {model}; "
                      f"os.cpu_count()={os.cpu_count()}"}


def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch of one kernel, from counter runs of ``--traffic-run`` (FETCH_SIZE and
    WRITE_SIZE, each scaled by what it reads for the 1 GiB copy), as recorded in
    profiles/traffic.json; returns (bytes, a note naming that file and its run), or (None, None)."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None, None
    try:
        data = json.loads(f.read_text())
        rec = data.get(kernel_tag)
        if rec is None:
            return None, None
        return int(rec["traffic_bytes"]), f"profiles/traffic.json ({data.get('_run', 'counter run')})"
    except (ValueError, OSError, KeyError, TypeError, AttributeError):
        return None, None


def traffic_run(torch, ops, shape, make_inputs, tokens):
    src = torch.empty(512 << 20, dtype=torch.bfloat16, device="cuda").normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)                       # 1 GiB read + 1 GiB written
    torch.cuda.synchronize()
    del src, dst
    inp = make_inputs(shape, tokens, device="cuda")
    for _ in range(2):
        ops.fused_moe(inp.x, inp.logits, shape.top_k, inp.w_gate_up, inp.w_down, renormalize=shape.renormalize)
    dx, dl = inp.x[:64].contiguous(), inp.logits[:64].contiguous()
    for _ in range(2):   # the 64-token decode batch (weight-streaming kernels)
        ops.fused_moe(dx, dl, shape.top_k, inp.w_gate_up, inp.w_down, renormalize=shape.renormalize)
    torch.cuda.synchronize()
    print("traffic run done", flush=True)


def settle(fn, warmup, torch, min_s=0.05):
    """Run a suite case until at least ``min_s`` seconds of it have executed (and ``warmup``
    calls): a freshly drawn workload measured ~10 % slow over its first few milliseconds
    (DeepSeek-V2-Lite zipf, 0.85 ms on the first timing vs 0.77 ms on later ones)."""
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < min_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def timed_cold(fn, steps, warmup, torch, flush):
    """Mean ms of fn with the device caches flushed before every call (each call bracketed by
    HIP events on the launch stream, the flush outside them): weights of a small layer would
    otherwise be served from the 256 MB last-level cache after the first call.  The flush
    reads a 512 MB buffer (a write would leave dirty lines whose write-back overlaps fn)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        flush.sum()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / steps


def layer_case(name, inp, torch, ops, steps, warmup, flush, *, w8a8=False, fp8w=None, router_kw=None):
    """One fused-layer workload: warm and cache-cold times, tokens/s, TFLOP/s and HBM GB/s."""
    from easyinfra_amd.workloads import layer_flops, layer_bytes
    s = inp.shape
    T, H = inp.x.shape
    I = s.inter
    n_local = inp.w_gate_up.shape[0]
    wgu, wd, scales = inp.w_gate_up, inp.w_down, None
    if fp8w is not None:
        wgu, wd, scales = fp8w
    Is = inp.shared_down.shape[1] if inp.shared_down is not None else 0
    kw = dict(renormalize=s.renormalize, shared_gate_up=inp.shared_gate_up, shared_down=inp.shared_down,
              expert_range=inp.expert_range, w_scales=scales, w8a8=w8a8, **(router_kw or {}))
    f32 = wgu.dtype == torch.float32
    flags = 4 if w8a8 else 32 if f32 else 0
    ws = torch.empty(ops.fused_moe_workspace_bytes(T, H, I, s.n_experts, s.top_k, n_local, Is, out_dtype=inp.x.dtype,
                                                   flags=flags), dtype=torch.uint8, device=inp.x.device)
    fn = lambda: ops.fused_moe(inp.x, inp.logits, s.top_k, wgu, wd, workspace=ws, **kw)
    _, ids, _ = ops.fused_moe(inp.x, inp.logits, s.top_k, wgu, wd, return_routing=True, **kw)
    lo, hi = inp.expert_range or (0, s.n_experts)
    local = ids[(ids >= lo) & (ids < hi)]
    A = int(local.numel())
    touched = int(torch.unique(local).numel())
    settle(fn, warmup, torch)
    ms = timed(fn, steps, warmup, torch)
    ms_cold = timed_cold(fn, steps, 1, torch, flush)
    flops = layer_flops(A, T, H, I, Is)
    b_w = 1 if fp8w is not None else 4 if f32 else 2
    b_x = 4 if f32 else 2
    nbytes = layer_bytes(touched, T, s.n_experts, H, I, b_w, b_x, b_x, Is, fp8_scales=fp8w is not None)
    peak = FP8_PEAK_TFLOPS if w8a8 else FP32_PEAK_TFLOPS if f32 else BF16_PEAK_TFLOPS
    return {"case": name, "tokens": T, "assignments": A, "touched_experts": touched, "ms": round(ms, 4),
            "ms_cold": round(ms_cold, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 1), "frac_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / peak, 4),
            "hbm_GBps_cold": round(nbytes / (ms_cold * 1e-3) / 1e9, 1),
            "hbm_frac_cold": round(nbytes / (ms_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def gate_case(torch, ops, steps, warmup, flush):
    """The DeepSeek-V3 gate alone: 4096 tokens x 256 experts, 8 groups keep 4, top-8 (HBM-bound:
    logits in, ids and weights out)."""
    T, E, k = 4096, 256, 8
    g = torch.Generator(device="cuda").manual_seed(5)
    logits = torch.randn(T, E, device="cuda", generator=g) * 2
    bias = torch.randn(E, device="cuda", generator=g) * 0.1
    fn = lambda: ops.router_grouped_topk(logits, k, 8, 4, bias, True, 2.5)
    settle(fn, warmup, torch)
    ms = timed(fn, steps, warmup, torch)
    ms_cold = timed_cold(fn, steps, 1, torch, flush)
    nbytes = T * E * 4 + E * 4 + T * k * 8
    return {"case": f"DeepSeek-V3 gate alone T={T} E={E} k={k} (8 groups keep 4)", "tokens": T, "ms": round(ms, 4),
            "ms_cold": round(ms_cold, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
            "hbm_GBps_cold": round(nbytes / (ms_cold * 1e-3) / 1e9, 1),
            "hbm_frac_cold": round(nbytes / (ms_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def prologue_case(torch, ops, steps, warmup, flush, T, H, E, logits_bf16, name):
    """Residual add + RMSNorm + router logits (HBM-bound: two rows in, two rows out)."""
    g = torch.Generator(device="cuda").manual_seed(T + E)
    hid = torch.randn(T, H, device="cuda", generator=g).to(torch.bfloat16)
    res = torch.randn(T, H, device="cuda", generator=g).to(torch.bfloat16)
    w = torch.ones(H, device="cuda", dtype=torch.bfloat16)
    gw = (0.02 * torch.randn(E, H, device="cuda", generator=g)).to(torch.bfloat16)
    ws = torch.empty(max(ops.moe_prologue_workspace_bytes(T, H, E), 1), dtype=torch.uint8, device="cuda")
    fn = lambda: ops.moe_prologue(hid, res, w, 1e-6, gw, logits_bf16, workspace=ws)
    settle(fn, warmup, torch)
    ms = timed(fn, steps, warmup, torch)
    ms_cold = timed_cold(fn, steps, 1, torch, flush)
    nbytes = 4 * T * H * 2 + T * E * 4 + E * H * 2
    return {"case": f"MoE prologue (residual add + RMSNorm + router) {name} T={T} H={H} E={E}", "tokens": T,
            "ms": round(ms, 4), "ms_cold": round(ms_cold, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
            "hbm_GBps_cold": round(nbytes / (ms_cold * 1e-3) / 1e9, 1),
            "hbm_frac_cold": round(nbytes / (ms_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def suite(torch, ops, mix_inp, steps, warmup):
    """The other workloads of the layer, one GPU each: timings only (parity is in tests/)."""
    from easyinfra_amd.workloads import SHAPES, make_inputs
    dev = mix_inp.x.device
    flush = torch.ones(128 << 20, dtype=torch.float32, device=dev)   # 512 MB > the 256 MB last-level cache
    out = []
    inp = make_inputs(SHAPES["tiny-mixtral-fp32"], 512, device=dev)
    out.append(layer_case("tiny-mixtral-fp32 T=512 (fp32 layer, fp32 MFMA)", inp, torch, ops, steps, warmup, flush))
    del inp
    ds = SHAPES["deepseek-v2-lite"]
    skew = layer_case("deepseek-v2-lite T=4096 zipf(1.2) + 2 shared", make_inputs(ds, 4096, device=dev), torch, ops,
                      steps, warmup, flush)
    uni = layer_case("deepseek-v2-lite T=4096 uniform twin", make_inputs(ds, 4096, device=dev, uniform_twin=True),
                     torch, ops, steps, warmup, flush)
    skew["skew_over_uniform"] = round(skew["ms"] / uni["ms"], 3)
    out += [skew, uni]
    # a mid-size batch (72 rows per expert on average): the routed GEMMs on other tiles
    mid = layer_case("deepseek-v2-lite T=768 zipf(1.2) + 2 shared", make_inputs(ds, 768, device=dev), torch, ops,
                     steps, warmup, flush)
    mid_u = layer_case("deepseek-v2-lite T=768 uniform twin", make_inputs(ds, 768, device=dev, uniform_twin=True),
                       torch, ops, steps, warmup, flush)
    mid["skew_over_uniform"] = round(mid["ms"] / mid_u["ms"], 3)
    out += [mid, mid_u]
    # the DeepSeek-V3 gate (sigmoid, correction bias, 8 groups keep 4, scaling 2.5) routing the
    # same layer, and the gate alone at DeepSeek-V3's own size (4096 tokens, 256 experts, top-8)
    ds_inp = make_inputs(ds, 4096, device=dev)
    bias = torch.randn(ds.n_experts, device=dev, generator=torch.Generator(device=dev).manual_seed(3)) * 0.1
    v3 = dict(scoring_func="sigmoid", n_group=8, topk_group=4, e_score_correction_bias=bias,
              routed_scaling_factor=2.5)
    out.append(layer_case("deepseek-v2-lite T=4096 + 2 shared, DeepSeek-V3 gate (8 groups keep 4)", ds_inp, torch,
                          ops, steps, warmup, flush, router_kw=v3))
    del ds_inp
    out.append(gate_case(torch, ops, steps, warmup, flush))
    out.append(prologue_case(torch, ops, steps, warmup, flush, 8192, 4096, 8, True, "Mixtral-8x7B"))
    out.append(prologue_case(torch, ops, steps, warmup, flush, 4096, 7168, 256, False, "DeepSeek-V3"))
    qw = SHAPES["qwen3-30b-a3b-local32"]
    for T in (1, 32, 256, 768, 2048):
        hot = layer_case(f"qwen3-30b-a3b local 32/128 T={T} hot:cold 8:1", make_inputs(qw, T, device=dev), torch, ops,
                         steps, warmup, flush)
        twin = layer_case(f"qwen3-30b-a3b local 32/128 T={T} uniform twin",
                          make_inputs(qw, T, device=dev, uniform_twin=True), torch, ops, steps, warmup, flush)
        hot["skew_over_uniform_cold"] = round(hot["ms_cold"] / twin["ms_cold"], 3)
        out += [hot, twin]
    qgu, sgu = ops.quantize_weights_fp8(mix_inp.w_gate_up)
    qd, sd = ops.quantize_weights_fp8(mix_inp.w_down)
    for T in (8192, 64):
        sub = mix_inp if T == mix_inp.x.shape[0] else type(mix_inp)(mix_inp.shape, mix_inp.x[:T].contiguous(),
                                                                     mix_inp.logits[:T].contiguous(),
                                                                     mix_inp.w_gate_up, mix_inp.w_down)
        out.append(layer_case(f"mixtral-8x7b fp8-e4m3 W8A8 T={T}", sub, torch, ops, steps, warmup, flush, w8a8=True,
                              fp8w=(qgu, qd, (sgu, sd))))
        # W8A16 (e4m3 weights widened to bf16, bf16 MFMA): the fp8 mode within 5e-2 rel-L2 of the bf16 layer
        out.append(layer_case(f"mixtral-8x7b fp8-e4m3 W8A16 T={T}", sub, torch, ops, steps, warmup, flush,
                              fp8w=(qgu, qd, (sgu, sd))))
    return out


def profile_case(torch, ops, spec):
    from easyinfra_amd.workloads import SHAPES, make_inputs
    parts = spec.split(":")
    if parts[0] == "copy":   # counter calibration: a 1 GiB device copy (1 GiB read + 1 GiB written)
        src = torch.empty(512 << 20, dtype=torch.bfloat16, device="cuda").normal_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print("profile case done:", spec, flush=True)
        return
    if parts[0] == "prologue":   # prologue:T:H:E[:f32] -- residual add + RMSNorm + router logits
        T, H, E = (int(v) for v in parts[1:4])
        g = torch.Generator(device="cuda").manual_seed(T + E)
        hid = torch.randn(T, H, device="cuda", generator=g).to(torch.bfloat16)
        res = torch.randn(T, H, device="cuda", generator=g).to(torch.bfloat16)
        w = torch.ones(H, device="cuda", dtype=torch.bfloat16)
        gw = (0.02 * torch.randn(E, H, device="cuda", generator=g)).to(torch.bfloat16)
        ws = torch.empty(max(ops.moe_prologue_workspace_bytes(T, H, E), 1), dtype=torch.uint8, device="cuda")
        flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
        for _ in range(12):
            flush.sum()
            ops.moe_prologue(hid, res, w, 1e-6, gw, "f32" not in parts[4:], workspace=ws)
        torch.cuda.synchronize()
        print("profile case done:", spec, flush=True)
        return
    shape, T = SHAPES[parts[0]], int(parts[1])
    inp = make_inputs(shape, T, device="cuda", uniform_twin="uniform" in parts[2:])
    wgu, wd, scales = inp.w_gate_up, inp.w_down, None   # the workload's own dtype (fp32: the fp32 layer)
    w8a8 = "w8a8" in parts[2:]
    if w8a8 or "w8a16" in parts[2:]:   # e4m3 weights (per-channel scales), activations e4m3 too for w8a8
        qgu, sgu = ops.quantize_weights_fp8(wgu)
        qd, sd = ops.quantize_weights_fp8(wd)
        wgu, wd, scales = qgu, qd, (sgu, sd)
    flush = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
    for _ in range(12):
        flush.sum()
        ops.fused_moe(inp.x, inp.logits, shape.top_k, wgu, wd, renormalize=shape.renormalize,
                      shared_gate_up=inp.shared_gate_up, shared_down=inp.shared_down,
                      expert_range=inp.expert_range, w_scales=scales, w8a8=w8a8)
    torch.cuda.synchronize()
    print("profile case done:", spec, flush=True)


def main():
    args = parse()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.trace_last)
        return
    if args.counter_summary:
        counter_summary(args.counter_summary, args.fetch_scale, args.write_scale, args.kernel_filter)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the MoE expert path is built and measured on a single "
              "MI355X (multi-GPU expert parallelism is out of scope); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from easyinfra_amd import ops
    from easyinfra_amd.workloads import MIXTRAL_8X7B, make_inputs, layer_flops, layer_bytes

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    shape = MIXTRAL_8X7B
    if args.traffic_run:
        traffic_run(torch, ops, shape, make_inputs, args.tokens)
        return
    if args.profile_case:
        profile_case(torch, ops, args.profile_case)
        return
    T = args.tokens
    inp = make_inputs(shape, T, device=dev)
    H, I, k = shape.hidden, shape.inter, shape.top_k
    n_local = inp.w_gate_up.shape[0]
    ws = torch.empty(ops.fused_moe_workspace_bytes(T, H, I, shape.n_experts, k, n_local), dtype=torch.uint8,
                     device=dev)

    def layer():
        ops.fused_moe(inp.x, inp.logits, k, inp.w_gate_up, inp.w_down, renormalize=shape.renormalize,
                      workspace=ws)

    ms = timed(layer, args.steps, args.warmup, torch)
    A = T * k
    flops = layer_flops(A, T, H, I)
    stages, down_split = stage_times(inp, args.steps, args.warmup, torch, ops)
    gu_flops = 4.0 * A * H * I
    gu_ms = stages["gate_up_silu"]
    achieved = gu_flops / (gu_ms * 1e-3) / 1e12
    traffic, traffic_src = traffic_from_profiles("gate_up_silu_prefill")
    roof = {"bound": "mfma", "kernel": "grouped_gemm_pp3p_kernel<2, 8, 0> (256x256 bf16 gate/up + SiLU*mul, persistent)",
            "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": traffic, "traffic_source": traffic_src,
            "flops_per_launch": gu_flops, "mean_launch_ms": round(gu_ms, 4),
            "launches_averaged": args.steps,
            "launches_note": f"the last {args.steps} of {2 * (args.warmup + args.steps)} launches of this kernel in the "
                             f"run: the layer's {args.warmup} + {args.steps} calls, then {args.warmup} warm-up and "
                             f"{args.steps} timed stage calls (HIP events on the launch stream)"}

    # decode batch (HBM-bound): the first decode-tokens rows of the same layer
    Td = args.decode_tokens
    dx, dl = inp.x[:Td].contiguous(), inp.logits[:Td].contiguous()
    dws = torch.empty(ops.fused_moe_workspace_bytes(Td, H, I, shape.n_experts, k, n_local), dtype=torch.uint8,
                      device=dev)
    ids_d, _ = ops.router_topk(dl, k, shape.renormalize)
    touched = int(torch.unique(ids_d).numel())
    dms = timed(lambda: ops.fused_moe(dx, dl, k, inp.w_gate_up, inp.w_down, renormalize=shape.renormalize,
                                      workspace=dws), max(args.steps, 20), args.warmup, torch)
    dbytes = layer_bytes(touched, Td, shape.n_experts, H, I, 2, 2, 2)
    decode = {"tokens": Td, "ms": round(dms, 4), "tokens_per_s": round(Td / (dms * 1e-3), 1),
              "hbm_GBps": round(dbytes / (dms * 1e-3) / 1e9, 1),
              "hbm_frac": round(dbytes / (dms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "touched_experts": touched}

    cases = None if args.no_suite else suite(torch, ops, inp, max(5, args.steps // 2), 2)

    cpu = None
    if args.cpu_tokens > 0:
        cpu = cpu_baseline(inp, args.cpu_tokens, args.cpu_runs, torch)

    line = {
        "metric": METRIC, "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, router logits x@gate_w)",
        "config": {"workload": "Mixtral-8x7B-shape MoE layer prefill", "tokens": T, "hidden": H, "inter": I,
                   "experts": shape.n_experts, "top_k": k, "router": "softmax, top-2, renormalised",
                   "weights": "bf16", "parallelism": "single GPU"},
        "layer": {"tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                  "frac_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                  "gflop": round(flops / 1e9, 1)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "decode": decode,
        "kernels_ms": {k_: round(v, 4) for k_, v in stages.items()},
        "down_k_split": down_split,
        "suite": cases,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
