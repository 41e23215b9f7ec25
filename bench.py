#!/usr/bin/env python3
"""Benchmark: one FP8 W8A8 Mega MoE layer (one GPU's expert-parallel share: 32 local experts,
H=4096, I=2048, top-6) per step, through the drop-in API ``fp8_w8a8_mega_moe``.

Default workload = BASELINE config 1 (decode, HBM-bound): 8x128 = 1024 source tokens routed
top-6 over 256 global experts from softmax(N(0,1)) logits, only experts 0..31 kept (~768 rows).
Synthetic seeded data, random-init weights N(0, 1/sqrt(K)) quantised channelwise to e4m3.

Timing: W warm-up layers, then K timed layers. Before every layer a 1 GiB buffer is read (a
reduction) to flush the L2/MALL outside the timed events -- a read, so no dirty lines are left
whose write-back would be charged to the layer; each layer is bracketed by HIP events on the
stream it runs on. A second pass launches the five stages separately with events between them
to attribute time per kernel (roofline of the dominant kernel). The CPU baseline is the
repository's own oracle (a restatement of the reference's dequantise-and-matmul baseline) on
the host cores, on a bounded sample of the same workload.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

E_LOCAL, HIDDEN, INTER, TOPK = 32, 4096, 2048, 6
HBM_PEAK_BPS = 8.0e12       # MI355X HBM3E
FP8_PEAK_FLOPS = 5.0e15     # MI355X dense FP8 MFMA

CONFIGS = {
    "c0": dict(id=0, tokens=64, global_experts=None, routing="softmax",
               workload="c0 T=64, 32 local experts (CPU-plumbing config)"),
    "c1": dict(id=1, tokens=1024, global_experts=256, routing="softmax",
               workload="c1 decode T=128: 8x128 source tokens, top-6 of 256 experts, 0-31 kept"),
    "c2": dict(id=2, tokens=32768, global_experts=256, routing="softmax",
               workload="c2 crossover T=4096: 8x4096 source tokens, top-6 of 256, 0-31 kept"),
    "c3": dict(id=3, tokens=262144, global_experts=256, routing="softmax",
               workload="c3 prefill T=32768: 8x32768 source tokens, top-6 of 256, 0-31 kept"),
    "c4": dict(id=4, tokens=8192, global_experts=None, routing="zipf",
               workload="c4 skew T=8192: top-6 i.i.d. Zipf(1.2) over 28 experts, 4 empty"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(rows: int, touched: int) -> dict:
    """Bytes per layer and per kernel, the reference's formula
    (tests/test_mega_moe_dcu.py:352-366) split by kernel."""
    h, i = HIDDEN, INTER
    layer = (touched * (2 * i * h + h * i) + touched * (2 * i + h) * 4 + rows * (h + 4)
             + rows * (i + 4) * 2 + rows * h * 2)
    gemm1 = touched * 2 * i * h + touched * 2 * i * 4 + rows * (h + 4) + rows * 2 * i * 2
    gemm2 = touched * h * i + touched * h * 4 + rows * (i + 4) + rows * h * 2
    return dict(layer=layer, gemm1=gemm1, gemm2=gemm2)


# kernel names as rocprofv3 reports them: the 8-wave persistent kernel (decode-sized configs)
# or the 4-wave WIDE kernel (many rows per expert)
PROFILE_KERNELS = {"gemm1": ("grouped_gemm_kernel<true, true, false>", "wide_gemm_kernel<true, true>"),
                   "gemm2": ("grouped_gemm_kernel<false, false, false>", "wide_gemm_kernel<false, false>")}


def profiled_traffic(config_id: str, kernel: str):
    """HBM bytes per dispatch of `kernel` measured by the two rocprofv3 --pmc passes
    (FETCH_SIZE, WRITE_SIZE, calibrated on a plain copy) recorded in
    profiles/megamoe_layer_<config>_*.md, or None when that config has no profile."""
    import glob

    names = PROFILE_KERNELS[kernel]
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", f"megamoe_layer_{config_id}_*.md"))):
        for line in open(path):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) == 4 and cells[0] in names and cells[3].isdigit():
                return int(cells[3]), os.path.relpath(path, ROOT)
    return None


def make_inputs(cfg: dict, torch, mm):
    """Seeded synthetic inputs drawn on the GPU (seed 1234 + config id)."""
    seed = 1234 + cfg["id"]
    s = cfg["tokens"]
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((s, HIDDEN), generator=g, device="cuda").to(torch.bfloat16)
    if cfg["routing"] == "zipf":
        perm = torch.randperm(E_LOCAL, generator=g, device="cuda")
        live = perm[4:]
        p = torch.arange(1, live.numel() + 1, device="cuda", dtype=torch.float64) ** (-1.2)
        p = (p / p.sum()).float()
        draws = torch.multinomial(p, s * TOPK, replacement=True, generator=g)
        idx = live[draws].view(s, TOPK).to(torch.int64)
        w = torch.rand((s, TOPK), generator=g, device="cuda") + 0.05
        w = w / w.sum(-1, keepdim=True)
    else:
        ge = cfg["global_experts"] or E_LOCAL
        logits = torch.randn((s, ge), generator=g, device="cuda")
        w, idx = torch.topk(torch.softmax(logits, -1), TOPK, dim=-1)
        w = w / w.sum(-1, keepdim=True)
        idx = torch.where(idx < E_LOCAL, idx, torch.full_like(idx, -1)).to(torch.int64)
    x_fp8, x_sf = mm.cast_to_fp8_channelwise(x)
    w1 = (torch.randn((E_LOCAL, 2 * INTER, HIDDEN), generator=g, device="cuda")
          / math.sqrt(HIDDEN)).to(torch.bfloat16)
    w2 = (torch.randn((E_LOCAL, HIDDEN, INTER), generator=g, device="cuda")
          / math.sqrt(INTER)).to(torch.bfloat16)
    l1, l2 = mm.transform_fp8_weights_for_mega_moe(w1, w2)
    del w1, w2, x
    return x_fp8, x_sf, idx.contiguous(), w.float().contiguous(), l1, l2


def cpu_baseline(x_fp8, x_sf, idx, w, l1, l2, y_gpu, budget_s: float, torch):
    """Time the oracle (K2-form dequant pipeline) on the host cores on a bounded sample:
    the experts [0, n) of the same workload (all 32 when it fits the budget)."""
    from oracle import megamoe_oracle as O

    threads = torch.get_num_threads()
    xc, sc, ic, wc = x_fp8.cpu(), x_sf.cpu(), idx.cpu(), w.cpu()
    l1c = (l1[0].cpu(), l1[1].cpu())
    l2c = (l2[0].cpu(), l2[1].cpu())
    total_rows = int(((ic >= 0) & (ic < E_LOCAL) & (wc != 0)).sum())
    n_exp = E_LOCAL
    # rough cost model from one timed expert, then shrink the sample to the budget
    t_start = time.perf_counter()
    ic1 = torch.where(ic < 1, ic, torch.full_like(ic, -1))
    O.mega_moe_forward(xc, sc, ic1, wc, (l1c[0][:1], l1c[1][:1]), (l2c[0][:1], l2c[1][:1]))
    per_exp = time.perf_counter() - t_start
    n_exp = max(1, min(E_LOCAL, int(budget_s / max(per_exp, 1e-3))))
    icn = torch.where(ic < n_exp, ic, torch.full_like(ic, -1))
    l1n = (l1c[0][:n_exp].contiguous(), l1c[1][:n_exp].contiguous())
    l2n = (l2c[0][:n_exp].contiguous(), l2c[1][:n_exp].contiguous())
    t0 = time.perf_counter()
    tr = O.mega_moe_forward(xc, sc, icn, wc, l1n, l2n)
    dt = time.perf_counter() - t0
    rows = tr.routing.num_rows
    parity = None
    if n_exp == E_LOCAL:
        parity = O.calc_diff(y_gpu.cpu(), tr.y)
    # scale to a whole layer by FLOPs (rows) -- weights dequant scales with experts, rows with
    # rows; the sample keeps both proportional to the full layer
    scale = total_rows / max(rows, 1)
    us_layer = dt * scale * 1e6
    return dict(value=round(us_layer, 1), unit="us/layer", cores=threads, kind="port",
                sample=f"oracle forward (fp32 dequant matmuls, weight dequant included) on "
                       f"experts 0..{n_exp - 1}: {rows} of {total_rows} routed rows, "
                       f"{dt:.2f} s, scaled by rows", parity_calc_diff=parity)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c1", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-stage-timing", action="store_true")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after timing, copy a buffer of this many MiB device-to-device once "
                         "(a known-size kernel that calibrates rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs one GPU's expert-parallel share; --gpus must be 1 "
              "(multi-GPU dispatch/combine is not built)", file=sys.stderr)
        return 2

    import torch

    from deepgemm_amd import megamoe as mm

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    torch.cuda.set_device(0)
    cfg = CONFIGS[args.config]
    log(f"config {args.config}: {cfg['workload']}")
    x_fp8, x_sf, idx, w, l1, l2 = make_inputs(cfg, torch, mm)
    s = cfg["tokens"]
    buf = mm.get_symm_buffer_for_mega_moe(None, E_LOCAL, s, TOPK, HIDDEN, INTER)
    buf.x[:s].copy_(x_fp8)
    buf.x_sf[:s].copy_(x_sf)
    buf.topk_idx[:s].copy_(idx)
    buf.topk_weights[:s].copy_(w)
    y = torch.empty((s, HIDDEN), dtype=torch.bfloat16, device="cuda")
    # Cache flush between steps: READ 1 GiB (a reduction), which evicts L2/MALL without leaving
    # dirty lines whose write-back would be charged to the next layer.
    flush = torch.ones((1 << 28,), dtype=torch.float32, device="cuda")

    def flush_cache():
        flush.sum()

    def layer():
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf)

    log(f"warmup {args.warmup}")
    for _ in range(max(1, args.warmup)):
        layer()
    torch.cuda.synchronize()
    counts = buf.scratch_view("counts").cpu()
    rows = int(counts.sum())
    touched = int((counts > 0).sum())
    mode = buf._large_opt_3stage_mode
    schedule = {"auto": "auto (per-expert engine)", "force": "tile engine",
                "off": "streaming engine"}[mode]
    stream_experts = int(((counts > 0) & (counts <= 64)).sum())
    log(f"routed rows R={rows}, touched experts={touched}, schedule={schedule}, "
        f"experts on the streaming engine={stream_experts if mode == 'auto' else '-'}")

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for i in range(args.steps):
        flush_cache()
        starts[i].record()
        layer()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = [a.elapsed_time(b) for a, b in zip(starts, ends)]
    med_ms = statistics.median(ms)
    log(f"layer: median {med_ms * 1e3:.1f} us, min {min(ms) * 1e3:.1f} us")

    stage_ms = None
    if not args.no_stage_timing:
        # The stages as the layer runs them: routing and GEMM1 are one launch when GEMM1 routes
        # in-kernel (small task counts), so they are timed together; the GEMM1 roofline below
        # uses that launch.
        call = mm.LayerCall(y, l1, l2, buf)
        groups = [("route_gemm1", 0, 1), ("requant", 2, 2), ("gemm2", 3, 3), ("combine", 4, 4)]
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(groups) + 1)]
              for _ in range(args.steps)]
        for i in range(args.steps):
            flush_cache()
            ev[i][0].record()
            for j, (_, first, last) in enumerate(groups):
                call.run(first, last)
                ev[i][j + 1].record()
        torch.cuda.synchronize()
        stage_ms = {name: statistics.median(ev[i][j].elapsed_time(ev[i][j + 1])
                                            for i in range(args.steps))
                    for j, (name, _, _) in enumerate(groups)}
        log("stages (median us): " + ", ".join(f"{k}={v * 1e3:.1f}" for k, v in stage_ms.items()))

    flops = 6.0 * rows * HIDDEN * INTER
    nbytes = algorithmic_bytes(rows, touched)
    t_s = med_ms * 1e-3
    tflops = flops / t_s / 1e12
    hbm_frac = nbytes["layer"] / t_s / HBM_PEAK_BPS
    mfma_frac = flops / t_s / FP8_PEAK_FLOPS
    bound = "hbm" if nbytes["layer"] and flops / nbytes["layer"] < FP8_PEAK_FLOPS / HBM_PEAK_BPS \
        else "mfma"

    roofline = None
    if stage_ms is not None:
        stage_ms["gemm1"] = stage_ms.pop("route_gemm1")
        dom = max(("gemm1", "gemm2"), key=lambda k: stage_ms[k])
        dom_s = stage_ms[dom] * 1e-3
        prof = profiled_traffic(args.config, dom)
        traffic = prof[0] if prof else None
        if bound == "hbm":
            achieved = nbytes[dom] / dom_s / 1e9
            roofline = dict(kernel=dom, bound="hbm", achieved=round(achieved, 1),
                            peak=HBM_PEAK_BPS / 1e9, unit="GB/s",
                            frac=round(achieved * 1e9 / HBM_PEAK_BPS, 4), traffic=traffic,
                            algorithmic_bytes=nbytes[dom], avg_us=round(stage_ms[dom] * 1e3, 2),
                            traffic_source=prof[1] if prof else None)
        else:
            kflops = 2.0 * rows * HIDDEN * (2 * INTER if dom == "gemm1" else INTER)
            achieved = kflops / dom_s / 1e12
            roofline = dict(kernel=dom, bound="mfma", achieved=round(achieved, 1),
                            peak=FP8_PEAK_FLOPS / 1e12, unit="TFLOP/s",
                            frac=round(achieved * 1e12 / FP8_PEAK_FLOPS, 4), traffic=traffic,
                            algorithmic_flops=kflops, avg_us=round(stage_ms[dom] * 1e3, 2),
                            traffic_source=prof[1] if prof else None)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)")
        cpu = cpu_baseline(x_fp8, x_sf, idx, w, l1, l2, y, args.cpu_budget_s, torch)
        log(f"cpu baseline: {cpu['value']} us/layer on {cpu['cores']} threads; "
            f"parity calc_diff={cpu.get('parity_calc_diff')}")

    out = {
        "metric": "us per MoE layer (FP8 W8A8 Mega MoE, one GPU's EP share)",
        "value": round(med_ms * 1e3, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(med_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded N(0,1) tokens/logits, N(0,1/sqrt(K)) weights)",
        "config": {"workload": cfg["workload"], "config_id": args.config, "tokens": s,
                   "experts": E_LOCAL, "hidden": HIDDEN, "intermediate": INTER, "topk": TOPK,
                   "routed_rows": rows, "touched_experts": touched, "schedule": schedule},
        "min_us": round(min(ms) * 1e3, 2),
        "fp8_tflops": round(tflops, 2),
        "hbm_frac": round(hbm_frac, 4),
        "mfma_frac": round(mfma_frac, 4),
        "layer_bound": bound,
        "algorithmic_bytes": nbytes["layer"],
        "flops": flops,
        "stage_us": None if stage_ms is None else {k: round(v * 1e3, 2) for k, v in stage_ms.items()},
        "wall_s_timed_loop_incl_flush": round(wall, 4),
        "flush": "1 GiB read (reduction) before every step, outside the timed events",
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib << 20
        src = torch.ones((n,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        out["calibration_copy_bytes"] = n
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
