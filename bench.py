#!/usr/bin/env python3
"""Benchmark: one FP8 W8A8 Mega MoE layer (one GPU's expert-parallel share: 32 local experts,
H=4096, I=2048, top-6) per step, through the drop-in API ``fp8_w8a8_mega_moe``.

Headline workload (``value``) = BASELINE config 1 (decode, HBM-bound): 8x128 = 1024 source
tokens routed top-6 over 256 global experts from softmax(N(0,1)) logits, only experts 0..31
kept (~768 rows). The same run also times configs 2-4 (T=4096 crossover, T=32768 prefill,
Zipf-skewed T=8192) and reports each under ``per_config``. Synthetic seeded data,
random-init weights N(0, 1/sqrt(K)) quantised channelwise to e4m3.

Timing: W warm-up layers, then K timed layers per config. Before every layer a 1 GiB buffer is
read (a reduction) to flush the L2/MALL outside the timed events -- a read, so no dirty lines
are left whose write-back would be charged to the layer; each layer is bracketed by HIP events
on the stream it runs on (`value`: the median; it includes the ~5-6 us by which a kernel that
follows a recorded event starts late). A second pass runs the same whole-layer calls through
mmoe_forward_profile, which launches each of the layer's kernels with its own start and stop
event (hipExtLaunchKernel: the dispatch's timestamps, as a kernel trace reads them): the
per-kernel times (`stage_us`) and the dominant kernel's roofline come from there, so they are
the kernels as they run inside the layer. The CPU baseline is the repository's own oracle (a
restatement of the reference's dequantise-and-matmul baseline) on all host cores, over whole
layers: c0 x10, c1 x3, c2/c3/c4 x1 (medians).

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

E_LOCAL, HIDDEN, INTER, TOPK = 32, 4096, 2048, 6
HBM_PEAK_BPS = 8.0e12       # MI355X HBM3E
FP8_PEAK_FLOPS = 5.0e15     # MI355X dense FP8 MFMA

CONFIGS = {
    "c0": dict(id=0, tokens=64, global_experts=None, routing="softmax", cpu_reps=10,
               workload="c0 T=64, 32 local experts (CPU-plumbing config)"),
    "c1": dict(id=1, tokens=1024, global_experts=256, routing="softmax", cpu_reps=3,
               workload="c1 decode T=128: 8x128 source tokens, top-6 of 256 experts, 0-31 kept"),
    "c2": dict(id=2, tokens=32768, global_experts=256, routing="softmax", cpu_reps=1,
               workload="c2 crossover T=4096: 8x4096 source tokens, top-6 of 256, 0-31 kept"),
    "c3": dict(id=3, tokens=262144, global_experts=256, routing="softmax", cpu_reps=1,
               workload="c3 prefill T=32768: 8x32768 source tokens, top-6 of 256, 0-31 kept"),
    "c4": dict(id=4, tokens=8192, global_experts=None, routing="zipf", cpu_reps=1,
               workload="c4 skew T=8192: top-6 i.i.d. Zipf(1.2) over 28 experts, 4 empty"),
    # EP shares between c1 and c2 (not BASELINE configs; run only when named in --configs):
    # T=448 puts at most 128 rows on an expert (the 8-wave kernels' 128-row STREAM items), T=1024
    # one WIDE row block an expert
    "m1": dict(id=5, tokens=3584, global_experts=256, routing="softmax", cpu_reps=1,
               workload="m1 EP share T=448: 8x448 source tokens, top-6 of 256, 0-31 kept"),
    "m2": dict(id=6, tokens=8192, global_experts=256, routing="softmax", cpu_reps=1,
               workload="m2 EP share T=1024: 8x1024 source tokens, top-6 of 256, 0-31 kept"),
}
HEADLINE = "c1"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(rows: int, touched: int) -> dict:
    """Bytes per layer and per kernel, the reference's formula
    (tests/test_mega_moe_dcu.py:352-366) split by kernel."""
    h, i = HIDDEN, INTER
    layer = (touched * (2 * i * h + h * i) + touched * (2 * i + h) * 4 + rows * (h + 4)
             + rows * (i + 4) * 2 + rows * h * 2)
    # GEMM1 applies the SwiGLU x route weight in its epilogue: it writes y [R, I] in bf16 (the
    # reference's fused output), not h [R, 2I]
    gemm1 = touched * 2 * i * h + touched * 2 * i * 4 + rows * (h + 4) + rows * i * 2
    gemm2 = touched * h * i + touched * h * 4 + rows * (i + 4) + rows * h * 2
    # the decode pipeline runs the whole layer (routing through the combine) in one launch
    return dict(layer=layer, gemm1=gemm1, gemm2=gemm2, pipeline=layer)


# kernel names as rocprofv3 reports them: the 8-wave persistent kernel (decode-sized configs)
# or the 4-wave WIDE kernel (many rows per expert)
PROFILE_KERNELS = {"gemm1": ("grouped_gemm_kernel<true, true, false>", "wide_gemm_kernel<true, true, 256>"),
                   "gemm2": ("grouped_gemm_kernel<false, false, false>", "wide_gemm_kernel<false, false, 256>"),
                   "pipeline": ("decode_pipeline_kernel",)}


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


def make_weights(torch, mm, seed: int):
    """W1 ~ N(0, 1/sqrt(H)) [E, 2I, H], W2 ~ N(0, 1/sqrt(I)) [E, H, I], drawn on the GPU and
    transformed by the package (channelwise e4m3 cast + Marlin)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w1 = (torch.randn((E_LOCAL, 2 * INTER, HIDDEN), generator=g, device="cuda")
          / math.sqrt(HIDDEN)).to(torch.bfloat16)
    w2 = (torch.randn((E_LOCAL, HIDDEN, INTER), generator=g, device="cuda")
          / math.sqrt(INTER)).to(torch.bfloat16)
    l1, l2 = mm.transform_fp8_weights_for_mega_moe(w1, w2)
    del w1, w2
    return l1, l2


def make_tokens(cfg: dict, torch, mm):
    """Seeded synthetic tokens and routing drawn on the GPU (seed 1234 + config id)."""
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
    del x
    return x_fp8, x_sf, idx.contiguous(), w.float().contiguous()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


class CpuOracle:
    """The oracle (K2-form dequantise-and-matmul pipeline) on the host cores, on CPU copies of
    the weights unpacked from Marlin once (outside the timing)."""

    def __init__(self, l1, l2, torch):
        from oracle import megamoe_oracle as O

        self.O = O
        self.torch = torch
        self.l1 = (l1[0].cpu(), l1[1].cpu())
        self.l2 = (l2[0].cpu(), l2[1].cpu())
        self.unpacked = (O.marlin_unpack(self.l1[0], 2 * INTER, HIDDEN),
                         O.marlin_unpack(self.l2[0], HIDDEN, INTER))

    def run(self, xc, sc, ic, wc):
        """One whole oracle layer; returns (seconds, routed rows, trace). The trace keeps only
        what the pipeline produces (no extra SwiGLU pass for the checks)."""
        t0 = time.perf_counter()
        tr = self.O.mega_moe_forward(xc, sc, ic, wc, self.l1, self.l2, unpacked_weights=self.unpacked,
                                     keep_y_act=False)
        return time.perf_counter() - t0, tr.routing.num_rows, tr


def calc_diff_blocks(a, b, block: int = 16384) -> float:
    """calc_diff = 1 - 2*sum(xy)/sum(x^2+y^2) in float64 (deep_gemm/testing/numeric.py:5-11),
    summed over row blocks so that a 262,144-row output needs no whole float64 copies."""
    num = den = 0.0
    for i in range(0, a.shape[0], block):
        x, y = a[i:i + block].double(), b[i:i + block].double()
        num += float((x * y).sum())
        den += float((x * x + y * y).sum())
    return 0.0 if den == 0.0 else 1.0 - 2.0 * num / den


def cpu_full_layer(oracle: CpuOracle, inputs, y_gpu, reps: int):
    """The whole layer `reps` times on the host cores: median (and all reps), plus the parity
    of the last run against the GPU's output."""
    xc, sc, ic, wc = (t.cpu() for t in inputs)
    times, tr = [], None
    for _ in range(reps):
        dt, rows, tr = oracle.run(xc, sc, ic, wc)
        times.append(dt)
    return dict(median_s=statistics.median(times), reps_s=[round(t, 3) for t in times],
                rows=rows, parity_calc_diff=calc_diff_blocks(y_gpu.cpu(), tr.y))


class LayerProfiler:
    """Whole-layer calls through mmoe_forward_profile: each kernel launch of the layer carries
    its own start and stop event (hipExtLaunchKernel), so the events read the kernels' durations
    inside the layer (the dispatch's timestamps). Events are made once through the HIP runtime
    that the process already loaded."""

    STAGES = {0: "route", 1: "gemm1", 2: "requant", 3: "gemm2", 4: "combine", 5: "pipeline"}
    CAP = 16  # launches timed per call

    def __init__(self, torch, mm, y, l1, l2, buf, steps: int):
        import ctypes

        self.ct = ctypes
        self.torch, self.mm = torch, mm
        path = next(line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line)
        self.hip = ctypes.CDLL(path)
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        schedule = mm._eager_schedule(mm._large_opt_3stage_mode(), mm._large_opt_3stage_threshold(),
                                      y.size(0))
        self.args = mm._forward_args(y, l1, l2, None, buf, None, schedule)
        self.keep = (y, l1, l2, buf)
        self.events = []
        for _ in range(steps):
            arr = (ctypes.c_void_p * (2 * self.CAP))()
            for j in range(2 * self.CAP):
                ev = ctypes.c_void_p()
                assert self.hip.hipEventCreate(ctypes.byref(ev)) == 0
                arr[j] = ev.value
            self.events.append(arr)
        self.stages = [(ctypes.c_int32 * self.CAP)() for _ in range(steps)]
        self.count = [ctypes.c_int32() for _ in range(steps)]

    def launch(self, i: int) -> None:
        ct = self.ct
        st = self.mm._capi.load().mmoe_forward_profile(
            ct.byref(self.args), self.mm._stream_handle(), ct.cast(self.events[i], ct.c_void_p),
            self.CAP, self.stages[i], ct.byref(self.count[i]))
        self.mm._capi.check(st, "mmoe_forward_profile")

    def read(self):
        """Per call: [(stage name, ms)] in launch order (after a synchronize)."""
        out = []
        for arr, stg, cnt in zip(self.events, self.stages, self.count):
            step = []
            for j in range(min(cnt.value, self.CAP)):
                ms = self.ct.c_float()
                assert self.hip.hipEventElapsedTime(self.ct.byref(ms), arr[2 * j], arr[2 * j + 1]) == 0
                step.append((self.STAGES[stg[j]], ms.value))
            out.append(step)
        return out

    def close(self) -> None:
        for arr in self.events:
            for ev in arr:
                self.hip.hipEventDestroy(ev)
        self.events = []


def time_config(name: str, cfg: dict, l1, l2, args, torch, mm, flush_cache):
    """Times the layer (and its stages) on one config; returns (result dict, inputs, y)."""
    log(f"config {name}: {cfg['workload']}")
    inputs = make_tokens(cfg, torch, mm)
    x_fp8, x_sf, idx, w = inputs
    s = cfg["tokens"]
    buf = mm.get_symm_buffer_for_mega_moe(None, E_LOCAL, s, TOPK, HIDDEN, INTER)
    buf.x[:s].copy_(x_fp8)
    buf.x_sf[:s].copy_(x_sf)
    buf.topk_idx[:s].copy_(idx)
    buf.topk_weights[:s].copy_(w)
    y = torch.empty((s, HIDDEN), dtype=torch.bfloat16, device="cuda")

    def layer():
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf)

    # the one-launch decode pipeline (routing, GEMM1, requant, GEMM2 and the combine) is the
    # only kernel that writes the per-block row maxima: whether it ran is read back from them
    buf.scratch_view("pmax").fill_(-1.0)
    for _ in range(max(1, args.warmup)):
        layer()
    torch.cuda.synchronize()
    counts = buf.scratch_view("counts").cpu()
    rows = int(counts.sum())
    pipeline = rows > 0 and bool((buf.scratch_view("pmax")[:rows] >= 0).all())
    touched = int((counts > 0).sum())
    log(f"  routed rows R={rows}, touched experts={touched}, largest expert={int(counts.max())}")

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
    log(f"  layer: median {med_ms * 1e3:.1f} us, min {min(ms) * 1e3:.1f} us")

    stage_ms = kernel_ms = None
    launches = None
    if not args.no_stage_timing:
        # The same whole-layer calls, each kernel launched with its own start and stop event:
        # the kernels' durations inside the layer (a dual launch's kernel that returns at once
        # counts in its stage; with the decode pipeline the layer is one launch).
        prof = LayerProfiler(torch, mm, y, l1, l2, buf, args.steps)
        for i in range(args.steps):
            flush_cache()
            prof.launch(i)
        torch.cuda.synchronize()
        per = prof.read()
        prof.close()
        names = [n for n in LayerProfiler.STAGES.values() if any(n == m for step in per for m, _ in step)]
        stage_ms = {n: statistics.median(sum(ms for m, ms in step if m == n) for step in per) for n in names}
        # the roofline's kernel time: the stage's longest launch (a dual launch's other kernel
        # returns at once; it counts in stage_us but did none of the stage's work)
        kernel_ms = {n: statistics.median(max(ms for m, ms in step if m == n) for step in per) for n in names}
        launches = [m for m, _ in per[0]]
        log("  kernels in the layer (median us): " + ", ".join(f"{k}={v * 1e3:.1f}" for k, v in stage_ms.items())
            + f"; launches {launches}")

    flops = 6.0 * rows * HIDDEN * INTER
    nbytes = algorithmic_bytes(rows, touched)
    t_s = med_ms * 1e-3
    bound = "hbm" if flops / max(nbytes["layer"], 1) < FP8_PEAK_FLOPS / HBM_PEAK_BPS else "mfma"
    roofline = None
    if stage_ms is not None:
        dom = "pipeline" if pipeline else max(("gemm1", "gemm2"), key=lambda k: stage_ms[k])
        dom_ms = kernel_ms[dom]
        dom_s = dom_ms * 1e-3
        prof_traffic = profiled_traffic(name, dom)
        timing = ("the kernel's own start/stop events (hipExtLaunchKernel) in whole-layer calls, "
                  "median over the steps (of a dual launch, the kernel that ran)")
        if bound == "hbm":
            achieved = nbytes[dom] / dom_s / 1e9
            roofline = dict(kernel=dom, bound="hbm", achieved=round(achieved, 1),
                            peak=HBM_PEAK_BPS / 1e9, unit="GB/s",
                            frac=round(achieved * 1e9 / HBM_PEAK_BPS, 4),
                            traffic=prof_traffic[0] if prof_traffic else None,
                            algorithmic_bytes=nbytes[dom], avg_us=round(dom_ms * 1e3, 2),
                            # the layer's bytes over the per-call event time (`value`, which also
                            # holds the event marker's start delay)
                            frac_of_layer_time=round(nbytes["layer"] / t_s / HBM_PEAK_BPS, 4),
                            timing=timing, traffic_source=prof_traffic[1] if prof_traffic else None)
        else:
            kflops = 2.0 * rows * HIDDEN * {"gemm1": 2 * INTER, "gemm2": INTER, "pipeline": 3 * INTER}[dom]
            achieved = kflops / dom_s / 1e12
            roofline = dict(kernel=dom, bound="mfma", achieved=round(achieved, 1),
                            peak=FP8_PEAK_FLOPS / 1e12, unit="TFLOP/s",
                            frac=round(achieved * 1e12 / FP8_PEAK_FLOPS, 4),
                            traffic=prof_traffic[0] if prof_traffic else None,
                            algorithmic_flops=kflops, avg_us=round(dom_ms * 1e3, 2),
                            frac_of_layer_time=round(flops / t_s / FP8_PEAK_FLOPS, 4),
                            timing=timing, traffic_source=prof_traffic[1] if prof_traffic else None)
    res = {
        "workload": cfg["workload"], "tokens": s, "routed_rows": rows, "touched_experts": touched,
        "largest_expert_rows": int(counts.max()),
        "us_median": round(med_ms * 1e3, 2), "us_min": round(min(ms) * 1e3, 2),
        "fp8_tflops": round(flops / t_s / 1e12, 2),
        "hbm_frac": round(nbytes["layer"] / t_s / HBM_PEAK_BPS, 4),
        "mfma_frac": round(flops / t_s / FP8_PEAK_FLOPS, 4),
        "layer_bound": bound, "algorithmic_bytes": nbytes["layer"], "flops": flops,
        "stage_us": None if stage_ms is None else {k: round(v * 1e3, 2) for k, v in stage_ms.items()},
        "launches": launches,
        "roofline": roofline, "wall_s_timed_loop_incl_flush": round(wall, 4),
    }
    del buf
    return res, inputs, y


def hipblaslt_gemm1(torch, rows: int, steps: int, flush_cache) -> dict:
    """hipBLASLt's FP8 GEMM (torch._scaled_mm) at a config's GEMM1 shape, for comparison only:
    [rows, H] x [H, 2I] e4m3 -> bf16, once with tensor-wise scales and once with per-row x
    per-column scales (what the layer needs; its GEMM1 also gathers the rows, which this does
    not). Median of `steps` calls, each after the cache flush, between two events."""
    m = (rows + 255) // 256 * 256
    g = torch.Generator(device="cuda").manual_seed(7)
    a = (torch.randn((m, HIDDEN), generator=g, device="cuda") * 0.5).to(torch.float8_e4m3fn)
    b = (torch.randn((2 * INTER, HIDDEN), generator=g, device="cuda") * 0.02).to(torch.float8_e4m3fn)
    sa = torch.rand((m, 1), generator=g, device="cuda") + 0.5
    sb = torch.rand((1, 2 * INTER), generator=g, device="cuda") + 0.5
    one = torch.ones((), device="cuda")
    out = {"rows": m, "n": 2 * INTER, "k": HIDDEN}
    for mode, (x, y) in (("tensorwise", (one, one)), ("rowwise", (sa, sb))):
        try:
            torch._scaled_mm(a, b.t(), scale_a=x, scale_b=y, out_dtype=torch.bfloat16)
            torch.cuda.synchronize()
        except Exception as exc:  # a scaling mode this torch/hipBLASLt does not offer
            out[mode] = f"unsupported: {str(exc)[:100]}"
            continue
        ts = []
        for _ in range(steps):
            flush_cache()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            torch._scaled_mm(a, b.t(), scale_a=x, scale_b=y, out_dtype=torch.bfloat16)
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        med = statistics.median(ts)
        out[mode] = {"us_median": round(med * 1e3, 1),
                     "tflops": round(2.0 * m * 2 * INTER * HIDDEN / (med * 1e-3) / 1e12, 1)}
        log(f"  hipBLASLt FP8 GEMM {m}x{2 * INTER}x{HIDDEN} {mode}: {out[mode]}")
    return out


def calibrate(torch, mib: int) -> dict:
    """Two known-size kernels for the rocprof byte counters of a profiling run: a read of
    `mib` MiB (a reduction: FETCH = mib MiB) and a device-to-device copy of `mib` MiB
    (FETCH = WRITE = mib MiB)."""
    n = mib << 20
    src = torch.ones((n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    src.view(torch.float32).sum()
    dst.copy_(src)
    torch.cuda.synchronize()
    return {"read_bytes": n, "copy_bytes": n}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="c0,c1,c2,c3,c4",
                    help="configs to time, comma-separated; the headline value is c1's (or the "
                         "first one's when c1 is not among them)")
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="time this one config only (same as --configs NAME)")
    ap.add_argument("--cpu-reps", type=int, default=0,
                    help="CPU baseline reps of every config's whole layer (0: c0 x10, c1 x3, "
                         "c2-c4 x1)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-stage-timing", action="store_true")
    ap.add_argument("--compare-hipblaslt", action="store_true",
                    help="also time hipBLASLt's FP8 GEMM (torch._scaled_mm) at each config's GEMM1 "
                         "shape (comparison only; reported under per_config.*.hipblaslt_gemm1)")
    ap.add_argument("--calibrate-mib", type=int, default=0,
                    help="after timing, read and copy a buffer of this many MiB once (known-size "
                         "kernels that calibrate rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs one GPU's expert-parallel share on one GPU; --gpus "
              "must be 1 (every GPU box here has one GPU, and the multi-GPU dispatch/combine "
              "is not built)", file=sys.stderr)
        return 2
    names = [args.config] if args.config else [c.strip() for c in args.configs.split(",") if c.strip()]
    for n in names:
        if n not in CONFIGS:
            ap.error(f"unknown config {n}")
    headline = HEADLINE if HEADLINE in names else names[0]

    import torch

    from deepgemm_amd import megamoe as mm

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    torch.cuda.set_device(0)
    # Cache flush between steps: READ 1 GiB (a reduction), which evicts L2/MALL without leaving
    # dirty lines whose write-back would be charged to the next layer.
    flush = torch.ones((1 << 28,), dtype=torch.float32, device="cuda")

    def flush_cache():
        flush.sum()

    log("weights: drawing and transforming on the GPU")
    l1, l2 = make_weights(torch, mm, seed=1234 + CONFIGS[headline]["id"])
    oracle = None
    if not args.no_cpu_baseline:
        torch.set_num_threads(os.cpu_count() or 1)
        oracle = CpuOracle(l1, l2, torch)
    per_config, cpu = {}, None
    for name in names:
        res, inputs, y = time_config(name, CONFIGS[name], l1, l2, args, torch, mm, flush_cache)
        if oracle is not None:
            reps = args.cpu_reps or CONFIGS[name]["cpu_reps"]
            log(f"  cpu baseline: the whole layer x{reps} on {torch.get_num_threads()} threads")
            full = cpu_full_layer(oracle, inputs, y, reps)
            base = dict(value=round(full["median_s"] * 1e6, 1), unit="us/layer",
                        cores=torch.get_num_threads(), kind="port",
                        sample=f"whole {name} layer ({full['rows']} routed rows), oracle "
                               f"dequantise-and-matmul pipeline (K2 form) from FP8 inputs and "
                               f"weights, median of {reps} reps {full['reps_s']} s",
                        os_cpu_count=os.cpu_count(), torch_threads=torch.get_num_threads(),
                        cpu_model=cpu_model(), parity_calc_diff=full["parity_calc_diff"])
            res["cpu_us"] = base["value"]
            res["cpu_sample"] = base["sample"]
            res["cpu_parity_calc_diff"] = full["parity_calc_diff"]
            if name == headline:
                cpu = base
            log(f"  cpu baseline: {base['value']} us/layer; parity calc_diff="
                f"{full['parity_calc_diff']:.2e}")
        if args.compare_hipblaslt:
            res["hipblaslt_gemm1"] = hipblaslt_gemm1(torch, res["routed_rows"], args.steps, flush_cache)
        per_config[name] = res
        del inputs, y
        torch.cuda.empty_cache()

    h = per_config[headline]
    out = {
        "metric": "us per MoE layer (FP8 W8A8 Mega MoE, one GPU's EP share)",
        "value": h["us_median"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["us_median"] / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate, bf16 out)",
        "data": "synthetic (seeded N(0,1) tokens/logits, N(0,1/sqrt(K)) weights)",
        "config": {"workload": h["workload"], "config_id": headline, "tokens": h["tokens"],
                   "experts": E_LOCAL, "hidden": HIDDEN, "intermediate": INTER, "topk": TOPK,
                   "routed_rows": h["routed_rows"], "touched_experts": h["touched_experts"],
                   "schedule": "auto (per-expert engine)"},
        "min_us": h["us_min"],
        "fp8_tflops": h["fp8_tflops"],
        "hbm_frac": h["hbm_frac"],
        "mfma_frac": h["mfma_frac"],
        "layer_bound": h["layer_bound"],
        "stage_us": h["stage_us"],
        "roofline": h["roofline"],
        "cpu_baseline": cpu,
        "per_config": per_config,
        "flush": "1 GiB read (reduction) before every step, outside the timed events",
    }
    if args.calibrate_mib > 0:
        out["calibration"] = calibrate(torch, args.calibrate_mib)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
