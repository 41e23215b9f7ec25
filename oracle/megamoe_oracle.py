"""CPU oracle for the FP8 W8A8 channelwise Mega MoE forward -- TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU with torch/numpy, the algorithm of the reference's
``megamoe.fp8_w8a8_mega_moe`` (yuguo-Jack/DeepGEMM, DCU half) in the form of its own
correctness baseline (``tests/test_mega_moe_dcu.py:188-323``):

    route (scatter) -> dequant GEMM1 -> K2 SwiGLU*weight + per-token e4m3 requant
    -> dequant GEMM2 -> slot-ordered top-k sum.

It is the checker of the HIP path, never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it. The
product (``deepgemm_amd``) never imports anything under ``oracle/`` and fails loudly when its
HIP library is missing.

Pinning (what checks each function, beyond retyping it) -- see tests/test_oracle.py:
  calc_diff                 closed forms (identical inputs -> 0, x vs -x -> 2, zero -> 0)
  e4m3 cast (torch)         exhaustive against the independent C restatement of the OCP
                            e4m3 RNE (oracle/megamoe_oracle.c) on every e4m3 grid point,
                            every midpoint and +-1 ulp around each
  cast_to_fp8_channelwise   known answers: amax 448 -> scale 1 and exact bytes; zero row
                            -> scale 1e-4/448 and zero bytes; grid values exact
  marlin pack/unpack        brute force of the byte-offset formula over every (e, r, k)
                            and round trip
  route                     brute force (python loops) on small cases, C restatement on
                            large ones, invariants (counts = histogram, rows contiguous
                            per expert, inverse index, every valid task exactly once)
  grouped_gemm_dequant      one-hot weights (GEMM = gather, exact), small-integer operands
                            (exact in fp32), float64 matmul on random inputs
  swiglu_quant_k2           hand-computed rows: w=0 row, gate=0 row, amax<1e-4 row,
                            clamp hit, and float64 recomputation of y, amax, scale
  combine                   float64 sum + bf16 RNE of exact-sum cases
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np
import torch

E4M3_MAX = 448.0
AMAX_FLOOR = 1.0e-4


# ----------------------------------------------------------------------------------------
# metric
# ----------------------------------------------------------------------------------------
def calc_diff(x: torch.Tensor, y: torch.Tensor) -> float:
    """1 - 2*sum(xy)/sum(x^2+y^2) in float64; deep_gemm/testing/numeric.py:5-11."""
    x = x.double()
    y = y.double()
    denominator = (x * x + y * y).sum()
    if float(denominator) == 0.0:
        return 0.0
    return float(1.0 - 2.0 * (x * y).sum() / denominator)


# ----------------------------------------------------------------------------------------
# quantisation helpers (megamoe/__init__.py:51-98)
# ----------------------------------------------------------------------------------------
def fdiv(num: float, den: torch.Tensor) -> torch.Tensor:
    """Correctly rounded fp32 num/den. (torch evaluates ``scalar / tensor`` as
    ``reciprocal(tensor) * scalar``, which is off by 1 ulp now and then; the reference's
    kernels divide in fp32, e.g. ``448.0f / clamped_amax`` in
    megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:352.)"""
    den = den.float()
    return torch.div(torch.full_like(den, float(num)), den)


def e4m3_from_f32(v: torch.Tensor) -> torch.Tensor:
    """Clip to +-448 then round-to-nearest-even into e4m3fn (the K2 conversion:
    megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:53-55, :121-142)."""
    return torch.clamp(v.float(), -E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)


def cast_to_fp8_channelwise(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row scale = max(amax,1e-4)/448; q = e4m3(x/scale). megamoe/__init__.py:51-56."""
    if x.dim() != 2:
        raise ValueError("channelwise FP8 cast expects a 2D tensor")
    scale = x.abs().float().amax(dim=1).clamp(min=AMAX_FLOOR) / E4M3_MAX
    fp8 = (x.float() / scale.view(-1, 1)).to(torch.float8_e4m3fn)
    return fp8.contiguous(), scale.float().contiguous()


def cast_grouped_weight_to_fp8_channelwise(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Channelwise cast of a grouped weight [G, R, K]. megamoe/__init__.py:59-78 (the
    reference chunks the rows only to bound memory; the result is row-independent)."""
    if w.dim() != 3:
        raise ValueError("MegaMoE grouped weights must be 3D tensors")
    g, r, k = w.shape
    fp8, scale = cast_to_fp8_channelwise(w.reshape(g * r, k))
    return fp8.reshape(g, r, k).contiguous(), scale.reshape(g, r).contiguous()


def marlin_pack(w: torch.Tensor) -> torch.Tensor:
    """[G,R,K] -> [G,R/16,K*16] Marlin nt_kpack2 permute. megamoe/__init__.py:81-98."""
    g, r, k = w.shape
    if r % 16 or k % 16:
        raise ValueError("DCU W8A8 MegaMoE Marlin weights require rows and K divisible by 16")
    return (w.reshape(g, r // 16, 16, k // 16, 16).permute(0, 1, 3, 2, 4).contiguous()
            .reshape(g, r // 16, k * 16))


def marlin_unpack(wm: torch.Tensor, rows: int, k: int) -> torch.Tensor:
    """Inverse of marlin_pack: [G,R/16,K*16] -> [G,R,K]."""
    g = wm.shape[0]
    return (wm.reshape(g, rows // 16, k // 16, 16, 16).permute(0, 1, 3, 2, 4).contiguous()
            .reshape(g, rows, k))


def marlin_offset(e: int, r: int, kk: int, rows: int, k: int) -> int:
    """Byte offset of element (e, r, kk) in the Marlin layout;
    deep_gemm/include/deep_gemm/layout/mega_moe_dcu.cuh:50-66."""
    return ((e * (rows // 16) + r // 16) * k + (kk // 16) * 16) * 16 + (r % 16) * 16 + kk % 16


def transform_fp8_weights_for_mega_moe(l1: torch.Tensor, l2: torch.Tensor):
    """megamoe/__init__.py:280-289."""
    l1_fp8, l1_s = cast_grouped_weight_to_fp8_channelwise(l1)
    l2_fp8, l2_s = cast_grouped_weight_to_fp8_channelwise(l2)
    return (marlin_pack(l1_fp8), l1_s), (marlin_pack(l2_fp8), l2_s)


# ----------------------------------------------------------------------------------------
# routing (a5-a7)
# ----------------------------------------------------------------------------------------
@dataclass
class Routing:
    counts: np.ndarray        # int32 [E]
    offsets: np.ndarray       # int32 [E+1]
    output_index: np.ndarray  # int32 [S, K]  row or -1
    row_token: np.ndarray     # int32 [R]
    row_slot: np.ndarray      # int32 [R]
    row_weight: np.ndarray    # float32 [R]
    m_indices: np.ndarray     # int32 [R]

    @property
    def num_rows(self) -> int:
        return int(self.offsets[-1])


def route(topk_idx, topk_weights, num_experts: int) -> Routing:
    """Deterministic routing.

    Validity: 0 <= e < E and w != 0 (deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:352).
    Rows are expert-contiguous with tight exclusive-scan offsets (the baseline scatter:
    csrc/kernels/mega_moe_baseline_hip.cu:37-96). Inside an expert the reference's order is
    atomic-arrival; the canonical order used here is ascending task index token*K+slot
    (what the reference yields when its atomics serialise)."""
    idx = np.asarray(topk_idx.cpu() if torch.is_tensor(topk_idx) else topk_idx).astype(np.int64)
    w = np.asarray(topk_weights.cpu() if torch.is_tensor(topk_weights) else topk_weights)
    w = w.astype(np.float32)
    s, k = idx.shape
    e_flat = idx.reshape(-1)
    w_flat = w.reshape(-1)
    valid = (e_flat >= 0) & (e_flat < num_experts) & (w_flat != 0.0)
    tasks = np.nonzero(valid)[0]
    experts = e_flat[tasks]
    counts = np.bincount(experts, minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    order = tasks[np.argsort(experts, kind="stable")]
    out_idx = np.full(s * k, -1, dtype=np.int32)
    out_idx[order] = np.arange(order.size, dtype=np.int32)
    return Routing(
        counts=counts,
        offsets=offsets,
        output_index=out_idx.reshape(s, k),
        row_token=(order // k).astype(np.int32),
        row_slot=(order % k).astype(np.int32),
        row_weight=w_flat[order].astype(np.float32),
        m_indices=e_flat[order].astype(np.int32),
    )


def route_bruteforce(topk_idx, topk_weights, num_experts: int) -> Routing:
    """Pure-python loop version of route() for small cases (independent restatement)."""
    idx = np.asarray(topk_idx).astype(np.int64)
    w = np.asarray(topk_weights).astype(np.float32)
    s, k = idx.shape
    buckets = [[] for _ in range(num_experts)]
    for t in range(s):
        for j in range(k):
            e = int(idx[t, j])
            if 0 <= e < num_experts and w[t, j] != 0.0:
                buckets[e].append((t, j))
    counts = np.array([len(b) for b in buckets], dtype=np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    out_idx = np.full((s, k), -1, dtype=np.int32)
    row_token, row_slot, row_weight, m_ind = [], [], [], []
    row = 0
    for e in range(num_experts):
        offsets[e] = row
        for (t, j) in buckets[e]:
            out_idx[t, j] = row
            row_token.append(t)
            row_slot.append(j)
            row_weight.append(w[t, j])
            m_ind.append(e)
            row += 1
    offsets[num_experts] = row
    return Routing(counts, offsets, out_idx, np.array(row_token, np.int32),
                   np.array(row_slot, np.int32), np.array(row_weight, np.float32),
                   np.array(m_ind, np.int32))


# ----------------------------------------------------------------------------------------
# GEMMs, SwiGLU requant, combine (a8-a11)
# ----------------------------------------------------------------------------------------
def grouped_gemm_dequant(a_fp8: torch.Tensor, a_scale: torch.Tensor, w_fp8: torch.Tensor,
                         w_scale: torch.Tensor, m_indices, offsets,
                         out_dtype=torch.bfloat16, acc_dtype=torch.float32) -> torch.Tensor:
    """out[r, n] = ((sum_k a[r,k] * w[e,n,k]) * a_scale[r]) * w_scale[e,n], e = m_indices[r],
    rows expert-contiguous per ``offsets``; w_fp8 is row-major [E, N, K] (un-Marlined).
    The reference's baseline runs deepgemm.m_grouped_fp8_gemm_nt_contiguous
    (tests/test_mega_moe_dcu.py:245-279); its accumulation order is not published (parity
    unpinned at the bit level), so this is the plain fp32 dequantise-and-matmul."""
    r_total = a_fp8.shape[0]
    n = w_fp8.shape[1]
    out = torch.zeros((r_total, n), dtype=out_dtype)
    offs = [int(v) for v in offsets]
    for e in range(len(offs) - 1):
        lo, hi = offs[e], offs[e + 1]
        if hi <= lo:
            continue
        a = a_fp8[lo:hi].to(acc_dtype)
        b = w_fp8[e].to(acc_dtype)
        acc = (a @ b.t()).float()
        acc = acc * a_scale[lo:hi].float().view(-1, 1)
        acc = acc * w_scale[e].float().view(1, -1)
        out[lo:hi] = acc.to(out_dtype)
    return out


def swiglu_k2(h: torch.Tensor, route_weight: torch.Tensor, clamp: Optional[float]) -> torch.Tensor:
    """The fp32 SwiGLU x route weight of K2 (megamoe/dcu_megamoe_large_opt/K2_fused/
    k2_fused_ext.cu:283-340): g = min(h_gate, c); u = clamp(h_up, -c, c);
    y = g*(1/(1+exp(-g)))*u*w, left to right."""
    inter = h.shape[1] // 2
    g = h[:, :inter].float()
    u = h[:, inter:].float()
    if clamp is not None and math.isfinite(clamp):
        c = float(clamp)
        u = torch.clamp(u, -c, c)
        g = torch.clamp(g, max=c)
    w = route_weight.float().view(-1, 1)
    return g * fdiv(1.0, 1.0 + torch.exp(-g)) * u * w


def swiglu_quant_k2(h: torch.Tensor, route_weight: torch.Tensor,
                    clamp: Optional[float]) -> Tuple[torch.Tensor, torch.Tensor]:
    """K2: megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:254-377.
    y = swiglu_k2(h, w, c); a = max(max|y|, 1e-4); q = e4m3(clip(y*(448/a))); scale = a/448.
    Rows with w == 0 -> q = 0 and scale = 1e-4/448."""
    rows, two_i = h.shape
    inter = two_i // 2
    y = swiglu_k2(h, route_weight, clamp)
    amax = y.abs().amax(dim=1) if inter > 0 else torch.zeros(rows)
    a = torch.clamp(amax, min=AMAX_FLOOR)
    inv = fdiv(E4M3_MAX, a).view(-1, 1)
    q = e4m3_from_f32(y * inv)
    scale = a / E4M3_MAX
    zero_rows = route_weight.float() == 0.0
    if bool(zero_rows.any()):
        q[zero_rows] = torch.zeros((int(zero_rows.sum()), inter), dtype=torch.float8_e4m3fn)
        scale = torch.where(zero_rows, torch.full_like(scale, AMAX_FLOOR / E4M3_MAX), scale)
    return q.contiguous(), scale.float().contiguous()


def combine(part: torch.Tensor, output_index, num_tokens: int) -> torch.Tensor:
    """y[t] = bf16(sum over valid slots s, in slot order, of f32(part[output_index[t,s]])).
    csrc/kernels/mega_moe_baseline_hip.cu:98-127 (apply_topk_weights=False) and the fused
    reduce deep_gemm/include/deep_gemm/impls/mega_moe_dcu.cuh:706-760."""
    oi = torch.as_tensor(np.asarray(output_index), dtype=torch.long)
    h = part.shape[1] if part.dim() == 2 else 0
    acc = torch.zeros((num_tokens, h), dtype=torch.float32)
    pf = part.float()
    for s in range(oi.shape[1]):
        col = oi[:num_tokens, s]
        ok = col >= 0
        if bool(ok.any()):
            contrib = torch.zeros((num_tokens, h), dtype=torch.float32)
            contrib[ok] = pf[col[ok]]
            acc = acc + contrib
    return acc.to(torch.bfloat16)


@dataclass
class ForwardTrace:
    routing: Routing
    h: torch.Tensor
    y_act: torch.Tensor
    act: torch.Tensor
    act_scale: torch.Tensor
    part: torch.Tensor
    y: torch.Tensor


def mega_moe_forward(x_fp8: torch.Tensor, x_sf: torch.Tensor, topk_idx, topk_weights,
                     l1_weights, l2_weights, num_tokens: Optional[int] = None,
                     activation_clamp: Optional[float] = None,
                     stats: Optional[torch.Tensor] = None,
                     unpacked_weights=None, keep_y_act: bool = True) -> ForwardTrace:
    """The whole layer on the CPU (fp32 dequant matmuls), K2-form numerics.

    ``l1_weights = (W1 Marlin [E,2I/16,H*16] e4m3, sw1 [E,2I] f32)``, ``l2_weights`` likewise
    with [E,H/16,I*16]; ``unpacked_weights`` may pass pre-unpacked row-major weights to skip
    the inverse permute. ``stats`` (int32 [E]) is accumulated in place like
    cumulative_local_expert_recv_stats (mega_moe_dcu.cuh:418-425). ``keep_y_act=False`` leaves
    the trace's SwiGLU output (y before the requant) out: the pipeline itself does not need it
    (the CPU baseline's timing)."""
    w1m, sw1 = l1_weights
    w2m, sw2 = l2_weights
    num_experts = w1m.shape[0]
    two_i = sw1.shape[1]
    hidden = sw2.shape[1]
    inter = two_i // 2
    s = x_fp8.shape[0] if num_tokens is None else int(num_tokens)
    idx = topk_idx[:s]
    tw = topk_weights[:s]
    rt = route(idx, tw, num_experts)
    if stats is not None:
        stats += torch.as_tensor(rt.counts, dtype=stats.dtype)
    if unpacked_weights is None:
        w1 = marlin_unpack(w1m.cpu(), two_i, hidden)
        w2 = marlin_unpack(w2m.cpu(), hidden, inter)
    else:
        w1, w2 = unpacked_weights
    tok = torch.as_tensor(rt.row_token, dtype=torch.long)
    a = x_fp8[:s].cpu()[tok]
    a_s = x_sf[:s].cpu()[tok]
    h = grouped_gemm_dequant(a, a_s, w1, sw1.cpu(), rt.m_indices, rt.offsets)
    rw = torch.as_tensor(rt.row_weight)
    act, act_s = swiglu_quant_k2(h, rw, activation_clamp)
    part = grouped_gemm_dequant(act, act_s, w2, sw2.cpu(), rt.m_indices, rt.offsets)
    y = combine(part, rt.output_index, s)
    y_act = swiglu_k2(h, rw, activation_clamp) if keep_y_act else None
    return ForwardTrace(rt, h, y_act, act, act_s, part, y)


# ----------------------------------------------------------------------------------------
# synthetic inputs (the configs of the benchmark, generated on the CPU, seeded)
# ----------------------------------------------------------------------------------------
def make_routing(num_tokens: int, num_experts_local: int, topk: int, gen: torch.Generator,
                 global_experts: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(N(0,1) logits) -> top-k -> renormalise; ids >= local experts -> -1."""
    ge = num_experts_local if global_experts is None else global_experts
    logits = torch.randn((num_tokens, ge), generator=gen, dtype=torch.float32)
    probs = torch.softmax(logits, dim=-1)
    w, idx = torch.topk(probs, topk, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    idx = torch.where(idx < num_experts_local, idx, torch.full_like(idx, -1))
    return idx.to(torch.int64).contiguous(), w.float().contiguous()


def make_layer_inputs(num_tokens: int, num_experts: int, hidden: int, inter: int, topk: int,
                      seed: int, global_experts: Optional[int] = None):
    """Seeded small-shape inputs: x ~ N(0,1), W1 ~ N(0,1/sqrt(H)), W2 ~ N(0,1/sqrt(I))."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((num_tokens, hidden), generator=gen).to(torch.bfloat16)
    w1 = (torch.randn((num_experts, 2 * inter, hidden), generator=gen) / math.sqrt(hidden))
    w2 = (torch.randn((num_experts, hidden, inter), generator=gen) / math.sqrt(inter))
    idx, tw = make_routing(num_tokens, num_experts, topk, gen, global_experts)
    x_fp8, x_sf = cast_to_fp8_channelwise(x)
    l1, l2 = transform_fp8_weights_for_mega_moe(w1.to(torch.bfloat16), w2.to(torch.bfloat16))
    return dict(x_fp8=x_fp8, x_sf=x_sf, topk_idx=idx, topk_weights=tw, l1=l1, l2=l2)
