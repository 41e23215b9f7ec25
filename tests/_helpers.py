"""Shared input builders for the GPU parity tests (seeded; CPU and GPU see the same bytes)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import megamoe_oracle as O


def zipf_routing(num_tokens: int, num_experts: int, topk: int, gen: torch.Generator,
                 s: float = 1.2, zero_experts: int = 4):
    """Config-4 routing: slots drawn i.i.d. with replacement from Zipf(s) over the experts,
    with `zero_experts` randomly chosen experts given zero mass (empty groups)."""
    perm = torch.randperm(num_experts, generator=gen)
    live = perm[zero_experts:]
    ranks = torch.arange(1, live.numel() + 1, dtype=torch.float64)
    p = ranks ** (-s)
    p = p / p.sum()
    draws = torch.multinomial(p.float(), num_tokens * topk, replacement=True, generator=gen)
    idx = live[draws].view(num_tokens, topk).to(torch.int64)
    w = torch.rand((num_tokens, topk), generator=gen) + 0.05
    w = w / w.sum(dim=-1, keepdim=True)
    return idx.contiguous(), w.float().contiguous()


def make_weights_gpu(num_experts: int, hidden: int, inter: int, seed: int, mm):
    """W1 ~ N(0, 1/sqrt(H)) [E, 2I, H], W2 ~ N(0, 1/sqrt(I)) [E, H, I] drawn on the GPU and
    transformed by the package (channelwise cast + Marlin)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w1 = (torch.randn((num_experts, 2 * inter, hidden), generator=g, device="cuda",
                      dtype=torch.float32) / math.sqrt(hidden)).to(torch.bfloat16)
    w2 = (torch.randn((num_experts, hidden, inter), generator=g, device="cuda",
                      dtype=torch.float32) / math.sqrt(inter)).to(torch.bfloat16)
    l1, l2 = mm.transform_fp8_weights_for_mega_moe(w1, w2)
    del w1, w2
    return l1, l2


def make_tokens(num_tokens: int, hidden: int, num_experts: int, topk: int, seed: int,
                global_experts=None, routing=None):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((num_tokens, hidden), generator=gen).to(torch.bfloat16)
    if routing == "zipf":
        idx, w = zipf_routing(num_tokens, num_experts, topk, gen)
    else:
        idx, w = O.make_routing(num_tokens, num_experts, topk, gen, global_experts)
    x_fp8, x_sf = O.cast_to_fp8_channelwise(x)
    return x_fp8, x_sf, idx, w


def run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2, num_tokens=None, clamp=None, stats=None,
              y=None, **kw):
    s = x_fp8.shape[0] if num_tokens is None else num_tokens
    buf.x[:x_fp8.shape[0]].copy_(x_fp8)
    buf.x_sf[:x_fp8.shape[0]].copy_(x_sf)
    buf.topk_idx[:x_fp8.shape[0]].copy_(idx)
    buf.topk_weights[:x_fp8.shape[0]].copy_(w)
    if y is None:
        y = torch.empty((s, buf.hidden), dtype=torch.bfloat16, device="cuda")
    mm.fp8_w8a8_mega_moe(y, l1, l2, buf, cumulative_local_expert_recv_stats=stats,
                         activation_clamp=clamp, **kw)
    return y


def cpu_weights(l1, l2):
    return (l1[0].cpu(), l1[1].cpu()), (l2[0].cpu(), l2[1].cpu())


def log(msg: str) -> None:
    print(msg, flush=True)
