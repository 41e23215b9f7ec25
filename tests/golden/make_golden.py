"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The reference holds no golden vectors, known-answer files or fixtures for this path (every
check in tests/test_mega_moe_dcu.py is computed at run time from random on-device inputs), and
it cannot run here (gfx938-only extension). These fixtures therefore come from this repo's
CPU oracle, after the oracle itself is pinned by tests/test_oracle.py (closed forms, brute
force, the independent C restatement). They freeze:

  e4m3_table.npz    the 256 OCP e4m3 codes and their values, computed here from the format's
                    definition (sign, 4-bit exponent with bias 7, 3-bit mantissa, subnormals,
                    0x7f/0xff NaN), plus f32 probes (grid points, midpoints, +-1 ulp, beyond
                    +-448) with their round-to-nearest-even code after clipping to +-448;
  layer_small.npz   one small layer (S=24, E=4, H=128, I=128, K=3) whose routing exercises
                    every rule of the reference's scan (deep_gemm/include/deep_gemm/impls/
                    mega_moe_dcu.cuh:352): ids -1 and >= E, zero weights and duplicate
                    experts within a token; inputs (FP8 bytes, scales, Marlin weights) and the
                    oracle's outputs (counts, offsets, output_index, row_token, requantised
                    act + act_scale, partial rows, y).

Inputs are plain arrays (np.load with allow_pickle=False); no file is executed when loaded.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import megamoe_oracle as O  # noqa: E402


def e4m3_value(code: int) -> float:
    """Value of an OCP e4m3 (fn) code from the format definition."""
    s = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return float("nan")
    if exp == 0:
        return s * (man / 8.0) * 2.0 ** -6
    return s * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


def e4m3_rne_code(v: float) -> int:
    """Round-to-nearest-even code of f32 v after clipping to +-448, by search over the grid."""
    v = float(np.float32(v))
    v = min(448.0, max(-448.0, v))
    best, best_err = None, None
    for code in range(256):
        q = e4m3_value(code)
        if q != q:
            continue
        if q == 0.0 and code == 0x80:
            continue  # -0 only for negative zero inputs, handled below
        err = abs(q - v)
        if best is None or err < best_err or (err == best_err and (code & 1) == 0 and (best & 1)):
            best, best_err = code, err
    if best == 0 and np.signbit(np.float32(v)):
        return 0x80
    return best


def make_e4m3_table(path: str) -> None:
    codes = np.arange(256, dtype=np.uint8)
    values = np.array([e4m3_value(int(c)) for c in codes], dtype=np.float32)
    finite = sorted(set(float(v) for v in values if np.isfinite(v) and v >= 0))
    probes = []
    for a, b in zip(finite[:-1], finite[1:]):
        mid = (a + b) / 2.0
        probes += [a, mid, float(np.nextafter(np.float32(mid), np.float32(-1))),
                   float(np.nextafter(np.float32(mid), np.float32(1)))]
    probes += [448.0, 464.0, 480.0, 1e6, 2.0 ** -10, 2.0 ** -9, 3 * 2.0 ** -11]
    probes = np.array(probes + [-p for p in probes], dtype=np.float32)
    expect = np.array([e4m3_rne_code(float(p)) for p in probes], dtype=np.uint8)
    np.savez_compressed(path, codes=codes, values=values, probes=probes, probe_codes=expect)


def make_layer_small(path: str) -> None:
    s, e, h, i, k = 24, 4, 128, 128, 3
    d = O.make_layer_inputs(s, e, h, i, k, seed=4242)
    idx = d["topk_idx"].clone()
    tw = d["topk_weights"].clone()
    # every routing rule: invalid ids, ids beyond the local experts, zero weights, duplicates
    idx[0, 0] = -1
    idx[1, 1] = e
    idx[2, 2] = e + 7
    tw[3, 0] = 0.0
    idx[4, 1] = idx[4, 0]
    idx[5, :] = -1
    tr = O.mega_moe_forward(d["x_fp8"], d["x_sf"], idx, tw, d["l1"], d["l2"])
    rt = tr.routing
    np.savez_compressed(
        path,
        shape=np.array([s, e, h, i, k], dtype=np.int64),
        x_fp8=d["x_fp8"].view(torch.uint8).numpy(),
        x_sf=d["x_sf"].numpy(),
        topk_idx=idx.numpy(),
        topk_weights=tw.numpy(),
        w1=d["l1"][0].view(torch.uint8).numpy(),
        sw1=d["l1"][1].numpy(),
        w2=d["l2"][0].view(torch.uint8).numpy(),
        sw2=d["l2"][1].numpy(),
        counts=np.asarray(rt.counts, dtype=np.int32),
        offsets=np.asarray(rt.offsets, dtype=np.int32),
        output_index=np.asarray(rt.output_index, dtype=np.int32),
        row_token=np.asarray(rt.row_token, dtype=np.int32),
        act=tr.act.view(torch.uint8).numpy(),
        act_scale=tr.act_scale.numpy(),
        part=tr.part.float().numpy(),
        y=tr.y.float().numpy(),
    )


def main() -> None:
    make_e4m3_table(os.path.join(HERE, "e4m3_table.npz"))
    make_layer_small(os.path.join(HERE, "layer_small.npz"))
    for f in ("e4m3_table.npz", "layer_small.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
