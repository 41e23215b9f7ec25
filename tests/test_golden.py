"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the oracle and its C restatement reproduce the frozen e4m3 table and the frozen small
layer. GPU: the HIP layer on the frozen inputs -- routing bit-exact, output within the bar.
"""
import os

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import megamoe_oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def test_e4m3_codes_round_trip():
    t = _load("e4m3_table.npz")
    codes, values = t["codes"], t["values"]
    finite = np.isfinite(values)
    got = O.e4m3_from_f32(torch.from_numpy(values[finite])).view(torch.uint8).numpy()
    assert np.array_equal(got, codes[finite])
    # the table's values decode back through torch's e4m3fn
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(dec), ~finite)
    assert np.array_equal(dec[finite], values[finite])


def test_e4m3_probes_match_table():
    t = _load("e4m3_table.npz")
    probes, expect = t["probes"], t["probe_codes"]
    got = O.e4m3_from_f32(torch.from_numpy(probes)).view(torch.uint8).numpy()
    assert np.array_equal(got, expect)
    lib = c_oracle()
    out = np.zeros_like(expect)
    lib.oracle_e4m3_from_f32_array(out.ctypes.data, probes.ctypes.data, probes.size)
    assert np.array_equal(out, expect)


def _layer_inputs(g):
    s, e, h, i, k = (int(v) for v in g["shape"])
    x_fp8 = torch.from_numpy(g["x_fp8"]).view(torch.float8_e4m3fn)
    x_sf = torch.from_numpy(g["x_sf"])
    idx = torch.from_numpy(g["topk_idx"])
    w = torch.from_numpy(g["topk_weights"])
    l1 = (torch.from_numpy(g["w1"]).view(torch.float8_e4m3fn), torch.from_numpy(g["sw1"]))
    l2 = (torch.from_numpy(g["w2"]).view(torch.float8_e4m3fn), torch.from_numpy(g["sw2"]))
    return (s, e, h, i, k), x_fp8, x_sf, idx, w, l1, l2


def test_oracle_reproduces_golden_layer():
    g = _load("layer_small.npz")
    _, x_fp8, x_sf, idx, w, l1, l2 = _layer_inputs(g)
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1, l2)
    rt = tr.routing
    assert np.array_equal(rt.counts, g["counts"])
    assert np.array_equal(rt.offsets, g["offsets"])
    assert np.array_equal(rt.output_index, g["output_index"])
    assert np.array_equal(rt.row_token, g["row_token"])
    # float parts: fp32 matmul order may differ between BLAS builds, so allow rare bf16 flips
    act = tr.act.view(torch.uint8).numpy()
    assert (act != g["act"]).mean() < 1e-3
    assert O.calc_diff(tr.y.float(), torch.from_numpy(g["y"])) < 1e-7
    # the routing rules the fixture exercises
    assert g["output_index"][0, 0] == -1 and g["output_index"][1, 1] == -1
    assert g["output_index"][2, 2] == -1 and g["output_index"][3, 0] == -1
    assert (g["output_index"][5] == -1).all() and not g["y"][5].any()


@pytest.mark.gpu
def test_hip_layer_on_golden_inputs(cuda):
    from deepgemm_amd import megamoe as mm

    g = _load("layer_small.npz")
    (s, e, h, i, k), x_fp8, x_sf, idx, w, l1, l2 = _layer_inputs(g)
    print(f"golden layer S={s} E={e} H={h} I={i} K={k}", flush=True)
    buf = mm.get_symm_buffer_for_mega_moe(None, e, s, k, h, i)
    buf.x[:s].copy_(x_fp8.to(cuda))
    buf.x_sf[:s].copy_(x_sf.to(cuda))
    buf.topk_idx[:s].copy_(idx.to(cuda))
    buf.topk_weights[:s].copy_(w.to(cuda))
    y = torch.empty((s, h), dtype=torch.bfloat16, device=cuda)
    mm.fp8_w8a8_mega_moe(y, (l1[0].to(cuda), l1[1].to(cuda)), (l2[0].to(cuda), l2[1].to(cuda)), buf)
    torch.cuda.synchronize()
    assert np.array_equal(buf.scratch_view("counts").cpu().numpy(), g["counts"])
    assert np.array_equal(buf.scratch_view("output_index").cpu().numpy()[:s], g["output_index"])
    r = int(g["offsets"][-1])
    assert np.array_equal(buf.scratch_view("row_token")[:r].cpu().numpy(), g["row_token"])
    d = O.calc_diff(y.float().cpu(), torch.from_numpy(g["y"]))
    print(f"  calc_diff={d:.3e}", flush=True)
    assert d <= 1e-3
    assert not y[5].any()
