"""GPU parity of the gfx950 HIP path against the CPU oracle (through the C ABI).

Bars: routing (counts, offsets, output_index, row tables, stats) bit-exact; conversions and
layout kernels bit-exact; layer output calc_diff <= 1e-3 (north star), checked per stage."""
import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import megamoe_oracle as O
from tests._helpers import (cpu_weights, log, make_tokens, make_weights_gpu, run_layer,
                            zipf_routing)

pytestmark = pytest.mark.gpu

CALC_DIFF_BAR = 1e-3  # north star: calc_diff(y, oracle) <= 1e-3


@pytest.fixture(scope="module")
def mm(cuda):
    from deepgemm_amd import megamoe
    return megamoe


# ------------------------------------------------------------------ conversions / layout
def test_e4m3_conversion_matches_c_oracle(mm, cuda):
    from tests.test_oracle import _probe_floats
    f = _probe_floats()
    out = torch.empty(f.size, dtype=torch.uint8, device=cuda)
    inp = torch.from_numpy(f).to(cuda)
    log(f"e4m3 conversion: {f.size} probes")
    mm._capi.check(mm._capi.load().mmoe_debug_f32_to_e4m3(out.data_ptr(), inp.data_ptr(), f.size,
                                                          mm._stream_handle()))
    ref = np.empty(f.size, dtype=np.uint8)
    c_oracle().oracle_e4m3_from_f32_array(ref.ctypes.data, f.ctypes.data, f.size)
    got = out.cpu().numpy()
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{f[bad[:8]]} gpu={got[bad[:8]]} ref={ref[bad[:8]]}"


@pytest.mark.parametrize("rows,cols", [(1, 16), (37, 4096), (300, 2048), (5, 130)])
def test_cast_fp8_channelwise_bitwise(mm, cuda, rows, cols):
    gen = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn((rows, cols), generator=gen) * 3).to(torch.bfloat16)
    x[0, :] = 0.0  # an all-zero row: scale 1e-4/448
    log(f"cast rows={rows} cols={cols}")
    q, s = mm.cast_to_fp8_channelwise(x.to(cuda))
    qr, sr = O.cast_to_fp8_channelwise(x)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))


def test_marlin_pack_bitwise(mm, cuda):
    w = torch.randint(0, 256, (3, 64, 256), dtype=torch.uint8).view(torch.float8_e4m3fn)
    log("marlin pack")
    got = mm.weight8bit_nt_kpack2_marlin(w.to(cuda)).cpu()
    assert torch.equal(got.view(torch.uint8), O.marlin_pack(w).view(torch.uint8))


# ------------------------------------------------------------------ routing
ROUTE_CASES = {
    # name: (S, E, K, global experts or "zipf"/"invalid")
    "tiny": (5, 4, 3, None),
    "c0": (64, 32, 6, None),
    "c1": (1024, 32, 6, 256),
    "ragged": (777, 32, 6, 256),
    "zipf": (3000, 32, 6, "zipf"),
    "wide": (2500, 40, 8, 64),
    "chunked": (20000, 32, 6, 256),  # 120,000 tasks: count + scatter kernels over 117 chunks
    # just past the one-workgroup kernel (16,384 tasks): 17 chunks, the last of 2 tasks; 32 full
    # chunks over 256 experts
    "chunks_ragged": (2731, 32, 6, 256),
    "chunks_e256": (4096, 256, 8, None),
}


def _route_inputs(name):
    s, e, k, g = ROUTE_CASES[name]
    gen = torch.Generator().manual_seed(100 + s)
    if g == "zipf":
        idx, w = zipf_routing(s, e, k, gen)
    else:
        idx, w = O.make_routing(s, e, k, gen, g)
    # sprinkle invalid cases: zero weights, ids out of range on both sides
    if s > 4:
        w[1, 0] = 0.0
        idx[2, 1] = e
        idx[3, 0] = -7
    return idx, w, e, k


@pytest.mark.parametrize("name", list(ROUTE_CASES))
def test_routing_bit_exact(mm, cuda, name):
    idx, w, e, k = _route_inputs(name)
    s = idx.shape[0]
    hidden, inter = 256, 128
    log(f"routing case={name} S={s} E={e} K={k}")
    buf = mm.SymmBuffer(None, e, s, k, hidden, inter)
    buf.topk_idx[:s].copy_(idx)
    buf.topk_weights[:s].copy_(w)
    l1 = (torch.zeros((e, 2 * inter // 16, hidden * 16), dtype=torch.float8_e4m3fn, device=cuda),
          torch.ones((e, 2 * inter), device=cuda))
    l2 = (torch.zeros((e, hidden // 16, inter * 16), dtype=torch.float8_e4m3fn, device=cuda),
          torch.ones((e, hidden), device=cuda))
    stats0 = torch.randint(0, 100, (e,), dtype=torch.int32)
    stats = stats0.to(cuda)
    mm.route_only(s, l1, l2, buf, stats)
    torch.cuda.synchronize()
    ref = O.route(idx, w, e)
    r = ref.num_rows
    assert np.array_equal(buf.scratch_view("counts").cpu().numpy(), ref.counts)
    assert np.array_equal(buf.scratch_view("offsets").cpu().numpy(), ref.offsets)
    assert buf.scratch_view("meta")[0].item() == r
    assert np.array_equal(buf.scratch_view("output_index")[:s].cpu().numpy(), ref.output_index)
    assert np.array_equal(buf.scratch_view("row_token")[:r].cpu().numpy(), ref.row_token)
    assert np.array_equal(buf.scratch_view("m_indices")[:r].cpu().numpy(), ref.m_indices)
    assert np.array_equal(buf.scratch_view("row_weight")[:r].cpu().numpy(), ref.row_weight)
    assert torch.equal(stats.cpu(), stats0 + torch.from_numpy(ref.counts))


# ------------------------------------------------------------------ the layer
def _stage_checks(buf, tr, s, clamp=None):
    r = tr.routing.num_rows
    assert buf.scratch_view("meta")[3].item() == 0, "decode pipeline: a bounded wait ran out"
    # GEMM1's SwiGLU x weight output, rounded to bf16 by every GEMM1 kernel (as the reference's
    # fused path rounds its activation)
    y_act = buf.scratch_view("y")[:r].cpu().float()
    assert O.calc_diff(y_act, tr.y_act) < 1e-5, "GEMM1 + SwiGLU x weight output"
    amax = buf.scratch_view("amax")[:r].cpu()
    assert torch.equal(amax, y_act.abs().amax(dim=1)), "row max |y|"
    act_s = buf.scratch_view("act_scale")[:r].cpu()
    assert torch.equal(act_s, torch.clamp(amax, min=1e-4) / 448.0), "act_scale from amax"
    # requant is exact given y: e4m3(clip(y * 448/a))
    inv = O.fdiv(448.0, torch.clamp(amax, min=1e-4)).view(-1, 1)
    requant = O.e4m3_from_f32(y_act * inv).view(torch.uint8)
    got = buf.scratch_view("act")[:r].cpu().view(torch.uint8)
    bad = (got != requant).nonzero()
    if bad.numel():
        detail = [(int(i), int(j), float(y_act[i, j]), float((y_act * inv)[i, j]), int(got[i, j]),
                   int(requant[i, j])) for i, j in bad[:8].tolist()]
        pytest.fail(f"per-row requant: {bad.shape[0]} mismatches in rows "
                    f"{sorted(set(bad[:, 0].tolist()))[:16]}; (row, col, y, y*inv, gpu, ref): "
                    f"{detail}")
    assert torch.allclose(act_s, tr.act_scale, rtol=2e-2, atol=0)
    act = buf.scratch_view("act")[:r].cpu()
    deq = act.float() * act_s.view(-1, 1)
    deq_ref = tr.act.float() * tr.act_scale.view(-1, 1)
    # The oracle quantizes f32 y. bf16 y (the reference fused path's rounding) moves a code by
    # one e4m3 step wherever its rounding crosses a code boundary: about one element in 60 (bf16
    # keeps 5 more mantissa bits than e4m3), at ~6% each: measured 6-8e-5.
    d_act = O.calc_diff(deq, deq_ref)
    log(f"  requant: calc_diff(act) = {d_act:.2e}")
    assert d_act < 5e-4, "SwiGLU requant"
    part = buf.scratch_view("part")[:r].cpu()
    if buf.scratch_view("meta")[2].item() == 1:
        # GEMM2 wrote the rows of single-slot tokens straight to y: row_dest names exactly those
        # rows (their token), and part holds the others
        row_dest = buf.scratch_view("row_dest")[:r].cpu().numpy()
        tok = np.asarray(tr.routing.row_token)[:r]
        slots = (np.asarray(tr.routing.output_index) >= 0).sum(axis=1)
        assert np.array_equal(row_dest, np.where(slots[tok] == 1, tok, -1)), "row_dest"
        keep = torch.from_numpy(row_dest < 0)
        assert O.calc_diff(part[keep], tr.part[keep]) < 1e-3, "GEMM2 partials"
    else:
        assert O.calc_diff(part, tr.part) < 1e-3, "GEMM2 partials"


def _combine_bitwise(mm, buf, y, l1, l2, s, clamp):
    """y is bitwise the slot-ordered fp32 sum (bf16 RNE) of GEMM2's own rows. When GEMM2 wrote
    single-slot tokens straight to y (meta[2] == 1), GEMM2 runs again with that switched off
    (meta[2] = 0, its only input besides the row table) so that every row is in part: this
    pins the direct rows (a one-term sum, -0 stored as +0) and the combine alike."""
    meta = buf.scratch_view("meta")
    if meta[2].item() == 1:
        meta[2] = 0
        mm.LayerCall(torch.empty_like(y), l1, l2, buf, activation_clamp=clamp).run(3, 3)
        torch.cuda.synchronize()
    r = int(meta[0].item())
    part = buf.scratch_view("part")[:r].cpu()
    oi = buf.scratch_view("output_index")[:s].cpu().numpy()
    expect = O.combine(part, oi, s)
    got = y.cpu()
    bad = (got.view(torch.int16) != expect.view(torch.int16)).nonzero()
    assert bad.numel() == 0, f"combine not bitwise at {bad[:8].tolist()}"


@pytest.mark.parametrize("cfg", [
    # (S, E, H, I, K, global experts, clamp)
    (16, 4, 256, 128, 3, None, None),
    (33, 8, 512, 256, 6, 16, None),
    (64, 8, 512, 384, 4, None, 10.0),
    # many rows per expert: the 4-wave tile kernel (GEMM2 with a partial column block; GEMM1
    # on the 8-wave kernel because k % 256 != 0), then both GEMMs on it with ragged row blocks
    (2048, 4, 640, 256, 6, 16, None),
    (1500, 5, 768, 256, 6, 8, None),
    # >= 16 tokens a CU: the whole-row combine; most tokens have one routed slot (direct rows)
    (4500, 4, 256, 256, 2, 16, None),
    # ~100 rows an expert: one 128-row STREAM item (4 row tiles) a column block, with K not a
    # multiple of the 512-byte chunk in both GEMMs (128-k chunks, one-step ring)
    (100, 4, 640, 384, 4, None, None),
    # GEMM1's in-kernel routing over more than one 64-expert scan chunk (S*K <= 8192), up to
    # its largest expert count (255: expert ids in a byte)
    (512, 160, 256, 128, 8, None, None),
    (300, 255, 256, 128, 6, None, None),
])
def test_layer_small_shapes(mm, cuda, cfg):
    s, e, hdim, inter, k, g, clamp = cfg
    log(f"layer small cfg={cfg}")
    x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=s + e, global_experts=g)
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=s * 3 + e, mm=mm)
    buf = mm.SymmBuffer(None, e, s, k, hdim, inter)
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2, clamp=clamp)
    torch.cuda.synchronize()
    l1c, l2c = cpu_weights(l1, l2)
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c, activation_clamp=clamp)
    # the shapes with many rows per expert run GEMM1 on the 4-wave kernel
    assert (buf.scratch_view("meta")[1].item() == 1) == (s * k > 8192 and s * k >= 256 * e and hdim % 256 == 0)
    # GEMM2 (k = I) on the 4-wave kernel writes single-slot tokens straight to y
    assert (buf.scratch_view("meta")[2].item() == 1) == (s * k > 8192 and s * k >= 256 * e and inter % 256 == 0)
    _stage_checks(buf, tr, s, clamp)
    _combine_bitwise(mm, buf, y, l1, l2, s, clamp)
    d = O.calc_diff(y.cpu(), tr.y)
    log(f"  calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR


# other models' expert shapes, one GPU's EP share of 32 experts: (S, H, I, top-k, global
# experts or None for all local). H = 7168 keeps GEMM1's K off the decode pipeline's 2048-byte
# chunks (the 8-wave kernels with in-kernel routing run at decode); I = 1536 keeps GEMM2's K off
# it; the prefill sizes run the WIDE kernels.
OTHER_MODEL_CASES = {
    "h7168_top8_decode": (512, 7168, 2048, 8, 256),
    "h7168_top8_prefill": (1536, 7168, 2048, 8, None),
    "i1536_top8_decode": (1024, 4096, 1536, 8, 128),
    "i1536_top8_prefill": (1536, 4096, 1536, 8, None),
}


@pytest.mark.parametrize("case", list(OTHER_MODEL_CASES))
def test_layer_other_model_shapes(mm, cuda, case):
    """The layer at other MoE models' expert shapes (a DeepSeek-like hidden size of 7168 with
    top-8, a Qwen-like expert width of 1536 with top-8): every stage against the oracle, the
    combine bitwise, and the output within the bar, at a decode and a prefill size."""
    s, hdim, inter, k, g = OTHER_MODEL_CASES[case]
    e = 32
    log(f"layer other-model case={case}")
    x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=4242 + s + hdim, global_experts=g)
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=777 + inter, mm=mm)
    buf = mm.get_symm_buffer_for_mega_moe(None, e, s, k, hdim, inter)
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    l1c, l2c = cpu_weights(l1, l2)
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c)
    wide = s * k > 8192 and s * k >= 256 * e
    assert (buf.scratch_view("meta")[1].item() == 1) == wide
    _stage_checks(buf, tr, s, None)
    _combine_bitwise(mm, buf, y, l1, l2, s, None)
    d = O.calc_diff(y.cpu(), tr.y)
    log(f"  R={tr.routing.num_rows} calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR
    del l1, l2, l1c, l2c


@pytest.fixture(scope="module")
def full_weights(mm):
    """Full-shape weights (32 experts, H=4096, I=2048), drawn on the GPU, plus CPU copies."""
    log("full weights: drawing on GPU")
    l1, l2 = make_weights_gpu(32, 4096, 2048, seed=1234, mm=mm)
    torch.cuda.synchronize()
    l1c, l2c = cpu_weights(l1, l2)
    unpacked = (O.marlin_unpack(l1c[0], 4096, 4096), O.marlin_unpack(l2c[0], 4096, 2048))
    return l1, l2, l1c, l2c, unpacked


# case: (S, global experts or "zipf", activation_clamp, GEMM1 kernel: "8wave" or "wide")
FULL_SHAPE_CASES = {
    "c0": (64, None, None, "8wave"),
    "c1_128": (1024, 256, None, "8wave"),
    "ragged_77": (77, 64, None, "8wave"),
    "clamp10": (96, None, 10.0, "8wave"),
    "wide_2048": (2048, None, None, "wide"),
    # eager calls whose task bound selects WIDE by a small margin: the routing's largest expert
    # row count chooses on the device, the 8-wave kernels up to 128 rows (an EP share of 2048
    # tokens: 1555 rows, at most 63 an expert, one STREAM chunk each; of 2304: 1697 rows, 68 in
    # the largest, two chunks for it; of 4096: 3046 rows, 65..117 rows in every expert), WIDE
    # above (of 5120: 3858 rows, 144 in the largest)
    "ep_2048": (2048, 256, None, "8wave"),
    "ep_2304": (2304, 256, None, "8wave"),
    "ep_4096": (4096, 256, None, "8wave"),
    "ep_5120": (5120, 256, None, "wide"),
    # clamp 1.0 binds on both sides of the gate and of the up value (h ~ N(0, 1)): the 8-wave
    # epilogue on the STREAM engine (c1 routing), on the TILE engine (Zipf: experts with more
    # than 128 rows), and the WIDE kernel's requant from h
    "clamp1_stream": (1024, 256, 1.0, "8wave"),
    "clamp1_tile": (600, "zipf", 1.0, "8wave"),
    "clamp1_wide": (2048, None, 1.0, "wide"),
}


def _assert_clamp_binds(h: torch.Tensor, clamp: float, min_frac: float = 0.05):
    """At least min_frac of the gate values lie above +c and below -c, and so do the up values:
    the clamp changes values on every side it applies to, and gate values below -c (which the
    one-sided K2 gate clamp leaves alone) are common."""
    inter = h.shape[1] // 2
    g, u = h[:, :inter].float(), h[:, inter:].float()
    fracs = {"gate>c": (g > clamp).float().mean().item(), "gate<-c": (g < -clamp).float().mean().item(),
             "up>c": (u > clamp).float().mean().item(), "up<-c": (u < -clamp).float().mean().item()}
    log(f"  clamp {clamp}: fractions beyond it {fracs}")
    for k, v in fracs.items():
        assert v >= min_frac, f"clamp does not bind: {k} on {v:.3f} of the values"


def _assert_every_engine(counts):
    """The auto schedule's three per-expert cases occur: STREAM in one 64-row chunk (1..64
    rows), STREAM in two chunks (65..128) and TILE (more than 128)."""
    assert ((counts > 0) & (counts <= 64)).any()
    assert ((counts > 64) & (counts <= 128)).any()
    assert (counts > 128).any()


@pytest.mark.parametrize("case", list(FULL_SHAPE_CASES))
def test_layer_full_shape(mm, cuda, full_weights, case):
    l1, l2, l1c, l2c, unpacked = full_weights
    s, g, clamp, kernel = FULL_SHAPE_CASES[case]
    log(f"layer full-shape case={case} S={s}")
    if g == "zipf":
        x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=1234 + s, routing="zipf")
    else:
        x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=1234 + s, global_experts=g)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048)
    stats = torch.zeros(32, dtype=torch.int32, device=cuda)
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2, clamp=clamp, stats=stats)
    torch.cuda.synchronize()
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c, activation_clamp=clamp,
                            unpacked_weights=unpacked)
    assert np.array_equal(stats.cpu().numpy(), tr.routing.counts)
    assert (buf.scratch_view("meta")[1].item() == 1) == (kernel == "wide")
    assert (buf.scratch_view("meta")[2].item() == 1) == (kernel == "wide")
    if case.startswith("ep_"):  # the routing launch's largest expert row count
        assert buf.scratch_view("meta")[4].item() == int(tr.routing.counts.max())
    if clamp is not None and clamp < 5.0:
        _assert_clamp_binds(tr.h, clamp)
    if g == "zipf":  # the TILE engine (more than 128 rows) next to one- and two-chunk STREAM experts
        _assert_every_engine(tr.routing.counts)
    _stage_checks(buf, tr, s, clamp)
    _combine_bitwise(mm, buf, y, l1, l2, s, clamp)
    d = O.calc_diff(y.cpu(), tr.y)
    log(f"  calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR


@pytest.mark.parametrize("mode", ["auto", "1", "0"])
def test_layer_every_schedule_matches_oracle_and_is_deterministic(mm, cuda, full_weights,
                                                                  monkeypatch, mode):
    """MEGAMOE_DCU_USE_LARGE_OPT_3STAGE = auto (per-expert engine), 1 (tile engine everywhere),
    0 (streaming engine everywhere): every schedule meets the bar on a mixed load (experts
    with few and with many rows) and repeated calls are bitwise identical."""
    l1, l2, l1c, l2c, unpacked = full_weights
    s = 600
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=99, routing="zipf")
    monkeypatch.setenv("MEGAMOE_DCU_USE_LARGE_OPT_3STAGE", mode)
    buf = mm.SymmBuffer(None, 32, 768, 6, 4096, 2048)
    log(f"schedule mode={mode}")
    y1 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2).clone()
    y2 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c, unpacked_weights=unpacked)
    _assert_every_engine(tr.routing.counts)
    d = O.calc_diff(y1.cpu(), tr.y)
    log(f"  calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR


@pytest.mark.parametrize("mode,wide", [("auto", False), ("1", True), ("0", False)])
def test_eager_dual_applies_to_the_auto_schedule_only(mm, cuda, full_weights, monkeypatch, mode, wide):
    """An EP share of 2048 tokens (1555 routed rows, at most 63 an expert; the task bound selects
    WIDE): the auto schedule's dual launch lets the routing choose the 8-wave kernels (every
    expert within the streaming engine's 128 rows), while a caller-set engine keeps the host's
    choice -- WIDE for the tile engine (=1), the streaming engine for =0 (which never selects
    WIDE). Each meets the bar against the oracle."""
    l1, l2, l1c, l2c, unpacked = full_weights
    s = 2048
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=1234 + s, global_experts=256)
    monkeypatch.setenv("MEGAMOE_DCU_USE_LARGE_OPT_3STAGE", mode)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048)
    log(f"eager dual: schedule mode={mode}")
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    meta = buf.scratch_view("meta")
    assert (meta[1].item() == 1) == wide, "WIDE GEMM1 exactly when expected"
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c, unpacked_weights=unpacked)
    assert int(tr.routing.counts.max()) <= 128
    d = O.calc_diff(y.cpu(), tr.y)
    log(f"  calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR


@pytest.mark.parametrize("s", [512, 2048])
def test_layer_zipf_empty_experts(mm, cuda, full_weights, s):
    l1, l2, l1c, l2c, unpacked = full_weights
    log(f"layer zipf skew with empty experts S={s}")
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=4, routing="zipf")
    buf = mm.SymmBuffer(None, 32, s, 6, 4096, 2048)
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c, unpacked_weights=unpacked)
    assert (tr.routing.counts == 0).sum() >= 4
    d = O.calc_diff(y.cpu(), tr.y)
    log(f"  calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR


def _prefill_tokens_gpu(mm, s, global_experts, seed):
    """Tokens of the prefill configs drawn on the GPU: x ~ N(0,1) cast per token to e4m3;
    logits N(0,1) [S, global experts] -> softmax -> top-6 -> renormalised, ids outside the 32
    local experts -> -1."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((s, 4096), generator=g, device="cuda").to(torch.bfloat16)
    x_fp8, x_sf = mm.cast_to_fp8_channelwise(x)
    del x
    logits = torch.randn((s, global_experts), generator=g, device="cuda")
    w, idx = torch.topk(torch.softmax(logits, -1), 6, dim=-1)
    w = (w / w.sum(-1, keepdim=True)).float().contiguous()
    idx = torch.where(idx < 32, idx, torch.full_like(idx, -1)).to(torch.int64).contiguous()
    return x_fp8, x_sf, idx, w


def _zipf_tokens_gpu(mm, s, seed):
    """Tokens of the skew config c4 drawn on the GPU: x as above; the 6 slots of a token drawn
    i.i.d. (with replacement, so a token can hold one expert twice) from Zipf(1.2) over 28 of
    the 32 experts, 4 chosen experts left empty; route weights uniform in [0.05, 1.05),
    normalised."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((s, 4096), generator=g, device="cuda").to(torch.bfloat16)
    x_fp8, x_sf = mm.cast_to_fp8_channelwise(x)
    del x
    live = torch.randperm(32, generator=g, device="cuda")[4:]
    p = torch.arange(1, live.numel() + 1, device="cuda", dtype=torch.float64) ** (-1.2)
    draws = torch.multinomial((p / p.sum()).float(), s * 6, replacement=True, generator=g)
    idx = live[draws].view(s, 6).to(torch.int64).contiguous()
    w = torch.rand((s, 6), generator=g, device="cuda") + 0.05
    w = (w / w.sum(-1, keepdim=True)).float().contiguous()
    return x_fp8, x_sf, idx, w


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_layer_prefill_full_scale_sampled(mm, cuda, full_weights, cfg):
    """The prefill configs at full scale through the WIDE kernels:
    - c2: T = 4096 a rank (32,768 source tokens, same routing as c3; ~24.7K routed rows, the
      decode/prefill crossover);
    - c3: T = 32768 a rank (262,144 source tokens, top-6 of 256 global experts, experts 0..31
      local; ~196K routed rows);
    - c4: 8192 tokens, Zipf-skewed slots over 28 local experts (49,152 rows, the hottest
      expert ~15K of them, so its tiles span several XCDs' item ranges; 4 empty experts;
      repeated (token, expert) slots).
    The oracle's whole layer (1.2-10 TFLOP on the host) is out of reach, so the checks are the
    size-independent ones:
    - routing bit-exact over all tasks;
    - h, the requant and GEMM2 on a sample of rows (every expert's first and last row, the
      rows around 256-row tile boundaries, random rows) against the oracle's dequantised
      matmuls of those rows;
    - the combine bitwise on sampled tokens with several slots, zero rows for tokens without
      one, and the direct rows of single-slot tokens equal to their GEMM2 row;
    - a second call bitwise identical."""
    l1, l2, l1c, l2c, unpacked = full_weights
    w1u, w2u = unpacked
    if cfg in ("c2", "c3"):
        s = 8 * (4096 if cfg == "c2" else 32768)
        x_fp8, x_sf, idx, w = _prefill_tokens_gpu(mm, s, 256, seed=1236 if cfg == "c2" else 1237)
    else:
        s = 8192
        x_fp8, x_sf, idx, w = _zipf_tokens_gpu(mm, s, seed=1238)
    log(f"prefill full scale {cfg} S={s}")
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048)
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    meta = buf.scratch_view("meta").cpu()
    assert meta[1].item() == 1 and meta[2].item() == 1, "the WIDE kernels (direct rows)"

    # routing, all tasks
    ref = O.route(idx.cpu(), w.cpu(), 32)
    r = ref.num_rows
    log(f"  routed rows {r}")
    assert meta[0].item() == r
    assert np.array_equal(buf.scratch_view("counts").cpu().numpy(), ref.counts)
    assert np.array_equal(buf.scratch_view("offsets").cpu().numpy(), ref.offsets)
    assert np.array_equal(buf.scratch_view("output_index")[:s].cpu().numpy(), ref.output_index)
    assert np.array_equal(buf.scratch_view("row_token")[:r].cpu().numpy(), ref.row_token)
    assert np.array_equal(buf.scratch_view("row_weight")[:r].cpu().numpy(), ref.row_weight)
    if cfg == "c4":  # the skew the config is for
        tiles = (ref.counts + 255) // 256 * 16  # 256 x 256 tiles an expert
        assert (ref.counts == 0).sum() == 4
        assert tiles.max() > 2 * tiles.sum() / 8, "hottest expert over 2+ XCD item ranges"
        srt = np.sort(idx.cpu().numpy(), axis=1)
        assert (srt[:, 1:] == srt[:, :-1]).any(), "repeated (token, expert) slots"

    # sampled rows
    gen = np.random.default_rng(5)
    picks = set()
    for e in range(32):
        lo, hi = int(ref.offsets[e]), int(ref.offsets[e + 1])
        if hi <= lo:
            continue
        picks.update({lo, hi - 1})
        for b in range(lo + 255, hi, 256 * 7):  # tile boundaries (255 | 256) of some blocks
            picks.update({b, min(b + 1, hi - 1)})
    picks.update(int(v) for v in gen.integers(0, r, 32))
    rows = torch.tensor(sorted(picks), dtype=torch.long)
    tok = torch.from_numpy(ref.row_token)[rows].long()
    exp = torch.from_numpy(ref.m_indices)[rows].long()
    xr = x_fp8.view(torch.uint8)[tok.to(cuda)].cpu().view(torch.float8_e4m3fn)
    xsr = x_sf[tok.to(cuda)].cpu()
    y16 = buf.scratch_view("y", r)[rows.to(cuda)].cpu()
    act = buf.scratch_view("act", r).view(torch.uint8)[rows.to(cuda)].cpu().view(torch.float8_e4m3fn)
    act_s = buf.scratch_view("act_scale", r)[rows.to(cuda)].cpu()
    h_ref = torch.empty((rows.numel(), 2 * 2048), dtype=torch.bfloat16)
    part_ref = torch.empty((rows.numel(), 4096), dtype=torch.bfloat16)
    for e in exp.unique().tolist():
        sel = (exp == e).nonzero().view(-1)
        acc = xr[sel].float() @ w1u[e].float().t()
        h_ref[sel] = ((acc * xsr[sel].view(-1, 1)) * l1c[1][e].view(1, -1)).to(torch.bfloat16)
        acc2 = act[sel].float() @ w2u[e].float().t()  # GEMM2 of the GPU's own act rows
        part_ref[sel] = ((acc2 * act_s[sel].view(-1, 1)) * l2c[1][e].view(1, -1)).to(torch.bfloat16)
    # GEMM1 + SwiGLU x weight (bf16 y) against the oracle formula on the
    # same rows: h = bf16(acc * x_scale * w_scale), y = SwiGLU(h) x route weight
    y_ref = O.swiglu_k2(h_ref, torch.from_numpy(ref.row_weight)[rows], None)
    d_y = O.calc_diff(y16.float(), y_ref)
    log(f"  {rows.numel()} sampled rows: calc_diff(y) = {d_y:.2e}")
    assert d_y < 1e-5, "GEMM1 + SwiGLU x weight (sampled rows)"
    # requant of the GPU's y rows: scales and codes exact
    y_act = y16.float()
    amax = y_act.abs().amax(dim=1)
    assert torch.equal(buf.scratch_view("amax", r)[rows.to(cuda)].cpu(), amax)
    assert torch.equal(act_s, torch.clamp(amax, min=1e-4) / 448.0)
    inv = O.fdiv(448.0, torch.clamp(amax, min=1e-4)).view(-1, 1)
    codes = O.e4m3_from_f32(y_act * inv).view(torch.uint8)
    assert torch.equal(act.view(torch.uint8), codes), "requant codes"
    # GEMM2 rows: part, or y for a row whose token has a single routed slot
    row_dest = buf.scratch_view("row_dest", r)[rows.to(cuda)].cpu()
    part = buf.scratch_view("part", r)[rows.to(cuda)].cpu()
    direct = row_dest >= 0
    if bool(direct.any()):
        part[direct] = y[row_dest[direct].long().to(cuda)].cpu()
    d_p = O.calc_diff(part.float(), part_ref.float())
    log(f"  calc_diff(GEMM2 rows) = {d_p:.2e} ({int(direct.sum())} of them direct y rows)")
    assert d_p < 1e-4, "GEMM2 rows (sampled)"

    # combine on sampled tokens
    slots = (ref.output_index >= 0).sum(axis=1)
    tsel = []
    for want in (0, 2, 3):
        cand = np.nonzero(slots == want if want < 3 else slots >= want)[0]
        tsel.extend(int(v) for v in cand[:: max(1, cand.size // 24)][:24])
    tsel = torch.tensor(sorted(set(tsel)), dtype=torch.long)
    oi = torch.from_numpy(ref.output_index)[tsel]
    part_all = buf.scratch_view("part", r)
    got = y[tsel.to(cuda)].cpu()
    expect = torch.zeros((tsel.numel(), 4096), dtype=torch.float32)
    for k in range(6):
        col = oi[:, k]
        ok = col >= 0
        if bool(ok.any()):
            expect[ok] += part_all[col[ok].long().to(cuda)].cpu().float()
    expect = expect.to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), expect.view(torch.int16)), "combine (sampled tokens)"

    y1 = y.clone()
    run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2, y=y)
    torch.cuda.synchronize()
    assert torch.equal(y1, y), "two calls bitwise identical"


def test_wide_claim_counters_return_to_zero(mm, cuda):
    """The WIDE GEMMs claim items from per-XCD counters in route_scratch when a workgroup has few
    items; the last workgroup of each GEMM resets them, so after a call (and after a GEMM2 run on
    its own) they read zero again, and a second call on the same scratch is bitwise identical.
    The zero-fill counters (sched[0, 9:12]: chunks of 64 tokens whose zero rows idle WIDE
    workgroups wrote, and each GEMM's workgroups out of tiles) are the exception: the combine reads
    them, and the next call's routing launch zeroes them."""
    s, e, hdim, inter, k = 2048, 4, 512, 256, 6
    x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=31, global_experts=8)
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=32, mm=mm)
    buf = mm.SymmBuffer(None, e, s, k, hdim, inter)
    log("WIDE claim counters")
    y1 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2).clone()
    torch.cuda.synchronize()
    assert buf.scratch_view("meta")[1].item() == 1, "the WIDE GEMM1 ran"
    sched = buf.scratch_view("sched").cpu()  # [GEMM1, GEMM2] x 16
    sched[0, 9:12] = 0
    assert torch.all(sched == 0)
    mm.LayerCall(torch.empty_like(y1), l1, l2, buf).run(3, 3)  # GEMM2 alone
    torch.cuda.synchronize()
    sched = buf.scratch_view("sched").cpu()
    sched[0, 9:12] = 0
    assert torch.all(sched == 0)
    y2 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_decode_pipeline_counters_and_row_maxima(mm, cuda, full_weights):
    """The one-launch decode pipeline (GEMM1 + requant + GEMM2 of the 8-wave kernel on the
    256-CU chip, S*K <= 8192): GEMM1's per-block row maxima are exactly the blocks' max |y| and
    reduce to the requant's row amax; its hand-off counters read zero after a whole call and
    after a call that stops before the combine; calls on the same scratch are bitwise equal."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the decode pipeline runs on the whole 256-CU MI355X only")
    l1, l2, l1c, l2c, unpacked = full_weights
    s = 512
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=77)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048)
    log("decode pipeline counters and row maxima")
    y1 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2).clone()
    torch.cuda.synchronize()
    assert buf.scratch_view("meta")[3].item() == 0
    assert torch.all(buf.scratch_view("pipe").cpu() == 0)
    r = int(buf.scratch_view("meta")[0].item())
    y = buf.scratch_view("y")[:r].cpu().float()
    pmax = buf.scratch_view("pmax")[:r].cpu()
    assert torch.equal(pmax, y.view(r, 64, 32).abs().amax(dim=2)), "per-block row maxima"
    assert torch.equal(buf.scratch_view("amax")[:r].cpu(), pmax.amax(dim=1)), "row amax"
    buf.scratch_view("pmax").fill_(-1.0)
    mm.LayerCall(torch.empty_like(y1), l1, l2, buf).run(0, 3)  # stops before the combine
    torch.cuda.synchronize()
    assert bool((buf.scratch_view("pmax")[:r] >= 0).all()), "the pipeline ran"
    assert torch.all(buf.scratch_view("pipe").cpu() == 0)
    y2 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("e,s,g", [(96, 512, 256), (160, 1024, 256)])
def test_decode_pipeline_many_experts(mm, cuda, e, s, g):
    """The one-launch decode pipeline over more than 64 local experts (its group plan scans the
    experts in 64-wide chunks) with several groups a workgroup: every stage against the oracle,
    the combine bitwise, counters back at zero."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the decode pipeline runs on the whole 256-CU MI355X only")
    log(f"decode pipeline E={e} S={s}")
    l1, l2 = make_weights_gpu(e, 4096, 2048, seed=500 + e, mm=mm)
    torch.cuda.synchronize()
    l1c, l2c = cpu_weights(l1, l2)
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, e, 6, seed=600 + e, global_experts=g)
    buf = mm.get_symm_buffer_for_mega_moe(None, e, s, 6, 4096, 2048)
    buf.scratch_view("pmax").fill_(-1.0)
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    tr = O.mega_moe_forward(x_fp8, x_sf, idx, w, l1c, l2c)
    r = tr.routing.num_rows
    assert (tr.routing.counts > 0).sum() > 64 and tr.routing.counts.max() <= 64
    assert bool((buf.scratch_view("pmax")[:r] >= 0).all()), "the pipeline ran"
    assert torch.all(buf.scratch_view("pipe").cpu() == 0)
    _stage_checks(buf, tr, s)
    _combine_bitwise(mm, buf, y, l1, l2, s, None)
    d = O.calc_diff(y.cpu(), tr.y)
    log(f"  calc_diff={d:.3e}")
    assert d <= CALC_DIFF_BAR
    del l1, l2


def test_caller_scratch_reused_across_shapes(mm, cuda, full_weights):
    """One caller-owned route_scratch, zero-filled once, serves mmoe_forward calls of different
    shapes in turn through the C ABI: an all-local 1024-token call (6144 rows: its y spans
    25 MB), a 200-token call, an all-local 4096-token prefill call (the WIDE kernels), and the
    first call again. Each is bitwise equal to the same call on a fresh zero-filled scratch and
    reports status 0, and the decode pipeline's counters read zero after each: they sit at
    offset 0 in every layout, and every call leaves them zero."""
    import ctypes

    l1, l2 = full_weights[0], full_weights[1]
    lib = mm._capi.load()
    cases = ((1024, None), (200, 64), (4096, None), (1024, None))
    bufs = [mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048) for s, _ in cases]
    need = max(b.route_scratch.numel() for b in bufs)
    shared = torch.zeros((need,), dtype=torch.int8, device=cuda)
    status = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    for (s, g), buf in zip(cases, bufs):
        log(f"shared scratch: S={s} global experts={g}")
        x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=900 + s, global_experts=g)
        _load_bucket(buf, x_fp8, x_sf, idx, w)
        y_ref = torch.empty((s, 4096), dtype=torch.bfloat16, device=cuda)
        mm.fp8_w8a8_mega_moe(y_ref, l1, l2, buf)
        y = torch.full((s, 4096), 7.0, dtype=torch.bfloat16, device=cuda)
        schedule = mm._eager_schedule(mm._large_opt_3stage_mode(), mm._large_opt_3stage_threshold(), s)
        args = mm._forward_args(y, l1, l2, None, buf, None, schedule)
        args.route_scratch = shared.data_ptr()
        args.route_scratch_bytes = shared.numel()
        assert lib.mmoe_forward(ctypes.byref(args), mm._stream_handle()) == 0
        assert lib.mmoe_scratch_status(shared.data_ptr(), ctypes.cast(status.data_ptr(),
                                       ctypes.POINTER(ctypes.c_int32)), mm._stream_handle()) == 0
        torch.cuda.synchronize()
        assert int(status.item()) == 0, f"S={s}: status"
        pipe = shared[:mm._capi.MMOE_PIPE_INTS * 4].view(torch.int32)
        assert torch.all(pipe.cpu() == 0), f"S={s}: pipeline counters left nonzero"
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), f"S={s}: output"


def test_layer_no_routed_rows(mm, cuda):
    """Every slot invalid -> y == 0 exactly (no partial contributes)."""
    s, e, hdim, inter = 10, 4, 256, 128
    x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, 2, seed=1)
    idx[:] = -1
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=2, mm=mm)
    buf = mm.SymmBuffer(None, e, s, 2, hdim, inter)
    log("layer with no routed rows")
    y = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    assert torch.all(y.cpu() == 0)


# ------------------------------------------------------------------ graph-bucket mode
# Every replay is checked against the oracle on its prefix (routing bit-exact, calc_diff of y),
# as the reference checks each replayed token count against its dequantise-and-matmul baseline
# (tests/test_mega_moe_dcu.py:563-715, comparison at :646-668), and bitwise against an eager call
# of this library on the same prefix. Each token count is replayed twice, with the eager work and
# host synchronisations in between, and both replays are checked.
def _load_bucket(buf, x_fp8, x_sf, idx, w):
    s = x_fp8.shape[0]
    for t, src in ((buf.x, x_fp8), (buf.x_sf, x_sf), (buf.topk_idx, idx), (buf.topk_weights, w)):
        t[:s].copy_(src.to(t.device))


def _capture_bucket(mm, y, l1, l2, buf, flag):
    """Warm-up on a side stream, then capture one call in graph mode (the reference's order,
    tests/test_mega_moe_dcu.py:618-631)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, **{flag: True})
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, **{flag: True})
    return graph


def _oracle_prefix_check(buf, n, tr, y, unpacked=None):
    """The replay's routing equals the oracle's on the prefix (counts, output_index) and its
    y[:n] is within the north-star bar of the oracle's."""
    assert np.array_equal(buf.scratch_view("counts").cpu().numpy(), tr.routing.counts), f"n={n}: counts"
    assert np.array_equal(buf.scratch_view("output_index")[:n].cpu().numpy(),
                          tr.routing.output_index), f"n={n}: output_index"
    d = O.calc_diff(y[:n].cpu(), tr.y)
    log(f"    n={n}: routed rows {tr.routing.num_rows}, calc_diff vs oracle {d:.3e}")
    assert d <= CALC_DIFF_BAR, f"n={n}: calc_diff {d}"


@pytest.mark.parametrize("flag", ["big_fused_cuda_graph", "stages_fused_cuda_graph"])
@pytest.mark.parametrize("bucket", [(200, 8, 16), (2048, 4, 16), (3000, 8, None), (2000, 64, None)])
def test_graph_capture_replay_runtime_tokens(mm, cuda, flag, bucket):
    """Capture once at the bucket size, replay with several device token counts: every replay
    matches the oracle on its prefix, equals an eager call on that prefix (bitwise, when the eager
    call ran the same GEMM1 kernel) and leaves rows past the prefix untouched. The large buckets'
    row bound selects the 4-wave WIDE GEMMs, so both those and the 8-wave kernels are captured
    and the routed rows choose on the device: WIDE from max(8193, 256 * E) rows (the 3000-token
    bucket's full replays), the 8-wave kernels below (short prefixes). An eager call chooses by
    its largest expert's rows instead, so the two can run different GEMM1 kernels, which round y
    differently (the WIDE epilogue stores it in bf16, the 8-wave one in f32): then the oracle
    bar alone applies. Buckets of more than 8192 tasks also leave the routing to GEMM1 when the
    live tasks fit in it; the 64-expert bucket does so without selecting WIDE (fewer than 256
    rows per expert)."""
    s_max, e, g = bucket
    hdim, inter, k = 512, 256, 6
    x_fp8, x_sf, idx, w = make_tokens(s_max, hdim, e, k, seed=21, global_experts=g)
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=22, mm=mm)
    l1c, l2c = cpu_weights(l1, l2)
    buf = mm.get_symm_buffer_for_mega_moe(None, e, s_max, k, hdim, inter)
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y = torch.zeros((s_max, hdim), dtype=torch.bfloat16, device=cuda)
    log(f"graph mode {flag} bucket={bucket}: warm-up then capture")
    graph = _capture_bucket(mm, y, l1, l2, buf, flag)
    ref_buf = mm.SymmBuffer(None, e, s_max, k, hdim, inter)
    wide_min = max(8193, 256 * e)
    kinds = set()
    bitwise = 0
    for n in (s_max, 57, 1, 0, 133, s_max - 77):
        tr = O.mega_moe_forward(x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1c, l2c) if n > 0 else None
        y_ref = run_layer(mm, ref_buf, x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1, l2) if n > 0 else None
        ref_wide = n > 0 and bool(ref_buf.scratch_view("meta")[1].item() == 1)
        for rep in range(2):
            log(f"  replay {rep} with runtime tokens={n}")
            y.fill_(7.0)
            buf.cuda_graph_num_tokens.fill_(n)
            graph.replay()
            torch.cuda.synchronize()
            meta = buf.scratch_view("meta").cpu()
            live_ids = idx[:n]
            routed = int(((live_ids >= 0) & (live_ids < e) & (w[:n] != 0)).sum())
            assert int(meta[0].item()) == routed, f"n={n}: routed rows of this replay"
            assert int(meta[3].item()) == 0, f"n={n}: status"
            wide = bool(meta[1].item() == 1)
            assert wide == (routed >= wide_min), f"n={n}: kernel choice for R={routed}"
            kinds.add(wide)
            if n > 0:
                _oracle_prefix_check(buf, n, tr, y)
                if wide == ref_wide:
                    assert torch.equal(y[:n], y_ref), f"replay n={n}"
                    bitwise += 1
            assert torch.all(y[n:] == 7.0), f"rows past the prefix were written (n={n})"
    assert bitwise > 0, "no replay ran the same GEMM1 kernel as its eager call"
    if g is None:  # every slot local: the full replays run WIDE (if the rows select it) and the
        # short ones the 8-wave kernels
        assert kinds == ({True, False} if s_max * k >= wide_min else {False})


def test_graph_full_shape_both_kernels(mm, cuda, full_weights):
    """The production shape in a 2048-token bucket (every slot local: a WIDE row bound): a full
    replay runs the WIDE kernels, a short one the 8-wave kernels with GEMM1 routing in-kernel,
    also on both sides of the in-kernel routing's task limit (1365 tokens = 8190 tasks: 8-wave;
    1366 = 8196: WIDE). Every replay matches the oracle on its prefix, is bitwise equal to an
    eager call on the same prefix, and leaves rows past it alone."""
    l1, l2, l1c, l2c, unpacked = full_weights
    s_max = 2048
    x_fp8, x_sf, idx, w = make_tokens(s_max, 4096, 32, 6, seed=333, global_experts=None)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y = torch.zeros((s_max, 4096), dtype=torch.bfloat16, device=cuda)
    log("full-shape graph: warm-up and capture at 2048 tokens")
    graph = _capture_bucket(mm, y, l1, l2, buf, "stages_fused_cuda_graph")
    ref_buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    for n, wide in ((s_max, True), (100, False), (1365, False), (1366, True)):
        tr = O.mega_moe_forward(x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1c, l2c, unpacked_weights=unpacked)
        y_ref = run_layer(mm, ref_buf, x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1, l2)
        for rep in range(2):
            log(f"  replay {rep} with runtime tokens={n}")
            y.fill_(7.0)
            buf.cuda_graph_num_tokens.fill_(n)
            graph.replay()
            torch.cuda.synchronize()
            meta = buf.scratch_view("meta").cpu()
            assert int(meta[0]) == 6 * n and bool(meta[1] == 1) == wide, f"n={n}: kernel choice"
            assert int(meta[3]) == 0, f"n={n}: status"
            _oracle_prefix_check(buf, n, tr, y)
            assert torch.equal(y[:n].view(torch.int16), y_ref.view(torch.int16)), f"replay n={n}"
            assert torch.all(y[n:] == 7.0)


def test_graph_decode_pipeline_bucket(mm, cuda, full_weights):
    """The production decode bucket: the full shape (32 local of 256 global experts, H = 4096,
    I = 2048, top-6) in a 1024-token bucket, so its 6144 tasks (<= 8192) put the one-launch
    decode pipeline in the graph, which reads cuda_graph_num_tokens on the device. Replays at
    n = 1024, 777, 128, 1, 0: the pipeline ran (it alone writes the per-block row maxima), no
    bounded wait ran out (status 0) and its counters are back at zero; the routing of the prefix
    is bit-exact and y[:n] within the bar of the oracle's, bitwise equal to an eager call on the
    prefix; rows past n are untouched."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the decode pipeline runs on the whole 256-CU MI355X only")
    l1, l2, l1c, l2c, unpacked = full_weights
    s_max = 1024
    x_fp8, x_sf, idx, w = make_tokens(s_max, 4096, 32, 6, seed=1234 + s_max, global_experts=256)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    assert buf.cuda_graph_max_tokens_per_rank == s_max and buf.num_max_tokens_per_rank == 1152
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y = torch.zeros((s_max, 4096), dtype=torch.bfloat16, device=cuda)
    log("decode-bucket graph: warm-up and capture at 1024 tokens")
    graph = _capture_bucket(mm, y, l1, l2, buf, "big_fused_cuda_graph")
    ref_buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    for n in (1024, 777, 128, 1, 0):
        tr = O.mega_moe_forward(x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1c, l2c,
                                unpacked_weights=unpacked) if n > 0 else None
        y_ref = run_layer(mm, ref_buf, x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1, l2) if n > 0 else None
        for rep in range(2):
            log(f"  replay {rep} with runtime tokens={n}")
            y.fill_(7.0)
            buf.scratch_view("pmax").fill_(-1.0)
            buf.cuda_graph_num_tokens.fill_(n)
            graph.replay()
            torch.cuda.synchronize()
            meta = buf.scratch_view("meta").cpu()
            r = int(meta[0])
            assert int(meta[3]) == 0, f"n={n}: a bounded wait ran out"
            assert int(meta[1]) == 0, f"n={n}: the pipeline's GEMM1 is the 8-wave one"
            assert torch.all(buf.scratch_view("pipe").cpu() == 0), f"n={n}: pipeline counters"
            if n > 0:
                assert r == tr.routing.num_rows
                assert bool((buf.scratch_view("pmax")[:r] >= 0).all()), f"n={n}: the pipeline ran"
                _oracle_prefix_check(buf, n, tr, y)
                assert torch.equal(y[:n].view(torch.int16), y_ref.view(torch.int16)), f"replay n={n}"
            else:
                assert r == 0
            assert torch.all(y[n:] == 7.0), f"n={n}: rows past the prefix were written"


def test_decode_pipeline_repeated_runs_bitwise(mm, cuda, full_weights):
    """The c1 decode layer (one launch whose workgroups hand rows to each other through counters
    and device-coherent loads) 50 times eagerly and 50 times as graph replays: every output is
    bitwise the first one (a race in a hand-off would show as a differing bit). Stops at the
    first mismatch."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the decode pipeline runs on the whole 256-CU MI355X only")
    l1, l2 = full_weights[0], full_weights[1]
    s = 1024
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=1234 + s, global_experts=256)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048)
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y = torch.empty((s, 4096), dtype=torch.bfloat16, device=cuda)
    buf.scratch_view("pmax").fill_(-1.0)
    mm.fp8_w8a8_mega_moe(y, l1, l2, buf)
    torch.cuda.synchronize()
    r = int(buf.scratch_view("meta")[0])
    assert bool((buf.scratch_view("pmax")[:r] >= 0).all()), "the pipeline ran"
    first = y.clone()
    log("decode pipeline: 50 eager calls")
    for i in range(50):
        y.fill_(7.0)
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf)
        torch.cuda.synchronize()
        assert int(buf.scratch_view("meta")[3]) == 0, f"eager call {i}: status"
        assert torch.equal(y.view(torch.int16), first.view(torch.int16)), f"eager call {i} differs"
    graph = _capture_bucket(mm, y, l1, l2, buf, "big_fused_cuda_graph")
    log("decode pipeline: 50 graph replays")
    for i in range(50):
        y.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert int(buf.scratch_view("meta")[3]) == 0, f"replay {i}: status"
        assert torch.equal(y.view(torch.int16), first.view(torch.int16)), f"replay {i} differs"


def test_decode_pipeline_failed_wait_is_reported(mm, cuda, full_weights, monkeypatch):
    """MMOE_DEBUG_NO_WAIT, set from the host, makes every bounded wait of the decode pipeline give
    up at its first poll (every kernel still runs to its end; the data it then reads are in
    bounds, only possibly stale). The call's status counts those waits: mmoe_scratch_status
    through the C ABI and last_call_status read it, and MEGAMOE_DEBUG_CHECK=1 makes the API raise.
    The next ordinary call on the same scratch reports 0 again and is bitwise the first call."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the decode pipeline runs on the whole 256-CU MI355X only")
    import ctypes

    l1, l2 = full_weights[0], full_weights[1]
    s = 1024
    x_fp8, x_sf, idx, w = make_tokens(s, 4096, 32, 6, seed=1234 + s, global_experts=256)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s, 6, 4096, 2048)
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y_ok = torch.empty((s, 4096), dtype=torch.bfloat16, device=cuda)
    mm.fp8_w8a8_mega_moe(y_ok, l1, l2, buf)
    assert mm.last_call_status(buf) == 0
    lib = mm._capi.load()
    log("decode pipeline with every bounded wait giving up at once (C ABI)")
    y = torch.empty_like(y_ok)
    args = mm._forward_args(y, l1, l2, None, buf, None, mm._capi.MMOE_SCHEDULE_AUTO)
    args.debug_flags = mm._capi.MMOE_DEBUG_NO_WAIT
    assert lib.mmoe_forward(ctypes.byref(args), mm._stream_handle()) == 0
    out = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    assert lib.mmoe_scratch_status(buf.route_scratch.data_ptr(),
                                   ctypes.cast(out.data_ptr(), ctypes.POINTER(ctypes.c_int32)),
                                   mm._stream_handle()) == 0
    torch.cuda.synchronize()
    failed = int(out.item())
    log(f"  status: {failed} waits ran out")
    assert failed > 0
    assert mm.last_call_status(buf) == failed
    assert torch.all(buf.scratch_view("pipe").cpu() == 0), "counters back at zero all the same"
    log("the same through the API with MEGAMOE_DEBUG_CHECK=1")
    orig = mm._forward_args

    def forced(*a, **k):
        fa = orig(*a, **k)
        fa.debug_flags = mm._capi.MMOE_DEBUG_NO_WAIT
        return fa

    monkeypatch.setenv("MEGAMOE_DEBUG_CHECK", "1")
    monkeypatch.setattr(mm, "_forward_args", forced)
    with pytest.raises(RuntimeError, match="bounded waits ran out"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf)
    monkeypatch.setattr(mm, "_forward_args", orig)
    y.fill_(7.0)
    mm.fp8_w8a8_mega_moe(y, l1, l2, buf)  # checked: raises if the status is not 0
    torch.cuda.synchronize()
    assert mm.last_call_status(buf) == 0
    assert torch.equal(y.view(torch.int16), y_ok.view(torch.int16))


def _sampled_oracle_check(mm, buf, n, y, x_fp8, x_sf, idx, w, l1c, l2c, unpacked, seed):
    """A token's output depends only on its own input and slots, so the oracle layer over a
    sample of tokens is the oracle of those tokens in the whole layer: routing of the whole
    prefix bit-exact (counts, output_index), and y of ~200 sampled tokens (with and without
    local slots) within the bar."""
    ref = O.route(idx[:n].cpu(), w[:n].cpu(), 32)
    assert np.array_equal(buf.scratch_view("counts").cpu().numpy(), ref.counts), f"n={n}: counts"
    assert np.array_equal(buf.scratch_view("output_index")[:n].cpu().numpy(),
                          ref.output_index), f"n={n}: output_index"
    gen = np.random.default_rng(seed)
    sel = torch.from_numpy(np.sort(gen.choice(n, size=min(n, 200), replace=False))).long()
    dsel = sel.to(x_fp8.device)
    xs = x_fp8.view(torch.uint8)[dsel].cpu().view(torch.float8_e4m3fn)
    tr = O.mega_moe_forward(xs, x_sf[dsel].cpu(), idx[dsel].cpu(), w[dsel].cpu(),
                            l1c, l2c, unpacked_weights=unpacked)
    d = O.calc_diff(y[sel.to(y.device)].cpu(), tr.y)
    log(f"    n={n}: {sel.numel()} sampled tokens, calc_diff vs oracle {d:.3e}")
    assert d <= CALC_DIFF_BAR
    return ref


def test_graph_ep_share_mid_bucket(mm, cuda, full_weights):
    """An EP share between the decode and prefill buckets (5120 tokens a rank, 256 global
    experts: its bound selects WIDE, ~3.9K routed rows): every replay below 8193 routed rows runs
    the 8-wave kernels of the dual launch -- 128-row STREAM items, the TILE engine for the few
    experts above 128 rows -- and 1365 tokens (8190 tasks) route in GEMM1 itself. Each replay
    matches the oracle on its prefix, is bitwise equal to an eager call on it where that call
    ran the same GEMM1 kernel, and leaves the rows past it alone."""
    l1, l2, l1c, l2c, unpacked = full_weights
    s_max = 5120
    x_fp8, x_sf, idx, w = make_tokens(s_max, 4096, 32, 6, seed=1234 + s_max, global_experts=256)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y = torch.zeros((s_max, 4096), dtype=torch.bfloat16, device=cuda)
    log("mid EP-share graph: warm-up and capture at 5120 tokens")
    graph = _capture_bucket(mm, y, l1, l2, buf, "stages_fused_cuda_graph")
    ref_buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    bitwise = 0
    largest_full = 0
    for n in (s_max, 3584, 2000, 1365):
        tr = O.mega_moe_forward(x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1c, l2c, unpacked_weights=unpacked)
        assert tr.routing.num_rows < 8193
        largest_full = max(largest_full, int(tr.routing.counts.max()))
        y_ref = run_layer(mm, ref_buf, x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1, l2)
        torch.cuda.synchronize()
        ref_wide = bool(ref_buf.scratch_view("meta")[1].item() == 1)
        for rep in range(2):
            log(f"  replay {rep} with runtime tokens={n}")
            y.fill_(7.0)
            buf.cuda_graph_num_tokens.fill_(n)
            graph.replay()
            torch.cuda.synchronize()
            meta = buf.scratch_view("meta").cpu()
            assert int(meta[0]) == tr.routing.num_rows and int(meta[3]) == 0, f"n={n}"
            assert int(meta[1]) == 0, f"n={n}: the 8-wave GEMM1 ran"
            _oracle_prefix_check(buf, n, tr, y, unpacked)
            if not ref_wide:
                assert torch.equal(y[:n].view(torch.int16), y_ref.view(torch.int16)), f"replay n={n}"
                bitwise += 1
            assert torch.all(y[n:] == 7.0), f"rows past the prefix were written (n={n})"
    assert bitwise > 0
    assert largest_full > 128, "an expert on the TILE engine in the full replay"


def test_graph_ep_share_zero_rows(mm, cuda, full_weights):
    """An EP share (256 global experts, ~45% of the tokens without a local slot) in a
    65536-token bucket (~49K routed rows: 14 WIDE tiles a workgroup, the static deal): a full
    replay runs the WIDE kernels, whose idle workgroups write the zero rows of live tokens without
    a slot (the combine skips the chunks they claimed: the claim counter is past zero); a short
    one the 8-wave kernels. Every replay: routing bit-exact and sampled tokens within the bar of
    the oracle, bitwise equal to an eager call on the same prefix (zero rows included: y starts at
    7.0), rows past the prefix left alone."""
    l1, l2, l1c, l2c, unpacked = full_weights
    s_max = 65536
    x_fp8, x_sf, idx, w = _prefill_tokens_gpu(mm, s_max, 256, seed=444)
    buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    _load_bucket(buf, x_fp8, x_sf, idx, w)
    y = torch.zeros((s_max, 4096), dtype=torch.bfloat16, device=cuda)
    log("EP-share graph: warm-up and capture at 65536 tokens")
    graph = _capture_bucket(mm, y, l1, l2, buf, "stages_fused_cuda_graph")
    ref_buf = mm.get_symm_buffer_for_mega_moe(None, 32, s_max, 6, 4096, 2048)
    for n, wide in ((s_max, True), (1024, False), (s_max - 77, True)):
        y_ref = torch.full((n, 4096), 7.0, dtype=torch.bfloat16, device=cuda)
        run_layer(mm, ref_buf, x_fp8[:n], x_sf[:n], idx[:n], w[:n], l1, l2, y=y_ref)
        torch.cuda.synchronize()
        unrouted = (idx[:n] < 0) | (idx[:n] >= 32)
        zero_rows = unrouted.all(dim=1)
        assert int(zero_rows.sum()) > n // 3, "many tokens without a local slot"
        assert torch.all(y_ref[zero_rows] == 0)
        for rep in range(2):
            log(f"  replay {rep} with runtime tokens={n}")
            y.fill_(7.0)
            buf.cuda_graph_num_tokens.fill_(n)
            graph.replay()
            torch.cuda.synchronize()
            meta = buf.scratch_view("meta").cpu()
            assert bool(meta[1].item() == 1) == wide, f"n={n}: kernel choice"
            assert int(meta[3]) == 0, f"n={n}: status"
            if wide:  # idle WIDE workgroups claimed zero-row chunks
                assert int(buf.scratch_view("sched")[0, 9].item()) > 0, f"n={n}: zero rows claimed"
            if rep == 0:
                _sampled_oracle_check(mm, buf, n, y, x_fp8, x_sf, idx, w, l1c, l2c, unpacked, n)
            assert torch.equal(y[:n].view(torch.int16), y_ref.view(torch.int16)), f"replay n={n}"
            assert torch.all(y[n:] == 7.0)
        del y_ref


# ------------------------------------------------------------------ pre/post-process
@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
def test_deepep_pre_post_process(mm, cuda, ids_dtype):
    s, e, k, hdim = 300, 8, 4, 512
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn((s, hdim), generator=gen)).to(torch.bfloat16)
    x_fp8, x_sf = O.cast_to_fp8_channelwise(x)
    idx = torch.randint(-1, e, (s, k), generator=gen).to(ids_dtype)
    w = torch.rand((s, k), generator=gen)
    ref = O.route(idx.to(torch.int64), torch.ones_like(w), e)  # preprocess ignores weights
    counts = torch.from_numpy(ref.counts).to(torch.int32)
    log(f"preprocess ids={ids_dtype}")
    gx, gs, rw, mi, oi = mm.deepep_deepgemm_preprocess_channelwise(
        x_fp8.to(cuda), x_sf.to(cuda), idx.to(cuda), w.to(cuda), counts.to(cuda), int(ref.num_rows))
    torch.cuda.synchronize()
    r = ref.num_rows
    assert np.array_equal(oi.cpu().numpy(), ref.output_index)
    assert np.array_equal(mi[:r].cpu().numpy(), ref.m_indices)
    tok = torch.from_numpy(ref.row_token).long()
    assert torch.equal(gx[:r].cpu().view(torch.uint8), x_fp8[tok].view(torch.uint8))
    assert torch.equal(gs[:r].cpu(), x_sf[tok])
    exp_w = w.reshape(-1)[torch.from_numpy(ref.row_token).long() * k
                          + torch.from_numpy(ref.row_slot).long()]
    assert torch.equal(rw[:r].cpu(), exp_w)
    # postprocess: gather-sum of arbitrary l2_out rows, with and without weights
    l2_out = (torch.randn((max(r, 1), hdim), generator=gen)).to(torch.bfloat16)
    for apply_w in (False, True):
        log(f"postprocess apply_w={apply_w}")
        y = torch.empty((s, hdim), dtype=torch.bfloat16, device=cuda)
        mm.deepep_deepgemm_postprocess_channelwise(y, l2_out.to(cuda), idx.to(cuda), w.to(cuda),
                                                   oi, apply_topk_weights=apply_w)
        torch.cuda.synchronize()
        acc = torch.zeros((s, hdim))
        oic = oi.cpu().long()
        for j in range(k):
            ok = (oic[:, j] >= 0) & (idx[:, j] >= 0)
            v = l2_out.float()[oic[ok, j]]
            if apply_w:
                v = v * w[ok, j].view(-1, 1)
            acc[ok] += v
        assert torch.equal(y.cpu(), acc.to(torch.bfloat16))


def test_api_flag_and_tensor_errors(mm, cuda, monkeypatch):
    """The reference's flag and tensor checks raise the same exception types and messages
    (megamoe/__init__.py:343-410, csrc/apis/mega_dcu.hpp:355-433, large_opt.py:381, :526,
    mega_moe_fused_hip.cu:87-91), in the same order: the staged paths refuse fast_math=False
    before any tensor check, the persistent path after them."""
    s, e, hdim, inter, k = 16, 4, 256, 128, 3
    log("api flag/tensor errors")
    x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=5)
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=6, mm=mm)
    buf = mm.SymmBuffer(None, e, s, k, hdim, inter)
    y = torch.empty((s, hdim), dtype=torch.bfloat16, device=cuda)
    # 16 tokens <= the default threshold 128: the persistent path
    with pytest.raises(RuntimeError, match="persistent fused path requires fast_math"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, fast_math=False)
    with pytest.raises(RuntimeError, match="y must be BF16"):
        mm.fp8_w8a8_mega_moe(y.float(), l1, l2, buf, fast_math=False)
    with pytest.raises(RuntimeError, match="persistent fused path requires fast_math"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, big_fused_cuda_graph=True, fast_math=False)
    with pytest.raises(RuntimeError, match="large-opt DCU MegaMoE graph path requires fast_math"):
        mm.fp8_w8a8_mega_moe(y.float(), l1, l2, buf, stages_fused_cuda_graph=True, fast_math=False)
    # a threshold below the token count: the staged path, refused before the tensor checks
    monkeypatch.setenv("MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD", "8")
    staged_buf = mm.SymmBuffer(None, e, s, k, hdim, inter)
    with pytest.raises(RuntimeError, match="large-opt DCU MegaMoE path requires fast_math"):
        mm.fp8_w8a8_mega_moe(y.float(), l1, l2, staged_buf, fast_math=False)
    monkeypatch.delenv("MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD")
    with pytest.raises(ValueError, match="choose only one"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, big_fused_cuda_graph=True,
                             stages_fused_cuda_graph=True)
    with pytest.raises(ValueError, match="dispatch_num_tokens must be in"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, dispatch_num_tokens=s + 1)
    with pytest.raises(RuntimeError, match="recipe"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, recipe=(1, 1, 64))
    with pytest.raises(RuntimeError, match="swiglu only"):
        mm.fp8_w8a8_mega_moe(y, l1, l2, buf, activation="gelu")
    with pytest.raises(RuntimeError, match="y must be BF16"):
        mm.fp8_w8a8_mega_moe(y.float(), l1, l2, buf)
    with pytest.raises(RuntimeError, match="FP8 E4M3 L1 weights"):
        mm.fp8_w8a8_mega_moe(y, (l1[0].view(torch.uint8), l1[1]), l2, buf)
    # the layer still runs after the refusals
    y2 = run_layer(mm, buf, x_fp8, x_sf, idx, w, l1, l2)
    torch.cuda.synchronize()
    assert torch.isfinite(y2.float()).all()
