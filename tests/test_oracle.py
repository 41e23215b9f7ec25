"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP path.

Every check here is independent of the formula it checks: closed forms, brute force,
a second restatement in C, exact special cases, or float64 recomputation."""
import math

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import megamoe_oracle as O


# ------------------------------------------------------------------ calc_diff
def test_calc_diff_closed_forms():
    x = torch.randn(1000, dtype=torch.float64)
    assert O.calc_diff(x, x) == pytest.approx(0.0, abs=1e-15)
    assert O.calc_diff(x, -x) == pytest.approx(2.0, abs=1e-12)
    assert O.calc_diff(torch.zeros(10), torch.zeros(10)) == 0.0
    # orthogonal vectors of equal norm -> 1
    a = torch.tensor([1.0, 0.0])
    b = torch.tensor([0.0, 1.0])
    assert O.calc_diff(a, b) == pytest.approx(1.0)
    # y = 2x: 1 - 2*2/(1+4) = 0.2
    assert O.calc_diff(x, 2 * x) == pytest.approx(0.2, abs=1e-12)


# ------------------------------------------------------------------ e4m3
def _e4m3_grid():
    lib = c_oracle()
    vals = np.array([lib.oracle_e4m3_to_f32(b) for b in range(256)], dtype=np.float32)
    return vals


def _probe_floats():
    grid = _e4m3_grid()
    finite = np.sort(np.unique(grid[np.isfinite(grid)]))
    mids = (finite[:-1].astype(np.float64) + finite[1:]) / 2.0
    pts = np.concatenate([finite.astype(np.float64), mids])
    pts32 = pts.astype(np.float32)
    up = np.nextafter(pts32, np.float32(np.inf))
    dn = np.nextafter(pts32, np.float32(-np.inf))
    rng = np.random.default_rng(0)
    rnd = (rng.standard_normal(200000) * np.exp(rng.uniform(-12, 7, 200000))).astype(np.float32)
    extra = np.array([448.0, 449.0, 464.0, 470.0, 480.0, 1e6, -1e6, 0.0, -0.0, 1e-30, -1e-30],
                     dtype=np.float32)
    return np.concatenate([pts32, up, dn, rnd, extra]).astype(np.float32)


def test_e4m3_torch_vs_c_restatement():
    """torch's e4m3fn cast (after the +-448 clip) == the C restatement of OCP RNE on every
    grid point, every midpoint (ties to even), +-1 float ulp around both, 200K random."""
    lib = c_oracle()
    f = _probe_floats()
    out_c = np.empty(f.size, dtype=np.uint8)
    lib.oracle_e4m3_from_f32_array(out_c.ctypes.data, f.ctypes.data, f.size)
    out_t = O.e4m3_from_f32(torch.from_numpy(f)).view(torch.uint8).numpy()
    bad = np.nonzero(out_c != out_t)[0]
    assert bad.size == 0, f"mismatch at {f[bad[:5]]}: c={out_c[bad[:5]]} torch={out_t[bad[:5]]}"


def test_e4m3_known_answers():
    lib = c_oracle()
    assert lib.oracle_e4m3_from_f32(448.0) == 0x7E
    assert lib.oracle_e4m3_from_f32(-448.0) == 0xFE
    assert lib.oracle_e4m3_from_f32(1000.0) == 0x7E  # clipped, saturating
    assert lib.oracle_e4m3_from_f32(1.0) == 0x38
    assert lib.oracle_e4m3_from_f32(2.0 ** -9) == 0x01  # smallest subnormal
    assert lib.oracle_e4m3_from_f32(2.0 ** -10) == 0x00  # tie -> even (0)
    assert lib.oracle_e4m3_from_f32(3 * 2.0 ** -10) == 0x02  # 1.5 ulp -> tie -> even (2)
    assert lib.oracle_e4m3_from_f32(1.0625) == 0x38  # tie between 1 and 1.125 -> even
    assert lib.oracle_e4m3_from_f32(1.1875) == 0x3A  # tie between 1.125 and 1.25 -> even


# ------------------------------------------------------------------ channelwise cast
def test_cast_known_answers():
    x = torch.zeros((3, 32), dtype=torch.bfloat16)
    x[0, 5] = 448.0
    x[0, 6] = -2.0
    x[2, :] = torch.tensor([1.0, -0.5, 0.25, 2.0] * 8, dtype=torch.bfloat16)
    q, s = O.cast_to_fp8_channelwise(x)
    assert s[0].item() == 1.0
    assert q[0].float()[5].item() == 448.0 and q[0].float()[6].item() == -2.0
    assert s[1].item() == pytest.approx(1e-4 / 448.0, rel=1e-7)
    assert torch.all(q[1].view(torch.uint8) == 0)
    # row 2: amax 2 -> scale 2/448; x/scale = 224*x exactly representable (224, 112, 56, 448)
    assert s[2].item() == pytest.approx(2.0 / 448.0, rel=1e-7)
    assert torch.equal(q[2].float(), (x[2].float() * 224.0))


# ------------------------------------------------------------------ Marlin
def test_marlin_offset_bruteforce_and_roundtrip():
    lib = c_oracle()
    g, r, k = 2, 32, 48
    w = torch.randint(0, 256, (g, r, k), dtype=torch.uint8)
    wm = O.marlin_pack(w).reshape(-1)
    for e in range(g):
        for rr in range(r):
            for kk in range(k):
                off = O.marlin_offset(e, rr, kk, r, k)
                assert off == lib.oracle_marlin_offset(e, rr, kk, r, k)
                assert wm[off] == w[e, rr, kk]
    assert torch.equal(O.marlin_unpack(O.marlin_pack(w), r, k), w)


# ------------------------------------------------------------------ routing
def _routing_cases():
    rng = np.random.default_rng(7)
    cases = []
    # random with invalid ids and zero weights
    idx = rng.integers(-3, 12, size=(37, 4)).astype(np.int64)
    w = rng.random((37, 4)).astype(np.float32)
    w[rng.random((37, 4)) < 0.1] = 0.0
    cases.append((idx, w, 8))
    # duplicates (same expert twice in a token)
    idx = rng.integers(0, 3, size=(20, 6)).astype(np.int64)
    cases.append((idx, rng.random((20, 6)).astype(np.float32) + 0.1, 4))
    # empty
    cases.append((np.zeros((0, 6), np.int64), np.zeros((0, 6), np.float32), 4))
    # all invalid
    cases.append((np.full((5, 2), -1, np.int64), np.ones((5, 2), np.float32), 4))
    # huge ids (int64 beyond int32)
    idx = np.array([[2 ** 40, 1], [3, -2 ** 40]], dtype=np.int64)
    cases.append((idx, np.ones((2, 2), np.float32), 4))
    return cases


def _assert_routing_equal(a: O.Routing, b: O.Routing):
    for f in ("counts", "offsets", "output_index", "row_token", "row_slot", "row_weight",
              "m_indices"):
        np.testing.assert_array_equal(getattr(a, f), getattr(b, f), err_msg=f)


@pytest.mark.parametrize("case", range(5))
def test_route_vs_bruteforce(case):
    idx, w, e = _routing_cases()[case]
    _assert_routing_equal(O.route(idx, w, e), O.route_bruteforce(idx, w, e))


def _c_route(idx, w, e):
    lib = c_oracle()
    s, k = idx.shape
    counts = np.zeros(e, np.int32)
    offsets = np.zeros(e + 1, np.int32)
    oi = np.zeros(s * k, np.int32)
    n = max(s * k, 1)
    rt = np.zeros(n, np.int32)
    rs = np.zeros(n, np.int32)
    rw = np.zeros(n, np.float32)
    mi = np.zeros(n, np.int32)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    w = np.ascontiguousarray(w, dtype=np.float32)
    r = lib.oracle_route(idx.ctypes.data, w.ctypes.data, s, k, e, counts.ctypes.data,
                         offsets.ctypes.data, oi.ctypes.data, rt.ctypes.data, rs.ctypes.data,
                         rw.ctypes.data, mi.ctypes.data)
    return O.Routing(counts, offsets, oi.reshape(s, k), rt[:r], rs[:r], rw[:r], mi[:r])


def test_route_vs_c_restatement_large():
    gen = torch.Generator().manual_seed(3)
    idx, w = O.make_routing(20000, 32, 6, gen, global_experts=256)
    _assert_routing_equal(O.route(idx, w, 32), _c_route(idx.numpy(), w.numpy(), 32))
    for c in _routing_cases():
        _assert_routing_equal(O.route(*c), _c_route(*c))


def test_route_invariants():
    gen = torch.Generator().manual_seed(11)
    idx, w = O.make_routing(3000, 32, 6, gen, global_experts=256)
    rt = O.route(idx, w, 32)
    valid = (idx.numpy() >= 0) & (idx.numpy() < 32) & (w.numpy() != 0)
    assert rt.counts.sum() == valid.sum() == rt.num_rows
    assert np.array_equal(rt.counts, np.bincount(idx.numpy()[valid], minlength=32))
    # rows contiguous per expert, ascending task inside an expert, inverse index exact
    for e in range(32):
        seg = slice(rt.offsets[e], rt.offsets[e + 1])
        assert np.all(rt.m_indices[seg] == e)
        task = rt.row_token[seg].astype(np.int64) * 6 + rt.row_slot[seg]
        assert np.all(np.diff(task) > 0)
    oi = rt.output_index
    t, s = np.nonzero(oi >= 0)
    assert np.array_equal(rt.row_token[oi[t, s]], t)
    assert np.array_equal(rt.row_slot[oi[t, s]], s)
    assert np.array_equal(np.sort(oi[oi >= 0]), np.arange(rt.num_rows))
    assert np.all(oi[~valid] == -1)


# ------------------------------------------------------------------ GEMM
def test_gemm_one_hot_weights_is_a_gather():
    """W[e, n, k] = 1 at k = perm_e[n] -> out[r, n] = a[r, perm[n]] * a_s[r] * w_s[n] exactly."""
    torch.manual_seed(0)
    e_cnt, n, k, r = 3, 32, 48, 10
    a = (torch.randn(r, k) * 8).to(torch.float8_e4m3fn)
    a_s = torch.rand(r) + 0.5
    w = torch.zeros(e_cnt, n, k)
    perms = [torch.randint(0, k, (n,)) for _ in range(e_cnt)]
    for e in range(e_cnt):
        w[e, torch.arange(n), perms[e]] = 1.0
    w = w.to(torch.float8_e4m3fn)
    w_s = torch.full((e_cnt, n), 0.5)
    m = np.array([0, 0, 0, 1, 1, 2, 2, 2, 2, 2], np.int32)
    offs = np.array([0, 3, 5, 10])
    out = O.grouped_gemm_dequant(a, a_s, w, w_s, m, offs, out_dtype=torch.float32)
    for row in range(r):
        e = m[row]
        exp = a[row].float()[perms[e]] * a_s[row] * 0.5
        assert torch.equal(out[row], exp)


def test_gemm_small_integers_exact_and_float64():
    torch.manual_seed(1)
    a = torch.randint(-4, 5, (6, 64)).float().to(torch.float8_e4m3fn)
    w = torch.randint(-4, 5, (2, 16, 64)).float().to(torch.float8_e4m3fn)
    a_s = torch.ones(6)
    w_s = torch.ones(2, 16)
    offs = np.array([0, 2, 6])
    m = np.array([0, 0, 1, 1, 1, 1], np.int32)
    out = O.grouped_gemm_dequant(a, a_s, w, w_s, m, offs, out_dtype=torch.float32)
    ref = torch.cat([a[:2].double() @ w[0].double().t(), a[2:].double() @ w[1].double().t()])
    assert torch.equal(out.double(), ref)
    # random fp8 operands: fp32 oracle vs float64 matmul
    a = (torch.randn(40, 512) * 20).to(torch.float8_e4m3fn)
    w = (torch.randn(1, 64, 512) * 20).to(torch.float8_e4m3fn)
    out = O.grouped_gemm_dequant(a, torch.ones(40), w, torch.ones(1, 64), np.zeros(40, np.int32),
                                 np.array([0, 40]), out_dtype=torch.float32)
    ref = a.double() @ w[0].double().t()
    assert O.calc_diff(out, ref) < 1e-12


# ------------------------------------------------------------------ fp32 division
def test_fdiv_is_correctly_rounded():
    """O.fdiv == the float64 quotient rounded once to float32 (a correctly rounded fp32 divide),
    on values where torch's reciprocal-then-multiply for scalar/tensor differs."""
    rng = np.random.default_rng(3)
    a = (rng.random(200000) * 10 + 1e-4).astype(np.float32)
    exact = (448.0 / a.astype(np.float64)).astype(np.float32)
    got = O.fdiv(448.0, torch.from_numpy(a)).numpy()
    assert np.array_equal(got, exact)
    recip = (448.0 / torch.from_numpy(a)).numpy()
    assert not np.array_equal(recip, exact), "torch scalar/tensor path expected to differ"


# ------------------------------------------------------------------ SwiGLU + requant
def test_swiglu_quant_special_rows():
    inter = 8
    h = torch.zeros((4, 2 * inter), dtype=torch.bfloat16)
    # row 0: weight 0 -> zero row, scale 1e-4/448
    h[0] = 1.0
    # row 1: gate 0 -> y = 0 -> amax floor
    h[1, inter:] = 3.0
    # row 2: gate 2, up 1, w 1 -> y = 2*sigmoid(2) everywhere -> all bytes 448
    h[2, :inter] = 2.0
    h[2, inter:] = 1.0
    # row 3: clamp 1.5: gate 4 -> 1.5, up -9 -> -1.5
    h[3, :inter] = 4.0
    h[3, inter:] = -9.0
    w = torch.tensor([0.0, 1.0, 1.0, 0.5])
    q, s = O.swiglu_quant_k2(h, w, None)
    assert torch.all(q[0].view(torch.uint8) == 0) and s[0].item() == pytest.approx(1e-4 / 448)
    assert torch.all(q[1].view(torch.uint8) == 0) and s[1].item() == pytest.approx(1e-4 / 448)
    y2 = 2.0 / (1.0 + math.exp(-2.0))
    assert s[2].item() == pytest.approx(y2 / 448.0, rel=1e-6)
    assert torch.all(q[2].float() == 448.0)
    qc, sc = O.swiglu_quant_k2(h, w, 1.5)
    y3 = 1.5 / (1.0 + math.exp(-1.5)) * -1.5 * 0.5
    assert sc[3].item() == pytest.approx(abs(y3) / 448.0, rel=1e-6)
    assert torch.all(qc[3].float() == -448.0)


def _k2_scalar(g: float, u: float, w: float, c):
    """One channel of the staged K2 rule in float64 scalars: the gate is clamped from above
    only, the up value on both sides (k2_fused_ext.cu:318-327), then g*sigmoid(g)*u*w."""
    if c is not None:
        u = min(c, max(-c, u))
        g = min(c, g)
    return g / (1.0 + math.exp(-g)) * u * w


def test_swiglu_clamp_is_one_sided_on_the_gate():
    """The K2 clamp (megamoe/dcu_megamoe_large_opt/K2_fused/k2_fused_ext.cu:318-327) limits
    the gate from above only: a gate below -c passes through unclamped. Rows cover a gate
    below -c, a gate above +c, an up value above +c and below -c, and values inside +-c, each
    checked against float64 scalars. A two-sided gate clamp (the persistent fused kernel's,
    mega_moe_dcu_tiles.cuh:540-542) differs materially on the gate < -c entries, so the
    assertions below tell the two rules apart."""
    c = 1.0
    gate = [-3.0, -2.5, -0.5, 0.25, 0.75, 2.0, 4.0, -6.0]
    up = [0.5, -2.5, 3.0, -0.75, 0.5, -4.0, 1.25, -0.5]
    inter = len(gate)
    h = torch.tensor([gate + up], dtype=torch.bfloat16)  # all values exact in bf16
    w = torch.tensor([0.75])
    y = O.swiglu_k2(h, w, c)[0].double()
    want = torch.tensor([_k2_scalar(g, u, 0.75, c) for g, u in zip(gate, up)], dtype=torch.float64)
    assert torch.allclose(y, want, rtol=2e-6, atol=1e-7)
    # gate -3 stays -3: y = -3*sigmoid(-3)*0.5*0.75, not -1*sigmoid(-1)*0.5*0.75
    assert y[0].item() == pytest.approx(-3.0 / (1.0 + math.exp(3.0)) * 0.5 * 0.75, rel=1e-6)
    two_sided = torch.tensor([_k2_scalar(max(-c, g), u, 0.75, c) for g, u in zip(gate, up)],
                             dtype=torch.float64)
    below = torch.tensor([g < -c for g in gate])
    assert bool(((y - two_sided).abs()[below] > 0.02).all()), "two-sided gate clamp not excluded"
    assert torch.allclose(y[~below], two_sided[~below], rtol=2e-6, atol=1e-7)
    # the up clamp is two-sided: up 3.0 -> 1.0 and -4.0 -> -1.0
    assert y[2].item() == pytest.approx(-0.5 / (1.0 + math.exp(0.5)) * 1.0 * 0.75, rel=1e-6)
    assert y[5].item() == pytest.approx(1.0 / (1.0 + math.exp(-1.0)) * -1.0 * 0.75, rel=1e-6)
    # no clamp: every value as given
    y_none = O.swiglu_k2(h, w, None)[0].double()
    want_none = torch.tensor([_k2_scalar(g, u, 0.75, None) for g, u in zip(gate, up)],
                             dtype=torch.float64)
    assert torch.allclose(y_none, want_none, rtol=2e-6, atol=1e-7)
    # the requant of the clamped row: scale from its own max |y|, codes from y * 448/a
    q, s = O.swiglu_quant_k2(h, w, c)
    amax = float(want.abs().max())
    assert s[0].item() == pytest.approx(amax / 448.0, rel=1e-6)
    deq = q[0].float().double() * s[0].double()
    assert torch.all((deq - want).abs() <= want.abs() * 0.0625 + amax / 448 * 2 ** -9)
    assert inter == 8


def test_swiglu_quant_float64_recompute():
    torch.manual_seed(5)
    h = (torch.randn(64, 256) * 3).to(torch.bfloat16)
    w = torch.rand(64)
    q, s = O.swiglu_quant_k2(h, w, None)
    g = h[:, :128].double()
    u = h[:, 128:].double()
    y = g * torch.sigmoid(g) * u * w.double().view(-1, 1)
    amax = y.abs().amax(dim=1).clamp(min=1e-4)
    assert torch.allclose(s.double(), amax / 448.0, rtol=1e-6)
    deq = q.float().double() * s.double().view(-1, 1)
    # e4m3 has 3 mantissa bits: |err| <= 2^-4 relative (+ subnormal floor)
    assert torch.all((deq - y).abs() <= y.abs() * 0.0625 + amax.view(-1, 1) / 448 * 2 ** -9 + 1e-12)


# ------------------------------------------------------------------ combine
def test_combine_exact_sum():
    part = torch.tensor([[1.0, 2.0], [0.5, -2.0], [4.0, 8.0]], dtype=torch.bfloat16)
    oi = np.array([[0, 1, -1], [2, -1, -1], [-1, -1, -1]], np.int32)
    y = O.combine(part, oi, 3)
    assert torch.equal(y.float(), torch.tensor([[1.5, 0.0], [4.0, 8.0], [0.0, 0.0]]))
    # rounding: 1 + 2^-8 + 2^-8 -> bf16(1.0078125) = 1.0078125 (exactly representable)
    part = torch.tensor([[1.0], [2 ** -8], [2 ** -8]], dtype=torch.bfloat16)
    y = O.combine(part, np.array([[0, 1, 2]], np.int32), 1)
    assert y.float().item() == 1.0078125


# ------------------------------------------------------------------ full layer (tiny)
def test_forward_small_vs_float64_pipeline():
    """Whole oracle layer vs a float64 restatement of the maths (no fp8 rounding differences
    other than the requant, which both share)."""
    inp = O.make_layer_inputs(16, 4, 256, 128, 3, seed=42)
    tr = O.mega_moe_forward(inp["x_fp8"], inp["x_sf"], inp["topk_idx"], inp["topk_weights"],
                            inp["l1"], inp["l2"])
    w1 = O.marlin_unpack(inp["l1"][0], 256, 256).double() * inp["l1"][1].double().unsqueeze(-1)
    w2 = O.marlin_unpack(inp["l2"][0], 256, 128).double() * inp["l2"][1].double().unsqueeze(-1)
    x = inp["x_fp8"].double() * inp["x_sf"].double().view(-1, 1)
    y = torch.zeros(16, 256, dtype=torch.float64)
    for t in range(16):
        for s in range(3):
            e = int(inp["topk_idx"][t, s])
            if e < 0:
                continue
            hh = w1[e] @ x[t]
            g, u = hh[:128], hh[128:]
            act = g * torch.sigmoid(g) * u * float(inp["topk_weights"][t, s])
            y[t] += w2[e] @ act
    assert O.calc_diff(tr.y, y) < 1e-3
