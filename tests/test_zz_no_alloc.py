"""The allocation-free entry point mmoe_forward_static (static device scratch) against
mmoe_forward (caller-provided route_scratch), through the C ABI: bitwise equal outputs and
stats on two calls in a row, the second with a smaller input, and the size limit refused on
the host."""
import ctypes

import pytest
import torch

from tests._helpers import log, make_tokens, make_weights_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mm(cuda):
    from deepgemm_amd import megamoe
    return megamoe


def _static_call(mm, y, l1, l2, buf, stats=None, clamp=None):
    """mmoe_forward_static with the same arguments as the API call, minus the scratch."""
    args = mm._forward_args(y, l1, l2, stats, buf, clamp, mm._capi.MMOE_SCHEDULE_AUTO)
    args.route_scratch = None
    args.route_scratch_bytes = 0
    return mm._capi.load().mmoe_forward_static(ctypes.byref(args), mm._stream_handle())


def _load(buf, x_fp8, x_sf, idx, w):
    s = x_fp8.shape[0]
    buf.x[:s].copy_(x_fp8.to(buf.x.device))
    buf.x_sf[:s].copy_(x_sf.to(buf.x.device))
    buf.topk_idx[:s].copy_(idx.to(buf.x.device))
    buf.topk_weights[:s].copy_(w.to(buf.x.device))


def _static_status(mm):
    """mmoe_scratch_status of the static scratch (NULL route_scratch) on this device."""
    out = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    st = mm._capi.load().mmoe_scratch_status(None, ctypes.cast(out.data_ptr(),
                                                               ctypes.POINTER(ctypes.c_int32)),
                                             mm._stream_handle())
    assert st == 0, mm._capi.status_string(st)
    return int(out.item())


def test_static_scratch_matches_mmoe_forward(mm, cuda):
    e, hdim, inter, k = 32, 4096, 2048, 6
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=4321, mm=mm)
    # call 1: the decode config's size (1024 tokens, capacity 1152); call 2: the same capacity
    # with every slot local (6144 rows: its y alone spans 25 MB of the static array); call 3:
    # a smaller input with a layout of its own, whose sections sit where call 2's y and partial
    # rows were (its pipeline counters start at zero only because they sit at offset 0 in every
    # layout and each call leaves them zero)
    for s, g, clamp in ((1024, 256, None), (1024, None, None), (200, 64, 1.0)):
        log(f"static scratch: S={s} clamp={clamp}")
        x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=77 + s, global_experts=g)
        buf = mm.get_symm_buffer_for_mega_moe(None, e, s, k, hdim, inter)
        _load(buf, x_fp8, x_sf, idx, w)
        stats_ref = torch.zeros(e, dtype=torch.int32, device=cuda)
        stats_got = torch.zeros(e, dtype=torch.int32, device=cuda)
        y_ref = torch.empty((s, hdim), dtype=torch.bfloat16, device=cuda)
        mm.fp8_w8a8_mega_moe(y_ref, l1, l2, buf, cumulative_local_expert_recv_stats=stats_ref,
                             activation_clamp=clamp)
        y_got = torch.full((s, hdim), 7.0, dtype=torch.bfloat16, device=cuda)
        st = _static_call(mm, y_got, l1, l2, buf, stats_got, clamp)
        assert st == 0, mm._capi.status_string(st)
        torch.cuda.synchronize()
        assert _static_status(mm) == 0, f"S={s}: status of the static call"
        assert torch.equal(y_got.view(torch.int16), y_ref.view(torch.int16)), f"S={s}"
        assert torch.equal(stats_got, stats_ref)
        assert int(stats_ref.sum()) > 0


def test_static_scratch_wide_path(mm, cuda):
    """A small shape with many rows per expert runs the prefill (WIDE) kernels, whose work-claim
    counters then live in the static scratch too; twice in a row, bitwise equal to
    mmoe_forward."""
    e, hdim, inter, k = 4, 512, 256, 6
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=4322, mm=mm)
    for s in (2048, 1536):
        log(f"static scratch, WIDE path: S={s}")
        x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=99 + s, global_experts=8)
        buf = mm.get_symm_buffer_for_mega_moe(None, e, s, k, hdim, inter)
        _load(buf, x_fp8, x_sf, idx, w)
        y_ref = torch.empty((s, hdim), dtype=torch.bfloat16, device=cuda)
        mm.fp8_w8a8_mega_moe(y_ref, l1, l2, buf)
        torch.cuda.synchronize()
        assert buf.scratch_view("meta")[1].item() == 1, "the WIDE GEMM1 ran"
        y_got = torch.full((s, hdim), 7.0, dtype=torch.bfloat16, device=cuda)
        st = _static_call(mm, y_got, l1, l2, buf)
        assert st == 0, mm._capi.status_string(st)
        torch.cuda.synchronize()
        assert torch.equal(y_got.view(torch.int16), y_ref.view(torch.int16)), f"S={s}"


def test_static_scratch_stream_items(mm, cuda):
    """Top-8 over an expert width of 1536 (GEMM2's K keeps it off the one-launch pipeline): the
    8-wave kernels route in-kernel and stream every expert, those above 64 rows as one 128-row
    item a column block; twice in a row, the second call smaller, bitwise equal to
    mmoe_forward."""
    e, hdim, inter, k = 32, 4096, 1536, 8
    l1, l2 = make_weights_gpu(e, hdim, inter, seed=4323, mm=mm)
    for s in (1024, 512):
        log(f"static scratch, 8-wave STREAM items: S={s}")
        x_fp8, x_sf, idx, w = make_tokens(s, hdim, e, k, seed=55 + s, global_experts=128)
        buf = mm.get_symm_buffer_for_mega_moe(None, e, s, k, hdim, inter)
        _load(buf, x_fp8, x_sf, idx, w)
        y_ref = torch.empty((s, hdim), dtype=torch.bfloat16, device=cuda)
        mm.fp8_w8a8_mega_moe(y_ref, l1, l2, buf)
        torch.cuda.synchronize()
        assert buf.scratch_view("meta")[1].item() == 0, "the 8-wave GEMM1 ran"
        if s == 1024:
            assert int(buf.scratch_view("counts").max()) > 64, "an expert on a 128-row item"
        y_got = torch.full((s, hdim), 7.0, dtype=torch.bfloat16, device=cuda)
        st = _static_call(mm, y_got, l1, l2, buf)
        assert st == 0, mm._capi.status_string(st)
        torch.cuda.synchronize()
        assert torch.equal(y_got.view(torch.int16), y_ref.view(torch.int16)), f"S={s}"


def test_static_scratch_limit_is_refused(mm, cuda):
    """A capacity whose scratch exceeds MMOE_STATIC_SCRATCH_BYTES returns
    MMOE_ERR_STATIC_SCRATCH before any launch."""
    e, hdim, inter, k = 32, 4096, 2048, 6
    s = 2048  # 170 MiB of scratch
    need = ctypes.c_int64()
    mm._capi.load().mmoe_route_scratch_bytes(1, e, s, k, hdim, inter, ctypes.byref(need))
    assert need.value > mm._capi.MMOE_STATIC_SCRATCH_BYTES
    buf = mm.SymmBuffer(None, e, s, k, hdim, inter)
    l1 = (torch.zeros((e, 2 * inter // 16, hdim * 16), dtype=torch.float8_e4m3fn, device=cuda),
          torch.ones((e, 2 * inter), device=cuda))
    l2 = (torch.zeros((e, hdim // 16, inter * 16), dtype=torch.float8_e4m3fn, device=cuda),
          torch.ones((e, hdim), device=cuda))
    y = torch.empty((s, hdim), dtype=torch.bfloat16, device=cuda)
    st = _static_call(mm, y, l1, l2, buf)
    assert st == mm._capi.MMOE_ERR_STATIC_SCRATCH
    assert "static" in mm._capi.status_string(st)
