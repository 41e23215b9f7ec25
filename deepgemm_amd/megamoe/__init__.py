"""MI355X (gfx950) FP8 W8A8 channelwise Mega MoE -- drop-in for the reference's ``megamoe``.

Same public names, signatures, tensor layouts and error types as the reference's
``megamoe/__init__.py`` (yuguo-Jack/DeepGEMM, DCU half, :461-473). The layer itself runs in
hand-written gfx950 HIP kernels behind the C ABI of ``include/megamoe_hip.h``
(``libmegamoe_hip.so``), called through ctypes with raw device pointers and the current HIP
stream. This build is one GPU's expert-parallel share: ``group`` must be ``None`` or a
single-rank process group and every expert id outside ``[0, num_experts)`` is not routed here.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
from types import SimpleNamespace
from typing import Optional, Tuple

import torch

from . import _capi

_LARGE_OPT_FORCE_VALUES = {"1", "true", "yes", "on", "large_opt", "3stage"}
_LARGE_OPT_AUTO_VALUES = {"auto", "threshold", "adaptive"}
_LARGE_OPT_THRESHOLD_ENV = "MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD"
_LARGE_OPT_DEFAULT_THRESHOLD = 128


def _align(value: int, alignment: int) -> int:
    return ((value + alignment - 1) // alignment) * alignment


def _is_hip_backend() -> bool:
    return getattr(torch.version, "hip", None) is not None


def _large_opt_3stage_mode() -> str:
    """megamoe/__init__.py:25-31."""
    value = os.getenv("MEGAMOE_DCU_USE_LARGE_OPT_3STAGE", "auto").strip().lower()
    if value in _LARGE_OPT_FORCE_VALUES:
        return "force"
    if value in _LARGE_OPT_AUTO_VALUES:
        return "auto"
    return "off"


def _large_opt_3stage_threshold() -> int:
    """megamoe/__init__.py:34-35."""
    return int(os.getenv(_LARGE_OPT_THRESHOLD_ENV, str(_LARGE_OPT_DEFAULT_THRESHOLD)))


def _schedule_for_mode(mode: str) -> int:
    """auto -> per-expert engine choice on the device; force -> tile engine; off -> streaming
    engine (see fp8_mega_moe)."""
    if mode == "force":
        return _capi.MMOE_SCHEDULE_STAGED
    if mode == "off":
        return _capi.MMOE_SCHEDULE_PERSISTENT
    return _capi.MMOE_SCHEDULE_AUTO


def _eager_schedule(mode: str, threshold: int, dispatch_tokens: int) -> int:
    """Schedule of an eager call. The reference runs its persistent fused kernel for
    ``dispatch_tokens <= threshold`` in auto mode and the staged K1/K2/K3 path above it
    (megamoe/__init__.py:38-43, :408-428). Here the persistent counterpart is the streaming
    engine for every expert (MMOE_SCHEDULE_PERSISTENT); above the threshold auto keeps the
    per-expert engine choice on the device. ``force`` and ``off`` ignore the threshold, as in
    the reference."""
    if mode == "auto" and dispatch_tokens <= threshold:
        return _capi.MMOE_SCHEDULE_PERSISTENT
    return _schedule_for_mode(mode)


def _is_current_stream_capturing() -> bool:
    checker = getattr(torch.cuda, "is_current_stream_capturing", None)
    return bool(checker()) if checker is not None else False


def _stream_handle() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------------------
# casts and weight layout (megamoe/__init__.py:51-98, :280-289)
# ---------------------------------------------------------------------------------------
def cast_to_fp8_channelwise(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row scale = max(amax, 1e-4)/448 and q = e4m3(x/scale); megamoe/__init__.py:51-56.
    A contiguous bf16 tensor on the GPU goes through the gfx950 cast kernel (bitwise the same
    as the torch formula); anything else uses the torch formula itself."""
    if x.dim() != 2:
        raise ValueError("channelwise FP8 cast expects a 2D tensor")
    if x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and x.size(1) > 0:
        fp8 = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
        scale = torch.empty((x.size(0),), dtype=torch.float32, device=x.device)
        _capi.check(_capi.load().mmoe_cast_fp8_channelwise(
            fp8.data_ptr(), scale.data_ptr(), x.data_ptr(), x.size(0), x.size(1),
            _stream_handle()), "cast_to_fp8_channelwise")
        return fp8, scale
    scale = x.abs().float().amax(dim=1).clamp(min=1.0e-4) / 448.0
    fp8 = (x.float() / scale.view(-1, 1)).to(torch.float8_e4m3fn)
    return fp8.contiguous(), scale.float().contiguous()


def cast_grouped_weight_to_fp8_channelwise(
    weights: torch.Tensor,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """megamoe/__init__.py:59-78 (row-independent; chunking only bounds the torch path's
    temporaries, MEGAMOE_DCU_WEIGHT_CAST_CHUNK_ROWS)."""
    if weights.dim() != 3:
        raise ValueError("MegaMoE grouped weights must be 3D tensors")
    num_groups, rows, k = weights.shape
    flat = weights.reshape(num_groups * rows, k)
    if flat.is_cuda and flat.dtype == torch.bfloat16:
        fp8, scale = cast_to_fp8_channelwise(flat.contiguous())
        return fp8.reshape(num_groups, rows, k), scale.reshape(num_groups, rows)
    chunk_rows = int(os.getenv("MEGAMOE_DCU_WEIGHT_CAST_CHUNK_ROWS", "8192"))
    if chunk_rows <= 0 or flat.size(0) <= chunk_rows:
        fp8, scale = cast_to_fp8_channelwise(flat)
    else:
        fp8 = torch.empty(flat.shape, dtype=torch.float8_e4m3fn, device=flat.device)
        scale = torch.empty((flat.size(0),), dtype=torch.float32, device=flat.device)
        for offset in range(0, flat.size(0), chunk_rows):
            end = min(offset + chunk_rows, flat.size(0))
            f, s = cast_to_fp8_channelwise(flat[offset:end])
            fp8[offset:end].copy_(f)
            scale[offset:end].copy_(s)
    return fp8.reshape(num_groups, rows, k).contiguous(), scale.reshape(num_groups, rows).contiguous()


def weight8bit_nt_kpack2_marlin(weight: torch.Tensor, k_tile: int = 16,
                                n_tile: int = 16) -> torch.Tensor:
    """[G,R,K] -> [G,R/16,K*16] Marlin nt_kpack2; megamoe/__init__.py:81-98."""
    if weight.dim() != 3:
        raise ValueError("MegaMoE Marlin weight layout expects a 3D grouped weight tensor")
    if k_tile != 16 or n_tile != 16:
        raise ValueError("DCU W8A8 MegaMoE currently supports only 16x16 kpack2 Marlin tiles")
    num_groups, rows, k = weight.shape
    if rows % n_tile != 0 or k % k_tile != 0:
        raise ValueError("DCU W8A8 MegaMoE Marlin weights require rows and K divisible by 16")
    if weight.is_cuda and weight.element_size() == 1:
        src = weight.contiguous()
        out = torch.empty((num_groups, rows // 16, k * 16), dtype=weight.dtype, device=weight.device)
        _capi.check(_capi.load().mmoe_marlin_pack(out.data_ptr(), src.data_ptr(), num_groups, rows,
                                                  k, _stream_handle()), "marlin pack")
        return out
    return (weight.reshape(num_groups, rows // n_tile, n_tile, k // k_tile, k_tile)
            .permute(0, 1, 3, 2, 4).contiguous().reshape(num_groups, rows // n_tile, k * n_tile))


def transform_fp8_weights_for_mega_moe(l1_weights: torch.Tensor, l2_weights: torch.Tensor):
    """megamoe/__init__.py:280-289."""
    l1_fp8, l1_scale = cast_grouped_weight_to_fp8_channelwise(l1_weights)
    l2_fp8, l2_scale = cast_grouped_weight_to_fp8_channelwise(l2_weights)
    return ((weight8bit_nt_kpack2_marlin(l1_fp8), l1_scale),
            (weight8bit_nt_kpack2_marlin(l2_fp8), l2_scale))


def get_mega_moe_hip_build_config():
    """megamoe/__init__.py:101-110 over csrc/apis/mega_dcu.hpp:28-39."""
    config = json.loads(_capi.load().mmoe_build_config().decode())
    config["large_opt_3stage_env"] = "MEGAMOE_DCU_USE_LARGE_OPT_3STAGE"
    config["large_opt_3stage_auto_values"] = sorted(_LARGE_OPT_AUTO_VALUES)
    config["large_opt_3stage_threshold_env"] = _LARGE_OPT_THRESHOLD_ENV
    config["large_opt_3stage_default_threshold"] = _LARGE_OPT_DEFAULT_THRESHOLD
    config["large_opt_3stage_shape"] = "single GPU: experts<=256, topk<=16, H,I % 128 == 0"
    config["large_opt_3stage_selection"] = ("auto: per expert on device (<=128 rows: streaming "
                                            "engine, else 256x256 MFMA tiles); every GEMM on "
                                            "the 4-wave 256x256 kernel when S*K > 8192 and "
                                            ">= 256 rows per expert on average")
    config["cuda_graph_max_tokens_source"] = "requested num_max_tokens_per_rank"
    config["cuda_graph_execution"] = "explicit_big_fused_or_large_opt_3stage"
    return config


def get_token_alignment_for_mega_moe() -> int:
    return int(_capi.load().mmoe_token_alignment())


def _group_size(group) -> int:
    return 1 if group is None else int(group.size())


# ---------------------------------------------------------------------------------------
# SymmBuffer (megamoe/__init__.py:113-277)
# ---------------------------------------------------------------------------------------
class SymmBuffer:
    """Input staging views + route scratch for one GPU's share of the layer.

    Attribute views match the reference (csrc/apis/mega_dcu.hpp:119-151): ``x`` e4m3
    [Smax, H], ``x_sf`` f32 [Smax], ``topk_idx`` int64 [Smax, K], ``topk_weights`` f32
    [Smax, K], ``cuda_graph_num_tokens`` int32 [1], ``route_scratch`` int8. The reference's
    IPC peer setup has no counterpart: this build is single-GPU (``group`` None or size 1)."""

    def __init__(self, group, num_experts: int, num_max_tokens_per_rank: int, num_topk: int,
                 hidden: int, intermediate_hidden: int, use_fp8_dispatch: bool = True,
                 activation: str = "swiglu",
                 cuda_graph_max_tokens_per_rank: Optional[int] = None):
        if not _is_hip_backend():
            raise RuntimeError("megamoe is the HIP/DCU MegaMoE package")
        if _group_size(group) != 1:
            raise RuntimeError(
                "this MI355X build runs one GPU's expert-parallel share; pass group=None or a "
                "single-rank group (multi-GPU dispatch/combine is not built)")
        self.group = group
        self.num_experts = num_experts
        self.num_max_tokens_per_rank = num_max_tokens_per_rank
        self.num_topk = num_topk
        self.hidden = hidden
        self.intermediate_hidden = intermediate_hidden
        self._large_opt_3stage_mode = _large_opt_3stage_mode()
        self._large_opt_3stage_threshold = _large_opt_3stage_threshold()
        self.cuda_graph_max_tokens_per_rank = int(
            cuda_graph_max_tokens_per_rank
            if cuda_graph_max_tokens_per_rank is not None else num_max_tokens_per_rank)
        if (self.cuda_graph_max_tokens_per_rank <= 0
                or self.cuda_graph_max_tokens_per_rank > self.num_max_tokens_per_rank):
            raise ValueError("cuda_graph_max_tokens_per_rank must be in "
                             f"1..{self.num_max_tokens_per_rank}")
        lib = _capi.load()
        layout = _capi.SymmLayout()
        _capi.check(lib.mmoe_symm_buffer_layout(1, num_experts, num_max_tokens_per_rank, num_topk,
                                                hidden, intermediate_hidden,
                                                ctypes.byref(layout)), "SymmBuffer")
        nbytes = ctypes.c_int64()
        _capi.check(lib.mmoe_route_scratch_bytes(1, num_experts, num_max_tokens_per_rank,
                                                 num_topk, hidden, intermediate_hidden,
                                                 ctypes.byref(nbytes)), "SymmBuffer")
        self.layout = layout
        self.scratch_layout = _capi.ScratchLayout()
        _capi.check(lib.mmoe_route_scratch_layout(1, num_experts, num_max_tokens_per_rank,
                                                  num_topk, hidden, intermediate_hidden,
                                                  ctypes.byref(self.scratch_layout)),
                    "SymmBuffer")
        self.buffer = torch.zeros((layout.total_bytes,), dtype=torch.int8, device="cuda")
        # zeroed once: the prefill GEMMs' work-claim counters live here (a full call's routing
        # stage zeroes them too, and the GEMMs leave them at zero)
        self.route_scratch = torch.zeros((nbytes.value,), dtype=torch.int8, device="cuda")
        t = num_max_tokens_per_rank

        def view(off, count, dtype, shape):
            nb = count * torch.empty((), dtype=dtype).element_size()
            return self.buffer[off:off + nb].view(dtype).view(*shape)

        self.x = view(layout.x_offset, t * hidden, torch.float8_e4m3fn, (t, hidden))
        self.x_sf = view(layout.x_sf_offset, t, torch.float32, (t,))
        self.topk_idx = view(layout.topk_idx_offset, t * num_topk, torch.int64, (t, num_topk))
        self.topk_weights = view(layout.topk_weights_offset, t * num_topk, torch.float32,
                                 (t, num_topk))
        empty = self.buffer[:0]
        self.l1_acts = empty.view(torch.float8_e4m3fn)
        self.l1_acts_sf = empty.view(torch.float32)
        self.l2_acts = empty.view(torch.float8_e4m3fn)
        self.l2_acts_sf = empty.view(torch.float32)
        self.cuda_graph_num_tokens = view(layout.runtime_num_tokens_offset, 1, torch.int32, (1,))
        self.cuda_graph_num_tokens.fill_(self.cuda_graph_max_tokens_per_rank)
        ptr = self.buffer.data_ptr()
        self.handle = SimpleNamespace(buffer_ptrs=[ptr], buffer_ptr=ptr, signal_ptrs=[0],
                                      signal_buffer_ptr=0)

    def destroy(self):
        if self.handle is not None:
            torch.cuda.synchronize()
        self.handle = None
        self.buffer = None
        self.group = None
        self.x = None
        self.x_sf = None
        self.topk_idx = None
        self.topk_weights = None
        self.route_scratch = None
        self.cuda_graph_num_tokens = None

    # -- stage-parity views into route_scratch (debug; valid after a call) --
    def scratch_view(self, name: str, num_rows: Optional[int] = None) -> torch.Tensor:
        """Intermediate tensors of the last call: counts, offsets, meta, output_index,
        row_token, row_weight, m_indices, act_scale, amax (max |y| per row), y (SwiGLU x
        weight, bf16), act (requantised y), part (GEMM2 rows), row_dest (the token whose y
        row GEMM2 wrote directly for a row, else -1; built in calls with the WIDE GEMMs, where
        those rows' part is not written; meta[2] == 1 then), sched and pipe (the GEMMs' work
        counters, zero between calls), pmax (per row, max |y| of each 64-column block of GEMM1's
        output; written by the one-launch decode pipeline only). meta[1] == 1 when GEMM1 ran on
        the WIDE kernel."""
        l = self.scratch_layout
        e, t, k = self.num_experts, self.num_max_tokens_per_rank, self.num_topk
        rows = int(l.row_capacity if num_rows is None else num_rows)
        spec = {
            "counts": (l.counts_offset, torch.int32, (e,)),
            "offsets": (l.offsets_offset, torch.int32, (e + 1,)),
            "meta": (l.meta_offset, torch.int32, (16,)),
            "output_index": (l.output_index_offset, torch.int32, (t, k)),
            "row_token": (l.row_token_offset, torch.int32, (rows,)),
            "row_weight": (l.row_weight_offset, torch.float32, (rows,)),
            "m_indices": (l.m_indices_offset, torch.int32, (rows,)),
            "act_scale": (l.act_scale_offset, torch.float32, (rows,)),
            "amax": (l.amax_offset, torch.float32, (rows,)),
            "y": (l.y_offset, torch.bfloat16, (rows, self.intermediate_hidden)),
            "act": (l.act_offset, torch.float8_e4m3fn, (rows, self.intermediate_hidden)),
            "part": (l.part_offset, torch.bfloat16, (rows, self.hidden)),
            "row_dest": (l.row_dest_offset, torch.int32, (rows,)),
            "sched": (l.sched_offset, torch.int32, (2, 16)),
            "pipe": (l.pipe_offset, torch.int32, (_capi.MMOE_PIPE_INTS,)),
            "pmax": (l.pmax_offset, torch.float32,
                     (min(rows, 8192), 2 * self.intermediate_hidden // 64)),
        }
        off, dtype, shape = spec[name]
        n = 1
        for d in shape:
            n *= d
        nb = n * torch.empty((), dtype=dtype).element_size()
        return self.route_scratch[off:off + nb].view(dtype).view(*shape)


def get_symm_buffer_for_mega_moe(group, num_experts: int, num_max_tokens_per_rank: int,
                                 num_topk: int, hidden: int, intermediate_hidden: int,
                                 use_fp8_dispatch: bool = True,
                                 activation: str = "swiglu") -> SymmBuffer:
    """megamoe/__init__.py:252-277: capacity aligned to the token alignment (384)."""
    requested = int(num_max_tokens_per_rank)
    aligned = _align(num_max_tokens_per_rank, get_token_alignment_for_mega_moe())
    return SymmBuffer(group, num_experts, aligned, num_topk, hidden, intermediate_hidden,
                      use_fp8_dispatch, activation, cuda_graph_max_tokens_per_rank=requested)


# ---------------------------------------------------------------------------------------
# DeepEP-style pre/post-process (csrc/apis/mega_dcu.hpp:222-336)
# ---------------------------------------------------------------------------------------
def deepep_deepgemm_preprocess_channelwise(recv_x: torch.Tensor, recv_x_scale: torch.Tensor,
                                           recv_topk_ids: torch.Tensor,
                                           recv_topk_weights: torch.Tensor,
                                           num_recv_tokens_per_expert: torch.Tensor,
                                           all_tokens: int):
    """Returns (grouped_x, grouped_x_scale, route_weights, m_indices, output_index)."""
    if not (recv_x.is_cuda and recv_x_scale.is_cuda and recv_topk_ids.is_cuda
            and recv_topk_weights.is_cuda and num_recv_tokens_per_expert.is_cuda):
        raise RuntimeError("DeepEP preprocess tensors must be CUDA/HIP tensors")
    if recv_x.dtype != torch.float8_e4m3fn:
        raise RuntimeError("DeepEP preprocess expects FP8 E4M3 recv_x")
    if recv_x_scale.dtype != torch.float32 or recv_topk_weights.dtype != torch.float32:
        raise RuntimeError("DeepEP preprocess scales and weights must be FP32")
    if recv_topk_ids.dtype not in (torch.int64, torch.int32):
        raise RuntimeError("DeepEP preprocess topk ids must be int64 or int32")
    if num_recv_tokens_per_expert.dtype != torch.int32:
        raise RuntimeError("num_recv_tokens_per_expert must be int32")
    if not (recv_x.is_contiguous() and recv_x_scale.is_contiguous()
            and recv_topk_ids.is_contiguous() and recv_topk_weights.is_contiguous()
            and num_recv_tokens_per_expert.is_contiguous()):
        raise RuntimeError("DeepEP preprocess tensors must be contiguous")
    if recv_x.dim() != 2:
        raise RuntimeError("recv_x must be [tokens, hidden]")
    if recv_topk_ids.dim() != 2 or recv_topk_weights.dim() != 2:
        raise RuntimeError("topk ids/weights must be [tokens, topk]")
    if recv_topk_ids.shape != recv_topk_weights.shape:
        raise RuntimeError("topk ids/weights shape mismatch")
    if recv_topk_ids.size(0) != recv_x.size(0):
        raise RuntimeError("topk rows must match recv_x")
    if recv_x_scale.numel() != recv_x.size(0):
        raise RuntimeError("channelwise recv_x_scale must have one value per received token")
    if all_tokens < 0:
        raise RuntimeError("all_tokens must be non-negative")
    rows = max(int(all_tokens), 1)
    hidden = recv_x.size(1)
    recv_rows = recv_x.size(0)
    topk = recv_topk_ids.size(1)
    num_experts = num_recv_tokens_per_expert.numel()
    dev = recv_x.device
    grouped_x = torch.empty((rows, hidden), dtype=torch.float8_e4m3fn, device=dev)
    grouped_x_scale = torch.empty((rows,), dtype=torch.float32, device=dev)
    route_weights = torch.zeros((rows,), dtype=torch.float32, device=dev)
    m_indices = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    output_index = torch.full((recv_rows, topk), -1, dtype=torch.int32, device=dev)
    lib = _capi.load()
    ws_bytes = ctypes.c_int64()
    _capi.check(lib.mmoe_deepep_preprocess_workspace_bytes(recv_rows, topk, num_experts, rows,
                                                           ctypes.byref(ws_bytes)),
                "deepep_deepgemm_preprocess_channelwise")
    ws = torch.empty((max(ws_bytes.value, 1),), dtype=torch.int8, device=dev)
    _capi.check(lib.mmoe_deepep_preprocess_channelwise(
        grouped_x.data_ptr(), grouped_x_scale.data_ptr(), route_weights.data_ptr(),
        m_indices.data_ptr(), output_index.data_ptr(), recv_x.data_ptr(),
        recv_x_scale.data_ptr(), recv_topk_ids.data_ptr(), recv_topk_weights.data_ptr(),
        num_recv_tokens_per_expert.data_ptr(), rows, recv_rows, topk, hidden, num_experts,
        1 if recv_topk_ids.dtype == torch.int64 else 0, ws.data_ptr(), ws_bytes.value,
        _stream_handle()), "deepep_deepgemm_preprocess_channelwise")
    return grouped_x, grouped_x_scale, route_weights, m_indices, output_index


def deepep_deepgemm_postprocess_channelwise(recv_y: torch.Tensor, l2_out: torch.Tensor,
                                            recv_topk_ids: torch.Tensor,
                                            recv_topk_weights: torch.Tensor,
                                            output_index: torch.Tensor,
                                            apply_topk_weights: bool = False):
    """recv_y[t] = bf16(sum over valid slots of l2_out[output_index[t,s]] (x w if asked))."""
    if not (recv_y.is_cuda and l2_out.is_cuda and recv_topk_ids.is_cuda
            and recv_topk_weights.is_cuda and output_index.is_cuda):
        raise RuntimeError("DeepEP postprocess tensors must be CUDA/HIP tensors")
    if recv_y.dtype != torch.bfloat16 or l2_out.dtype != torch.bfloat16:
        raise RuntimeError("DeepEP postprocess expects BF16 tensors")
    if recv_topk_ids.dtype not in (torch.int64, torch.int32):
        raise RuntimeError("DeepEP postprocess topk ids must be int64 or int32")
    if recv_topk_weights.dtype != torch.float32:
        raise RuntimeError("DeepEP postprocess topk weights must be FP32")
    if output_index.dtype != torch.int32:
        raise RuntimeError("output_index must be int32")
    if not (recv_y.is_contiguous() and l2_out.is_contiguous() and recv_topk_ids.is_contiguous()
            and recv_topk_weights.is_contiguous() and output_index.is_contiguous()):
        raise RuntimeError("DeepEP postprocess tensors must be contiguous")
    if recv_y.dim() != 2 or l2_out.dim() != 2:
        raise RuntimeError("recv_y/l2_out must be 2D")
    if recv_topk_ids.dim() != 2 or recv_topk_weights.dim() != 2 or output_index.dim() != 2:
        raise RuntimeError("topk ids/weights/output_index must be 2D")
    if recv_topk_ids.shape != recv_topk_weights.shape or recv_topk_ids.shape != output_index.shape:
        raise RuntimeError("topk ids/weights/output_index shape mismatch")
    if recv_y.size(0) != recv_topk_ids.size(0):
        raise RuntimeError("recv_y rows mismatch")
    if recv_y.size(1) != l2_out.size(1):
        raise RuntimeError("hidden size mismatch")
    _capi.check(_capi.load().mmoe_deepep_postprocess_channelwise(
        recv_y.data_ptr(), l2_out.data_ptr(), recv_topk_ids.data_ptr(),
        recv_topk_weights.data_ptr(), output_index.data_ptr(), recv_y.size(0),
        recv_topk_ids.size(1), recv_y.size(1), 1 if recv_topk_ids.dtype == torch.int64 else 0,
        1 if apply_topk_weights else 0, _stream_handle()),
        "deepep_deepgemm_postprocess_channelwise")


# ---------------------------------------------------------------------------------------
# the layer (megamoe/__init__.py:328-452; csrc/apis/mega_dcu.hpp:338-518)
# ---------------------------------------------------------------------------------------
def _validate_layer_tensors(y, l1_weights, l2_weights, stats, sym_buffer, recipe, activation):
    """The TORCH_CHECKs of fp8_mega_moe_impl (csrc/apis/mega_dcu.hpp:355-433), same texts."""
    rm, rn, rk = recipe
    if not (rm == 1 and rn == 1 and rk == 32):
        raise RuntimeError("DCU W8A8 MegaMoE expects recipe=(1,1,32)")
    if activation != "swiglu":
        raise RuntimeError("DCU W8A8 MegaMoE supports swiglu only")
    if y.dtype != torch.bfloat16:
        raise RuntimeError("y must be BF16")
    if not y.is_cuda or not y.is_contiguous():
        raise RuntimeError("y must be a contiguous CUDA/HIP tensor")
    if sym_buffer.buffer is None or sym_buffer.buffer.dtype != torch.int8:
        raise RuntimeError("sym_buffer must be int8")
    rs = sym_buffer.route_scratch
    if rs is None or not rs.is_cuda:
        raise RuntimeError("route_scratch must be CUDA/HIP memory")
    if rs.dtype != torch.int8:
        raise RuntimeError("route_scratch must be int8")
    if not rs.is_contiguous():
        raise RuntimeError("route_scratch must be contiguous")
    w1, sw1 = l1_weights
    w2, sw2 = l2_weights
    if w1.dtype != torch.float8_e4m3fn:
        raise RuntimeError("DCU MegaMoE expects FP8 E4M3 L1 weights")
    if w2.dtype != torch.float8_e4m3fn:
        raise RuntimeError("DCU MegaMoE expects FP8 E4M3 L2 weights")
    if sw1.dtype != torch.float32 or sw2.dtype != torch.float32:
        raise RuntimeError("DCU MegaMoE expects FP32 channelwise weight scales")
    if w1.dim() != 3 or w2.dim() != 3:
        raise RuntimeError("weights must be grouped 3D tensors")
    if sw1.dim() != 2 or sw2.dim() != 2:
        raise RuntimeError("weight scales must be [expert,row]")
    for t in (w1, sw1, w2, sw2):
        if not t.is_cuda or not t.is_contiguous():
            raise RuntimeError("weights and scales must be contiguous CUDA/HIP tensors")
    num_experts_per_rank = w1.size(0)
    hidden = y.size(1)
    if sw1.size(1) % 2 != 0:
        raise RuntimeError("invalid L1 scale shape")
    inter = sw1.size(1) // 2
    if sym_buffer.num_experts != num_experts_per_rank:
        raise RuntimeError("invalid expert count")
    if (2 * inter) % 16 or hidden % 16 or inter % 16:
        raise RuntimeError("DCU MegaMoE Marlin weights require rows and K divisible by 16")
    if w1.size(1) != 2 * inter // 16 or w1.size(2) != hidden * 16:
        raise RuntimeError("invalid Marlin L1 weight shape, expected [expert, rows/16, K*16]")
    if w2.size(1) != hidden // 16 or w2.size(2) != inter * 16:
        raise RuntimeError("invalid Marlin L2 weight shape, expected [expert, rows/16, K*16]")
    if sw1.size(0) != num_experts_per_rank or sw1.size(1) != 2 * inter:
        raise RuntimeError("invalid L1 scale shape")
    if sw2.size(0) != num_experts_per_rank or sw2.size(1) != hidden:
        raise RuntimeError("invalid L2 scale shape")
    if y.size(0) > sym_buffer.num_max_tokens_per_rank:
        raise RuntimeError("too many tokens")
    if hidden != sym_buffer.hidden or inter != sym_buffer.intermediate_hidden:
        raise RuntimeError("sym_buffer is too small for the requested DCU MegaMoE capacity")
    if stats is not None:
        if stats.dtype != torch.int32:
            raise RuntimeError("stats must be int32")
        if stats.numel() != num_experts_per_rank:
            raise RuntimeError("stats must have num_experts_per_rank elements")
        if not stats.is_cuda or not stats.is_contiguous():
            raise RuntimeError("stats must be a contiguous CUDA/HIP tensor")
    return hidden, inter


def _forward_args(y, l1_weights, l2_weights, stats, sym_buffer, activation_clamp, schedule,
                  runtime_num_tokens=None) -> _capi.ForwardArgs:
    w1, sw1 = l1_weights
    w2, sw2 = l2_weights
    clamp = math.inf if activation_clamp is None else float(activation_clamp)
    args = _capi.ForwardArgs(
        y=y.data_ptr(), x=sym_buffer.x.data_ptr(), x_sf=sym_buffer.x_sf.data_ptr(),
        topk_idx=sym_buffer.topk_idx.data_ptr(), topk_weights=sym_buffer.topk_weights.data_ptr(),
        w1=w1.data_ptr(), w1_sf=sw1.data_ptr(), w2=w2.data_ptr(), w2_sf=sw2.data_ptr(),
        stats=_ptr(stats), route_scratch=sym_buffer.route_scratch.data_ptr(),
        route_scratch_bytes=sym_buffer.route_scratch.numel(),
        sym_buffer_bytes=sym_buffer.buffer.numel(),
        runtime_num_tokens=_ptr(runtime_num_tokens),
        num_tokens=y.size(0), num_max_tokens=sym_buffer.num_max_tokens_per_rank,
        num_experts=sym_buffer.num_experts, num_topk=sym_buffer.num_topk,
        hidden=sym_buffer.hidden, intermediate=sym_buffer.intermediate_hidden,
        activation_clamp=clamp, schedule=schedule, debug_flags=0)
    return args


_DEBUG_CHECK_ENV = "MEGAMOE_DEBUG_CHECK"


def last_call_status(sym_buffer: SymmBuffer) -> int:
    """Status of the last layer call on ``sym_buffer`` (synchronises the current stream): 0 when
    its output is valid, else the number of bounded waits of the one-launch decode pipeline that
    ran out (``mmoe_scratch_status``). Such a wait only runs out when other work holds the GPU's
    CUs far longer than any of the layer's own items; the layer then still ends, but ``y`` is not
    valid."""
    out = torch.empty((1,), dtype=torch.int32, device=sym_buffer.route_scratch.device)
    _capi.check(_capi.load().mmoe_scratch_status(sym_buffer.route_scratch.data_ptr(),
                                                 ctypes.cast(out.data_ptr(),
                                                             ctypes.POINTER(ctypes.c_int32)),
                                                 _stream_handle()), "last_call_status")
    return int(out.item())


def _check_status(sym_buffer: SymmBuffer) -> None:
    """MEGAMOE_DEBUG_CHECK=1: after an eager call, synchronise and raise RuntimeError when the
    call's status reports bounded waits that ran out (off by default: it costs a host sync)."""
    if os.getenv(_DEBUG_CHECK_ENV, "0").strip().lower() not in ("1", "true", "yes", "on"):
        return
    if _is_current_stream_capturing():
        return
    failed = last_call_status(sym_buffer)
    if failed != 0:
        raise RuntimeError(f"DCU MegaMoE decode pipeline: {failed} bounded waits ran out (the "
                           "GPU's CUs were held by other work); the layer output is not valid")


def _launch_layer(y, l1_weights, l2_weights, stats, sym_buffer, activation_clamp, schedule,
                  runtime_num_tokens=None, entry="mmoe_forward"):
    args = _forward_args(y, l1_weights, l2_weights, stats, sym_buffer, activation_clamp, schedule,
                         runtime_num_tokens)
    fn = getattr(_capi.load(), entry)
    _capi.check(fn(ctypes.byref(args), _stream_handle()), "fp8_mega_moe")
    if entry == "mmoe_forward":
        _check_status(sym_buffer)


class LayerCall:
    """A prepared layer call whose stages can be launched one at a time (profiling, stage
    parity). ``run(first, last)`` launches stages [first, last] on the current stream:
    0 route, 1 GEMM1 with the fused SwiGLU x weight, 2 requant, 3 GEMM2, 4 combine."""

    STAGES = ("route", "gemm1_swiglu", "requant", "gemm2", "combine")

    def __init__(self, y, l1_weights, l2_weights, sym_buffer, activation_clamp=None,
                 staged: Optional[bool] = None, stats=None):
        _validate_layer_tensors(y, l1_weights, l2_weights, stats, sym_buffer, (1, 1, 32),
                                "swiglu")
        if staged is None:
            schedule = _schedule_for_mode(sym_buffer._large_opt_3stage_mode)
        else:
            schedule = _capi.MMOE_SCHEDULE_STAGED if staged else _capi.MMOE_SCHEDULE_PERSISTENT
        self._keep = (y, l1_weights, l2_weights, sym_buffer, stats)
        self.args = _forward_args(y, l1_weights, l2_weights, stats, sym_buffer,
                                  activation_clamp, schedule)

    def run(self, first: int = 0, last: int = 4) -> None:
        _capi.check(_capi.load().mmoe_forward_stages(ctypes.byref(self.args), first, last,
                                                     _stream_handle()), "fp8_mega_moe")


def fp8_mega_moe(
    y: torch.Tensor,
    l1_weights: Tuple[torch.Tensor, torch.Tensor],
    l2_weights: Tuple[torch.Tensor, torch.Tensor],
    sym_buffer: SymmBuffer,
    cumulative_local_expert_recv_stats: Optional[torch.Tensor] = None,
    recipe: Tuple[int, int, int] = (1, 1, 32),
    activation: str = "swiglu",
    activation_clamp: Optional[float] = None,
    fast_math: bool = True,
    big_fused_cuda_graph: bool = False,
    stages_fused_cuda_graph: bool = False,
    dispatch_num_tokens: Optional[int] = None,
):
    """The layer; writes ``y`` in place and returns None (megamoe/__init__.py:328-449).

    Schedules: the reference's persistent small-T kernel and staged large-T path become two
    tile engines of one persistent grouped GEMM, chosen per expert on the device from its
    routed rows (the row counts exist only there). ``MEGAMOE_DCU_USE_LARGE_OPT_3STAGE``
    keeps its meaning: ``auto`` (default) = the streaming engine for every expert when the
    call's token count is at most ``MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD`` (default
    128, the reference's persistent-path rule), else the per-expert choice; ``1``/``3stage`` =
    tile engine everywhere; ``0``/``off`` = streaming engine everywhere. Every choice computes
    the same layer, bit for bit. Graph modes use the mode alone (the token count of a replay is
    only known on the device). Flags, ``dispatch_num_tokens`` and graph-mode rules are
    validated exactly as in the reference. Graph modes read the device token count ``sym_buffer.cuda_graph_num_tokens`` at
    run time; the launch sequence allocates nothing and never synchronises, so it captures."""
    call_y = y
    if big_fused_cuda_graph and stages_fused_cuda_graph:
        raise ValueError("choose only one of big_fused_cuda_graph or stages_fused_cuda_graph")
    graph_mode = big_fused_cuda_graph or stages_fused_cuda_graph
    mode = getattr(sym_buffer, "_large_opt_3stage_mode", None) or _large_opt_3stage_mode()
    threshold = getattr(sym_buffer, "_large_opt_3stage_threshold", None)
    if threshold is None:
        threshold = _large_opt_3stage_threshold()
    runtime_tokens = None
    # fast_math=False is refused where the reference refuses it: the staged paths check it
    # first (megamoe/large_opt.py:381, :526), the persistent kernel after the tensor checks
    # (csrc/kernels/mega_moe_fused_hip.cu:87-91)
    persistent_no_fast_math = False
    if graph_mode:
        graph_max_tokens = int(sym_buffer.cuda_graph_max_tokens_per_rank)
        capture_rows = int(y.size(0))
        if capture_rows < graph_max_tokens:
            raise ValueError(
                "CUDA graph mode requires y to have at least "
                f"{graph_max_tokens} rows; pass a fixed graph-bucket output "
                "buffer and consume only the valid prefix")
        if cumulative_local_expert_recv_stats is not None:
            raise ValueError("CUDA graph mode does not support cumulative_local_expert_recv_stats")
        if stages_fused_cuda_graph and mode == "off":
            raise RuntimeError("stages_fused_cuda_graph=True requires "
                               "MEGAMOE_DCU_USE_LARGE_OPT_3STAGE=auto or 1")
        if stages_fused_cuda_graph and not fast_math:
            raise RuntimeError("large-opt DCU MegaMoE graph path requires fast_math")
        persistent_no_fast_math = not fast_math
        call_y = y[:graph_max_tokens] if capture_rows != graph_max_tokens else y
        runtime_tokens = sym_buffer.cuda_graph_num_tokens
        schedule = _schedule_for_mode(mode)
    else:
        if _is_current_stream_capturing():
            raise RuntimeError(
                "DCU MegaMoE CUDA Graph capture requires an explicit graph mode: "
                "pass big_fused_cuda_graph=True for the persistent fused path or "
                "stages_fused_cuda_graph=True for the staged K1/K2/K3 path. "
                "Capturing the eager auto-dispatch path is not graph-bucket safe.")
        dispatch_tokens = int(y.size(0)) if dispatch_num_tokens is None else int(dispatch_num_tokens)
        if dispatch_tokens < 0 or dispatch_tokens > int(sym_buffer.num_max_tokens_per_rank):
            raise ValueError("dispatch_num_tokens must be in "
                             f"0..{int(sym_buffer.num_max_tokens_per_rank)}")
        staged = mode == "force" or (mode == "auto" and dispatch_tokens > threshold)
        if staged and not fast_math:
            raise RuntimeError("large-opt DCU MegaMoE path requires fast_math")
        persistent_no_fast_math = not fast_math
        schedule = _eager_schedule(mode, threshold, dispatch_tokens)
    _validate_layer_tensors(call_y, l1_weights, l2_weights, cumulative_local_expert_recv_stats,
                            sym_buffer, recipe, activation)
    if persistent_no_fast_math:
        raise RuntimeError("DCU MegaMoE W8A8 channelwise persistent fused path requires fast_math")
    _launch_layer(call_y, l1_weights, l2_weights, cumulative_local_expert_recv_stats, sym_buffer,
                  activation_clamp, schedule, runtime_tokens)


fp8_w8a8_mega_moe = fp8_mega_moe


def route_only(y_rows: int, l1_weights, l2_weights, sym_buffer: SymmBuffer,
               cumulative_local_expert_recv_stats: Optional[torch.Tensor] = None) -> None:
    """Run only the routing stage of the layer for ``y_rows`` tokens (stage parity): fills
    counts/offsets/output_index/row tables readable through ``sym_buffer.scratch_view``."""
    y = torch.empty((y_rows, sym_buffer.hidden), dtype=torch.bfloat16, device="cuda")
    _validate_layer_tensors(y, l1_weights, l2_weights, cumulative_local_expert_recv_stats,
                            sym_buffer, (1, 1, 32), "swiglu")
    _launch_layer(y, l1_weights, l2_weights, cumulative_local_expert_recv_stats, sym_buffer,
                  None, _capi.MMOE_SCHEDULE_AUTO, None, entry="mmoe_route")


__all__ = [
    "SymmBuffer",
    "cast_to_fp8_channelwise",
    "cast_grouped_weight_to_fp8_channelwise",
    "weight8bit_nt_kpack2_marlin",
    "get_mega_moe_hip_build_config",
    "get_symm_buffer_for_mega_moe",
    "transform_fp8_weights_for_mega_moe",
    "deepep_deepgemm_preprocess_channelwise",
    "deepep_deepgemm_postprocess_channelwise",
    "fp8_mega_moe",
    "fp8_w8a8_mega_moe",
    "last_call_status",
]

__version__ = "0.1"
