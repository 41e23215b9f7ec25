"""ctypes binding of include/megamoe_hip.h (libmegamoe_hip.so, built for gfx950).

The library is the only compute path: nothing here falls back to another implementation. If
the shared library is missing it is built in-tree with hipcc; if that fails, loading raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libmegamoe_hip.so")

MMOE_OK = 0
MMOE_ERR_STATIC_SCRATCH = -15
MMOE_STATIC_SCRATCH_BYTES = 128 << 20
MMOE_PIPE_INTS = 4928
MMOE_SCRATCH_STATUS_OFFSET = MMOE_PIPE_INTS * 4 + 3 * 4
MMOE_DEBUG_NO_WAIT = 1
MMOE_STAGE_PIPELINE = 5
MMOE_SCHEDULE_AUTO = 0
MMOE_SCHEDULE_PERSISTENT = 1
MMOE_SCHEDULE_STAGED = 2

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_p = ctypes.c_void_p


class SymmLayout(ctypes.Structure):
    _fields_ = [
        ("total_bytes", c_i64),
        ("runtime_num_tokens_offset", c_i64),
        ("x_offset", c_i64),
        ("x_sf_offset", c_i64),
        ("topk_idx_offset", c_i64),
        ("topk_weights_offset", c_i64),
    ]


class ScratchLayout(ctypes.Structure):
    _fields_ = [
        ("total_bytes", c_i64),
        ("row_capacity", c_i64),
        ("num_chunks", c_i64),
        ("counts_offset", c_i64),
        ("offsets_offset", c_i64),
        ("meta_offset", c_i64),
        ("chunk_counts_offset", c_i64),
        ("output_index_offset", c_i64),
        ("row_token_offset", c_i64),
        ("row_weight_offset", c_i64),
        ("m_indices_offset", c_i64),
        ("act_scale_offset", c_i64),
        ("amax_offset", c_i64),
        ("y_offset", c_i64),
        ("act_offset", c_i64),
        ("part_offset", c_i64),
        ("row_dest_offset", c_i64),
        ("sched_offset", c_i64),
        ("pipe_offset", c_i64),
        ("pmax_offset", c_i64),
    ]


class ForwardArgs(ctypes.Structure):
    _fields_ = [
        ("y", c_p),
        ("x", c_p),
        ("x_sf", c_p),
        ("topk_idx", c_p),
        ("topk_weights", c_p),
        ("w1", c_p),
        ("w1_sf", c_p),
        ("w2", c_p),
        ("w2_sf", c_p),
        ("stats", c_p),
        ("route_scratch", c_p),
        ("route_scratch_bytes", c_i64),
        ("sym_buffer_bytes", c_i64),
        ("runtime_num_tokens", c_p),
        ("num_tokens", c_i32),
        ("num_max_tokens", c_i32),
        ("num_experts", c_i32),
        ("num_topk", c_i32),
        ("hidden", c_i32),
        ("intermediate", c_i32),
        ("activation_clamp", ctypes.c_float),
        ("schedule", c_i32),
        ("debug_flags", c_i32),
    ]


# exported symbol -> (restype, argtypes); tests check that this matches the header
SIGNATURES = {
    "mmoe_token_alignment": (ctypes.c_int, []),
    "mmoe_symm_buffer_layout": (ctypes.c_int, [ctypes.c_int] * 6 + [ctypes.POINTER(SymmLayout)]),
    "mmoe_route_scratch_bytes": (ctypes.c_int, [ctypes.c_int] * 6 + [ctypes.POINTER(c_i64)]),
    "mmoe_route_scratch_layout": (ctypes.c_int,
                                  [ctypes.c_int] * 6 + [ctypes.POINTER(ScratchLayout)]),
    "mmoe_build_config": (ctypes.c_char_p, []),
    "mmoe_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mmoe_forward": (ctypes.c_int, [ctypes.POINTER(ForwardArgs), c_p]),
    "mmoe_forward_static": (ctypes.c_int, [ctypes.POINTER(ForwardArgs), c_p]),
    "mmoe_scratch_status": (ctypes.c_int, [c_p, ctypes.POINTER(c_i32), c_p]),
    "mmoe_forward_profile": (ctypes.c_int, [ctypes.POINTER(ForwardArgs), c_p, c_p, ctypes.c_int,
                                            ctypes.POINTER(c_i32), ctypes.POINTER(c_i32)]),
    "mmoe_route": (ctypes.c_int, [ctypes.POINTER(ForwardArgs), c_p]),
    "mmoe_forward_stages": (ctypes.c_int, [ctypes.POINTER(ForwardArgs), ctypes.c_int,
                                           ctypes.c_int, c_p]),
    "mmoe_deepep_preprocess_workspace_bytes": (ctypes.c_int, [ctypes.c_int] * 4
                                               + [ctypes.POINTER(c_i64)]),
    "mmoe_deepep_preprocess_channelwise": (
        ctypes.c_int,
        [c_p] * 10 + [ctypes.c_int] * 6 + [c_p, c_i64, c_p]),
    "mmoe_deepep_postprocess_channelwise": (
        ctypes.c_int, [c_p] * 5 + [ctypes.c_int] * 5 + [c_p]),
    "mmoe_cast_fp8_channelwise": (ctypes.c_int, [c_p, c_p, c_p, c_i64, c_i64, c_p]),
    "mmoe_marlin_pack": (ctypes.c_int, [c_p, c_p, c_i64, c_i64, c_i64, c_p]),
    "mmoe_debug_f32_to_e4m3": (ctypes.c_int, [c_p, c_p, c_i64, c_p]),
}

_lock = threading.Lock()
_lib = None


def _build_library() -> None:
    from .. import build as _build

    _build.build()


def check_fresh(path: str = LIB_PATH) -> None:
    """Raise when the library was built from other sources or flags than those in the tree
    (the hash build() records next to it differs from the tree's), so that a kernel edit
    without a rebuild never runs a stale binary."""
    from .. import build as _build

    if os.path.abspath(path) != os.path.abspath(_build.LIB_PATH):
        return
    try:
        with open(_build.HASH_PATH) as fh:
            built = fh.read().strip()
    except OSError:
        built = None
    if built != _build.source_hash():
        raise OSError(f"{path} is stale: it was not built from the kernel sources in this tree "
                      "(run `python -m deepgemm_amd.build`)")


def load(path: str = LIB_PATH, build_if_missing: bool = True):
    """Load (building once if absent) the gfx950 library and declare every entry point.
    A library that does not match the tree's sources raises (check_fresh)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            if not build_if_missing:
                raise OSError(f"{path} is missing; run `python -m deepgemm_amd.build`")
            _build_library()
        check_fresh(path)
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def status_string(code: int) -> str:
    return load().mmoe_status_string(int(code)).decode()


def check(code: int, what: str = "") -> None:
    """Raise RuntimeError (the reference's TORCH_CHECK type) for a non-zero status."""
    if code != MMOE_OK:
        msg = status_string(code)
        raise RuntimeError(f"{what}: {msg}" if what else msg)
