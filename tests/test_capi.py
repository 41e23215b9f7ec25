"""C-ABI checks that need no GPU: the library loads, exports every symbol include/*.h declares,
and the host-side validation returns the reference's checks as status codes."""
import ctypes
import math
import os
import re

import pytest

from deepgemm_amd.megamoe import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "megamoe_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mmoe_[a-z0-9_]+)\s*\(", src)))


def _header_prototypes():
    src = open(os.path.join(ROOT, "include", "megamoe_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    protos = {}
    for m in re.finditer(r"\b(mmoe_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        if params == ["void"]:
            params = []
        protos[m.group(1)] = params
    return protos


def test_bindings_match_header_arity():
    protos = _header_prototypes()
    assert set(protos) == set(_header_functions())
    for name, params in protos.items():
        assert len(_capi.SIGNATURES[name][1]) == len(params), name


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    names = _header_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
        assert name in _capi.SIGNATURES, f"{name} not bound in _capi.SIGNATURES"


def test_struct_layouts_match_c_compiler(tmp_path):
    """sizeof/offsetof of every header struct as gcc lays it out == the ctypes mirrors (and the
    header's counter count == the binding's)."""
    structs = {"mmoe_forward_args": _capi.ForwardArgs, "mmoe_symm_layout": _capi.SymmLayout,
               "mmoe_scratch_layout": _capi.ScratchLayout}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "megamoe_hip.h"',
             'int main(void) {']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append('printf("MMOE_PIPE_INTS %d\\n", MMOE_PIPE_INTS);')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    import subprocess
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = dict(line.rsplit(" ", 1) for line in
               subprocess.run([str(exe)], capture_output=True, text=True,
                              check=True).stdout.split("\n") if line)
    assert int(out["MMOE_PIPE_INTS"]) == _capi.MMOE_PIPE_INTS
    for cname, py in structs.items():
        assert int(out[cname]) == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(py, fname).offset, f"{cname}.{fname}"


def test_token_alignment_and_build_config():
    lib = _capi.load()
    assert lib.mmoe_token_alignment() == 384
    import json
    cfg = json.loads(lib.mmoe_build_config().decode())
    assert cfg["operator"] == "fp8_w8a8_mega_moe" and cfg["arch"] == "gfx950"


def test_layouts():
    lib = _capi.load()
    sl = _capi.SymmLayout()
    assert lib.mmoe_symm_buffer_layout(1, 32, 384, 6, 4096, 2048, ctypes.byref(sl)) == 0
    assert sl.x_offset % 256 == 0 and sl.x_sf_offset >= sl.x_offset + 384 * 4096
    assert sl.topk_weights_offset >= sl.topk_idx_offset + 384 * 6 * 8
    assert sl.total_bytes >= sl.topk_weights_offset + 384 * 6 * 4
    nb = ctypes.c_int64()
    assert lib.mmoe_route_scratch_bytes(1, 32, 384, 6, 4096, 2048, ctypes.byref(nb)) == 0
    lay = _capi.ScratchLayout()
    assert lib.mmoe_route_scratch_layout(1, 32, 384, 6, 4096, 2048, ctypes.byref(lay)) == 0
    assert lay.total_bytes == nb.value
    assert lay.row_capacity >= 384 * 6
    offs = [lay.pipe_offset, lay.meta_offset, lay.counts_offset, lay.offsets_offset,
            lay.chunk_counts_offset, lay.output_index_offset, lay.row_token_offset,
            lay.row_weight_offset, lay.m_indices_offset, lay.act_scale_offset, lay.amax_offset,
            lay.y_offset, lay.act_offset, lay.part_offset, lay.row_dest_offset, lay.sched_offset,
            lay.pmax_offset]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert lay.part_offset + lay.row_capacity * 4096 * 2 <= lay.total_bytes


@pytest.mark.parametrize("shape", [
    (1, 32, 384, 6, 4096, 2048), (1, 32, 1152, 6, 4096, 2048), (1, 32, 200, 6, 4096, 2048),
    (1, 4, 16, 3, 256, 128), (1, 255, 300, 6, 256, 128), (1, 64, 2000, 6, 512, 256),
    (1, 1024, 8, 16, 128, 128), (1, 32, 0, 6, 4096, 2048),
])
def test_pipe_counters_and_status_sit_at_fixed_offsets(shape):
    """The decode pipeline's counters (which must read zero when a call starts; each call leaves
    them zero) are at offset 0 in every layout, and meta right after them, so one scratch can
    serve calls of any shape in turn without handing a call another section's bytes as its
    counters, and the status word is found without the shape."""
    lib = _capi.load()
    lay = _capi.ScratchLayout()
    assert lib.mmoe_route_scratch_layout(*shape, ctypes.byref(lay)) == 0
    assert lay.pipe_offset == 0
    assert lay.meta_offset == _capi.MMOE_PIPE_INTS * 4
    assert lay.meta_offset + 3 * 4 == _capi.MMOE_SCRATCH_STATUS_OFFSET
    others = [getattr(lay, f) for f, _ in _capi.ScratchLayout._fields_
              if f.endswith("_offset") and f not in ("pipe_offset", "meta_offset")]
    assert min(others) >= lay.meta_offset + 16 * 4


def test_scratch_status_rejects_null_output():
    lib = _capi.load()
    assert lib.mmoe_scratch_status(None, None, None) == -1


def test_debug_flags_are_validated():
    lib = _capi.load()
    assert lib.mmoe_forward(ctypes.byref(_args(debug_flags=2)), None) == -14


@pytest.mark.parametrize("args,code", [
    ((0, 32, 384, 6, 4096, 2048), -2),
    ((3, 32, 384, 6, 4096, 2048), -3),
    ((1, 32, 384, 6, 0, 2048), -4),
    ((1, 32, 384, 0, 4096, 2048), -10),
    ((1, 32, 384, 17, 4096, 2048), -10),
    # routed rows are counted in 32-bit integers by the kernels: at most 2^30 of them
    ((1, 32, (1 << 30) // 6 + 1, 6, 4096, 2048), -9),
])
def test_layout_validation_codes(args, code):
    lib = _capi.load()
    nb = ctypes.c_int64()
    assert lib.mmoe_route_scratch_bytes(*args, ctypes.byref(nb)) == code
    assert _capi.status_string(code) != "unknown status"


def _args(**kw):
    base = dict(num_tokens=4, num_max_tokens=384, num_experts=32, num_topk=6, hidden=4096,
                intermediate=2048, activation_clamp=math.inf, schedule=0, debug_flags=0,
                route_scratch_bytes=1 << 40, sym_buffer_bytes=1 << 40)
    base.update(kw)
    a = _capi.ForwardArgs()
    for k, v in base.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(num_tokens=385), -6),                 # too many tokens
    (dict(route_scratch_bytes=1024), -8),       # scratch too small
    (dict(sym_buffer_bytes=1024), -7),          # sym buffer too small
    (dict(hidden=4104), -5),                    # not divisible by 16
    (dict(hidden=4112), -9),                    # not a multiple of 128
    (dict(schedule=7), -11),
    (dict(num_topk=0), -10),
    (dict(), -1),                               # null data pointers
])
def test_forward_validation_without_gpu(kw, code):
    lib = _capi.load()
    assert lib.mmoe_forward(ctypes.byref(_args(**kw)), None) == code


def test_forward_zero_tokens_is_a_noop():
    lib = _capi.load()
    assert lib.mmoe_forward(ctypes.byref(_args(num_tokens=0)), None) == 0


def test_check_raises_runtime_error():
    with pytest.raises(RuntimeError, match="too many tokens"):
        _capi.check(-6, "fp8_mega_moe")


def test_stale_library_is_refused(monkeypatch):
    """A library whose recorded source hash differs from the tree's raises instead of loading
    (a kernel edit without a rebuild must not run the old binary)."""
    from deepgemm_amd import build as hip_build

    _capi.check_fresh()  # the tree's library is fresh
    monkeypatch.setattr(hip_build, "source_hash", lambda: "0" * 64)
    with pytest.raises(OSError, match="stale"):
        _capi.check_fresh()
