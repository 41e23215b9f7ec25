"""The bench's metric definitions, on the CPU: the algorithmic byte counts that its rooflines
divide by (the reference's formula, tests/test_mega_moe_dcu.py:352-366, split by kernel) and
its refusal of more than one GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

H, I = 4096, 2048


def test_layer_bytes_known_answer():
    # c1's routing (785 rows over all 32 local experts): the figure its HBM roofline is quoted on
    assert bench.algorithmic_bytes(785, 32)["layer"] == 819_225_804


def test_layer_bytes_from_first_principles():
    """Weights read once per touched expert (W1 [2I, H] and W2 [H, I] e4m3 plus their f32
    per-row scales); per routed row the x row with its scale, the requantized activation row
    with its scale written and read back, and the bf16 partial row."""
    for rows, touched in ((0, 0), (1, 1), (785, 32), (24_731, 32), (49_152, 28)):
        weights = touched * (2 * I * H + H * I) + touched * (2 * I + H) * 4
        per_row = (H + 4) + 2 * (I + 4) + 2 * H
        assert bench.algorithmic_bytes(rows, touched)["layer"] == weights + rows * per_row
        assert bench.algorithmic_bytes(rows, touched)["pipeline"] == weights + rows * per_row


def test_kernel_split():
    """GEMM1 reads W1, its scales and the x rows and writes y = SwiGLU(h) x w in bf16 [R, I];
    GEMM2 reads W2, its scales and the activation rows and writes the bf16 partial rows."""
    rows, touched = 3_046, 32
    b = bench.algorithmic_bytes(rows, touched)
    assert b["gemm1"] == touched * (2 * I * H + 2 * I * 4) + rows * (H + 4) + rows * I * 2
    assert b["gemm2"] == touched * (H * I + H * 4) + rows * (I + 4) + rows * H * 2
    # the layer counts the activation once written (GEMM1's output side, as the requant's act)
    # and once read (GEMM2's input), with y's bytes not part of it
    assert b["layer"] - b["gemm2"] - (touched * (2 * I * H + 2 * I * 4) + rows * (H + 4)) == rows * (I + 4)


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert res.returncode != 0
    assert "one GPU" in res.stdout + res.stderr
    assert res.stdout.strip() == "" or not res.stdout.lstrip().startswith("{")
