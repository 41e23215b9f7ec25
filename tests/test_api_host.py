"""Host-side logic of the Python API mirror (no GPU): the schedule knobs of
MEGAMOE_DCU_USE_LARGE_OPT_3STAGE and MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD
(megamoe/__init__.py:19-43, :408-428 of the reference)."""
import pytest

from deepgemm_amd import megamoe as mm
from deepgemm_amd.megamoe import _capi


@pytest.mark.parametrize("value,mode", [
    ("auto", "auto"), ("threshold", "auto"), ("ADAPTIVE", "auto"), (" auto ", "auto"),
    ("1", "force"), ("true", "force"), ("3stage", "force"), ("large_opt", "force"),
    ("0", "off"), ("off", "off"), ("anything-else", "off"),
])
def test_mode_env_values(monkeypatch, value, mode):
    monkeypatch.setenv("MEGAMOE_DCU_USE_LARGE_OPT_3STAGE", value)
    assert mm._large_opt_3stage_mode() == mode


def test_mode_default_is_auto(monkeypatch):
    monkeypatch.delenv("MEGAMOE_DCU_USE_LARGE_OPT_3STAGE", raising=False)
    assert mm._large_opt_3stage_mode() == "auto"


def test_threshold_env(monkeypatch):
    monkeypatch.delenv("MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD", raising=False)
    assert mm._large_opt_3stage_threshold() == 128
    monkeypatch.setenv("MEGAMOE_DCU_LARGE_OPT_3STAGE_TOKEN_THRESHOLD", "4096")
    assert mm._large_opt_3stage_threshold() == 4096


def test_threshold_selects_the_persistent_schedule_in_auto_mode():
    """auto: tokens <= threshold -> the streaming engine for every expert (the reference's
    persistent fused path); tokens > threshold (strict) -> the per-expert choice (its staged
    path). force/off ignore the threshold."""
    P, A, S = _capi.MMOE_SCHEDULE_PERSISTENT, _capi.MMOE_SCHEDULE_AUTO, _capi.MMOE_SCHEDULE_STAGED
    assert mm._eager_schedule("auto", 128, 0) == P
    assert mm._eager_schedule("auto", 128, 128) == P
    assert mm._eager_schedule("auto", 128, 129) == A
    assert mm._eager_schedule("auto", 0, 1) == A
    assert mm._eager_schedule("auto", 4096, 1024) == P
    for tokens in (0, 128, 129, 100000):
        assert mm._eager_schedule("force", 128, tokens) == S
        assert mm._eager_schedule("off", 128, tokens) == P


def test_graph_modes_use_the_mode_alone():
    assert mm._schedule_for_mode("auto") == _capi.MMOE_SCHEDULE_AUTO
    assert mm._schedule_for_mode("force") == _capi.MMOE_SCHEDULE_STAGED
    assert mm._schedule_for_mode("off") == _capi.MMOE_SCHEDULE_PERSISTENT


def test_removed_helpers_stay_removed():
    assert not hasattr(mm, "_large_opt_3stage_selected")
    assert not hasattr(mm, "_group_rank")
