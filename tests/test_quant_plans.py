"""The compressed-tensors dispatch decisions (no vLLM, no GPU): which dense schemes and MoE methods go to libr9k,
R9K_DISABLE's families and R9K_NVFP4's modes, as the reference's quant/ct.py get_scheme / get_quant_method
branches decide them (r9700_vllm/quant/ct.py:375-402, :417-428)."""
import pytest

from r9700_vllm.quant import ct


@pytest.mark.parametrize("kind, disabled, mode, want", [
    ("mxfp4", set(), None, "mxfp4"),
    ("mxfp4", {"linear"}, None, None),
    ("mxfp4", {"nvfp4", "moe"}, None, "mxfp4"),
    ("nvfp4", set(), "", "nvfp4-native"),
    ("nvfp4", set(), "NATIVE", "nvfp4-native"),
    ("nvfp4", set(), "mxfp4", "nvfp4-mxfp4"),
    ("nvfp4", {"nvfp4"}, "native", None),
    ("nvfp4", {"linear"}, "mxfp4", "nvfp4-mxfp4"),
    ("fp8", set(), None, None),
    (None, set(), None, None),
])
def test_dense_plan(kind, disabled, mode, want):
    assert ct.dense_plan(kind, disabled, mode) == want


@pytest.mark.parametrize("kind, cutlass, disabled, want", [
    ("nvfp4", False, set(), "nvfp4"),
    ("nvfp4", True, set(), "nvfp4"),           # decided from the checkpoint before any stock method exists
    ("nvfp4", False, {"nvfp4"}, None),
    ("nvfp4", False, {"moe"}, "nvfp4"),
    ("mxfp4", False, set(), "mxfp4"),
    ("mxfp4", True, set(), None),              # the stock method's CUTLASS path is kept
    ("mxfp4", False, {"moe"}, None),
    ("mxfp4", False, {"nvfp4", "linear"}, "mxfp4"),
    (None, False, set(), None),
])
def test_moe_plan(kind, cutlass, disabled, want):
    assert ct.moe_plan(kind, cutlass, disabled) == want


def test_plans_read_the_environment(monkeypatch):
    monkeypatch.setenv("R9K_DISABLE", " moe , linear")
    monkeypatch.setenv("R9K_NVFP4", "mxfp4")
    assert ct.dense_plan("mxfp4") is None
    assert ct.dense_plan("nvfp4") == "nvfp4-mxfp4"
    assert ct.moe_plan("mxfp4") is None
    assert ct.moe_plan("nvfp4") == "nvfp4"
    monkeypatch.delenv("R9K_DISABLE")
    monkeypatch.delenv("R9K_NVFP4")
    assert ct.dense_plan("nvfp4") == "nvfp4-native"
    assert ct.moe_plan("mxfp4") == "mxfp4"
