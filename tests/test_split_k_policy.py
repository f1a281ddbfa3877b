"""Split-K knob of ``awq_fused_gemm`` (CPU only): the override precedence of the reference's
``_select_split_k`` (``vllm/kernels/triton/awq_fused_gemm.py:420-469``), with the expectations
of its guardrail tests (``tests/test_awq_fused_split_k.py:47-75``) and the cases those leave
open (an empty override, the kernel-policy key and its "auto" spellings).

The reference's auto rule (``470-501``) sizes a 16-24-program gfx1151 grid; here "auto" is 0 and
the library plans the partition for the MI355X, so the reference's auto expectations
(``test_awq_fused_split_k.py:78-150``) are not mirrored: every one of them asks for "auto".
"""
from __future__ import annotations

import importlib
from unittest import mock

import pytest

# the package re-exports the function of the same name; the tests need the module
F = importlib.import_module("litevllm_amd.awq_fused_gemm")

KEY = "FASTINFERENCE_AWQ_FUSED_GEMM_SPLIT_K"


@pytest.fixture(autouse=True)
def _clear_snapshot():
    F.set_awq_fused_tuning_config({})
    yield
    F.set_awq_fused_tuning_config({})


# ---- tests/test_awq_fused_split_k.py:47-75 ----
def test_tool_override_integer_forces_value():
    F.set_awq_fused_tuning_config({KEY: "3"}, locked=False)
    assert F._select_split_k(1, 4096, 4096) == 3


def test_tool_override_clamps_below_one():
    F.set_awq_fused_tuning_config({KEY: "0"}, locked=False)
    assert F._select_split_k(1, 65536, 65536) == 1


def test_tool_override_rejects_garbage_and_falls_to_one():
    F.set_awq_fused_tuning_config({KEY: "banana"}, locked=False)
    assert F._select_split_k(1, 65536, 65536) == 1


def test_locked_snapshot_forces_value():
    F.set_awq_fused_tuning_config({KEY: "5"}, locked=True)
    assert F._select_split_k(1, 4096, 4096) == 5


# ---- what the reference's rule gives for the cases its tests leave open ----
def test_empty_tool_override_forces_one():
    """A present but empty override is the tool override (``_tool_override_get`` returns it),
    and ``int("")`` raises, so the reference returns 1, not "auto"."""
    F.set_awq_fused_tuning_config({KEY: ""})
    assert F._select_split_k(1, 4096, 4096) == 1
    F.set_awq_fused_tuning_config({KEY: "  7 "})
    assert F._select_split_k(1, 4096, 4096) == 7


def test_tool_override_beats_policy():
    F.set_awq_fused_tuning_config({KEY: "2"})
    assert F._select_split_k(1, 4096, 4096, policy={"awq_fused_gemm_split_k": 8}) == 2


@pytest.mark.parametrize("raw,want", [(4, 4), ("6", 6), ("0", 1), (-3, 1), ("x", 1), ("", 0), ("auto", 0),
                                      (" AUTO ", 0), (None, 1)])
def test_policy_values(raw, want):
    """``kernel_policy["awq_fused_gemm_split_k"]``: integers clamp to >= 1, unparsable values
    force 1, ``""`` / ``"auto"`` (any case, padded) leave "auto" (0 here).  A present ``None``
    reaches the reference's final lookup as ``str(None)`` and forces 1."""
    assert F._select_split_k(1, 4096, 4096, policy={"awq_fused_gemm_split_k": raw}) == want


def test_policy_sources():
    """The policy comes from ``policy=``, else ``config["kernel_policy"]``, else a dict config
    itself, else ``config.kernel_policy`` (``awq_fused_gemm.py:80-94``)."""
    assert F._select_split_k(1, 8, 8, config={"kernel_policy": {"awq_fused_gemm_split_k": 3}}) == 3
    assert F._select_split_k(1, 8, 8, config={"awq_fused_gemm_split_k": 5}) == 5
    assert F._select_split_k(1, 8, 8, config=mock.Mock(kernel_policy={"awq_fused_gemm_split_k": "2"})) == 2
    assert F._select_split_k(1, 8, 8, config=mock.Mock(kernel_policy=None)) == 0
    assert F._select_split_k(1, 8, 8, config={"kernel_policy": {"awq_fused_gemm_split_k": 3}},
                             policy={"awq_fused_gemm_split_k": 6}) == 6


def test_auto_by_default():
    for m, n, k in ((1, 43008, 5376), (1, 5376, 21504), (4, 8192, 16384), (0, 8192, 16384), (1, 0, 16384)):
        assert F._select_split_k(m, n, k) == 0


def test_forced_value_reaches_ops(monkeypatch):
    """The knob is what ``awq_fused_gemm`` hands to ``ops.gemm``."""
    seen = []
    monkeypatch.setattr(F.ops, "gemm", lambda *a, **kw: seen.append(kw["split_k"]))
    monkeypatch.setattr(F.ops, "gemm_dims", lambda qw, layout: (64, 16))
    a = mock.Mock(shape=(1, 64))
    F.set_awq_fused_tuning_config({KEY: "4"})
    F.awq_fused_gemm(a, None, None, None, 32)
    F.set_awq_fused_tuning_config({})
    F.awq_fused_gemm(a, None, None, None, 32, policy={"awq_fused_gemm_split_k": "auto"})
    F.awq_fused_gemm(a, None, None, None, 32, policy={"awq_fused_gemm_split_k": ""})
    F.awq_fused_gemm(a, None, None, None, 32, policy={"awq_fused_gemm_split_k": "3"})
    assert seen == [4, 0, 0, 3]
