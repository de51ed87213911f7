"""KuiperMode's verify ledger, call log and strictness policy, on CPU tensors
(no kernel runs: CPU tensors are never offloaded)."""
import io
import math

import pytest
import torch

import kuillm_amd as kuipy

aten = torch.ops.aten


@pytest.fixture(autouse=True)
def _clean_ledger():
    kuipy.reset_verify()
    yield
    kuipy.reset_verify()


def _entry(op):
    return kuipy.verify_stats[str(op)]


@pytest.mark.parametrize("scale, fails", [(0.0, False), (1e-3, False), (0.5, True)])
def test_relative_error_against_tolerance(scale, fails):
    g = torch.Generator().manual_seed(1)
    ref = torch.randn(16, 16, generator=g, dtype=torch.float64)
    noise = torch.randn(16, 16, generator=g, dtype=torch.float64)
    out = ref + scale * noise * ref.norm() / noise.norm()     # rel error == scale exactly
    kuipy._verify_compare(aten.mm.default, out, ref, tol=2e-2)
    e = _entry(aten.mm.default)
    assert e["n"] == 1 and e["fail"] == int(fails)
    assert math.isclose(e["max_rel"], scale, rel_tol=1e-6, abs_tol=1e-12)
    assert (e["worst"] is not None) == fails


def test_error_is_measured_in_float64():
    # bf16 inputs whose difference is one bf16 ulp of a single element
    ref = torch.ones(1024, dtype=torch.bfloat16)
    out = ref.clone()
    out[7] = 1.0078125
    kuipy._verify_compare(aten.add.Tensor, out, ref, tol=1.0)
    assert math.isclose(_entry(aten.add.Tensor)["max_rel"], 0.0078125 / 32.0, rel_tol=1e-9)


def test_positions_not_finite_in_either_tensor_are_skipped():
    ref = torch.arange(12.0).reshape(3, 4)
    out = ref.clone()
    out[0, :] = float("nan")         # kernel wrote NaN where the reference is finite
    ref[2, :] = float("-inf")        # reference itself not finite there
    out[2, :] = 123.0
    kuipy._verify_compare(aten.mm.default, out, ref, tol=1e-6)
    assert _entry(aten.mm.default)["fail"] == 0 and _entry(aten.mm.default)["n"] == 1


def test_all_masked_output_is_not_counted():
    t = torch.full((2, 3), float("nan"))
    kuipy._verify_compare(aten.mm.default, t, t.clone(), tol=1e-6)
    assert _entry(aten.mm.default)["n"] == 0


def test_tuple_results_pair_in_order_and_skip_empty_and_integer_leaves():
    o = torch.randn(2, 5)
    out = (o, torch.empty(2, 0), torch.tensor([3, 1]), o * 2)
    ref = (o.clone(), torch.empty(2, 0), torch.tensor([0, 0]), o * 2)
    kuipy._verify_compare(aten.topk.default, out, ref, tol=1e-6)
    e = _entry(aten.topk.default)
    assert e["n"] == 2 and e["fail"] == 0      # the int64 leaf differs but is not compared


def test_shape_disagreement_is_a_failure():
    kuipy._verify_compare(aten.bmm.default, torch.zeros(2, 3), torch.zeros(3, 2), tol=1.0)
    e = _entry(aten.bmm.default)
    assert e["fail"] == 1 and "shape" in e["worst"]


def test_report_lists_each_op_and_returns_verdict():
    buf = io.StringIO()
    assert kuipy.print_verify_report(out_dev=buf) is None and "nothing" in buf.getvalue()
    a = torch.randn(4, 4)
    kuipy._verify_compare(aten.mm.default, a, a.clone(), tol=2e-2)
    kuipy._verify_compare(aten.bmm.default, a, a.clone(), tol=2e-2)
    buf = io.StringIO()
    assert kuipy.print_verify_report(out_dev=buf, tol=2e-2) is True
    text = buf.getvalue()
    assert "aten.mm.default" in text and "aten.bmm.default" in text and "PASS" in text
    kuipy._verify_compare(aten.mm.default, a, -a, tol=2e-2)
    buf = io.StringIO()
    assert kuipy.print_verify_report(out_dev=buf, tol=2e-2) is False
    assert "FAIL" in buf.getvalue()


def test_cpu_tensors_run_stock_pytorch_under_verify():
    A, B = torch.randn(8, 8), torch.randn(8, 8)
    with kuipy.KuiperMode(verify=True):
        out = torch.mm(A, B)
    assert torch.equal(out, A @ B)
    assert kuipy.verify_stats == {}


def test_call_log_skips_views(monkeypatch):
    monkeypatch.setattr(kuipy.C, "ENABLE_PRINT_PROFILING", True)
    kuipy.profile_data.clear()
    A = torch.randn(4, 4)
    with kuipy.KuiperMode():
        torch.mm(A, A)
        A.view(16)
        A.t()
        A.add_(1.0)                              # in place: launches a kernel
    logged = {str(f) for f in kuipy.profile_data}
    assert {"aten.mm.default", "aten.add_.Tensor"} <= logged
    assert "aten.view.default" not in logged and "aten.t.default" not in logged
    buf = io.StringIO()
    kuipy.print_profile_data(out_dev=buf)
    assert "aten.mm.default" in buf.getvalue() and "float32" in buf.getvalue()
    kuipy.profile_data.clear()


def test_dummy_print_mode_never_offloads(monkeypatch):
    calls = []
    monkeypatch.setattr(kuipy, "_offload", lambda *a: calls.append(a))
    monkeypatch.setattr(kuipy.KuiperMode, "dummy_print_mode", True)
    with kuipy.KuiperMode():
        torch.mm(torch.ones(2, 2), torch.ones(2, 2))
    assert calls == []
