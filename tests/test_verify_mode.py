"""The verify machinery (reference tests/test_verify_mode.py), CPU only."""
import io

import torch

import kuillm_amd as kuipy


class _F:  # stand-in for an aten OpOverload (only str() is used as the key)
    def __init__(self, name):
        self.name = name

    def __str__(self):
        return self.name


def setup_function():
    kuipy.reset_verify()


def test_matching_tensors_pass():
    a = torch.randn(8, 8)
    kuipy._verify_compare(_F("aten.mm"), a, a.clone(), tol=2e-2)
    s = kuipy.verify_stats["aten.mm"]
    assert s["n"] == 1 and s["fail"] == 0 and s["max_rel"] < 1e-6


def test_divergent_tensors_fail():
    a = torch.randn(8, 8)
    b = a + 0.5 * a.abs().mean()
    kuipy._verify_compare(_F("aten.mm"), a, b, tol=2e-2)
    s = kuipy.verify_stats["aten.mm"]
    assert s["fail"] == 1 and s["max_rel"] > 2e-2 and "rel=" in s["worst"]


def test_empty_reference_is_skipped():
    kuipy._verify_compare(_F("aten.sdpa"), torch.randn(2, 3, 1), torch.randn(2, 3, 0), tol=2e-2)
    s = kuipy.verify_stats["aten.sdpa"]
    assert s["n"] == 0 and s["fail"] == 0


def test_nonfinite_positions_are_ignored():
    out = torch.randn(4, 8)
    ref = out.clone()
    out[0] = float("nan")
    ref[0] = 0.0
    kuipy._verify_compare(_F("aten.sdpa"), out, ref, tol=2e-2)
    s = kuipy.verify_stats["aten.sdpa"]
    assert s["n"] == 1 and s["fail"] == 0


def test_tuple_outputs_compared_elementwise():
    a, b = torch.randn(4, 4), torch.randn(4)
    kuipy._verify_compare(_F("aten.sdpa"), (a, b), (a.clone(), b.clone()), tol=2e-2)
    assert kuipy.verify_stats["aten.sdpa"]["n"] == 2


def test_shape_mismatch_counts_as_failure():
    kuipy._verify_compare(_F("aten.x"), torch.randn(2, 3), torch.randn(3, 2), tol=2e-2)
    assert kuipy.verify_stats["aten.x"]["fail"] == 1


def test_report_pass_and_fail():
    a = torch.randn(8, 8)
    kuipy._verify_compare(_F("aten.mm"), a, a.clone(), tol=2e-2)
    buf = io.StringIO()
    assert kuipy.print_verify_report(out_dev=buf, tol=2e-2) is True and "PASS" in buf.getvalue()
    kuipy._verify_compare(_F("aten.bmm"), a, a + 1.0, tol=2e-2)
    buf = io.StringIO()
    assert kuipy.print_verify_report(out_dev=buf, tol=2e-2) is False and "FAIL" in buf.getvalue()


def test_mode_falls_through_on_cpu_tensors():
    # CPU tensors are never offloaded: results are stock PyTorch's
    A, B = torch.randn(8, 8), torch.randn(8, 8)
    with kuipy.KuiperMode(verify=True):
        out = torch.mm(A, B)
    assert torch.allclose(out, A @ B)
    assert not kuipy.verify_stats


def test_profile_recording(monkeypatch):
    monkeypatch.setattr(kuipy.C, "ENABLE_PRINT_PROFILING", True)
    kuipy.profile_data.clear()
    A, B = torch.randn(4, 4), torch.randn(4, 4)
    with kuipy.KuiperMode():
        torch.mm(A, B)
        A.view(16)          # a view launches nothing and is not recorded
    names = {str(f) for f, *_ in kuipy.profile_data}
    assert "aten.mm.default" in names and "aten.view.default" not in names
    buf = io.StringIO()
    kuipy.print_profile_data(out_dev=buf)
    assert "aten.mm.default" in buf.getvalue()
