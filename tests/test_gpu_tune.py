"""Autotuning on the GPU: the sweeps return parameters in range, the tuned
GEMM row limit routes calls to either kernel with the same results, and the
CLI writes a JSON file the registry reads back."""
import json

import numpy as np
import pytest
import torch

from kuillm_amd import kuiops as K
from kuillm_amd import ops, registry, tune
from oracle import kuiops_oracle as O

pytestmark = pytest.mark.gpu


def test_sweeps_in_range(cuda):
    m = tune.sweep_gemv_max_m(shapes=((1024, 2048),), rows=(1, 16, 64))
    assert m in (0, 1, 16, 64)
    r = tune.sweep_decode_max_rows(rows=(1, 4), s=512, hd=64, hkv=2)
    assert r in (0, 1, 4)


def test_gemv_row_limit_routes_both_kernels(cuda):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 1024, generator=g).to(torch.bfloat16)
    W = (torch.randn(1024, 512, generator=g) * 0.05).to(torch.bfloat16)
    ref = O.mm(x.float().numpy(), W.float().numpy())
    for lim in (0, 64):
        out = torch.ops.kuiops.mm(x.to(cuda), W.to(cuda), lim)
        err = np.abs(out.float().cpu().numpy() - ref) - (1e-2 + 1e-2 * np.abs(ref))
        assert err.max() <= 0
    impl = K.MmImpl({"MM": {"gemv_max_m": 0}})
    spec = impl.supported(torch.ops.aten.mm.default, (x.to(cuda), W.to(cuda)), {})
    assert impl.run(spec, (), {}).shape == (8, 512)


def test_tune_cli_writes_json(cuda, tmp_path):
    out = tmp_path / "tune.json"
    tune.main(["--out", str(out)])
    params = json.loads(out.read_text())
    assert 0 <= params["MM"]["gemv_max_m"] <= 64
    assert params["SDPA"]["decode_max_rows"] >= 0
    assert registry.load_tune_params(out)["MM"]["gemv_max_m"] == params["MM"]["gemv_max_m"]
