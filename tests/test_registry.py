"""Family gates and the registry, on the CPU with fake CUDA tensors (the
gates read shapes / dtypes / devices only).  Mirrors the reference's
negative tests (tests/test_jit_ops.py:63-73, 115-134, 158-165, 232-244;
tests/test_jit_general.py:61-71) with this build's wider acceptance."""
import json

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from kuillm_amd import kuiops as K
from kuillm_amd import registry

aten = torch.ops.aten


@pytest.fixture
def fake():
    with FakeTensorMode() as m:
        yield m


def cu(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="cuda", dtype=dtype)


def test_mm_gate(fake):
    impl = K.MmImpl({})
    assert impl.supported(aten.mm.default, (cu(64, 32), cu(32, 16)), {}) is not None
    # odd K and decode shapes are served (the reference needs M, N % 64 == 0)
    assert impl.supported(aten.mm.default, (cu(1, 63), cu(63, 11008)), {}) is not None
    assert impl.supported(aten.mm.default, (cu(8, 8), cu(9, 8)), {}) is None            # K mismatch
    assert impl.supported(aten.mm.default, (cu(8, 8), cu(8, 8, dtype=torch.float16)), {}) is None
    assert impl.supported(aten.mm.default, (cu(8, 8, dtype=torch.int32), cu(8, 8, dtype=torch.int32)), {}) is None
    assert impl.supported(aten.mm.default, (cu(2, 8, 8), cu(8, 8)), {}) is None


def test_mm_gate_rejects_cpu_tensors():
    impl = K.MmImpl({})
    assert impl.supported(aten.mm.default, (torch.randn(64, 64), torch.randn(64, 64)), {}) is None


def test_addmm_gate(fake):
    impl = K.AddmmImpl({})
    A, B = cu(32, 16), cu(16, 24)
    for C in (cu(32, 24), cu(24), cu(1, 24), cu(32, 1)):
        spec = impl.supported(aten.addmm.default, (C, A, B), {"alpha": 0.5, "beta": 2})
        assert spec is not None and spec[-2:] == (0.5, 2.0)
    assert impl.supported(aten.addmm.default, (cu(7), A, B), {}) is None                 # not broadcastable
    assert impl.supported(aten.addmm.default, (cu(24, dtype=torch.float32), A, B), {}) is None
    assert impl.supported(aten.addmm.default, (cu(24), A, B), {"alpha": cu(())}) is None  # tensor alpha


def test_bmm_gate(fake):
    impl = K.BmmImpl({})
    assert impl.supported(aten.bmm.default, (cu(5, 17, 9), cu(5, 9, 13)), {}) is not None
    assert impl.supported(aten.bmm.default, (cu(2, 4, 4), cu(3, 4, 4)), {}) is None       # batch mismatch
    assert impl.supported(aten.bmm.default, (cu(4, 4), cu(4, 4)), {}) is None             # 2-D is not bmm


def test_softmax_gate(fake):
    impl = K.SoftmaxImpl({})
    assert impl.supported(aten._softmax.default, (cu(8, 5, 33), 2, False), {}) is not None
    assert impl.supported(aten._softmax.default, (cu(8, 5, 33), -1, False), {}) is not None
    assert impl.supported(aten._softmax.default, (cu(16, 16), 0, False), {}) is None      # not last dim
    assert impl.supported(aten._softmax.default, (cu(16, 16), 1, True), {}) is None       # half_to_float


def test_sdpa_gate(fake):
    impl = K.SdpaImpl({})
    eff = aten._scaled_dot_product_efficient_attention.default
    fl = aten._scaled_dot_product_flash_attention.default
    q, k, v = cu(1, 8, 64, 128), cu(1, 2, 64, 128), cu(1, 2, 64, 128)
    spec = impl.supported(fl, (q, k, v, 0.0, True), {})
    assert spec is not None and spec[2] is True and abs(spec[1] - 128 ** -0.5) < 1e-12
    assert impl.supported(eff, (q, k, v, None, True, 0.0, True), {"scale": 0.3})[1] == 0.3
    spec = impl.supported(eff, (q, k, v, cu(1, 8, 64, 64), True), {})                    # explicit bias
    assert spec is not None and spec[-1].shape == (1, 8, 64, 64)
    assert impl.supported(eff, (q, k, v, cu(1, 1, 1, 64), True), {}) is not None         # broadcast mask
    assert impl.supported(eff, (q, k, v, cu(1, 8, 64, 63), True), {}) is None            # wrong key count
    assert impl.supported(eff, (q, k, v, cu(1, 8, 64, 64, dtype=torch.float32), True), {}) is None
    assert impl.supported(fl, (q, k, v, 0.1, False), {}) is None                         # dropout
    assert impl.supported(fl, (q, k, v, 0.0, False, True), {}) is None                   # debug mask
    assert impl.supported(fl, (cu(1, 3, 64, 128), k, v), {}) is None                     # 3 % 2 heads
    assert impl.supported(fl, (cu(1, 2, 8, 96), cu(1, 2, 8, 96), cu(1, 2, 8, 96)), {}) is not None  # padded
    # wide heads, e != ev and fp32 / fp64 (the reference gate's _FLOAT_DTYPES) take the general kernel
    assert impl.supported(fl, (cu(1, 2, 8, 160), cu(1, 2, 8, 160), cu(1, 2, 8, 160)), {}) is not None
    assert impl.supported(fl, (cu(1, 2, 8, 16), cu(1, 2, 8, 16), cu(1, 2, 8, 12)), {}) is not None
    assert impl.supported(fl, (cu(1, 2, 8, 2048), cu(1, 2, 8, 2048), cu(1, 2, 8, 2048)), {}) is None
    for dt in (torch.float32, torch.float64):
        assert impl.supported(fl, (cu(1, 2, 8, 64, dtype=dt), cu(1, 2, 8, 64, dtype=dt),
                                   cu(1, 2, 8, 64, dtype=dt)), {}) is not None
    assert impl.supported(fl, (cu(1, 2, 8, 64, dtype=torch.int32), cu(1, 2, 8, 64, dtype=torch.int32),
                               cu(1, 2, 8, 64, dtype=torch.int32)), {}) is None


def test_topk_gate(fake):
    impl = K.TopkImpl({})
    x = cu(4, 32000, dtype=torch.float32)
    assert impl.supported(aten.topk.default, (x, 50), {}) == (x, 50, 1, True, True)
    assert impl.supported(aten.topk.default, (x, 3, 0, False, False), {})[2:] == (0, False, False)
    assert impl.supported(aten.topk.default, (x, 2048), {}) is None
    assert impl.supported(aten.topk.default, (cu(4, 3, dtype=torch.int64), 1), {}) is None


def test_gather_gate(fake):
    impl = K.GatherImpl({})
    inp = cu(4, 4, dtype=torch.float32)
    assert impl.supported(aten.gather.default, (inp, 1, cu(4, 7, dtype=torch.int64)), {}) is not None
    assert impl.supported(aten.gather.default, (inp, 1, cu(4, 4, dtype=torch.int32)), {}) is None
    assert impl.supported(aten.gather.default, (inp, 1, cu(4, dtype=torch.int64)), {}) is None
    assert impl.supported(aten.gather.default, (inp, 1, cu(5, 4, dtype=torch.int64)), {}) is None
    assert impl.supported(aten.gather.default, (inp, 1, cu(4, 4, dtype=torch.int64)), {"sparse_grad": True}) is None


def test_index_gate(fake):
    impl = K.IndexImpl({})
    E = cu(32000, 64)
    ids = cu(1, 7, dtype=torch.int64)
    assert impl.supported(aten.index.Tensor, (E, [ids]), {}) == (0, [E, ids])
    assert impl.supported(aten.index.Tensor, (cu(2, 9, 4), [None, ids]), {})[0] == 1
    spec = impl.supported(aten.index.Tensor, (E, [ids, ids]), {})                          # two indices
    assert spec[0] == 0 and len(spec[1]) == 3
    assert impl.supported(aten.index.Tensor, (cu(2, 9, 4), [ids, None, ids]), {}) is None  # not adjacent
    assert impl.supported(aten.index.Tensor, (E, [cu(32000, dtype=torch.bool)]), {}) is None


def test_registry_maps_hot_ops():
    registry.reset()
    reg = registry.registry()
    expect = {aten.mm.default: K.MmImpl, aten.addmm.default: K.AddmmImpl, aten.bmm.default: K.BmmImpl,
              aten._softmax.default: K.SoftmaxImpl, aten.topk.default: K.TopkImpl,
              aten.gather.default: K.GatherImpl, aten.index.Tensor: K.IndexImpl,
              aten._scaled_dot_product_flash_attention.default: K.SdpaImpl,
              aten._scaled_dot_product_efficient_attention.default: K.SdpaImpl}
    for op, cls in expect.items():
        assert isinstance(reg[op], cls)
    assert registry.try_dispatch(aten.add.Tensor, (torch.ones(2), torch.ones(2)), {}) is None
    assert registry.try_dispatch(aten.mm.default, (torch.ones(2, 2), torch.ones(2, 2)), {}) is None


def test_tune_params_roundtrip(tmp_path, monkeypatch):
    f = tmp_path / "tune.json"
    registry.save_tune_params({"MM": {"impl": "auto", "gemv_max_m": 32}}, f)
    assert json.loads(f.read_text())["MM"]["gemv_max_m"] == 32
    monkeypatch.setattr(registry.C, "TUNE_FILE", f)
    registry.reset()
    assert registry.registry()[aten.mm.default].tune_params["gemv_max_m"] == 32
    monkeypatch.setattr(registry.C, "RE_TUNE", True)
    registry.reset()
    registry.registry()
    saved = json.loads(f.read_text())
    assert {"MM", "ADDMM", "SDPA"} <= set(saved)
    registry.reset()


def test_strictness_levels(monkeypatch):
    import kuillm_amd as kuipy

    def boom(*a, **k):
        raise RuntimeError("kernel failed")
    monkeypatch.setattr(registry, "try_dispatch", boom)
    monkeypatch.setattr(kuipy.C, "JIT_STRICTNESS", 1)
    with pytest.raises(RuntimeError, match="kernel failed"):
        kuipy._offload(aten.mm.default, (), {})
    monkeypatch.setattr(kuipy.C, "JIT_STRICTNESS", 0)
    assert kuipy._offload(aten.mm.default, (), {}) is None       # warn once, fall back
    monkeypatch.setattr(registry, "try_dispatch", lambda *a: None)
    monkeypatch.setattr(kuipy.C, "JIT_STRICTNESS", 2)
    with pytest.raises(kuipy.NotOffloaded):
        kuipy._offload(aten.mm.default, (), {})


def test_sampling_tail_gates(fake):
    sc = K.ScatterImpl({})
    s32 = cu(4, 9, dtype=torch.float32)
    i64 = cu(4, 9, dtype=torch.int64)
    assert sc.supported(aten.scatter.src, (s32, 1, i64, s32), {}) is not None
    assert sc.supported(aten.scatter.src, (cu(4, 9, dtype=torch.bool), 1, i64, cu(4, 9, dtype=torch.bool)), {}) \
        is not None
    assert sc.supported(aten.scatter.src, (s32, 1, cu(4, 9, dtype=torch.int32), s32), {}) is None     # int32 index
    assert sc.supported(aten.scatter.src, (s32, 1, i64, cu(4, 9, dtype=torch.float16)), {}) is None  # src dtype
    assert sc.supported(aten.scatter.src, (s32, 1, cu(5, 9, dtype=torch.int64), s32), {}) is None    # idx > self
    so = K.SortImpl({})
    assert so.supported(aten.sort.default, (cu(4, 32000, dtype=torch.float32),), {}) is not None
    spec = so.supported(aten.sort.stable, (cu(4, 7),), {"stable": True, "dim": 0, "descending": True})
    assert spec is not None and spec[1:] == (0, True)
    assert so.supported(aten.sort.default, (cu(4, 7, dtype=torch.int64),), {}) is None
    cs = K.CumsumImpl({})
    assert cs.supported(aten.cumsum.default, (cu(4, 7, dtype=torch.float32), 1), {}) is not None
    assert cs.supported(aten.cumsum.default, (cu(4, 7, dtype=torch.int64), -1), {}) is not None
    assert cs.supported(aten.cumsum.default, (cu(4, 7, dtype=torch.float32), 1), {"dtype": torch.float64}) is None
    assert cs.supported(aten.cumsum.default, (cu(4, 7, dtype=torch.bool), 1), {}) is None
    mn = K.MultinomialImpl({})
    assert mn.supported(aten.multinomial.default, (cu(4, 100, dtype=torch.float32), 1), {}) is not None
    assert mn.supported(aten.multinomial.default, (cu(4, 100, dtype=torch.float32), 5, True), {}) is not None
    assert mn.supported(aten.multinomial.default, (cu(4, 100, dtype=torch.float32), 5), {}) is None  # no replacement
    assert mn.supported(aten.multinomial.default, (cu(2, 4, 100, dtype=torch.float32), 1), {}) is None
    reg = registry.registry()
    for op in (aten.scatter.src, aten.sort.default, aten.sort.stable, aten.cumsum.default, aten.multinomial.default):
        assert op in reg


def test_tune_crossover_logic():
    from kuillm_amd import tune
    assert tune.pick_crossover([1, 2, 4, 8], lambda c: c <= 4) == 4
    assert tune.pick_crossover([1, 2, 4, 8], lambda c: c != 2) == 1          # first failure stops the sweep
    assert tune.pick_crossover([1, 2, 4], lambda c: False) == 0
    assert K._gemv_max_m({"gemv_max_m": 500}) == 64 and K._gemv_max_m({"gemv_max_m": -3}) == 0
    assert K._gemv_max_m(()) == 64
