"""Elementwise / mean / cat parity on the GPU: the kuiops kernels against the
oracle (bit-exact for the exact ops, within 4 fp32 ulps / 1 bf16 ulp for the
transcendental ones), against the aten golden fixtures, and through KuiperMode on an HF
Llama block (the ops the reference's ElementwiseImpl / MeanImpl / CatImpl
families serve, kuipy/registry.py:33-57)."""
import numpy as np
import pytest
import torch

import kuillm_amd as kuipy
from kuillm_amd import _lib, ops
from kuillm_amd.kuiops import CatImpl, ElementwiseImpl, MeanImpl
from oracle import kuiops_oracle as O

pytestmark = pytest.mark.gpu
aten = torch.ops.aten
BF = torch.bfloat16
DT = {"f32": torch.float32, "bf16": BF, "f16": torch.float16, "f64": torch.float64}


def npy(t):
    t = t.detach().cpu()
    return t.float().numpy() if t.dtype in (BF, torch.float16) else t.numpy()


def ulps(a, b, dt):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    if dt == "bf16":
        ia, ib = O.f32_to_bf16_bits(a).astype(np.int64), O.f32_to_bf16_bits(b).astype(np.int64)
    elif dt == "f16":
        ia, ib = a.astype(np.float16).view(np.int16).astype(np.int64), b.astype(np.float16).view(np.int16).astype(np.int64)
    else:
        ia, ib = a.view(np.int32).astype(np.int64), b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def run_family(func, *args, **kwargs):
    fam = {ElementwiseImpl: ElementwiseImpl({}), MeanImpl: MeanImpl({}), CatImpl: CatImpl({})}
    for cls, impl in fam.items():
        if (cls is ElementwiseImpl and func in ElementwiseImpl.OPS) or \
                (cls is MeanImpl and func == aten.mean.dim) or (cls is CatImpl and func == aten.cat.default):
            spec = impl.supported(func, args, kwargs)
            assert spec is not None, f"{func} refused"
            out = impl.run(spec, args, kwargs)
            assert out is not None
            return out
    raise AssertionError(func)


UNARY = [("neg", aten.neg.default, {}), ("silu", aten.silu.default, {}), ("cos", aten.cos.default, {}),
         ("sin", aten.sin.default, {}), ("exp", aten.exp.default, {}), ("rsqrt", aten.rsqrt.default, {"pos": 1}),
         ("sqrt", aten.sqrt.default, {"pos": 1})]
EXACT_UNARY = {"neg"}


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16", "f64"])
@pytest.mark.parametrize("name,func,opt", UNARY)
@pytest.mark.parametrize("n", [1, 7, 8, 4099, 1 << 18])
def test_unary_vs_oracle(cuda, dt, name, func, opt, n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g) * 3
    if opt.get("pos"):
        x = x.abs() + 0.01
    x = x.to(DT[dt])
    out = run_family(func, x.to(cuda))
    assert out.dtype == x.dtype and out.shape == x.shape
    comp = "f64" if dt == "f64" else "f32"
    ref = O.round_dtype(O.elementwise(name, npy(x), compute=comp), dt)
    got = npy(out)
    if dt == "f64":
        np.testing.assert_allclose(got, ref, rtol=1e-14, atol=1e-300)
    elif name in EXACT_UNARY or name == "sqrt":          # correctly rounded on both sides
        assert np.array_equal(got, ref)
    else:
        # transcendental: a few ulps of fp32 (HIP's expf / sinf / rsqrtf and
        # numpy's differ by ~1 ulp each; silu adds a division), one rounding
        # step of 16-bit storage
        lim = 4 if dt == "f32" else 1
        assert ulps(got, ref, dt).max() <= lim, name
        assert ulps(got, npy(func(x.to(cuda))), dt).max() <= lim, name      # stock aten on the GPU
    if name in EXACT_UNARY:
        assert torch.equal(out, func(x.to(cuda)))


BINARY = [("add", aten.add.Tensor), ("sub", aten.sub.Tensor), ("mul", aten.mul.Tensor), ("div", aten.div.Tensor)]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16", "f64"])
@pytest.mark.parametrize("name,func", BINARY)
@pytest.mark.parametrize("shapes", [((5, 33), (5, 33)), ((4, 7, 64), (4, 7, 1)), ((2, 3, 8), (8,)),
                                    ((3000,), ()), ((16, 1, 40), (1, 9, 40))])
def test_binary_broadcast_bit_exact(cuda, dt, name, func, shapes):
    g = torch.Generator().manual_seed(len(shapes[0]))
    a = (torch.randn(shapes[0], generator=g) * 2).to(DT[dt])
    b = (torch.randn(shapes[1], generator=g) + (3.0 if name == "div" else 0.0)).to(DT[dt])
    out = run_family(func, a.to(cuda), b.to(cuda))
    comp = "f64" if dt == "f64" else "f32"
    ref = O.round_dtype(O.elementwise(name, npy(a), npy(b), compute=comp), dt)
    assert out.shape == ref.shape
    assert np.array_equal(npy(out), ref)
    assert torch.equal(out, func(a.to(cuda), b.to(cuda)))          # stock aten on the GPU


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_golden_fixtures(cuda, golden, dt):
    def load(key):
        a = golden[f"ew_{dt}_{key}"]
        t = torch.from_numpy(a.view(np.int16)).view(BF) if dt == "bf16" else torch.from_numpy(a)
        return t.to(cuda)

    x, y, col = load("x"), load("y"), load("col")
    cases = {
        "neg": (aten.neg.default, (x,), {}), "sq": (aten.pow.Tensor_Scalar, (x, 2), {}),
        "p3": (aten.pow.Tensor_Scalar, (x, 3), {}), "add": (aten.add.Tensor, (x, y), {}),
        "add_a": (aten.add.Tensor, (x, y), {"alpha": 0.5}), "sub": (aten.sub.Tensor, (x, y), {}),
        "mul": (aten.mul.Tensor, (x, y), {}), "div": (aten.div.Tensor, (x, y), {}),
        "mulcol": (aten.mul.Tensor, (x, col), {}), "adds": (aten.add.Tensor, (x, 1e-6), {}),
        "muls": (aten.mul.Tensor, (x, 0.125), {}), "where": (aten.where.self, (x > 0, x, y), {}),
        "silu": (aten.silu.default, (x,), {}), "cos": (aten.cos.default, (x,), {}),
        "sin": (aten.sin.default, (x,), {}), "exp": (aten.exp.default, (x,), {}),
        "rsqrt": (aten.rsqrt.default, (y,), {}), "sqrt": (aten.sqrt.default, (y,), {}),
    }
    for key, (func, args, kw) in cases.items():
        out = npy(run_family(func, *args, **kw))
        want = golden[f"ew_{dt}_{key}"]
        want = O.bf16_bits_to_f32(want) if dt == "bf16" else want
        tol = 0 if key in ("neg", "sq", "p3", "add", "sub", "mul", "div", "mulcol", "adds", "muls", "where") else (4 if dt == "f32" else 1)
        if key == "add_a":
            tol = 1
        assert ulps(out, want, dt).max() <= tol, key
    assert np.array_equal(npy(run_family(aten.lt.Scalar, x, 0.5)), golden[f"ew_{dt}_lt"])
    assert np.array_equal(npy(run_family(aten.le.Tensor, x, y)), golden[f"ew_{dt}_le"])
    assert np.array_equal(npy(run_family(aten.eq.Scalar, x, 0.0)), golden[f"ew_{dt}_eq"])


def test_promotion_integer_and_bitwise_golden(cuda, golden):
    xb = torch.from_numpy(golden["ew_bf16_x"].view(np.int16)).view(BF).to(cuda)
    yf = torch.from_numpy(golden["ew_f32_y"]).to(cuda)
    out = run_family(aten.mul.Tensor, xb, yf)
    assert out.dtype == torch.float32 and np.array_equal(npy(out), golden["ew_mixed_out"])
    b1, b2 = (torch.from_numpy(golden[k]).to(cuda) for k in ("ew_b1", "ew_b2"))
    assert np.array_equal(npy(run_family(aten.bitwise_and.Tensor, b1, b2)), golden["ew_band"])
    assert np.array_equal(npy(run_family(aten.bitwise_or.Tensor, b1, b2)), golden["ew_bor"])
    assert np.array_equal(npy(run_family(aten.bitwise_not.default, b1)), golden["ew_bnot"])
    i = torch.from_numpy(golden["ew_i64"]).to(cuda)
    assert np.array_equal(npy(run_family(aten.add.Tensor, i, 3)), golden["ew_i64_add"])
    assert np.array_equal(npy(run_family(aten.mul.Tensor, i, i)), golden["ew_i64_mul"])
    r = run_family(aten.div.Tensor, i, 4)                    # true division promotes to fp32
    assert r.dtype == torch.float32 and torch.equal(r, i / 4)


def test_strided_and_special_operands(cuda):
    g = torch.Generator(device=cuda).manual_seed(3)
    a = torch.randn(64, 48, device=cuda, generator=g).to(BF)
    at = a.t()                                               # transposed view
    b = torch.randn(48, 64, device=cuda, generator=g).to(BF)
    assert torch.equal(run_family(aten.mul.Tensor, at, b), at * b)
    sl = a[:, 5:37]                                          # row-strided slice
    assert torch.equal(run_family(aten.add.Tensor, sl, 1.5), sl + 1.5)
    s0 = torch.tensor(2.0, device=cuda, dtype=BF)            # 0-d device tensor
    assert torch.equal(run_family(aten.mul.Tensor, a, s0), a * s0)
    cpu_scalar = torch.tensor(0.25, dtype=torch.float64)     # wrapped scalar on the CPU
    assert torch.equal(run_family(aten.mul.Tensor, a, cpu_scalar), a * 0.25)
    assert torch.equal(run_family(aten.sub.Tensor, a, b.t(), alpha=2), torch.sub(a, b.t(), alpha=2))
    x = torch.tensor([float("nan"), float("inf"), -0.0, 0.0, 1.0], device=cuda)
    assert torch.equal(run_family(aten.eq.Scalar, x, 0.0), x == 0.0)
    assert torch.equal(run_family(aten.ne.Tensor, x, x), x != x)
    w = run_family(aten.where.self, x > 0, x, 0.0)
    assert torch.equal(w, torch.where(x > 0, x, 0.0))
    e = torch.empty(0, 5, device=cuda)
    assert run_family(aten.neg.default, e).shape == (0, 5)
    big = torch.randn(3, 1000003, device=cuda)               # ragged tail, several blocks per lane
    assert torch.equal(run_family(aten.neg.default, big), -big)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f64"])
@pytest.mark.parametrize("shape", [(6, 100), (3, 5000), (2, 9, 2048), (1, 40000), (7, 1)])
def test_mean_vs_oracle(cuda, dt, shape):
    g = torch.Generator().manual_seed(shape[-1])
    x = torch.randn(*shape, generator=g).to(DT[dt])
    for keepdim in (True, False):
        out = run_family(aten.mean.dim, x.to(cuda), [-1], keepdim)
        ref = O.round_dtype(O.mean_lastdim(npy(x).astype(np.float64), keepdim), dt)
        assert out.shape == ref.shape
        if dt == "bf16":
            assert ulps(npy(out), ref, dt).max() <= 1
        else:
            np.testing.assert_allclose(npy(out), ref, rtol=1e-5 if dt == "f32" else 1e-12, atol=1e-6)
    xs = x.to(cuda)[..., : shape[-1] // 2 + 1]                 # strided rows
    ref = O.round_dtype(O.mean_lastdim(npy(x)[..., : shape[-1] // 2 + 1].astype(np.float64)), dt)
    got = npy(run_family(aten.mean.dim, xs, [-1]))
    if dt == "bf16":
        assert ulps(got, ref, dt).max() <= 1
    else:
        np.testing.assert_allclose(got, ref, rtol=1e-5 if dt == "f32" else 1e-12, atol=1e-6)


def test_mean_golden(cuda, golden):
    x = torch.from_numpy(golden["mean_bf16_x"].view(np.int16)).view(BF).to(cuda)
    out = run_family(aten.mean.dim, x, [-1], True)
    assert ulps(npy(out), O.bf16_bits_to_f32(golden["mean_bf16_out"]), "bf16").max() <= 1
    xf = torch.from_numpy(golden["mean_f32_x"]).to(cuda)
    np.testing.assert_allclose(npy(run_family(aten.mean.dim, xf, [-1])), golden["mean_f32_out"], rtol=1e-5)


def test_cat_bit_exact(cuda, golden):
    a = torch.from_numpy(golden["cat_a"].view(np.int16)).view(BF).to(cuda)
    b = torch.from_numpy(golden["cat_b"].view(np.int16)).view(BF).to(cuda)
    out = run_family(aten.cat.default, [a, b], 2)
    assert np.array_equal(npy(out), O.bf16_bits_to_f32(golden["cat_out"]))
    q = torch.from_numpy(golden["cat_q"]).to(cuda)
    rot = run_family(aten.cat.default, [-q[..., 8:], q[..., :8]], -1)     # rotate_half, strided slice input
    assert np.array_equal(npy(rot), golden["cat_rot"])
    g = torch.Generator(device=cuda).manual_seed(9)
    parts = [torch.randn(3, k, 5, device=cuda, generator=g) for k in (1, 0, 7, 2)]
    assert torch.equal(run_family(aten.cat.default, parts, 1), torch.cat(parts, 1))
    many = [torch.randint(0, 100, (4, 3), device=cuda, dtype=torch.int64) for _ in range(20)]
    assert torch.equal(run_family(aten.cat.default, many, 0), torch.cat(many, 0))
    odd = [torch.randn(5, 3, device=cuda).to(BF), torch.randn(5, 1, device=cuda).to(BF)]   # 2-byte copies
    assert torch.equal(run_family(aten.cat.default, odd, -1), torch.cat(odd, -1))
    kv = torch.randn(1, 8, 640, 64, device=cuda).to(BF)                   # KV-cache growth
    new = torch.randn(1, 8, 1, 64, device=cuda).to(BF)
    assert torch.equal(run_family(aten.cat.default, [kv, new], -2), torch.cat([kv, new], -2))


def test_hf_llama_block_under_kuiper_mode(cuda, monkeypatch):
    """A transformers Llama decoder layer under KuiperMode: its RMSNorm,
    rotary and SwiGLU elementwise ops, mean and cat run on the kuiops
    kernels (verify mode compares each against stock PyTorch)."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                      num_hidden_layers=1, vocab_size=100, max_position_embeddings=256, rms_norm_eps=1e-5)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    layer = LlamaDecoderLayer(cfg, 0).to(cuda, BF).eval()
    rope = LlamaRotaryEmbedding(cfg).to(cuda)
    h = torch.randn(2, 16, 256, device=cuda, dtype=BF)
    pos = torch.arange(16, device=cuda)[None].expand(2, 16)
    with torch.no_grad():
        pe = rope(h, pos)
        ref = layer(h, position_embeddings=pe)
        ref = ref[0] if isinstance(ref, tuple) else ref
    monkeypatch.setattr(kuipy.C, "ENABLE_PRINT_PROFILING", True)
    kuipy.profile_data.clear()
    kuipy.reset_verify()
    with torch.no_grad(), kuipy.KuiperMode(verify=True):
        pe2 = rope(h, pos)
        out = layer(h, position_embeddings=pe2)
        out = out[0] if isinstance(out, tuple) else out
    assert kuipy.print_verify_report() is True
    served = set(kuipy.verify_stats)
    assert {"aten.mul.Tensor", "aten.add.Tensor", "aten.rsqrt.default", "aten.pow.Tensor_Scalar",
            "aten.mean.dim", "aten.silu.default", "aten.cat.default", "aten.neg.default"} <= served, served
    rel = ((out.float() - ref.float()).norm() / ref.float().norm()).item()
    assert rel < 1e-2
    kuipy.profile_data.clear()


def test_rejections_fall_through(cuda):
    e = ElementwiseImpl({})
    x = torch.randn(4, device=cuda)
    assert e.supported(aten.add.Tensor, (x, torch.randn(4)), {}) is None          # CPU tensor operand
    assert e.supported(aten.silu.default, (torch.arange(4, device=cuda),), {}) is None   # int silu
    assert e.supported(aten.div.Tensor, (x, x), {"rounding_mode": "floor"}) is None
    assert MeanImpl({}).supported(aten.mean.dim, (x.view(2, 2), [0]), {}) is None  # not the last axis
    assert CatImpl({}).supported(aten.cat.default, ([x, x.double()], 0), {}) is None
    with pytest.raises(_lib.KuiopsError):
        ops.cat([torch.randn(2, 3, device=cuda), torch.randn(3, 3, device=cuda)], 1)
