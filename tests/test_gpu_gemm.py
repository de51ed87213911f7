"""GEMM parity on the GPU: mm / addmm / bmm / decode split-K against the numpy
oracle on the same seeded inputs, the aten golden fixtures, and size-free
properties at the BASELINE.json sizes.

Tolerance (north star): bf16 / f16 results within rel 1e-2 / abs 1e-2 of the
fp32-accumulate oracle, elementwise: |out - ref| <= 1e-2 + 1e-2 * |ref|.
fp32 results: allclose(rtol=1e-3, atol=1e-3) as the reference's tests
(tests/test_jit_ops.py:34-43)."""
import numpy as np
import pytest
import torch

from kuillm_amd import _lib, ops
from oracle import kuiops_oracle as O

pytestmark = pytest.mark.gpu
RTOL = ATOL = 1e-2


def npy(t):
    return t.detach().float().cpu().numpy() if t.dtype != torch.float64 else t.detach().cpu().numpy()


def gen(shape, dtype, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def assert_tol(out, ref, dtype):
    o = npy(out)
    if dtype in (torch.float32, torch.float64):
        np.testing.assert_allclose(o, ref, rtol=1e-3, atol=1e-3)
    else:
        err = np.abs(o - ref) - (ATOL + RTOL * np.abs(ref))
        assert err.max() <= 0, f"max excess {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


SHAPES = [(64, 64, 64), (128, 128, 64), (256, 512, 320), (300, 260, 72), (129, 1000, 136), (96, 80, 8)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_mm_vs_oracle(cuda, dtype, layout, M, N, K):
    A = gen((M, K), dtype, seed=1)
    B = gen((K, N), dtype, 0.5, seed=2)
    ref = O.mm(npy(A), npy(B))
    Bd = B.to(cuda) if layout == "row" else B.t().contiguous().to(cuda).t()
    out = ops.mm(A.to(cuda), Bd)
    assert out.dtype == dtype and out.shape == (M, N)
    assert_tol(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("M,N,K", [(4096, 8192, 64), (2048, 16384, 128)])
def test_mm_short_k_many_tiles(cuda, dtype, layout, M, N, K):
    """K of one or two 64-k stages and at least two 256x256 tiles per CU:
    the persistent short-K kernel, with B row-major (transposing fragment
    reads) or column-major (B^T rows staged like A)."""
    A = gen((M, K), dtype, seed=5)
    B = gen((K, N), dtype, 0.5, seed=6)
    Bd = B.to(cuda) if layout == "row" else B.t().contiguous().to(cuda).t()
    out = ops.mm(A.to(cuda), Bd)
    assert out.dtype == dtype and out.shape == (M, N)
    assert_tol(out, O.mm(npy(A), npy(B)), dtype)


@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("M,N,K", [(256, 512, 2048), (130, 384, 4096)])
def test_mm_few_tiles_splitk(cuda, layout, M, N, K):
    """Few output tiles and a long K: ops.mm takes split-K through the addmm
    entry point (workspace partials, fixed-order sum)."""
    A, B = gen((M, K), torch.bfloat16, seed=21), gen((K, N), torch.bfloat16, 0.02, seed=22)
    lib = _lib.load()
    assert lib.kuiops_query_workspace(_lib.OP_ADDMM, M, N, K) > 0      # the split path is taken
    Bd = B.to(cuda) if layout == "row" else B.t().contiguous().to(cuda).t()
    out = ops.mm(A.to(cuda), Bd)
    assert torch.equal(out, ops.mm(A.to(cuda), Bd))
    assert_tol(out, O.mm(npy(A), npy(B)), torch.bfloat16)


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (17, 9, 13), (64, 64, 64)])
def test_mm_f32_f64(cuda, M, N, K):
    for dt in (torch.float32, torch.float64):
        A, B = gen((M, K), dt, seed=3), gen((K, N), dt, seed=4)
        out = ops.mm(A.to(cuda), B.to(cuda))
        assert_tol(out, O.mm(npy(A), npy(B)), dt)


def test_mm_golden(cuda, golden):
    A, B = torch.from_numpy(golden["mm_f32_A"]), torch.from_numpy(golden["mm_f32_B"])
    np.testing.assert_allclose(npy(ops.mm(A.to(cuda), B.to(cuda))), golden["mm_f32_C"], rtol=1e-3, atol=1e-3)
    Ab = torch.from_numpy(golden["mm_bf16_A"].view(np.int16)).view(torch.bfloat16)
    Bb = torch.from_numpy(golden["mm_bf16_B"].view(np.int16)).view(torch.bfloat16)
    out = ops.mm(Ab.to(cuda), Bb.to(cuda))
    assert_tol(out, golden["mm_bf16_C32"], torch.bfloat16)
    # the kernel rounds the fp32 accumulator once: equal to the rounded oracle
    # up to fp32 summation order (at most one bf16 ulp)
    got = out.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.int32)
    exp = O.f32_to_bf16_bits(golden["mm_bf16_C32"]).astype(np.int32)
    assert np.abs(got - exp).max() <= 1


def test_mm_closed_forms(cuda):
    # integer-valued bf16 operands: every product and partial sum is exact in fp32
    g = torch.Generator().manual_seed(5)
    A = torch.randint(-4, 5, (256, 512), generator=g).to(torch.bfloat16)
    B = torch.randint(-4, 5, (512, 384), generator=g).to(torch.bfloat16)
    out = ops.mm(A.to(cuda), B.to(cuda)).float().cpu()
    exact = A.double() @ B.double()
    small = exact.abs() <= 256          # exactly representable in bf16
    assert torch.equal(out[small], exact[small].float())
    eye = torch.eye(512, dtype=torch.bfloat16)
    assert torch.equal(ops.mm(A.to(cuda), eye.to(cuda)).cpu(), A)


# Shapes that take the 4-wave 256x256 kernel (K % 128 == 0, K >= 512, at
# least 128 tiles) with partial edge tiles in M and N.
WAVE_SHAPES = [(2000, 4100, 640), (4096, 2056, 512), (1288, 6400, 1024)]


@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("M,N,K", WAVE_SHAPES)
@pytest.mark.parametrize("kind", ["row", "full", "none"])
def test_addmm_wave_kernel_edges(cuda, layout, M, N, K, kind):
    """Large-tile kernel paths: ragged last tiles, the three addend kinds
    (bias row, full C, beta = 0) with alpha / beta != 1, and both B layouts,
    every output against the oracle."""
    A = gen((M, K), torch.bfloat16, seed=11)
    B = gen((K, N), torch.bfloat16, 0.05, seed=12)
    C = gen((N,) if kind == "row" else (M, N), torch.bfloat16, seed=13)
    alpha, beta = (0.5, 0.0) if kind == "none" else (0.5, 2.0)
    Bd = B.to(cuda) if layout == "row" else B.t().contiguous().to(cuda).t()
    out = ops.addmm(C.to(cuda), A.to(cuda), Bd, beta=beta, alpha=alpha)
    assert out.shape == (M, N)
    assert_tol(out, O.addmm(npy(C), npy(A), npy(B), alpha, beta), torch.bfloat16)


@pytest.mark.parametrize("layout", ["row", "col"])
def test_mm_wave_kernel_f32_out(cuda, layout):
    """bf16 operands, fp32 output, on the large-tile kernel (ragged N)."""
    M, N, K = 2048, 4104, 768
    A = gen((M, K), torch.bfloat16, seed=14)
    B = gen((K, N), torch.bfloat16, 0.05, seed=15)
    Bd = B.to(cuda) if layout == "row" else B.t().contiguous().to(cuda).t()
    out = ops.mm(A.to(cuda), Bd, out_dtype=torch.float32)
    assert out.dtype == torch.float32 and out.shape == (M, N)
    ref = O.mm(npy(A), npy(B))
    np.testing.assert_allclose(npy(out), ref, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("alpha,beta", [(1.0, 1.0), (0.5, 2.0)])
def test_addmm_golden(cuda, golden, dtype, alpha, beta):
    dt = "f32" if dtype == torch.float32 else "bf16"
    tag = "11" if alpha == 1.0 else "052"

    def t(name):
        a = golden[f"addmm_{dt}_{name}"]
        return (torch.from_numpy(a) if dt == "f32" else torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)).to(cuda)
    A, B, C2, C1 = t("A"), t("B"), t("C2"), t("C1")
    out2 = ops.addmm(C2, A, B, beta=beta, alpha=alpha)
    out1 = ops.addmm(C1, A, B, beta=beta, alpha=alpha)
    ref2 = O.addmm(npy(C2), npy(A), npy(B), alpha, beta)
    ref1 = O.addmm(npy(C1), npy(A), npy(B), alpha, beta)
    assert_tol(out2, ref2, dtype)
    assert_tol(out1, ref1, dtype)


@pytest.mark.parametrize("M,N,K", [(128, 128, 8192), (64, 320, 4096), (256, 256, 2048)])
def test_addmm_splitk_deterministic(cuda, M, N, K):
    A, B = gen((M, K), torch.bfloat16, seed=6), gen((K, N), torch.bfloat16, 0.02, seed=7)
    bias = gen((N,), torch.bfloat16, 0.02, seed=8)
    Ad, Bd, bd = A.to(cuda), B.to(cuda), bias.to(cuda)
    out = ops.addmm(bd, Ad, Bd)
    again = ops.addmm(bd, Ad, Bd)
    assert torch.equal(out, again)            # fixed-order split-K reduction
    assert_tol(out, O.addmm(npy(bias), npy(A), npy(B)), torch.bfloat16)


def test_addmm_config0_cpu_shape(cuda, golden):
    # BASELINE config 0 (fp32 addmm, reduced columns) through the GPU kernels
    x, W, b = (torch.from_numpy(golden[k]).to(cuda) for k in ("cfg0_x", "cfg0_W", "cfg0_b"))
    np.testing.assert_allclose(npy(ops.addmm(b, x, W)), golden["cfg0_out"], rtol=1e-3, atol=1e-3)


def test_addmm_config0_full_shape(cuda):
    """BASELINE config 0 at its own shape: fp32 x[64,768]~N(0,1),
    W[768,3072]~N(0,.02), bias[3072]~N(0,.02), seed 0; every output against
    the oracle."""
    torch.manual_seed(0)
    x = torch.randn(64, 768)
    W = torch.randn(768, 3072) * 0.02
    b = torch.randn(3072) * 0.02
    out = ops.addmm(b.to(cuda), x.to(cuda), W.to(cuda))
    assert out.shape == (64, 3072) and out.dtype == torch.float32
    assert_tol(out, O.addmm(b.numpy(), x.numpy(), W.numpy()), torch.float32)


def test_addmm_full_size_prefill(cuda):
    """A[4096,4096]~N(0,1), B~N(0,.02), bias[4096]: every
    output against the oracle, repeatability, and bias linearity."""
    torch.manual_seed(0)
    A = torch.randn(4096, 4096, device=cuda).to(torch.bfloat16)
    B = (torch.randn(4096, 4096, device=cuda) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(4096, device=cuda) * 0.02).to(torch.bfloat16)
    out = ops.addmm(bias, A, B)
    assert torch.equal(out, ops.addmm(bias, A, B))
    assert_tol(out, O.addmm(npy(bias), npy(A), npy(B)), torch.bfloat16)
    # out(bias) - out(0) == bias up to output rounding
    out0 = ops.mm(A, B)
    d = (out.float() - out0.float() - bias.float()).abs()
    assert d.max().item() <= 2 * 2 ** -8 * out0.float().abs().max().item() + 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bmm_golden(cuda, golden, dtype):
    dt = "f32" if dtype == torch.float32 else "bf16"

    def t(name):
        a = golden[f"bmm_{dt}_{name}"]
        return (torch.from_numpy(a) if dt == "f32" else torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)).to(cuda)
    out = ops.bmm(t("A"), t("B"))
    assert out.shape == (5, 17, 13)
    assert_tol(out, O.bmm(npy(t("A")), npy(t("B"))), dtype)


@pytest.mark.parametrize("b,M,K,N", [(4, 64, 64, 64), (3, 130, 72, 200), (2, 256, 128, 512),
                                     (8, 1024, 640, 1024),     # batched 4-wave kernel (K >= 512)
                                     (6, 600, 128, 1800)])     # short-K 8-wave kernel, ragged tiles
def test_bmm_vs_oracle(cuda, b, M, K, N):
    A, B = gen((b, M, K), torch.bfloat16, seed=9), gen((b, K, N), torch.bfloat16, seed=10)
    assert_tol(ops.bmm(A.to(cuda), B.to(cuda)), O.bmm(npy(A), npy(B)), torch.bfloat16)
    # a K-contiguous B (transposed view) gives the same result
    Bt = B.transpose(1, 2).contiguous().to(cuda).transpose(1, 2)
    assert torch.equal(ops.bmm(A.to(cuda), Bt), ops.bmm(A.to(cuda), B.to(cuda)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b,M,K,N", [(8, 1024, 64, 4096),      # one 64-k stage
                                     (9, 1024, 128, 3840)])    # 540 tiles: uneven tiles per work-group
@pytest.mark.parametrize("layout", ["row", "col"])
def test_bmm_persistent_short_k(cuda, dtype, b, M, K, N, layout):
    """Short-K batched GEMM with at least two full tiles per CU: the
    persistent kernel that stores each tile while loading the next (B as
    given, or a K-contiguous transposed view as in q @ k^T)."""
    A, B = gen((b, M, K), dtype, seed=21), gen((b, K, N), dtype, seed=22)
    Bd = B.to(cuda) if layout == "row" else B.transpose(1, 2).contiguous().to(cuda).transpose(1, 2)
    out = ops.bmm(A.to(cuda), Bd)
    assert_tol(out, O.bmm(npy(A), npy(B)), dtype)


def test_bmm_full_size(cuda):
    """BASELINE config 2b: bmm 32 x [2048,128] x [128,2048]: every batch
    against the oracle in full."""
    torch.manual_seed(1)
    A = torch.randn(32, 2048, 128, device=cuda).to(torch.bfloat16)
    B = torch.randn(32, 128, 2048, device=cuda).to(torch.bfloat16)
    out = ops.bmm(A, B)
    An, Bn = npy(A), npy(B)
    for bi in range(0, 32, 8):
        assert_tol(out[bi:bi + 8], O.bmm(An[bi:bi + 8], Bn[bi:bi + 8]), torch.bfloat16)


@pytest.mark.parametrize("M", [1, 4, 16, 33, 64])
@pytest.mark.parametrize("layout", ["row", "col"])
def test_decode_gemm_vs_oracle(cuda, M, layout):
    """x[M,4096] @ W[4096,11008] (W~N(0,.02)), split-K."""
    x = gen((M, 4096), torch.bfloat16, seed=11)
    W = gen((4096, 11008), torch.bfloat16, 0.02, seed=12)
    Wd = W.to(cuda) if layout == "row" else W.t().contiguous().to(cuda).t()
    out = ops.mm(x.to(cuda), Wd)
    assert torch.equal(out, ops.mm(x.to(cuda), Wd))          # bitwise repeatable
    assert_tol(out, O.mm(npy(x), npy(W)), torch.bfloat16)


@pytest.mark.parametrize("M,N,K", [(4, 4096, 11008), (16, 2048, 8192), (1, 8192, 2048), (64, 4096, 4104),
                                   (5, 11008, 4104), (33, 11008, 1000)])
def test_decode_gemm_ragged_k_and_splits(cuda, M, N, K):
    """Row-major W shapes of the Llama decode projections: K not a multiple of
    the per-wave pipeline (the last K parts are short or empty), one or several
    K splits, and a W view with ldw > N."""
    x = gen((M, K), torch.bfloat16, seed=16)
    Wbig = gen((K, N + 64), torch.bfloat16, 0.02, seed=17)
    for W in (Wbig[:, :N].contiguous(), Wbig[:, 32:32 + N]):
        Wd = Wbig.to(cuda)[:, :N].contiguous() if W.is_contiguous() else Wbig.to(cuda)[:, 32:32 + N]
        out = ops.mm(x.to(cuda), Wd)
        assert torch.equal(out, ops.mm(x.to(cuda), Wd))
        assert_tol(out, O.mm(npy(x), npy(W)), torch.bfloat16)
        o32 = ops.mm(x.to(cuda), Wd, out_dtype=torch.float32)
        np.testing.assert_allclose(npy(o32), O.mm(npy(x), npy(W)), rtol=1e-4, atol=1e-4)


def test_decode_gemm_split_sequence_keeps_counters_zero(cuda):
    """Row-major decode GEMMs whose K split is summed by the last-arriving
    work-group of each strip: alternating shapes (different split counts and
    partial layouts over one workspace) stay exact and bitwise repeatable, and
    leave the workspace's arrival counters at zero."""
    shapes = [(16, 4096, 11008), (1, 2048, 8192), (4, 4096, 4096), (16, 2048, 8192), (1, 4096, 4096)]
    firsts = {}
    for rep in range(2):
        for (M, N, K) in shapes:
            x = gen((M, K), torch.bfloat16, seed=M + K)
            W = gen((K, N), torch.bfloat16, 0.02, seed=N)
            out = ops.mm(x.to(cuda), W.to(cuda))
            if rep == 0:
                assert_tol(out, O.mm(npy(x), npy(W)), torch.bfloat16)
                firsts[(M, N, K)] = out
            else:
                assert torch.equal(out, firsts[(M, N, K)])
    torch.cuda.synchronize()
    ws = ops.workspace_buffer(cuda, "gemv")
    assert not ws[:16384].any()


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("N,K", [(512, 8), (1000, 4104), (11008, 4096), (4104, 520), (2048, 8192)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_gemm_row_stream(cuda, M, N, K, dtype):
    """Row-streaming decode GEMM (M <= 2, row-major W, N >= 512): a ragged last
    512-column block, one 8-row group (K = 8), one or several K splits merged
    in split order, a strided W view, bias, fp32 output; bitwise repeatable."""
    x = gen((M, K), dtype, seed=21)
    Wbig = gen((K, N + 16), dtype, 0.02, seed=22)
    b = gen((N,), dtype, seed=23)
    ref = O.mm(npy(x), npy(Wbig[:, 8:8 + N]))
    Wd = Wbig.to(cuda)[:, 8:8 + N]
    out = ops.mm(x.to(cuda), Wd)
    assert torch.equal(out, ops.mm(x.to(cuda), Wd))
    assert_tol(out, ref, dtype)
    o32 = ops.mm(x.to(cuda), Wd, out_dtype=torch.float32)
    np.testing.assert_allclose(npy(o32), ref, rtol=1e-4, atol=1e-4)
    ob = ops.addmm(b.to(cuda), x.to(cuda), Wd)
    assert_tol(ob, O.addmm(npy(b), npy(x), npy(Wbig[:, 8:8 + N])), dtype)
    torch.cuda.synchronize()
    assert not ops.workspace_buffer(cuda, "gemv")[:16384].any()


@pytest.mark.parametrize("M", [1, 2])
def test_decode_gemm_row_stream_strided_x_and_nan(cuda, M):
    """Row-streaming decode GEMM with x a view whose row stride exceeds K, and
    a NaN in one x element: the NaN reaches every output of its row (as in
    aten) and nothing else."""
    K, N = 2048, 4096
    xb = gen((M, K + 24), torch.bfloat16, seed=31)
    W = gen((K, N), torch.bfloat16, 0.02, seed=32)
    x = xb.to(cuda)[:, 8:8 + K]
    out = ops.mm(x, W.to(cuda))
    assert_tol(out, O.mm(npy(xb[:, 8:8 + K]), npy(W)), torch.bfloat16)
    xn = xb.clone()
    xn[M - 1, 8 + 1000] = float("nan")
    outn = ops.mm(xn.to(cuda)[:, 8:8 + K], W.to(cuda))
    assert torch.isnan(outn[M - 1]).all()
    if M > 1:
        assert torch.equal(outn[:M - 1], out[:M - 1])


def test_decode_gemm_bias_odd_shapes(cuda):
    for (M, N, K) in [(3, 1000, 520), (1, 8, 8), (7, 4104, 4096)]:
        x, W = gen((M, K), torch.bfloat16, seed=13), gen((K, N), torch.bfloat16, 0.1, seed=14)
        b = gen((N,), torch.bfloat16, seed=15)
        out = ops.addmm(b.to(cuda), x.to(cuda), W.to(cuda))
        assert_tol(out, O.addmm(npy(b), npy(x), npy(W)), torch.bfloat16)
        # fp32 output straight from the accumulator
        o32 = ops.mm(x.to(cuda), W.to(cuda), out_dtype=torch.float32)
        np.testing.assert_allclose(npy(o32), O.mm(npy(x), npy(W)), rtol=1e-4, atol=1e-4)


def test_empty_and_degenerate(cuda):
    A = torch.zeros(0, 8, device=cuda, dtype=torch.bfloat16)
    assert ops.mm(A, torch.zeros(8, 4, device=cuda, dtype=torch.bfloat16)).shape == (0, 4)
    z = ops.mm(torch.zeros(3, 0, device=cuda, dtype=torch.bfloat16), torch.zeros(0, 5, device=cuda, dtype=torch.bfloat16))
    assert z.shape == (3, 5) and not z.any()
