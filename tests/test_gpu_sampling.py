"""Sampling tail parity on the GPU: softmax (tolerance), topk / gather /
index (bit-exact) against the oracle and the aten golden fixtures."""
import numpy as np
import pytest
import torch

from kuillm_amd import ops
from oracle import kuiops_oracle as O

pytestmark = pytest.mark.gpu


def npy(t):
    return t.detach().cpu().numpy() if t.dtype not in (torch.bfloat16,) else t.detach().float().cpu().numpy()


@pytest.mark.parametrize("shape", [(128, 64), (8, 5, 33), (4, 32000), (2, 1025), (3, 40000), (1, 1)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_softmax_vs_oracle(cuda, shape, dtype):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(*shape, generator=g) * 3).to(dtype)
    out = ops.softmax(x.to(cuda))
    ref = O.softmax(npy(x).astype(np.float64))
    tol = 1e-3 if dtype == torch.bfloat16 else 1e-6
    np.testing.assert_allclose(npy(out).astype(np.float64), ref, rtol=1e-2 if dtype == torch.bfloat16 else 1e-5,
                               atol=tol)
    np.testing.assert_allclose(npy(out).astype(np.float64).sum(-1), 1.0, atol=1e-3 if dtype != torch.bfloat16 else 3e-2)


def test_softmax_golden(cuda, golden):
    for tag in ("128x64", "8x5x33"):
        out = ops.softmax(torch.from_numpy(golden[f"softmax_{tag}_X"]).to(cuda))
        np.testing.assert_allclose(npy(out), golden[f"softmax_{tag}_Y"], rtol=1e-5, atol=1e-6)


def test_softmax_special_values(cuda):
    x = torch.tensor([[0.0, float("-inf"), 1.0, float("-inf")],
                      [float("nan"), 0.0, 1.0, 2.0],
                      [5.0, 5.0, 5.0, 5.0]], device=cuda)
    out = ops.softmax(x).cpu()
    ref = torch.softmax(x.cpu(), -1)
    assert torch.allclose(out[0], ref[0]) and out[0, 1] == 0
    assert torch.isnan(out[1]).all() and torch.isnan(ref[1]).all()
    assert torch.allclose(out[2], torch.full((4,), 0.25))
    big = torch.full((1, 50000), float("-inf"), device=cuda)
    big[0, 1234] = 3.0
    out = ops.softmax(big)
    assert out[0, 1234] == 1 and out.sum() == 1


def test_topk_golden(cuda, golden):
    X = torch.from_numpy(golden["topk_X"]).to(cuda)
    for kk in (1, 5, 64, 300):
        v, i = ops.topk(X, kk)
        assert np.array_equal(npy(v), golden[f"topk_{kk}_v"]) and np.array_equal(npy(i), golden[f"topk_{kk}_i"])
        v, i = ops.topk(X, kk, largest=False)
        assert np.array_equal(npy(v), golden[f"topk_{kk}_sv"]) and np.array_equal(npy(i), golden[f"topk_{kk}_si"])


def tie_free_rows(m, n, dtype, seed):
    """m rows of n distinct values, exactly representable in `dtype`."""
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.bfloat16:
        # distinct finite non-zero bf16 bit patterns of both signs
        pats = torch.cat([torch.arange(1, 0x7F80), torch.arange(0x8001, 0xFF80)])
        rows = [pats[torch.randperm(pats.numel(), generator=g)[:n]] for _ in range(m)]
        return torch.stack(rows).to(torch.int16).view(torch.bfloat16)
    vals = (torch.arange(n, dtype=torch.float32) - n / 2) / 1024
    return torch.stack([vals[torch.randperm(n, generator=g)] for _ in range(m)])


@pytest.mark.parametrize("m,n,k,dtype", [
    (1, 32000, 1, torch.float32), (4, 32000, 50, torch.float32), (3, 1000, 1000, torch.float32),
    (16, 777, 7, torch.float32), (2, 100000, 20, torch.float32),
    (1, 32000, 1, torch.bfloat16), (4, 32000, 50, torch.bfloat16), (3, 1000, 1000, torch.bfloat16)])
def test_topk_vs_oracle(cuda, m, n, k, dtype):
    x = tie_free_rows(m, n, dtype, seed=n + k)
    for largest in (True, False):
        v, i = ops.topk(x.to(cuda), k, largest=largest)
        rv, ri = O.topk(npy(x), k, largest=largest)
        assert np.array_equal(npy(i), ri) and np.array_equal(npy(v), rv)
        tv, ti = torch.topk(x.to(cuda), k, largest=largest)
        assert torch.equal(i, ti) and torch.equal(v, tv)


def test_topk_ties_and_nan(cuda):
    x = torch.tensor([[1.0, 3.0, 3.0, -1.0, 3.0, float("nan"), 2.0]], device=cuda)
    v, i = ops.topk(x, 4)
    rv, ri = O.topk(npy(x), 4)
    assert np.array_equal(npy(i), ri)          # NaN first, then ties by ascending index
    assert np.isnan(npy(v)[0, 0]) and np.array_equal(npy(v)[0, 1:], rv[0, 1:])
    v, i = ops.topk(x, 7, largest=False)
    assert np.array_equal(npy(i), O.topk(npy(x), 7, largest=False)[1])
    # a tie across the k-th place keeps the lowest indices
    y = torch.zeros(1, 5000, device=cuda)
    y[0, 4000:] = 1.0
    v, i = ops.topk(y, 1020)
    assert torch.equal(i[0, :1000].cpu(), torch.arange(4000, 5000))
    assert torch.equal(i[0, 1000:].cpu(), torch.arange(0, 20))
    with pytest.raises(Exception):
        ops.topk(y, 1100)                      # k above 1024 is outside the kernel


def test_topk_threshold_ties(cuda):
    """The register-resident path (n <= 32768, k <= 512): ties at the k-th
    place keep the lowest indices, and a row whose candidates overflow the
    sort buffer (all equal) takes the general path with the same answer."""
    y = torch.zeros(1, 5000, device=cuda)
    y[0, 4000:] = 1.0
    v, i = ops.topk(y, 300)
    assert torch.equal(i[0].cpu(), torch.arange(4000, 4300)) and bool((v == 1).all())
    z = torch.zeros(2, 32000, device=cuda)
    v, i = ops.topk(z, 10)
    assert torch.equal(i.cpu(), torch.arange(10).expand(2, 10))
    # softmax probabilities of random logits (the sampling tail's input)
    p = torch.softmax(torch.randn(3, 32000, generator=torch.Generator().manual_seed(9)), -1).to(cuda)
    for k in (1, 20, 50, 512):
        v, i = ops.topk(p, k)
        tv, ti = torch.topk(p, k)
        assert torch.equal(v, tv) and torch.equal(i, ti)


def test_topk_other_dim(cuda):
    x = torch.randn(50, 3, device=cuda)
    v, i = ops.topk(x, 5, dim=0)
    tv, ti = torch.topk(x, 5, dim=0)
    assert torch.equal(v, tv) and torch.equal(i, ti)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64, torch.uint8])
def test_gather_vs_oracle(cuda, golden, dtype):
    for shape, dim in (((8, 5), 1), ((8, 5), 0), ((4, 3, 6), 2)):
        tag = "x".join(map(str, shape)) + f"_d{dim}"
        inp = torch.from_numpy(golden[f"gather_{tag}_inp"] * 10).to(dtype)
        idx = torch.from_numpy(golden[f"gather_{tag}_idx"])
        out = ops.gather(inp.to(cuda), dim, idx.to(cuda))
        assert torch.equal(out.cpu(), torch.gather(inp, dim, idx))
        if dtype == torch.float32:
            assert np.array_equal(npy(out), O.gather(npy(inp), dim, npy(idx)))
    big = torch.randn(64, 32000, device=cuda)
    idx = torch.randint(0, 32000, (64, 50), device=cuda)
    assert torch.equal(ops.gather(big, 1, idx), torch.gather(big, 1, idx))


def test_gather_out_of_range_flag(cuda):
    inp = torch.randn(2, 3, device=cuda)
    with pytest.raises(IndexError):
        ops.gather(inp, 1, torch.tensor([[0, 3], [1, 2]], device=cuda), check=True)


def test_index_vs_oracle(cuda, golden):
    E = torch.from_numpy(golden["index_emb"])
    ids = torch.from_numpy(golden["index_ids"])
    assert np.array_equal(npy(ops.index(E.to(cuda), 0, ids.to(cuda))), golden["index_out"])
    T3, ids2 = torch.from_numpy(golden["index3_inp"]), torch.from_numpy(golden["index3_ids"])
    assert np.array_equal(npy(ops.index(T3.to(cuda), 1, ids2.to(cuda))), golden["index3_out"])
    # embedding lookup at the Llama config: 16-byte row copies
    emb = torch.randn(32000, 2048, device=cuda).to(torch.bfloat16)
    tok = torch.randint(0, 32000, (1, 512), device=cuda)
    assert torch.equal(ops.index(emb, 0, tok), emb[tok])
    with pytest.raises(IndexError):
        ops.index(emb, 0, torch.tensor([32000], device=cuda), check=True)


def test_index_multi_vs_oracle(cuda, golden):
    """Several int64 index tensors on adjacent axes: the reference app's
    bool-mask call (KERNELS.md:67), a middle-axis pair with negative indices,
    broadcast index shapes, bit-exact against the aten golden and the oracle."""
    import kuillm_amd as kuipy
    m = torch.from_numpy(golden["index2_mask"]).to(cuda)
    i0, i1 = (torch.from_numpy(golden[k]).to(cuda) for k in ("index2_i0", "index2_i1"))
    out = ops.index_multi(m, 0, [i0, i1])
    assert out.dtype == torch.bool and np.array_equal(out.cpu().numpy(), golden["index2_out"])
    t = torch.from_numpy(golden["index3d_inp"]).to(cuda)
    j0, j1 = (torch.from_numpy(golden[k]).to(cuda) for k in ("index3d_j0", "index3d_j1"))
    assert np.array_equal(npy(ops.index_multi(t, 1, [j0, j1])), golden["index3d_out"])
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 40, 50, 16, generator=g).to(torch.bfloat16)
    a, b = torch.randint(-40, 40, (6, 1), generator=g), torch.randint(0, 50, (1, 9), generator=g)
    got = ops.index_multi(x.to(cuda), 1, [a.to(cuda), b.to(cuda)])
    assert np.array_equal(got.view(torch.int16).cpu().numpy(),
                          O.index_multi(x.view(torch.int16).numpy(), 1, [a.numpy(), b.numpy()]))
    kuipy.reset_verify()
    with kuipy.KuiperMode(verify=True):
        r = m[i0, i1]                       # dispatched as aten.index.Tensor with two indices
        f = t[:, j0, j1]
    assert torch.equal(r, out) and np.array_equal(npy(f), golden["index3d_out"])
    with pytest.raises(IndexError):
        ops.index_multi(t, 1, [j0, torch.tensor([7, 0, 0, 0], device=cuda)], check=True)


# ------------------------------------------- sort / cumsum / scatter / sampling

def test_sort_golden(cuda, golden):
    """Stable sort with ties, NaN and signed zeros, both directions; a row
    wider than one 2048-key chunk (bit-exact values and indices)."""
    X = torch.from_numpy(golden["sort_X"]).to(cuda)
    for tag, desc in (("asc", False), ("desc", True)):
        v, i = ops.sort(X, descending=desc)
        np.testing.assert_array_equal(v.cpu().numpy(), golden[f"sort_{tag}_v"])
        np.testing.assert_array_equal(i.cpu().numpy(), golden[f"sort_{tag}_i"])
    v, i = ops.sort(torch.from_numpy(golden["sortw_X"]).to(cuda), descending=True)
    np.testing.assert_array_equal(i.cpu().numpy(), golden["sortw_i"])
    np.testing.assert_array_equal(v.cpu().numpy(), golden["sortw_v"])


@pytest.mark.parametrize("m,n,dtype", [(1, 32000, torch.float32), (3, 2048, torch.float32), (2, 2049, torch.float32), (1, 4097, torch.float32),
                                       (5, 1, torch.float32), (4, 7000, torch.bfloat16), (2, 513, torch.float16),
                                       (1, 131072, torch.float32),
                                       (17, 65536, torch.bfloat16),    # 32 chunks x 17 rows: the per-chunk rank pass
                                       (20, 32000, torch.float32)])    # 2048-key chunks, pairwise rank pass
def test_sort_vs_oracle(cuda, m, n, dtype):
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(m, n, generator=g) * 4).to(dtype)
    for desc in (False, True):
        v, i = ops.sort(x.to(cuda), descending=desc)
        rv, ri = O.sort(npy(x), descending=desc)
        np.testing.assert_array_equal(i.cpu().numpy(), ri)
        assert torch.equal(v.cpu(), x.gather(1, torch.from_numpy(ri)))
        # against aten's stable sort too
        tv, ti = torch.sort(x, descending=desc, stable=True)
        assert torch.equal(i.cpu(), ti)


def test_sort_dim_and_empty(cuda):
    x = torch.randn(6, 5, 4)
    v, i = ops.sort(x.to(cuda), dim=1)
    tv, ti = torch.sort(x, dim=1, stable=True)
    assert torch.equal(v.cpu(), tv) and torch.equal(i.cpu(), ti)
    v, i = ops.sort(torch.empty(3, 0, device=cuda))
    assert v.shape == (3, 0) and i.shape == (3, 0)


def test_cumsum_golden_and_vs_oracle(cuda, golden):
    y = ops.cumsum(torch.from_numpy(golden["cumsum_X"]).to(cuda))
    np.testing.assert_allclose(y.cpu().numpy(), golden["cumsum_Y"], rtol=1e-4, atol=1e-3)
    yi = ops.cumsum(torch.from_numpy(golden["cumsum_i64_X"]).to(cuda))
    np.testing.assert_array_equal(yi.cpu().numpy(), golden["cumsum_i64_Y"])
    x = torch.randn(3, 50000, dtype=torch.float64)
    np.testing.assert_allclose(ops.cumsum(x.to(cuda)).cpu().numpy(), O.cumsum(x.numpy()), rtol=1e-10, atol=1e-9)
    x = torch.rand(2, 32000)                  # probabilities: the top-p cumulative sums
    np.testing.assert_allclose(ops.cumsum(x.to(cuda)).cpu().numpy(), O.cumsum(x.numpy()), rtol=1e-5, atol=1e-3)
    # along another dim
    x = torch.randint(-5, 5, (4, 7, 3))
    assert torch.equal(ops.cumsum(x.to(cuda), dim=1).cpu(), torch.cumsum(x, 1))


def test_scatter_golden(cuda, golden):
    S = torch.from_numpy(golden["scatter_self"]).to(cuda)
    idx = torch.from_numpy(golden["scatter_idx"]).to(cuda)
    out = ops.scatter(S, 1, idx, torch.from_numpy(golden["scatter_src"]).to(cuda))
    np.testing.assert_array_equal(out.cpu().numpy(), golden["scatter_out"])
    mb = torch.from_numpy(golden["scatter_bool_src"]).to(cuda)
    np.testing.assert_array_equal(ops.scatter(mb, 1, idx, mb).cpu().numpy(), golden["scatter_bool_out"])
    # partial index along dim 0, self untouched elsewhere; out-of-range flagged
    base = torch.arange(12.0).view(3, 4)
    out = ops.scatter(base.to(cuda), 0, torch.tensor([[2, 0]], device=cuda), torch.tensor([[-1.0, -2.0]], device=cuda))
    assert torch.equal(out.cpu(), base.scatter(0, torch.tensor([[2, 0]]), torch.tensor([[-1.0, -2.0]])))
    with pytest.raises(IndexError):
        ops.scatter(base.to(cuda), 0, torch.tensor([[3, 0]], device=cuda), torch.ones(1, 2, device=cuda), check=True)


@pytest.mark.parametrize("m,n,ns", [(1, 32000, 1), (4, 1000, 16), (3, 7, 50), (2, 40000, 3)])
def test_multinomial_vs_oracle(cuda, m, n, ns):
    """Draws are the inverse CDF of the given uniforms: equal to the oracle's
    (fp64 CDF) for the same uniforms; zero weights are never drawn."""
    g = torch.Generator().manual_seed(m * n)
    p = torch.rand(m, n, generator=g) * (torch.rand(m, n, generator=g) > 0.3)
    p[:, 0] = 0.0
    u = torch.rand(m, ns, generator=g)
    d = ops.multinomial(p.to(cuda), ns, replacement=True, uniforms=u.to(cuda))
    np.testing.assert_array_equal(d.cpu().numpy(), O.multinomial(p.numpy(), u.numpy()))
    assert (p.gather(1, d.cpu()) > 0).all()


def test_multinomial_distribution_and_errors(cuda):
    p = torch.tensor([0.1, 0.0, 0.6, 0.3], device=cuda)
    d = ops.multinomial(p.expand(20000, 4).contiguous(), 1, generator=torch.Generator(device=cuda).manual_seed(1))
    freq = torch.bincount(d.view(-1).cpu(), minlength=4).float() / 20000
    assert freq[1] == 0
    assert torch.allclose(freq, p.cpu(), atol=0.015)
    with pytest.raises(RuntimeError):
        ops.multinomial(torch.tensor([[1.0, -0.5]], device=cuda), 1)
    with pytest.raises(RuntimeError):
        ops.multinomial(torch.zeros(2, 5, device=cuda), 1)


def test_top_p_filter_and_sampler_vs_oracle(cuda):
    """The HF top-p tail on the GPU (sort, softmax, cumsum, scatter, masked
    fill) keeps exactly the oracle's tokens (rows with a cumulative value
    within 1e-5 of the threshold are skipped: fp32 vs fp64 sums), and the
    sampler's draws equal the oracle's for the same uniforms."""
    g = torch.Generator().manual_seed(3)
    scores = torch.randn(4, 32000, generator=g) * 3
    for top_p in (0.5, 0.9):
        got = ops.top_p_filter(scores.to(cuda), top_p).cpu().numpy()
        exp = O.top_p_filter(scores.numpy(), top_p)
        vals, _ = O.sort(scores.numpy())
        cum = O.cumsum(O.softmax(vals))
        for r in range(4):
            if np.min(np.abs(cum[r] - (1 - top_p))) < 1e-5:
                continue
            np.testing.assert_array_equal(np.isinf(got[r]), np.isinf(exp[r]))
            np.testing.assert_array_equal(got[r][~np.isinf(got[r])], exp[r][~np.isinf(exp[r])])
    u = torch.rand(4, 1, generator=g)
    tok = ops.sample_top_p(scores.to(cuda), 0.9, uniforms=u.to(cuda)).cpu().numpy()
    probs = O.softmax(O.top_p_filter(scores.numpy(), 0.9))
    np.testing.assert_array_equal(tok, O.multinomial(probs, u.numpy())[:, 0])


@pytest.mark.parametrize("min_keep", [1, 5, 0, 40000])
def test_top_p_mask_kernel_matches_aten_sequence(cuda, min_keep):
    """The fused top-p mask equals the aten sequence it replaces (le.Scalar,
    setitem of the kept tail, scatter, masked_fill) on the same sorted
    indices and cumulative probabilities, bit for bit, including a NaN score
    (sorts last, never removed), ties and min_tokens_to_keep edge values."""
    g = torch.Generator().manual_seed(min_keep + 7)
    scores = (torch.randn(3, 32000, generator=g) * 3).to(cuda)
    scores[1, 100] = float("nan")
    scores[2, :50] = 1.0                                   # ties
    for top_p in (0.3, 0.9, 1.0):
        sv, si = ops.sort(scores, -1, descending=False)
        cum = ops.cumsum(ops.softmax(sv), -1)
        remove = cum <= (1 - top_p)
        remove[..., -min_keep:] = False
        mask = ops.scatter(remove, 1, si, remove)
        ref = scores.masked_fill(mask, -float("inf"))
        got = ops.top_p_filter(scores, top_p, min_tokens_to_keep=min_keep)
        assert torch.equal(torch.isnan(got), torch.isnan(ref))
        assert torch.equal(got.nan_to_num(0.0), ref.nan_to_num(0.0))


@pytest.mark.parametrize("m,n,dtype", [(1, 32000, torch.bfloat16), (3, 32000, torch.float32), (2, 1000, torch.float16),
                                       (1, 32768, torch.float32), (4, 7, torch.float32)])
def test_softmax_top1_matches_softmax_topk(cuda, m, n, dtype):
    """The fused greedy tail returns exactly topk(softmax(x.float()), 1):
    same probability bits, same index (lowest on ties), and advances the
    decode state by one."""
    g = torch.Generator().manual_seed(n + m)
    x = (torch.randn(m, n, generator=g) * 4).to(dtype).to(cuda)
    x[0, n // 2] = x[0].max()                      # a tie at the top: the lower index wins
    pos = torch.arange(m, dtype=torch.int32, device=cuda)
    kvl = pos + 10
    prob = torch.empty(m, dtype=torch.float32, device=cuda)
    _, idx = ops.softmax_top1(x, prob_out=prob, pos=pos, kv_len=kvl)
    pv, pi = ops.topk(ops.softmax(x.float()), 1)
    assert torch.equal(idx, pi.view(-1))
    if n > 1024:
        assert torch.equal(prob, pv.view(-1))
    else:   # rows of <= 1024 take the one-wave softmax kernel (another summation order)
        torch.testing.assert_close(prob, pv.view(-1), rtol=1e-6, atol=0)
    tv, ti = torch.topk(torch.softmax(x.float(), -1), 1)
    assert torch.equal(idx.cpu(), ti.view(-1).cpu())
    assert torch.equal(pos.cpu(), torch.arange(m, dtype=torch.int32) + 1)
    assert torch.equal(kvl.cpu(), torch.arange(m, dtype=torch.int32) + 11)


def test_softmax_top1_nan_row(cuda):
    x = torch.tensor([[0.5, float("nan"), 2.0, 2.0]], device=cuda)
    _, idx = ops.softmax_top1(x)
    _, ref = ops.topk(ops.softmax(x), 1)
    assert torch.equal(idx, ref.view(-1))
