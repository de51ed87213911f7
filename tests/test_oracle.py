"""Pins the numpy oracle (oracle/kuiops_oracle.py) against the golden vectors
written by stock aten (tests/golden/make_golden.py) and against closed forms
that catch dropped terms, wrong signs / indices and transposed operands."""
import math

import numpy as np
import pytest

from oracle import kuiops_oracle as O

rng = np.random.default_rng(0)


def bf(bits):
    return O.bf16_bits_to_f32(bits)


# ------------------------------------------------------------------ bf16

def test_bf16_rounding_matches_aten_golden(golden):
    # aten's bf16 mm result must equal the fp32-accumulated product rounded once
    c32 = golden["mm_bf16_C32"]
    got = O.f32_to_bf16_bits(c32)
    exp = golden["mm_bf16_C"]
    # aten CPU may accumulate in a different order: allow 1-ulp differences only
    diff = np.abs(got.astype(np.int32) - exp.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.9


def test_bf16_round_to_nearest_even_cases():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0, np.inf, -np.inf], dtype=np.float32)
    r = O.round_bf16(x)
    assert r[0] == 1.0
    assert r[1] == 1.0                       # tie -> even (mantissa 0)
    assert r[2] == 1.0 + 2 ** -6             # tie -> even (rounds up)
    assert r[3] == -2.5 and r[4] == 0.0 and np.isinf(r[5]) and r[6] == -np.inf
    assert np.isnan(O.round_bf16(np.array([np.nan], dtype=np.float32)))[0]


# ------------------------------------------------------------------ GEMM

def test_mm_golden(golden):
    np.testing.assert_allclose(O.mm(golden["mm_f32_A"], golden["mm_f32_B"]), golden["mm_f32_C"],
                               rtol=1e-5, atol=1e-4)
    A, B = bf(golden["mm_bf16_A"]), bf(golden["mm_bf16_B"])
    np.testing.assert_allclose(O.mm(A, B), golden["mm_bf16_C32"], rtol=1e-5, atol=1e-5)


def test_mm_closed_forms():
    A = rng.integers(-8, 8, size=(33, 40)).astype(np.float64)
    assert np.array_equal(O.mm(A, np.eye(40)), A)                    # identity
    B = rng.integers(-8, 8, size=(40, 21)).astype(np.float64)
    # one-hot rows pick rows of B (catches a transposed operand)
    onehot = np.zeros((5, 40)); onehot[np.arange(5), [3, 0, 39, 7, 7]] = 1
    assert np.array_equal(O.mm(onehot, B), B[[3, 0, 39, 7, 7]])
    # all-ones: every entry is K
    assert np.all(O.mm(np.ones((4, 17)), np.ones((17, 6))) == 17)
    # integer-valued products are exact: compare with a brute-force triple loop
    ref = np.array([[sum(A[i, k] * B[k, j] for k in range(40)) for j in range(21)] for i in range(33)])
    assert np.array_equal(O.mm(A, B), ref)
    with pytest.raises(ValueError):
        O.mm(A, B.T)


def test_addmm_golden_alpha_beta(golden):
    for dt in ("f32", "bf16"):
        A, B = golden[f"addmm_{dt}_A"], golden[f"addmm_{dt}_B"]
        C2, C1 = golden[f"addmm_{dt}_C2"], golden[f"addmm_{dt}_C1"]
        if dt == "bf16":
            A, B, C2, C1 = bf(A), bf(B), bf(C2), bf(C1)
        for tag, (al, be) in (("11", (1.0, 1.0)), ("052", (0.5, 2.0))):
            exp2, exp1 = golden[f"addmm_{dt}_out2_{tag}"], golden[f"addmm_{dt}_out1_{tag}"]
            got2 = O.addmm(C2, A, B, alpha=al, beta=be)
            got1 = O.addmm(C1, A, B, alpha=al, beta=be)
            if dt == "f32":
                np.testing.assert_allclose(got2, exp2, rtol=1e-4, atol=1e-4)
                np.testing.assert_allclose(got1, exp1, rtol=1e-4, atol=1e-4)
            else:
                np.testing.assert_allclose(got2, golden[f"addmm_{dt}_out2_{tag}_f32acc"], rtol=1e-5, atol=1e-4)
                # aten's bf16 output is the rounded value: within one bf16 ulp
                assert O.within(O.round_bf16(got2.astype(np.float32)), bf(exp2), rtol=2 ** -7, atol=1e-2)
                assert O.within(O.round_bf16(got1.astype(np.float32)), bf(exp1), rtol=2 ** -7, atol=1e-2)


def test_addmm_beta_zero_ignores_nan_addend():
    A = np.ones((2, 3)); B = np.ones((3, 2)); C = np.full((2, 2), np.nan)
    assert np.array_equal(O.addmm(C, A, B, alpha=2.0, beta=0.0), np.full((2, 2), 6.0))
    # sign of alpha / beta matters
    assert np.array_equal(O.addmm(np.ones(2), A, B, alpha=-1.0, beta=3.0), np.zeros((2, 2)))


def test_config0_addmm_golden(golden):
    got = O.addmm(golden["cfg0_b"], golden["cfg0_x"], golden["cfg0_W"])
    np.testing.assert_allclose(got, golden["cfg0_out"], rtol=1e-5, atol=1e-5)


def test_bmm_golden(golden):
    np.testing.assert_allclose(O.bmm(golden["bmm_f32_A"], golden["bmm_f32_B"]), golden["bmm_f32_C"],
                               rtol=1e-5, atol=1e-5)
    got = O.round_bf16(O.bmm(bf(golden["bmm_bf16_A"]), bf(golden["bmm_bf16_B"])).astype(np.float32))
    assert O.rel_frobenius(got, bf(golden["bmm_bf16_C"])) < 1e-2
    # batches are independent: permuting the batch permutes the output
    A, B = golden["bmm_f32_A"], golden["bmm_f32_B"]
    p = [3, 1, 4, 0, 2]
    np.testing.assert_allclose(O.bmm(A[p], B[p]), O.bmm(A, B)[p])


def test_splitk_order_is_fixed_and_close():
    A = rng.standard_normal((7, 1000)).astype(np.float32)
    B = rng.standard_normal((1000, 9)).astype(np.float32)
    full = O.mm(A, B)
    for s in (1, 3, 8):
        r1, r2 = O.splitk_mm(A, B, s), O.splitk_mm(A, B, s)
        assert np.array_equal(r1, r2)
        np.testing.assert_allclose(r1, full, rtol=1e-4, atol=1e-4)


# --------------------------------------------------------------- softmax

def test_softmax_golden(golden):
    for tag in ("128x64", "8x5x33"):
        np.testing.assert_allclose(O.softmax(golden[f"softmax_{tag}_X"]), golden[f"softmax_{tag}_Y"],
                                   rtol=1e-5, atol=1e-6)
        got = O.round_bf16(O.softmax(bf(golden[f"softmax_{tag}_Xb"])).astype(np.float32))
        assert O.within(got, bf(golden[f"softmax_{tag}_Yb"]), rtol=2 ** -7, atol=1e-3)


def test_softmax_closed_forms():
    assert np.allclose(O.softmax(np.full((3, 10), 4.2)), 0.1)              # uniform row
    x = rng.standard_normal((4, 50))
    assert np.allclose(O.softmax(x), O.softmax(x + 7.5))                   # shift invariance
    assert np.allclose(O.softmax(x).sum(-1), 1.0)
    big = np.array([[0.0, 1000.0, 0.0]])
    assert np.allclose(O.softmax(big), [[0, 1, 0]])                        # one hot at a huge margin
    two = np.array([[0.0, math.log(3.0)]])
    assert np.allclose(O.softmax(two), [[0.25, 0.75]])                     # sign of the exponent


# ------------------------------------------------------------------ SDPA

def test_sdpa_golden(golden):
    Q, K, V, bias = golden["sdpa_Q"], golden["sdpa_K"], golden["sdpa_V"], golden["sdpa_bias"]
    out, lse = O.sdpa(Q, K, V, scale=0.3, bias=bias)
    np.testing.assert_allclose(out, golden["sdpa_out_bias"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(lse, golden["sdpa_lse_bias"], rtol=1e-5, atol=1e-5)
    out, _ = O.sdpa(Q, K, V, causal=True)
    np.testing.assert_allclose(out, golden["sdpa_out_causal"], rtol=1e-4, atol=1e-5)
    out, _ = O.sdpa(Q, K, V)
    np.testing.assert_allclose(out, golden["sdpa_out_full"], rtol=1e-4, atol=1e-5)
    out, _ = O.sdpa(bf(golden["sdpa_bf16_Q"]), bf(golden["sdpa_bf16_K"]), bf(golden["sdpa_bf16_V"]), causal=True)
    np.testing.assert_allclose(out, golden["sdpa_bf16_out_causal"], rtol=1e-4, atol=1e-5)


def test_sdpa_closed_forms():
    q = rng.standard_normal((1, 2, 6, 8)); k = rng.standard_normal((1, 2, 9, 8))
    vconst = np.broadcast_to(rng.standard_normal((1, 2, 1, 8)), (1, 2, 9, 8))
    out, _ = O.sdpa(q, k, vconst)
    assert np.allclose(out, vconst[:, :, :6])                              # constant V -> V
    v = rng.standard_normal((1, 2, 9, 8))
    out, lse = O.sdpa(q, k[:, :, :1], v[:, :, :1])
    assert np.allclose(out, np.broadcast_to(v[:, :, :1], out.shape))       # one key -> V0
    assert np.allclose(lse, np.einsum("nhle,nhe->nhl", q, k[:, :, 0]) / math.sqrt(8))
    out, _ = O.sdpa(q, k, v, causal=True)
    assert np.allclose(out[:, :, 0], v[:, :, 0])                           # causal row 0 -> V0
    # brute force on one row
    sc = np.array([q[0, 1, 3] @ k[0, 1, j] / math.sqrt(8) for j in range(4)])
    w = np.exp(sc - sc.max()); w /= w.sum()
    assert np.allclose(out[0, 1, 3], (w[:, None] * v[0, 1, :4]).sum(0))
    # bottom-right alignment: the last query sees every key
    o_br, _ = O.sdpa(q[:, :, -1:], k, v, causal=True, align="bottom_right")
    o_full, _ = O.sdpa(q[:, :, -1:], k, v)
    assert np.allclose(o_br, o_full)
    # grouped-query heads read KV head h // (hq / hkv)
    q4 = rng.standard_normal((1, 4, 3, 8))
    og, _ = O.sdpa(q4, k, v)
    for h in range(4):
        oh, _ = O.sdpa(q4[:, h:h + 1], k[:, h // 2:h // 2 + 1], v[:, h // 2:h // 2 + 1])
        assert np.allclose(og[:, h:h + 1], oh)
    # a row with no visible key: out 0, lse -inf
    o0, l0 = O.sdpa(q[:, :, :1], k[:, :, :0], v[:, :, :0])
    assert np.all(o0 == 0) and np.all(np.isneginf(l0))


# ------------------------------------------------------------------ topk

def test_topk_golden(golden):
    X = golden["topk_X"]
    for kk in (1, 5, 64, 300):
        v, i = O.topk(X, kk)
        assert np.array_equal(v, golden[f"topk_{kk}_v"]) and np.array_equal(i, golden[f"topk_{kk}_i"])
        v, i = O.topk(X, kk, largest=False)
        assert np.array_equal(v, golden[f"topk_{kk}_sv"]) and np.array_equal(i, golden[f"topk_{kk}_si"])


def test_topk_ties_nan_and_brute_force():
    x = np.array([[1.0, 3.0, 3.0, -1.0, 3.0, np.nan, 2.0]], dtype=np.float32)
    v, i = O.topk(x, 4)
    assert np.isnan(v[0, 0]) and i[0, 0] == 5
    assert list(i[0, 1:]) == [1, 2, 4]                       # ties: ascending index
    v, i = O.topk(x, 2, largest=False)
    assert list(i[0]) == [3, 0]
    v, i = O.topk(x, 7, largest=False)
    assert i[0, -1] == 5                                     # NaN last when smallest
    for _ in range(20):
        row = rng.permutation(30).astype(np.float32)[None]
        k = int(rng.integers(1, 30))
        v, i = O.topk(row, k)
        assert list(v[0]) == sorted(row[0].tolist(), reverse=True)[:k]
        assert np.array_equal(row[0, i[0]], v[0])


# ------------------------------------------------------- gather / index

def test_gather_golden_and_loops(golden):
    for shape, dim in (((8, 5), 1), ((8, 5), 0), ((4, 3, 6), 2)):
        tag = "x".join(map(str, shape)) + f"_d{dim}"
        inp, idx = golden[f"gather_{tag}_inp"], golden[f"gather_{tag}_idx"]
        got = O.gather(inp, dim, idx)
        assert np.array_equal(got, golden[f"gather_{tag}_out"])
        for pos in np.ndindex(*idx.shape):
            src = list(pos); src[dim] = idx[pos]
            assert got[pos] == inp[tuple(src)]
    with pytest.raises(IndexError):
        O.gather(np.zeros((2, 2)), 1, np.array([[2, 0], [0, 0]]))


def test_index_golden(golden):
    assert np.array_equal(O.index(golden["index_emb"], 0, golden["index_ids"]), golden["index_out"])
    assert np.array_equal(O.index(golden["index3_inp"], 1, golden["index3_ids"]), golden["index3_out"])
    with pytest.raises(IndexError):
        O.index(np.zeros((3, 2)), 0, np.array([3]))


def test_verify_metric_ignores_nonfinite():
    a = rng.standard_normal((4, 8)); b = a.copy()
    a[0] = np.nan; b[0] = 0.0
    assert O.rel_frobenius(a, b) == 0.0
    assert O.rel_frobenius(a + 1.0, b) > 0.1


# ------------------------------------------- sort / cumsum / scatter / sampling

def test_sort_golden_ties_nan_zero(golden):
    X = golden["sort_X"]
    for tag, desc in (("asc", False), ("desc", True)):
        v, i = O.sort(X, descending=desc)
        np.testing.assert_array_equal(v, golden[f"sort_{tag}_v"])       # NaN == NaN positionally
        np.testing.assert_array_equal(i, golden[f"sort_{tag}_i"])
    v, i = O.sort(golden["sortw_X"], descending=True)
    np.testing.assert_array_equal(i, golden["sortw_i"])
    np.testing.assert_array_equal(v, golden["sortw_v"])


def test_sort_brute_force_stable():
    # python's sorted() is stable: ties keep index order; NaN last (ascending)
    x = rng.integers(-3, 4, size=40).astype(np.float32)
    x[[3, 17]] = np.nan
    x[5], x[6] = -0.0, 0.0
    key = lambda j: (1, 0.0) if np.isnan(x[j]) else (0, float(x[j]) + 0.0)  # noqa: E731
    order = sorted(range(40), key=key)
    v, i = O.sort(x)
    np.testing.assert_array_equal(i, order)
    rev = sorted(range(40), key=lambda j: (0, 0.0) if np.isnan(x[j]) else (1, -float(x[j]) + 0.0))
    np.testing.assert_array_equal(O.sort(x, descending=True)[1], rev)


def test_cumsum_golden_and_closed_forms(golden):
    np.testing.assert_allclose(O.cumsum(golden["cumsum_X"]), golden["cumsum_Y"], rtol=1e-4, atol=1e-3)
    np.testing.assert_array_equal(O.cumsum(golden["cumsum_i64_X"]), golden["cumsum_i64_Y"])
    np.testing.assert_array_equal(O.cumsum(np.ones((2, 9), np.int64)), np.tile(np.arange(1, 10), (2, 1)))
    x = rng.standard_normal((3, 50))
    c = O.cumsum(x)
    np.testing.assert_allclose(np.diff(c, axis=-1), x[:, 1:], atol=1e-12)   # differences give back x
    assert np.allclose(c[:, 0], x[:, 0])


def test_scatter_golden_and_loop(golden):
    out = O.scatter(golden["scatter_self"], 1, golden["scatter_idx"], golden["scatter_src"])
    np.testing.assert_array_equal(out, golden["scatter_out"])
    outb = O.scatter(golden["scatter_bool_src"], 1, golden["scatter_idx"], golden["scatter_bool_src"])
    np.testing.assert_array_equal(outb, golden["scatter_bool_out"])
    # scatter inverts gather along a permutation
    perm = golden["scatter_idx"]
    src = golden["scatter_src"]
    np.testing.assert_array_equal(O.gather(O.scatter(np.zeros_like(src), 1, perm, src), 1, perm), src)
    # a partial index only touches its targets
    base = np.arange(12, dtype=np.float32).reshape(3, 4)
    out = O.scatter(base, 0, np.array([[2, 0]]), np.array([[-1.0, -2.0]], np.float32))
    assert out[2, 0] == -1 and out[0, 1] == -2 and out[1, 1] == 5 and out[0, 0] == 0


def test_multinomial_inverse_cdf_closed_forms():
    # one-hot rows always draw their hot index
    p = np.zeros((3, 10)); p[0, 4] = 1; p[1, 0] = 0.3; p[2, 9] = 5
    u = rng.random((3, 6))
    np.testing.assert_array_equal(O.multinomial(p, u), np.array([[4] * 6, [0] * 6, [9] * 6]))
    # uniform weights: u in the middle of bucket k draws k
    n = 16
    u = (np.arange(n) + 0.5) / n
    np.testing.assert_array_equal(O.multinomial(np.ones((1, n)), u.reshape(1, -1))[0], np.arange(n))
    # zero weights are never drawn, also at the edges u = 0 and u -> 1
    p = np.array([[0, 0, 2, 0, 1, 0, 0]], dtype=np.float64)
    d = O.multinomial(p, np.array([[0.0, 0.5, 0.6666, 0.6667, 0.999999999]]))
    np.testing.assert_array_equal(d[0], [2, 2, 2, 4, 4])
    # against numpy's searchsorted on the CDF
    p = rng.random((4, 50)) * (rng.random((4, 50)) > 0.3)
    u = rng.random((4, 20))
    cdf = np.cumsum(p, axis=1)
    exp = np.stack([np.searchsorted(cdf[r], u[r] * cdf[r, -1], side="right") for r in range(4)])
    np.testing.assert_array_equal(O.multinomial(p, u), exp)
    with pytest.raises(ValueError):
        O.multinomial(np.array([[1.0, -1.0]]), np.array([[0.5]]))


def test_top_p_filter_matches_transformers():
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers.generation.logits_process")
    scores = (rng.standard_normal((3, 300)) * 3).astype(np.float32)
    for top_p in (0.5, 0.9, 0.95):
        warp = tr.TopPLogitsWarper(top_p=top_p)
        exp = warp(None, torch.from_numpy(scores.copy())).numpy()
        got = O.top_p_filter(scores, top_p)
        np.testing.assert_array_equal(np.isinf(got), np.isinf(exp))
        np.testing.assert_array_equal(got[~np.isinf(got)], exp[~np.isinf(exp)])


# ------------------------------------------------- multi-tensor index

def test_index_multi_against_aten_golden_and_numpy(golden):
    out = O.index_multi(golden["index2_mask"], 0, [golden["index2_i0"], golden["index2_i1"]])
    assert out.dtype == np.bool_ and np.array_equal(out, golden["index2_out"])
    out3 = O.index_multi(golden["index3d_inp"], 1, [golden["index3d_j0"], golden["index3d_j1"]])
    assert np.array_equal(out3, golden["index3d_out"])
    # numpy's own fancy indexing (the textbook routine) on a random case
    x = rng.standard_normal((4, 5, 6, 3))
    a, b = rng.integers(-5, 5, (2, 3)), rng.integers(0, 6, (1, 3))
    assert np.array_equal(O.index_multi(x, 1, [a, b]), x[:, a, b])
    # one index tensor reduces to the single-axis index
    ids = rng.integers(0, 5, (7,))
    assert np.array_equal(O.index_multi(x, 1, [ids]), O.index(x, 1, ids))
