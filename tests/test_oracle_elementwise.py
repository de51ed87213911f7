"""Pins the oracle's elementwise / mean / cat restatement
(oracle/kuiops_oracle.py) against stock-aten golden vectors
(tests/golden/make_golden.py) and against closed forms."""
import numpy as np
import pytest

from oracle import kuiops_oracle as O

EXACT = ("neg", "sq", "p3", "add", "sub", "mul", "div", "mulcol", "adds", "muls", "where")
# aten's CPU kernels are not correctly rounded for these (sqrt included)
TRANSC = ("silu", "cos", "sin", "exp", "rsqrt", "p15", "sqrt")


def _load(golden, dt, key):
    a = golden[f"ew_{dt}_{key}"]
    return O.bf16_bits_to_f32(a) if dt == "bf16" else a


def _oracle(golden, dt, key):
    x, y, col = (_load(golden, dt, k) for k in ("x", "y", "col"))
    E = O.elementwise
    table = {
        "neg": lambda: E("neg", x), "silu": lambda: E("silu", x), "cos": lambda: E("cos", x),
        "sin": lambda: E("sin", x), "exp": lambda: E("exp", x), "sq": lambda: E("pow", x, exponent=2),
        "p3": lambda: E("pow", x, exponent=3, store=dt), "p15": lambda: E("pow", np.abs(x), exponent=1.5),
        "rsqrt": lambda: E("rsqrt", y), "sqrt": lambda: E("sqrt", y), "add": lambda: E("add", x, y),
        "add_a": lambda: E("add", x, y, alpha=0.5), "sub": lambda: E("sub", x, y), "mul": lambda: E("mul", x, y),
        "div": lambda: E("div", x, y), "mulcol": lambda: E("mul", x, col), "adds": lambda: E("add", x, 1e-6),
        "muls": lambda: E("mul", x, 0.125), "where": lambda: E("where", E("gt", x, 0.0), x, y),
    }
    return O.round_dtype(table[key](), dt)


def _ulps(a, b, dt):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    if dt == "bf16":
        ia, ib = O.f32_to_bf16_bits(a).astype(np.int64), O.f32_to_bf16_bits(b).astype(np.int64)
    else:
        ia, ib = a.view(np.int32).astype(np.int64), b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("key", EXACT + ("add_a",))
def test_exact_ops_match_aten_bitwise(golden, dt, key):
    got = _oracle(golden, dt, key)
    want = _load(golden, dt, key)
    if key == "add_a":                       # a fused multiply-add either way: at most one rounding apart
        assert _ulps(got, want, dt).max() <= 1
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("key", TRANSC)
def test_transcendental_ops_within_two_ulps_of_aten(golden, dt, key):
    got = _oracle(golden, dt, key)
    want = _load(golden, dt, key)
    u = _ulps(got, want, dt)
    assert u.max() <= 2, (key, dt, u.max())
    if dt == "bf16":
        assert (u == 0).mean() > 0.95


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_comparisons_match_aten(golden, dt):
    x, y = _load(golden, dt, "x"), _load(golden, dt, "y")
    assert np.array_equal(O.elementwise("lt", x, 0.5), golden[f"ew_{dt}_lt"])
    assert np.array_equal(O.elementwise("le", x, y), golden[f"ew_{dt}_le"])
    assert np.array_equal(O.elementwise("eq", x, 0.0), golden[f"ew_{dt}_eq"])


def test_promotion_bitwise_and_integer_ops(golden):
    xb = O.bf16_bits_to_f32(golden["ew_bf16_x"])
    # bf16 * fp32 promotes to fp32: the bf16 values exactly, one fp32 product
    from_golden_y = golden["ew_f32_y"]
    assert np.array_equal(O.elementwise("mul", xb, from_golden_y), golden["ew_mixed_out"])
    b1, b2 = golden["ew_b1"], golden["ew_b2"]
    assert np.array_equal(O.elementwise("bitwise_and", b1, b2), golden["ew_band"])
    assert np.array_equal(O.elementwise("bitwise_or", b1, b2), golden["ew_bor"])
    assert np.array_equal(O.elementwise("bitwise_not", b1), golden["ew_bnot"])
    i = golden["ew_i64"]
    assert np.array_equal(O.elementwise("add", i, 3, compute="i64"), golden["ew_i64_add"])
    assert np.array_equal(O.elementwise("mul", i, i, compute="i64"), golden["ew_i64_mul"])


def test_elementwise_closed_forms():
    x = np.linspace(-30, 30, 121, dtype=np.float32)
    s = O.elementwise("silu", x)
    assert s[60] == 0.0                                   # silu(0) = 0
    np.testing.assert_allclose(s[-1], 30.0, rtol=1e-6)    # silu(x) -> x for large x
    np.testing.assert_allclose(s[0], 0.0, atol=1e-10)     # and -> 0 for very negative x
    np.testing.assert_allclose(O.elementwise("sin", x) ** 2 + O.elementwise("cos", x) ** 2, 1.0, rtol=1e-6)
    assert O.elementwise("rsqrt", np.float32([4.0, 0.25]))[0] == 0.5
    assert np.array_equal(O.elementwise("sub", x, x), np.zeros_like(x))
    assert np.array_equal(O.elementwise("add", x, x, alpha=0.0), x)
    assert np.array_equal(O.elementwise("sub", x, 1.0, alpha=-1.0), x + 1)   # a - (-1) * 1
    assert np.array_equal(O.elementwise("where", x > 0, x, 0.0), np.maximum(x, 0))
    assert np.array_equal(O.elementwise("pow", x, exponent=-1), np.float32(1) / x)
    # broadcast: a column times a row is the outer product
    r, c = np.arange(1, 5, dtype=np.float32), np.arange(1, 4, dtype=np.float32)[:, None]
    assert np.array_equal(O.elementwise("mul", r, c), np.outer(c[:, 0], r))


def test_mean_against_aten_and_closed_forms(golden):
    got = O.round_dtype(O.mean_lastdim(O.bf16_bits_to_f32(golden["mean_bf16_x"]), keepdim=True), "bf16")
    want = O.bf16_bits_to_f32(golden["mean_bf16_out"])
    assert got.shape == want.shape and _ulps(got, want, "bf16").max() <= 1
    got32 = O.mean_lastdim(golden["mean_f32_x"])
    np.testing.assert_allclose(got32, golden["mean_f32_out"], rtol=1e-5, atol=1e-7)
    c = np.full((3, 7), 2.5)
    assert np.array_equal(O.mean_lastdim(c), np.full(3, 2.5))              # constant rows
    assert O.mean_lastdim(np.arange(10.0)[None]).item() == 4.5           # (n - 1) / 2
    assert O.mean_lastdim(np.ones((2, 3, 4)), keepdim=True).shape == (2, 3, 1)


def test_cat_against_aten(golden):
    assert np.array_equal(O.cat([golden["cat_a"], golden["cat_b"]], dim=2), golden["cat_out"])
    q = golden["cat_q"]
    rot = O.cat([O.elementwise("neg", q[..., 8:]), q[..., :8]], dim=-1)
    assert np.array_equal(rot, golden["cat_rot"])
    parts = np.split(golden["cat_out"], [5], axis=2)                      # cat then split = identity
    assert np.array_equal(parts[0], golden["cat_a"]) and np.array_equal(parts[1], golden["cat_b"])
