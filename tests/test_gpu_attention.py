"""Flash SDPA parity on the GPU against the fp64 numpy oracle and the aten
golden fixtures.  Tolerance (north star): rel 1e-2 / abs 1e-2 elementwise on
the output; the LSE (fp32) within 1e-3 absolute."""
import math
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from kuillm_amd import ops
from oracle import kuiops_oracle as O

pytestmark = pytest.mark.gpu


def npy(t):
    return t.detach().float().cpu().numpy()


def gen(shape, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def close(out, ref, rtol=1e-2, atol=1e-2):
    o = npy(out)
    err = np.abs(o - ref) - (atol + rtol * np.abs(ref))
    assert err.max() <= 0, f"max excess {err.max():.3e}"


CASES = [  # n, hq, hkv, l, s, d, causal
    (1, 2, 2, 128, 128, 128, False),
    (1, 2, 2, 128, 128, 128, True),
    (2, 4, 2, 200, 200, 64, True),
    (1, 3, 3, 77, 300, 128, False),
    (1, 4, 1, 65, 65, 64, True),
    (2, 2, 2, 1, 1, 128, True),
    (1, 2, 2, 300, 100, 64, True),       # more queries than keys: late rows see every key
]


@pytest.mark.parametrize("n,hq,hkv,l,s,d,causal", CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sdpa_fwd_vs_oracle(cuda, n, hq, hkv, l, s, d, causal, dtype):
    q, k, v = gen((n, hq, l, d), dtype, 1), gen((n, hkv, s, d), dtype, 2), gen((n, hkv, s, d), dtype, 3)
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=causal)
    ref, lse_ref = O.sdpa(npy(q), npy(k), npy(v), causal=causal)
    assert out.shape == (n, hq, l, d) and lse.shape == (n, hq, l) and lse.dtype == torch.float32
    close(out, ref)
    np.testing.assert_allclose(npy(lse), lse_ref, atol=1e-3, rtol=1e-4)


def test_sdpa_golden(cuda, golden):
    def tb(name):
        return torch.from_numpy(golden[name].view(np.int16)).view(torch.bfloat16).to(cuda)
    out, _ = ops.sdpa(tb("sdpa_bf16_Q"), tb("sdpa_bf16_K"), tb("sdpa_bf16_V"), is_causal=True)
    close(out, golden["sdpa_bf16_out_causal"])


def bf16_np(a):
    return O.round_bf16(np.asarray(a, np.float32))


def test_sdpa_bias_golden(cuda, golden):
    """The reference family's own form: a full (N, H, L, S) additive bias
    with scale 0.3 (tests/test_jit_ops.py:173-193 shape, head dim 16, zero-
    padded to the kernel's 64 on the host).  Against the oracle on the
    bf16-rounded inputs, and against aten's fp32 result within the bf16
    input rounding."""
    Qf, Kf, Vf, Bf = (golden[k] for k in ("sdpa_Q", "sdpa_K", "sdpa_V", "sdpa_bias"))
    Q, K, V, B = (torch.from_numpy(a).to(cuda).to(torch.bfloat16) for a in (Qf, Kf, Vf, Bf))
    out, lse = ops.sdpa(Q, K, V, scale=0.3, bias=B)
    ref, lref = O.sdpa(bf16_np(Qf), bf16_np(Kf), bf16_np(Vf), scale=0.3, bias=bf16_np(Bf))
    close(out, ref)
    np.testing.assert_allclose(npy(lse), lref, atol=2e-3, rtol=1e-3)
    close(out, golden["sdpa_out_bias"], rtol=3e-2, atol=3e-2)
    np.testing.assert_allclose(npy(lse), golden["sdpa_lse_bias"], atol=5e-2)
    # the other golden cases at head dim 16 (padded the same way)
    out, _ = ops.sdpa(Q, K, V, is_causal=True)
    ref, _ = O.sdpa(bf16_np(Qf), bf16_np(Kf), bf16_np(Vf), causal=True)
    close(out, ref)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_full_bias_vs_oracle(cuda, d, causal):
    n, hq, hkv, l, s = 2, 4, 2, 150, 150
    q, k, v = gen((n, hq, l, d), seed=21), gen((n, hkv, s, d), seed=22), gen((n, hkv, s, d), seed=23)
    bias = gen((n, hq, l, s), seed=24)
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=causal, bias=bias.to(cuda))
    ref, lref = O.sdpa(npy(q), npy(k), npy(v), causal=causal, bias=npy(bias))
    close(out, ref)
    np.testing.assert_allclose(npy(lse), lref, atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("d", [64, 128])
def test_sdpa_left_padded_batch(cuda, d):
    """Batched generation with left padding (the reference app's call,
    KERNELS.md:64, infer.py:22-24): one additive mask (N, 1, 1, S) for every
    head and query, -inf on each sequence's padding, causal on top; rows
    whose every key is masked are left out, as verify mode leaves them out."""
    n, hq, hkv, s = 3, 8, 2, 257
    pads = [0, 13, 100]
    q, k, v = gen((n, hq, s, d), seed=31), gen((n, hkv, s, d), seed=32), gen((n, hkv, s, d), seed=33)
    mask = torch.zeros(n, 1, 1, s)
    for b, p in enumerate(pads):
        mask[b, ..., :p] = float("-inf")
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=True, bias=mask.to(torch.bfloat16).to(cuda))
    ref, lref = O.sdpa(npy(q), npy(k), npy(v), causal=True, bias=npy(mask))
    for b, p in enumerate(pads):
        close(out[b:b + 1, :, p:], ref[b:b + 1, :, p:])
        np.testing.assert_allclose(npy(lse)[b, :, p:], lref[b, :, p:], atol=2e-3, rtol=1e-3)
    # decode step of the same batch: one query per sequence over the cache
    qd = gen((n, hq, 1, d), seed=34)
    out, _ = ops.sdpa(qd.to(cuda), k.to(cuda), v.to(cuda), bias=mask.to(torch.bfloat16).to(cuda))
    ref, _ = O.sdpa(npy(qd), npy(k), npy(v), bias=npy(mask))
    close(out, ref)


@pytest.mark.parametrize("e", [16, 80, 96])
def test_sdpa_other_head_dims(cuda, e):
    q, k, v = gen((1, 4, 100, e), seed=41), gen((1, 2, 100, e), seed=42), gen((1, 2, 100, e), seed=43)
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=True)
    ref, lref = O.sdpa(npy(q), npy(k), npy(v), causal=True)
    assert out.shape == (1, 4, 100, e)
    close(out, ref)
    np.testing.assert_allclose(npy(lse), lref, atol=2e-3, rtol=1e-3)


def test_efficient_attention_with_bias_under_kuiper_mode(cuda):
    import kuillm_amd as kuipy
    aten = torch.ops.aten
    q, k, v = (gen((2, 4, 64, 128), seed=51 + i).to(cuda) for i in range(3))
    bias = gen((2, 4, 64, 64), seed=54).to(cuda)
    kuipy.reset_verify()
    with kuipy.KuiperMode(verify=True):
        out, lse, _, _ = aten._scaled_dot_product_efficient_attention(q, k, v, bias, True, 0.0, False)
    assert kuipy.print_verify_report() is True
    assert "aten._scaled_dot_product_efficient_attention.default" in kuipy.verify_stats
    ref, _ = O.sdpa(npy(q), npy(k), npy(v), bias=npy(bias))
    close(out, ref)


def test_sdpa_strided_views(cuda):
    # (B, S, H, D) storage seen as (B, H, S, D): HF's layout, no copies needed
    base = gen((2, 96, 4, 64), seed=4).to(cuda)
    q = base.transpose(1, 2)
    out, _ = ops.sdpa(q, q, q, is_causal=True)
    ref, _ = O.sdpa(npy(q), npy(q), npy(q), causal=True)
    close(out, ref)


def test_sdpa_closed_forms(cuda):
    q, k = gen((1, 2, 64, 128), seed=5).to(cuda), gen((1, 2, 256, 128), seed=6).to(cuda)
    vrow = gen((1, 2, 1, 128), seed=7).to(cuda)
    out, _ = ops.sdpa(q, k, vrow.expand(1, 2, 256, 128).contiguous())
    close(out, np.broadcast_to(npy(vrow), out.shape))           # constant V -> V
    v = gen((1, 2, 256, 128), seed=8).to(cuda)
    out, _ = ops.sdpa(q, k, v, is_causal=True)
    close(out[:, :, 0], npy(v[:, :, 0]))                        # causal row 0 -> V0


@pytest.mark.parametrize("S", [2048, 4096])
def test_sdpa_full_size_all_heads(cuda, S):
    """B=1, H=32, S, D=128 causal; every head against the
    oracle in full (output and log-sum-exp)."""
    torch.manual_seed(S)
    q = torch.randn(1, 32, S, 128, device=cuda).to(torch.bfloat16)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    out, lse = ops.sdpa(q, k, v, is_causal=True, scale=1 / math.sqrt(128))
    qn, kn, vn = npy(q), npy(k), npy(v)
    # one head per task: numpy's BLAS and ufuncs release the GIL
    with ThreadPoolExecutor(8) as pool:
        refs = list(pool.map(lambda h: O.sdpa(qn[:, h:h + 1], kn[:, h:h + 1], vn[:, h:h + 1], causal=True),
                             range(32)))
    close(out, np.concatenate([r[0] for r in refs], axis=1))
    np.testing.assert_allclose(npy(lse), np.concatenate([r[1] for r in refs], axis=1), atol=1e-3, rtol=1e-4)


DECODE = [  # n, hq, hkv, l, s, d
    (1, 32, 32, 1, 4096, 128),
    (1, 32, 8, 1, 600, 64),
    (1, 32, 8, 1, 768, 64),     # longest cache of the one-step row-wide kernel
    (1, 32, 8, 1, 769, 64),     # one key more: split-KV
    (1, 12, 4, 2, 300, 64),     # row-wide, 24 rows (no XCD regrouping)
    (1, 16, 4, 1, 384, 128),    # row-wide at head dim 128 (longest)
    (2, 8, 2, 1, 77, 128),
    (1, 4, 4, 1, 1, 64),
    (64, 32, 8, 1, 300, 64),    # 512 row groups of 4 rows: one split, 4-wave work-groups
    (70, 32, 8, 1, 520, 64),
]


@pytest.mark.parametrize("n,hq,hkv,l,s,d", DECODE)
def test_sdpa_decode_vs_oracle(cuda, n, hq, hkv, l, s, d):
    q, k, v = gen((n, hq, l, d), seed=9), gen((n, hkv, s, d), seed=10), gen((n, hkv, s, d), seed=11)
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda))          # non-causal -> split-KV kernel
    ref, lref = O.sdpa(npy(q), npy(k), npy(v))
    close(out, ref)
    np.testing.assert_allclose(npy(lse), lref, atol=1e-3, rtol=1e-4)
    again, _ = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda))
    assert torch.equal(out, again)


def test_sdpa_decode_empty_keys(cuda):
    """No visible keys.  A batch entry whose device kv_len is 0, on the
    split kernel over a 4096-key cache (its K / V loads are issued before the
    key count is known), and s = 0 through the C ABI with non-null K / V
    pointers: zero outputs and lse = -inf, the other entry unchanged."""
    from kuillm_amd import _lib
    q, k, v = gen((2, 32, 1, 128), seed=21), gen((2, 32, 4096, 128), seed=22), gen((2, 32, 4096, 128), seed=23)
    lens = torch.tensor([0, 4096], dtype=torch.int32, device=cuda)
    out, lse = ops.sdpa_decode(q.to(cuda), k.to(cuda), v.to(cuda), causal=False, return_lse=True, kv_len=lens)
    assert not out[0].float().any() and bool(torch.isneginf(lse[0]).all())
    ref, lref = O.sdpa(npy(q[1:]), npy(k[1:]), npy(v[1:]))
    close(out[1:], ref)
    np.testing.assert_allclose(npy(lse[1:]), lref, atol=1e-3, rtol=1e-4)

    lib = ops._lib_handle()
    q0 = q[:1, :4, :, :64].contiguous().to(cuda)
    kz = torch.zeros(1, 4, 1, 64, dtype=q0.dtype, device=cuda)
    o0 = torch.full((1, 4, 1, 64), 7.0, dtype=q0.dtype, device=cuda)
    l0 = torch.zeros(1, 4, 1, dtype=torch.float32, device=cuda)
    ws = ops.workspace(q0.device, lib.kuiops_query_workspace(_lib.OP_SDPA_DECODE, 4, 0, 64), "attn")
    st = _lib.strides3(*kz.stride()[:3])
    rc = lib.kuiops_sdpa_decode(1, 4, 4, 1, 0, 64, 64, _lib.BF16, q0.data_ptr(), _lib.strides3(*q0.stride()[:3]),
                                kz.data_ptr(), st, kz.data_ptr(), st, o0.data_ptr(), _lib.strides3(*o0.stride()[:3]),
                                l0.data_ptr(), 0.125, 0, None,
                                ws.data_ptr(), ws.numel(), None)
    torch.cuda.synchronize()
    assert rc == _lib.OK
    assert not o0.float().any() and bool(torch.isneginf(l0).all())


@pytest.mark.parametrize("l", [1, 2, 4])
def test_sdpa_decode_bottom_right_causal(cuda, l):
    # KV-cache decode step: the l new queries are the last l positions
    q, k, v = gen((1, 32, l, 64), seed=12), gen((1, 8, 530, 64), seed=13), gen((1, 8, 530, 64), seed=14)
    out, lse = ops.sdpa_decode(q.to(cuda), k.to(cuda), v.to(cuda), causal=True, return_lse=True)
    ref, lref = O.sdpa(npy(q), npy(k), npy(v), causal=True, align="bottom_right")
    close(out, ref)
    np.testing.assert_allclose(npy(lse), lref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("n,hq,hkv,l,s,d", [(2, 32, 8, 2048, 2048, 64), (1, 64, 64, 2048, 2304, 128)])
def test_sdpa_causal_paired_blocks(cuda, n, hq, hkv, l, s, d):
    """Grids large enough for paired causal query blocks (block p with block
    nqb-1-p, the second walked backwards over its keys): GQA, head dim 64,
    and more keys than queries (top-left causal alignment).  Sampled heads
    against the oracle, plus the same call on one head (a small grid that
    runs single blocks) must agree to rounding."""
    torch.manual_seed(l + s + d)
    q = torch.randn(n, hq, l, d, device=cuda).to(torch.bfloat16)
    k = torch.randn(n, hkv, s, d, device=cuda).to(torch.bfloat16)
    v = torch.randn(n, hkv, s, d, device=cuda).to(torch.bfloat16)
    out, lse = ops.sdpa(q, k, v, is_causal=True)
    g = hq // hkv
    for b, h in ((0, 0), (n - 1, hq - 1), (n - 1, hq // 2 + 1)):
        kh = h // g
        ref, lref = O.sdpa(npy(q[b:b + 1, h:h + 1]), npy(k[b:b + 1, kh:kh + 1]), npy(v[b:b + 1, kh:kh + 1]),
                           causal=True)
        close(out[b:b + 1, h:h + 1], ref)
        np.testing.assert_allclose(npy(lse[b:b + 1, h:h + 1]), lref, atol=1e-3, rtol=1e-4)
        single, _ = ops.sdpa(q[b:b + 1, h:h + 1].contiguous(), k[b:b + 1, kh:kh + 1].contiguous(),
                             v[b:b + 1, kh:kh + 1].contiguous(), is_causal=True)
        assert (single.float() - out[b:b + 1, h:h + 1].float()).abs().max().item() < 2e-2


# ------------------------------------------------ general SDPA (any float dtype, e != ev, wide heads)

def test_sdpa_fp32_golden(cuda, golden):
    """The reference family's own test case in fp32 (tests/test_jit_ops.py:173-193:
    N, H, L, S = 2, 3, 8, 10, head dim 16, a full float bias, scale 0.3) on
    kuiops_sdpa_general, against aten's fp32 outputs: the bias case, its LSE,
    causal and full attention."""
    Q, K, V, B = (torch.from_numpy(golden[k]).to(cuda) for k in ("sdpa_Q", "sdpa_K", "sdpa_V", "sdpa_bias"))
    out, lse = ops.sdpa(Q, K, V, scale=0.3, bias=B)
    assert out.dtype == torch.float32 and lse.dtype == torch.float32
    np.testing.assert_allclose(npy(out), golden["sdpa_out_bias"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(npy(lse), golden["sdpa_lse_bias"], rtol=1e-5, atol=1e-5)
    out, _ = ops.sdpa(Q, K, V, is_causal=True)
    np.testing.assert_allclose(npy(out), golden["sdpa_out_causal"], rtol=1e-4, atol=1e-5)
    out, _ = ops.sdpa(Q, K, V)
    np.testing.assert_allclose(npy(out), golden["sdpa_out_full"], rtol=1e-4, atol=1e-5)


GENERAL = [  # n, hq, hkv, l, s, e, ev
    (2, 3, 3, 8, 10, 16, 12),            # the reference test's e != ev shape
    (1, 4, 2, 37, 53, 64, 96),
    (1, 2, 1, 20, 70, 160, 160),         # head dims past the MFMA kernels
    (2, 2, 2, 9, 130, 256, 64),
    (1, 1, 1, 3, 1, 8, 1100 // 2),
]


@pytest.mark.parametrize("n,hq,hkv,l,s,e,ev", GENERAL)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("with_bias", [False, True])
def test_sdpa_general_vs_oracle(cuda, n, hq, hkv, l, s, e, ev, dtype, causal, with_bias):
    """kuiops_sdpa_general against the fp64 oracle: fp64 to 1e-12, fp32 to
    1e-5, bf16 at the north-star tolerance; LSE in natural log."""
    q, k, v = gen((n, hq, l, e), dtype, 31), gen((n, hkv, s, e), dtype, 32), gen((n, hkv, s, ev), dtype, 33)
    bias = gen((n, hq, l, s), dtype, 34) if with_bias else None
    scale = 0.3 if with_bias else None
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=causal, scale=scale,
                        bias=bias.to(cuda) if with_bias else None)
    ref, lref = O.sdpa(q.double().numpy(), k.double().numpy(), v.double().numpy(), causal=causal, scale=scale,
                       bias=bias.double().numpy() if with_bias else None)
    assert out.shape == (n, hq, l, ev) and out.dtype == dtype
    o = out.double().cpu().numpy()
    tol = {torch.float64: 1e-12, torch.float32: 1e-5, torch.bfloat16: 1e-2}[dtype]
    err = np.abs(o - ref) - (tol + tol * np.abs(ref))
    assert err.max() <= 0, f"max excess {err.max():.3e}"
    np.testing.assert_allclose(lse.double().cpu().numpy(), lref, rtol=1e-5, atol=1e-5)


def test_sdpa_general_masked_rows_and_broadcast_bias(cuda):
    """A broadcast padding mask (-inf on the first keys of one batch entry)
    and a row with every key masked: that row gives 0 and LSE -inf, as the
    oracle (and verify mode) treat it."""
    n, h, l, s, e, ev = 2, 2, 6, 9, 24, 40
    q, k, v = gen((n, h, l, e), torch.float32, 41), gen((n, h, s, e), torch.float32, 42), gen((n, h, s, ev), torch.float32, 43)
    mask = torch.zeros(n, 1, 1, s)
    mask[1, :, :, :4] = -math.inf
    mask_full = mask.expand(n, h, l, s).clone()
    mask_full[0, 1, 2, :] = -math.inf                 # one row sees no key
    out, lse = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), bias=mask_full.to(cuda))
    ref, lref = O.sdpa(q.numpy(), k.numpy(), v.numpy(), bias=mask_full.numpy())
    np.testing.assert_allclose(npy(out), ref, rtol=1e-5, atol=1e-5)
    assert float(out[0, 1, 2].abs().max()) == 0.0 and math.isinf(float(lse[0, 1, 2]))
    out2, _ = ops.sdpa(q.to(cuda), k.to(cuda), v.to(cuda), bias=mask.to(cuda))     # stride-0 broadcast
    ref2, _ = O.sdpa(q.numpy(), k.numpy(), v.numpy(), bias=np.broadcast_to(mask.numpy(), (n, h, l, s)))
    np.testing.assert_allclose(npy(out2), ref2, rtol=1e-5, atol=1e-5)


def test_sdpa_general_under_kuiper_mode(cuda):
    """The reference family's call (aten._scaled_dot_product_efficient_attention
    with a full fp32 bias, e != ev, scale 0.3: tests/test_jit_ops.py:173-193)
    is served by SdpaImpl (the general kernel) under KuiperMode instead of
    falling through: output and LSE against the oracle."""
    import kuillm_amd as kuipy
    from kuillm_amd import kuiops as K
    q, k = gen((2, 3, 8, 16), torch.float32, 51), gen((2, 3, 10, 16), torch.float32, 52)
    v, bias = gen((2, 3, 10, 12), torch.float32, 53), gen((2, 3, 8, 10), torch.float32, 54)
    func = torch.ops.aten._scaled_dot_product_efficient_attention.default
    args = (q.to(cuda), k.to(cuda), v.to(cuda), bias.to(cuda), True)
    impl = K.SdpaImpl({})
    spec = impl.supported(func, args, {"scale": 0.3})
    assert spec is not None
    out, lse = impl.run(spec, args, {"scale": 0.3})[:2]
    ref, lref = O.sdpa(q.double().numpy(), k.double().numpy(), v.double().numpy(), scale=0.3,
                       bias=bias.double().numpy())
    np.testing.assert_allclose(npy(out), ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(npy(lse)[..., :8], lref, rtol=1e-5, atol=1e-5)
    with kuipy.KuiperMode():
        out2 = func(*args, scale=0.3)[0]
    assert torch.equal(out2, out)
