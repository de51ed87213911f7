"""Writes the golden fixtures in this directory from stock aten on CPU.

The reference computes every hot-path op either with an un-vendored Kuiper
kernel that its tests hold to stock torch (tests/test_jit_ops.py:34-43), or
by falling through to stock aten (kuipy/__init__.py:161-164; always for
topk / index / causal SDPA).  Stock aten on CPU is therefore the reference's
own result for these ops.  Shapes follow the reference's tests
(tests/test_jit_ops.py:51-230) plus BASELINE.json config 0 at reduced size.

Fixtures are data only: inputs and aten outputs, bf16 stored as uint16 bits.
Re-run with:  python tests/golden/make_golden.py
"""
import math
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "golden.npz"


def bits(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def main():
    g = {}
    torch.manual_seed(0)
    # mm (MmImpl; tests/test_jit_general.py:50-59 uses 128x64 @ 64x128 f32)
    A = torch.randn(128, 64); B = torch.randn(64, 128)
    g["mm_f32_A"], g["mm_f32_B"], g["mm_f32_C"] = A.numpy(), B.numpy(), torch.mm(A, B).numpy()
    A = torch.randn(64, 96).bfloat16(); B = (torch.randn(96, 80) * 0.5).bfloat16()
    g["mm_bf16_A"], g["mm_bf16_B"] = bits(A), bits(B)
    g["mm_bf16_C32"] = (A.float() @ B.float()).numpy()          # fp32 accumulate, unrounded
    g["mm_bf16_C"] = bits(torch.mm(A, B))                        # aten bf16 result
    # addmm, test_jit_ops.py:98-112: 64^3, alpha/beta in {(1,1),(0.5,2)}, 2-D bias
    for dt in ("f32", "bf16"):
        tdt = torch.float32 if dt == "f32" else torch.bfloat16
        A = torch.randn(64, 64, dtype=tdt); B = torch.randn(64, 64, dtype=tdt)
        C2 = torch.randn(64, 64, dtype=tdt); C1 = torch.randn(64, dtype=tdt)
        g[f"addmm_{dt}_A"], g[f"addmm_{dt}_B"], g[f"addmm_{dt}_C2"], g[f"addmm_{dt}_C1"] = bits(A), bits(B), bits(C2), bits(C1)
        for tag, (al, be) in (("11", (1.0, 1.0)), ("052", (0.5, 2.0))):
            g[f"addmm_{dt}_out2_{tag}"] = bits(torch.addmm(C2, A, B, alpha=al, beta=be))
            g[f"addmm_{dt}_out1_{tag}"] = bits(torch.addmm(C1, A, B, alpha=al, beta=be))
            g[f"addmm_{dt}_out2_{tag}_f32acc"] = (be * C2.float() + al * (A.float() @ B.float())).numpy()
    # BASELINE config 0 (reduced rows): x~N(0,1), W~N(0,.02), bias~N(0,.02), fp32
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(8, 768, generator=gen); W = torch.randn(768, 3072, generator=gen) * 0.02
    b = torch.randn(3072, generator=gen) * 0.02
    g["cfg0_x"], g["cfg0_W"], g["cfg0_b"] = x.numpy(), W[:, :64].contiguous().numpy(), b[:64].contiguous().numpy()
    g["cfg0_out"] = torch.addmm(b[:64], x, W[:, :64]).numpy()
    # bmm, test_jit_ops.py:51-60
    for dt in ("f32", "bf16"):
        tdt = torch.float32 if dt == "f32" else torch.bfloat16
        A = torch.randn(5, 17, 9, dtype=tdt); B = torch.randn(5, 9, 13, dtype=tdt)
        g[f"bmm_{dt}_A"], g[f"bmm_{dt}_B"], g[f"bmm_{dt}_C"] = bits(A), bits(B), bits(torch.bmm(A, B))
    # softmax, test_jit_ops.py:141-155
    for shape in ((128, 64), (8, 5, 33)):
        tag = "x".join(map(str, shape))
        X = torch.randn(*shape)
        g[f"softmax_{tag}_X"], g[f"softmax_{tag}_Y"] = X.numpy(), torch.softmax(X, -1).numpy()
        Xb = X.bfloat16()
        g[f"softmax_{tag}_Xb"], g[f"softmax_{tag}_Yb"] = bits(Xb), bits(torch.softmax(Xb, -1))
    # sdpa: test_jit_ops.py:173-193 shape with a float bias, plus causal cases
    N, H, L, S, E = 2, 3, 8, 10, 16
    Q, K, V = torch.randn(N, H, L, E), torch.randn(N, H, S, E), torch.randn(N, H, S, E)
    bias = torch.randn(N, H, L, S)
    g["sdpa_Q"], g["sdpa_K"], g["sdpa_V"], g["sdpa_bias"] = Q.numpy(), K.numpy(), V.numpy(), bias.numpy()
    g["sdpa_out_bias"] = F.scaled_dot_product_attention(Q, K, V, attn_mask=bias, scale=0.3).numpy()
    g["sdpa_lse_bias"] = torch.logsumexp(Q @ K.transpose(-1, -2) * 0.3 + bias, -1).numpy()
    g["sdpa_out_causal"] = F.scaled_dot_product_attention(Q, K, V, is_causal=True).numpy()
    g["sdpa_out_full"] = F.scaled_dot_product_attention(Q, K, V).numpy()
    Qb = torch.randn(1, 4, 70, 64).bfloat16(); Kb = torch.randn(1, 4, 70, 64).bfloat16(); Vb = torch.randn(1, 4, 70, 64).bfloat16()
    g["sdpa_bf16_Q"], g["sdpa_bf16_K"], g["sdpa_bf16_V"] = bits(Qb), bits(Kb), bits(Vb)
    g["sdpa_bf16_out_causal"] = F.scaled_dot_product_attention(Qb.float(), Kb.float(), Vb.float(), is_causal=True).numpy()
    # topk: tie-free rows (distinct values), several k, both directions
    X = torch.randperm(4 * 300).reshape(4, 300).float() / 7.0 - 80.0
    g["topk_X"] = X.numpy()
    for kk in (1, 5, 64, 300):
        v, i = torch.topk(X, kk)
        g[f"topk_{kk}_v"], g[f"topk_{kk}_i"] = v.numpy(), i.numpy()
        v, i = torch.topk(X, kk, largest=False)
        g[f"topk_{kk}_sv"], g[f"topk_{kk}_si"] = v.numpy(), i.numpy()
    # gather, test_jit_ops.py:216-230
    for shape, dim in (((8, 5), 1), ((8, 5), 0), ((4, 3, 6), 2)):
        tag = "x".join(map(str, shape)) + f"_d{dim}"
        Inp = torch.randn(*shape)
        ish = list(shape); ish[dim] = max(1, shape[dim] - 1)
        Idx = torch.randint(0, shape[dim], ish)
        g[f"gather_{tag}_inp"], g[f"gather_{tag}_idx"], g[f"gather_{tag}_out"] = Inp.numpy(), Idx.numpy(), torch.gather(Inp, dim, Idx).numpy()
    # index: embedding-row gather and a middle-axis index with negative entries
    Emb = torch.randn(50, 12); ids = torch.randint(0, 50, (3, 7))
    g["index_emb"], g["index_ids"], g["index_out"] = Emb.numpy(), ids.numpy(), Emb[ids].numpy()
    T3 = torch.randn(2, 9, 4); ids2 = torch.tensor([[-1, 0, 3], [8, -9, 2]])
    g["index3_inp"], g["index3_ids"], g["index3_out"] = T3.numpy(), ids2.numpy(), T3[:, ids2].numpy()
    # sort (stable): ties, NaN, -0 / +0, both directions; a row wider than one sort chunk
    X = torch.randint(-20, 20, (3, 257)).float() / 4.0
    X[0, 5] = float("nan"); X[2, 100] = float("nan"); X[1, 7] = -0.0; X[1, 9] = 0.0; X[1, 11] = -0.0
    g["sort_X"] = X.numpy()
    for tag, desc in (("asc", False), ("desc", True)):
        v, i = torch.sort(X, descending=desc, stable=True)
        g[f"sort_{tag}_v"], g[f"sort_{tag}_i"] = v.numpy(), i.numpy()
    Xw = torch.randn(2, 5000)
    g["sortw_X"] = Xw.numpy()
    v, i = torch.sort(Xw, descending=True, stable=True)
    g["sortw_v"], g["sortw_i"] = v.numpy(), i.numpy()
    # cumsum: fp32 and int64 rows
    Xc = torch.randn(4, 3000)
    g["cumsum_X"], g["cumsum_Y"] = Xc.numpy(), torch.cumsum(Xc, -1).numpy()
    Xi = torch.randint(-1000, 1000, (3, 777))
    g["cumsum_i64_X"], g["cumsum_i64_Y"] = Xi.numpy(), torch.cumsum(Xi, -1).numpy()
    # scatter.src (ScatterImpl, kuipy/kuiops.py:757-807): permutation indices
    # (no repeated targets) in fp32 and bool, as the top-p filter uses it
    S = torch.randn(4, 9); perm = torch.stack([torch.randperm(9) for _ in range(4)]); src = torch.randn(4, 9)
    g["scatter_self"], g["scatter_idx"], g["scatter_src"] = S.numpy(), perm.numpy(), src.numpy()
    g["scatter_out"] = S.scatter(1, perm, src).numpy()
    mb = torch.rand(4, 9) > 0.5
    g["scatter_bool_src"], g["scatter_bool_out"] = mb.numpy(), mb.scatter(1, perm, mb).numpy()
    # elementwise / mean / cat (ElementwiseImpl / MeanImpl / CatImpl,
    # kuipy/kuiops.py:150-320, 810-921): bf16 and fp32 operands, a broadcast
    # column, python scalars, mixed bf16 * fp32 promotion
    ex = torch.randn(4, 33) * 2
    ey = torch.randn(4, 33) + 3.0                          # away from 0 for div
    ecol = torch.randn(4, 1)
    for dt in ("f32", "bf16"):
        tdt = torch.float32 if dt == "f32" else torch.bfloat16
        x, y, col = ex.to(tdt), ey.to(tdt), ecol.to(tdt)
        g[f"ew_{dt}_x"], g[f"ew_{dt}_y"], g[f"ew_{dt}_col"] = bits(x), bits(y), bits(col)
        for name, fn in (("neg", torch.neg), ("silu", F.silu), ("cos", torch.cos), ("sin", torch.sin),
                         ("exp", torch.exp), ("sq", lambda t: t.pow(2)), ("p3", lambda t: t.pow(3)),
                         ("p15", lambda t: t.abs().pow(1.5))):
            g[f"ew_{dt}_{name}"] = bits(fn(x))
        g[f"ew_{dt}_rsqrt"] = bits(torch.rsqrt(y))
        g[f"ew_{dt}_sqrt"] = bits(torch.sqrt(y))
        g[f"ew_{dt}_add"] = bits(x + y)
        g[f"ew_{dt}_add_a"] = bits(torch.add(x, y, alpha=0.5))
        g[f"ew_{dt}_sub"] = bits(x - y)
        g[f"ew_{dt}_mul"] = bits(x * y)
        g[f"ew_{dt}_div"] = bits(x / y)
        g[f"ew_{dt}_mulcol"] = bits(x * col)
        g[f"ew_{dt}_adds"] = bits(x + 1e-6)
        g[f"ew_{dt}_muls"] = bits(x * 0.125)
        g[f"ew_{dt}_lt"] = (x < 0.5).numpy()
        g[f"ew_{dt}_le"] = (x <= y).numpy()
        g[f"ew_{dt}_eq"] = (x == 0.0).numpy()
        g[f"ew_{dt}_where"] = bits(torch.where(x > 0, x, y))
    xb, yf = ex.bfloat16(), ey
    g["ew_mixed_out"] = (xb * yf).numpy()                  # bf16 * fp32 -> fp32
    bm1, bm2 = torch.rand(5, 9) > 0.5, torch.rand(5, 9) > 0.3
    g["ew_b1"], g["ew_b2"] = bm1.numpy(), bm2.numpy()
    g["ew_band"], g["ew_bor"], g["ew_bnot"] = (bm1 & bm2).numpy(), (bm1 | bm2).numpy(), (~bm1).numpy()
    ei = torch.randint(-50, 50, (6, 7))
    g["ew_i64"], g["ew_i64_add"], g["ew_i64_mul"] = ei.numpy(), (ei + 3).numpy(), (ei * ei).numpy()
    mx = torch.randn(6, 100).bfloat16()
    g["mean_bf16_x"], g["mean_bf16_out"] = bits(mx), bits(mx.mean(-1, keepdim=True))
    mxf = torch.randn(3, 5000)
    g["mean_f32_x"], g["mean_f32_out"] = mxf.numpy(), mxf.mean(-1).numpy()
    c1, c2 = torch.randn(2, 3, 5, 8).bfloat16(), torch.randn(2, 3, 7, 8).bfloat16()
    g["cat_a"], g["cat_b"], g["cat_out"] = bits(c1), bits(c2), bits(torch.cat([c1, c2], dim=2))
    q = torch.randn(2, 4, 6, 16)
    g["cat_q"], g["cat_rot"] = q.numpy(), torch.cat((-q[..., 8:], q[..., :8]), dim=-1).numpy()
    # index.Tensor with two int64 index tensors on a bool matrix: the
    # reference app's call T(2,bool)[T(4,int64),T(4,int64)] (KERNELS.md:67)
    bm = torch.rand(24, 30) > 0.5
    i0 = torch.randint(-24, 24, (2, 1, 3, 4)); i1 = torch.randint(0, 30, (1, 5, 3, 4))
    g["index2_mask"], g["index2_i0"], g["index2_i1"], g["index2_out"] = bm.numpy(), i0.numpy(), i1.numpy(), bm[i0, i1].numpy()
    t4 = torch.randn(3, 6, 7, 5)
    j0, j1 = torch.randint(0, 6, (4,)), torch.randint(-7, 7, (4,))
    g["index3d_inp"], g["index3d_j0"], g["index3d_j1"], g["index3d_out"] = t4.numpy(), j0.numpy(), j1.numpy(), t4[:, j0, j1].numpy()
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
