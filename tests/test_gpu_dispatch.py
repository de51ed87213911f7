"""End-to-end dispatch on the GPU: stock PyTorch calls inside KuiperMode run
the HIP kernels (checked by verify mode and by the native library being the
one loaded), fall through where unsupported, and the kernels are safe to
record in a HIP graph."""
import math

import pytest
import torch
import torch.nn.functional as F

import kuillm_amd as kuipy
from kuillm_amd import _lib, ops

pytestmark = pytest.mark.gpu


def test_kuiper_mode_integration(cuda, monkeypatch):
    # reference tests/test_jit_general.py:50-59, at strictness 2
    monkeypatch.setattr(kuipy.C, "JIT_STRICTNESS", 2)
    A = torch.randn(128, 64, device=cuda)
    B = torch.randn(64, 128, device=cuda)
    with kuipy.KuiperMode():
        o_mm = torch.mm(A, B)
    assert torch.allclose(o_mm, A @ B, atol=1e-3, rtol=1e-3)
    assert _lib.loaded()


def test_verify_mode_over_hot_ops(cuda):
    kuipy.reset_verify()
    torch.manual_seed(0)
    x = torch.randn(16, 256, device=cuda, dtype=torch.bfloat16)
    lin = torch.nn.Linear(256, 512, device=cuda, dtype=torch.bfloat16)
    q = torch.randn(1, 4, 256, 128, device=cuda, dtype=torch.bfloat16)
    logits = torch.randn(2, 32000, device=cuda)
    with torch.no_grad(), kuipy.KuiperMode(verify=True):
        y = lin(x)                                            # addmm, 1-D bias
        z = torch.bmm(q[0], q[0].transpose(1, 2))             # bmm with a K-contiguous B
        p = torch.softmax(logits, -1)                         # _softmax
        v, i = torch.topk(logits, 20)                         # topk
        g = torch.gather(logits, 1, i)                        # gather
        a = F.scaled_dot_product_attention(q, q, q, is_causal=True)
    assert kuipy.print_verify_report() is True
    names = set(kuipy.verify_stats)
    assert {"aten.addmm.default", "aten.bmm.default", "aten._softmax.default", "aten.topk.default",
            "aten.gather.default"} <= names
    assert torch.equal(g, v)
    ref = F.scaled_dot_product_attention(q.float(), q.float(), q.float(), is_causal=True)
    assert ((a.float() - ref).norm() / ref.norm()).item() < 1e-2


def test_unsupported_falls_through(cuda):
    # reference tests/test_jit_general.py:61-71: odd shapes / CPU tensors run stock
    A = torch.randn(128, 63, device=cuda)
    B = torch.randn(63, 128, device=cuda)
    with kuipy.KuiperMode():
        out = torch.mm(A, B)                                  # served by the SIMT kernel
        c = torch.mm(torch.randn(4, 4), torch.randn(4, 4))    # CPU: stock
        i = torch.randint(0, 5, (3,), device=cuda)
        s = torch.cumprod(torch.randn(10, device=cuda), 0)    # no family: stock
    assert torch.allclose(out, A @ B, atol=1e-3, rtol=1e-3)
    assert c.shape == (4, 4) and s.shape == (10,)


def test_hip_graph_replay_matches_eager(cuda):
    torch.manual_seed(1)
    x = torch.randn(4, 4096, device=cuda, dtype=torch.bfloat16)
    W = torch.randn(4096, 11008, device=cuda, dtype=torch.bfloat16) * 0.02
    q = torch.randn(1, 32, 1, 128, device=cuda, dtype=torch.bfloat16)
    k = torch.randn(1, 32, 700, 128, device=cuda, dtype=torch.bfloat16)
    logits = torch.randn(1, 32000, device=cuda)

    bias = torch.randn(11008, device=cuda, dtype=torch.bfloat16)

    def step():
        y = ops.mm(x, W)
        y1 = ops.mm(x[:1], W)                # row-streaming kernel, K split merged in-kernel
        y2 = ops.addmm(bias, x[:2], W)
        o, _ = ops.sdpa(q, k, k)
        p = ops.softmax(logits)
        t = ops.topk(p, 1)[1]
        return y, y1, y2, o, p, t

    eager = step()                   # also allocates the workspaces outside capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step()
    for rep in range(3):
        x.add_(0)                    # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b), f"replay {rep} differs"


def test_top_p_sampling_tail_under_kuiper_mode(cuda):
    """transformers' top-p warper and torch.multinomial inside KuiperMode:
    sort, softmax, cumsum, scatter and multinomial run on the kuiops kernels
    (verify mode checks the deterministic ones against stock PyTorch), and
    every drawn token survives the top-p filter."""
    tr = pytest.importorskip("transformers.generation.logits_process")
    kuipy.reset_verify()
    torch.manual_seed(0)
    scores = torch.randn(4, 32000, device=cuda) * 3
    warp = tr.TopPLogitsWarper(top_p=0.9)
    with torch.no_grad(), kuipy.KuiperMode(verify=True):
        filt = warp(None, scores)
        probs = torch.softmax(filt, -1)
        tok = torch.multinomial(probs, 1)
    assert kuipy.print_verify_report() is True
    names = set(kuipy.verify_stats)
    assert {"aten.sort.default", "aten.cumsum.default", "aten.scatter.src", "aten._softmax.default"} <= names
    ref = warp(None, scores)
    assert torch.equal(torch.isinf(filt), torch.isinf(ref))
    assert bool((probs.gather(1, tok) > 0).all())
