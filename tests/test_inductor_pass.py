"""The Inductor pass and the torch.ops.kuiops custom operators, on the CPU:
aten graphs traced with fake CUDA tensors are rewritten, the gates decide
which nodes move, and the rewritten graph still runs under fake tensors (the
fake kernels agree with the aten shapes)."""
import operator

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from kuillm_amd import inductor as KI
from kuillm_amd import library  # noqa: F401

aten = torch.ops.aten
K = torch.ops.kuiops


def cu(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="cuda", dtype=dtype)


def _targets(gm):
    return [n.target for n in gm.graph.nodes if n.op == "call_function" and n.target is not operator.getitem]


def _hot_path(x, w, b, q, k, v, idx):
    y = aten.mm(x, w)
    y2 = aten.addmm(b, x, w)
    a = aten._scaled_dot_product_flash_attention(q, k, v, 0.0, True, scale=0.125)
    p = aten._softmax(y.float(), -1, False)
    t = aten.topk(p, 5)
    g = aten.gather(p, 1, t[1])
    e = aten.index(w, [idx])
    bb = aten.bmm(q[0], k[0].transpose(1, 2))
    return t[0], a[0], y2, g, e, bb


def _args():
    return (cu(4, 64), cu(64, 128), cu(128), cu(1, 4, 16, 64), cu(1, 4, 16, 64), cu(1, 4, 16, 64),
            cu(3, dtype=torch.int64))


def test_every_hot_op_is_replaced():
    with FakeTensorMode():
        args = _args()
        gm = make_fx(_hot_path)(*args)
        before = [o.shape for o in gm(*args)]
        n = KI.replace_in_graph(gm.graph)
        gm.recompile()
        after = gm(*args)
    tg = _targets(gm)
    assert n == 8
    for op in (aten.mm.default, aten.addmm.default, aten._softmax.default, aten.topk.default,
               aten.gather.default, aten.index.Tensor, aten.bmm.default,
               aten._scaled_dot_product_flash_attention.default):
        assert op not in tg, op
    for op in (K.mm, K.addmm, K.softmax, K.topk, K.gather, K.index, K.bmm, K.sdpa):
        assert op.default in tg, op
    assert [o.shape for o in after] == before


def test_unsupported_nodes_stay():
    def f(x, w, q, k, v, idx):
        y = aten.mm(x, w)                                         # int32: not served
        a = aten._scaled_dot_product_flash_attention(q, k, v, 0.0, False)   # head dim 2048
        s = aten._softmax(q, 2, False)                            # not the last dim
        e = aten.index(q, [idx, None, idx])                       # index axes not adjacent
        return y, a[0], s, e
    with FakeTensorMode():
        args = (cu(4, 4, dtype=torch.int32), cu(4, 4, dtype=torch.int32), cu(1, 2, 8, 2048), cu(1, 2, 8, 2048),
                cu(1, 2, 8, 2048), cu(2, dtype=torch.int64))
        gm = make_fx(f)(*args)
        assert KI.replace_in_graph(gm.graph) == 0


def test_sdpa_lse_user_and_efficient_variant():
    def f(q, k, v):
        a = aten._scaled_dot_product_flash_attention(q, k, v, 0.0, True)
        e = aten._scaled_dot_product_efficient_attention(q, k, v, None, True, 0.0, False)
        return a[0], a[1], e[0], e[1]                              # efficient LSE is padded: kept
    with FakeTensorMode():
        qkv = [cu(1, 2, 40, 128) for _ in range(3)]
        gm = make_fx(f)(*qkv)
        ref = [o.shape for o in gm(*qkv)]
        assert KI.replace_in_graph(gm.graph) == 1
        gm.recompile()
        assert [o.shape for o in gm(*qkv)] == ref
    tg = _targets(gm)
    assert K.sdpa.default in tg and aten._scaled_dot_product_efficient_attention.default in tg


def test_cpu_tensors_are_not_served():
    with FakeTensorMode():
        gm = make_fx(lambda a, b: aten.mm(a, b))(torch.empty(4, 4), torch.empty(4, 4))
        assert KI.replace_in_graph(gm.graph) == 0


def test_custom_ops_have_no_cpu_kernel():
    with pytest.raises(NotImplementedError):
        K.mm(torch.ones(2, 2, dtype=torch.bfloat16), torch.ones(2, 2, dtype=torch.bfloat16))


def test_install_sets_and_restores_the_hook():
    import torch._inductor.config as ic
    prev = ic.post_grad_custom_post_pass
    with KI.enabled() as p:
        assert ic.post_grad_custom_post_pass is p
        assert isinstance(p.uuid(), str) and len(p.uuid()) == 64
    assert ic.post_grad_custom_post_pass is prev
