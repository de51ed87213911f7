"""Inductor pass: put the kuiops custom operators into compiled graphs.

``torch.compile`` lowers a model to an aten graph; this post-grad pass walks
it and replaces every hot-path aten node whose operands the kuiops kernels
serve with the matching ``torch.ops.kuiops`` op.  Inductor then calls those
ops as extern kernels and generates code only for the rest of the graph.
The decision is the op families' own ``supported()`` gate (the one
``KuiperMode`` uses, kuipy/registry.py:67-84), evaluated on the nodes' fake
tensors, so eager dispatch and compiled graphs agree on which calls are
offloaded.

    import kuillm_amd.inductor as ki
    with ki.enabled():
        model = torch.compile(model)
        model(*inputs)

or ``ki.install()`` / ``ki.uninstall()``.  ``replace_in_graph(graph)`` runs
the rewrite on any aten-level ``torch.fx.Graph`` whose nodes carry
``meta["val"]`` and returns the number of nodes replaced.
"""
from __future__ import annotations

import contextlib
import hashlib
import operator

import torch
from torch._inductor.custom_graph_pass import CustomGraphPass

from . import library  # noqa: F401  (defines torch.ops.kuiops)
from . import registry

aten = torch.ops.aten
K = torch.ops.kuiops


def _val(a):
    """A node argument with every fx.Node replaced by its fake value."""
    if isinstance(a, torch.fx.Node):
        return a.meta.get("val")
    if isinstance(a, (list, tuple)):
        return type(a)(_val(x) for x in a)
    return a


def _getitem_users(node):
    """{index: getitem node} for the live users of a tuple-valued node, or
    None if some user is not a getitem."""
    out = {}
    for u in node.users:
        if u.op != "call_function" or u.target is not operator.getitem:
            return None
        if u.users:
            out[u.args[1]] = u
    return out


def _rewrite(graph, node, spec):
    """Return (target, args, kwargs) of the kuiops node replacing ``node``,
    or None when the node's outputs cannot be mapped."""
    t = node.target
    if t is aten.mm.default:
        return K.mm.default, tuple(node.args[:2]), {}
    if t is aten.addmm.default:
        _, _, _, _, _, alpha, beta = spec
        return K.addmm.default, (node.args[0], node.args[1], node.args[2], beta, alpha), {}
    if t is aten.bmm.default:
        return K.bmm.default, tuple(node.args[:2]), {}
    if t is aten._softmax.default:
        return K.softmax.default, (node.args[0],), {}
    if t in (aten._scaled_dot_product_flash_attention.default,
             aten._scaled_dot_product_efficient_attention.default):
        _, scale, causal, _, _, bias = spec
        users = _getitem_users(node)
        # outputs 0 (attention) and 1 (log-sum-exp, fp32 [N, H, L]) map
        # onto kuiops.sdpa; the efficient kernel pads its LSE, so there
        # only the attention output may be used
        allowed = {0, 1} if t is aten._scaled_dot_product_flash_attention.default else {0}
        if users is None or not set(users) <= allowed:
            return None
        kw = {"is_causal": causal, "scale": scale}
        if bias is not None:
            kw["bias"] = node.args[3] if len(node.args) > 3 else node.kwargs["attn_bias"]
        return K.sdpa.default, tuple(node.args[:3]), kw
    if t is aten.topk.default:
        _, k, dim, largest, srt = spec
        return K.topk.default, (node.args[0], k, dim, largest, srt), {}
    if t is aten.gather.default:
        dim, _ = spec
        return K.gather.default, (node.args[0], dim, node.args[2]), {}
    if t is aten.index.Tensor:
        d, tensors = spec
        k = len(tensors) - 1
        if k == 1:
            return K.index.default, (node.args[0], d, node.args[1][d]), {}
        return K.index_multi.default, (node.args[0], d, list(node.args[1][d:d + k])), {}
    return None


def replace_in_graph(graph: torch.fx.Graph, record: list | None = None) -> int:
    """Replace every supported hot-path aten node with its kuiops op; the
    replaced aten targets are appended to ``record`` when given."""
    reg = registry.registry()
    n_replaced = 0
    for node in list(graph.nodes):
        if node.op != "call_function" or node.target not in reg:
            continue
        vals = _val(node.args)
        kw = _val(dict(node.kwargs))
        if any(v is None for v in vals if not isinstance(v, (int, float, bool, list, tuple))):
            continue
        impl = reg[node.target]
        spec = impl.supported(node.target, vals, kw)
        if spec is None:
            continue
        rw = _rewrite(graph, node, spec)
        if rw is None:
            continue
        target, args, kwargs = rw
        with graph.inserting_before(node):
            new = graph.call_function(target, args, kwargs)
        val = node.meta.get("val")
        if isinstance(val, (tuple, list)):
            if target is K.sdpa.default:
                new.meta["val"] = (val[0], val[1])
            else:
                new.meta["val"] = tuple(val)
            for u in list(node.users):
                if not u.users:
                    graph.erase_node(u)
        else:
            new.meta["val"] = val
        node.replace_all_uses_with(new)
        graph.erase_node(node)
        n_replaced += 1
        if record is not None:
            record.append(node.target)
    if n_replaced:
        graph.lint()
    return n_replaced


class KuiopsPostGradPass(CustomGraphPass):
    """``torch._inductor.config.post_grad_custom_post_pass`` hook."""

    def __init__(self):
        self.replaced = []          # aten targets replaced, over all graphs compiled

    def __call__(self, graph: torch.fx.Graph) -> None:
        replace_in_graph(graph, self.replaced)

    def uuid(self):
        # part of Inductor's FX-graph cache key: changes with this file
        with open(__file__, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()


_PASS = KuiopsPostGradPass()
_SAVED = []


def install() -> KuiopsPostGradPass:
    """Register the pass with Inductor (replacing any previous custom
    post-grad pass until ``uninstall()``)."""
    import torch._inductor.config as ic
    _SAVED.append(ic.post_grad_custom_post_pass)
    ic.post_grad_custom_post_pass = _PASS
    return _PASS


def uninstall() -> None:
    import torch._inductor.config as ic
    ic.post_grad_custom_post_pass = _SAVED.pop() if _SAVED else None


@contextlib.contextmanager
def enabled():
    p = install()
    try:
        yield p
    finally:
        uninstall()
