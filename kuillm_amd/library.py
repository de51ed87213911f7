"""PyTorch custom operators ``torch.ops.kuiops.*`` over the kuiops C ABI.

These are the callers the C ABI is built for: the ``kuiops`` op families
(``KuiperMode``) and the Inductor pass both go through them.  Each op has
  * a CUDA (HIP) kernel: the ``ops`` function, which enqueues the HIP
    kernels of libkuiops.so on the current stream;
  * a fake (meta) implementation, so the ops trace under ``torch.compile``,
    ``make_fx`` and FakeTensorMode without touching the device.
There is no CPU kernel: calling an op on CPU tensors raises
``NotImplementedError`` from the dispatcher, as a product op must not fall
back silently.

Schemas follow the aten ops they replace (mm, addmm, bmm, _softmax over the
last dim, scaled-dot-product attention returning (out, lse), topk, gather,
index, the elementwise maps, last-axis mean, cat) with the reference's argument meaning
(kuipy/kuiops.py:403-754).
"""
from __future__ import annotations

import torch

from . import ops

_LIB = torch.library.Library("kuiops", "DEF")

_SCHEMAS = {
    "mm": "mm(Tensor A, Tensor B, int gemv_max_m=64) -> Tensor",
    "addmm": "addmm(Tensor C, Tensor A, Tensor B, float beta=1.0, float alpha=1.0, int gemv_max_m=64) -> Tensor",
    "bmm": "bmm(Tensor A, Tensor B) -> Tensor",
    "softmax": "softmax(Tensor x) -> Tensor",
    "sdpa": "sdpa(Tensor q, Tensor k, Tensor v, bool is_causal=False, float? scale=None, "
            "int decode_max_rows=8, Tensor? bias=None) -> (Tensor, Tensor)",
    "sdpa_decode": "sdpa_decode(Tensor q, Tensor k, Tensor v, bool causal=True, float? scale=None) -> Tensor",
    "topk": "topk(Tensor x, int k, int dim=-1, bool largest=True, bool sorted=True) -> (Tensor, Tensor)",
    "gather": "gather(Tensor inp, int dim, Tensor idx) -> Tensor",
    "index": "index(Tensor inp, int dim, Tensor idx) -> Tensor",
    "index_multi": "index_multi(Tensor inp, int first, Tensor[] idxs) -> Tensor",
    "scatter": "scatter(Tensor inp, int dim, Tensor idx, Tensor src) -> Tensor",
    "sort": "sort(Tensor x, int dim=-1, bool descending=False) -> (Tensor, Tensor)",
    "cumsum": "cumsum(Tensor x, int dim) -> Tensor",
    "multinomial": "multinomial(Tensor probs, int num_samples, Tensor uniforms) -> Tensor",
    "elementwise": "elementwise(int op, Tensor[] inputs, ScalarType out_dtype, ScalarType compute_dtype, "
                   "float s0=1.0, float s1=0.0) -> Tensor",
    "mean_lastdim": "mean_lastdim(Tensor x, bool keepdim=False) -> Tensor",
    "cat": "cat(Tensor[] tensors, int dim=0) -> Tensor",
}
for _s in _SCHEMAS.values():
    _LIB.define(_s)


# ------------------------------------------------------------ HIP kernels

def _mm(A, B, gemv_max_m=64):
    return ops.mm(A, B, gemv_max_m=gemv_max_m)


def _addmm(C, A, B, beta=1.0, alpha=1.0, gemv_max_m=64):
    return ops.addmm(C, A, B, beta=beta, alpha=alpha, gemv_max_m=gemv_max_m)


def _bmm(A, B):
    return ops.bmm(A, B)


def _softmax(x):
    return ops.softmax(x)


def _sdpa(q, k, v, is_causal=False, scale=None, decode_max_rows=8, bias=None):
    return ops.sdpa(q, k, v, is_causal=is_causal, scale=scale, return_lse=True,
                    decode_max_rows=decode_max_rows, bias=bias)


def _sdpa_decode(q, k, v, causal=True, scale=None):
    return ops.sdpa_decode(q, k, v, scale=scale, causal=causal)[0]


def _topk(x, k, dim=-1, largest=True, sorted=True):
    v, i = ops.topk(x, k, dim=dim, largest=largest, sorted=sorted)
    return v.contiguous(), i.contiguous()      # the strides the fake kernel promises


def _gather(inp, dim, idx):
    return ops.gather(inp, dim, idx)


def _index(inp, dim, idx):
    return ops.index(inp, dim, idx)


def _index_multi(inp, first, idxs):
    return ops.index_multi(inp, first, list(idxs))


def _scatter(inp, dim, idx, src):
    return ops.scatter(inp, dim, idx, src)


def _sort(x, dim=-1, descending=False):
    v, i = ops.sort(x, dim=dim, descending=descending)
    return v.contiguous(), i.contiguous()


def _cumsum(x, dim):
    return ops.cumsum(x, dim).contiguous()


def _multinomial(probs, num_samples, uniforms):
    return ops.multinomial(probs, num_samples, replacement=True, uniforms=uniforms)


def _elementwise(op, inputs, out_dtype, compute_dtype, s0=1.0, s1=0.0):
    return ops.elementwise(op, list(inputs), out_dtype, compute_dtype, s0=s0, s1=s1)


def _mean_lastdim(x, keepdim=False):
    return ops.mean_lastdim(x, keepdim)


def _cat(tensors, dim=0):
    return ops.cat(list(tensors), dim)


for _name, _fn in (("mm", _mm), ("addmm", _addmm), ("bmm", _bmm), ("softmax", _softmax),
                   ("sdpa", _sdpa), ("sdpa_decode", _sdpa_decode), ("topk", _topk),
                   ("gather", _gather), ("index", _index), ("index_multi", _index_multi), ("scatter", _scatter), ("sort", _sort),
                   ("cumsum", _cumsum), ("multinomial", _multinomial), ("elementwise", _elementwise),
                   ("mean_lastdim", _mean_lastdim), ("cat", _cat)):
    _LIB.impl(_name, _fn, "CUDA")


# ------------------------------------------------- fake (meta) kernels

def _fake(name):
    return torch.library.register_fake(f"kuiops::{name}", lib=_LIB)


@_fake("mm")
def _mm_fake(A, B, gemv_max_m=64):
    return A.new_empty((A.shape[0], B.shape[1]))


@_fake("addmm")
def _addmm_fake(C, A, B, beta=1.0, alpha=1.0, gemv_max_m=64):
    return A.new_empty((A.shape[0], B.shape[1]))


@_fake("bmm")
def _bmm_fake(A, B):
    return A.new_empty((A.shape[0], A.shape[1], B.shape[2]))


@_fake("softmax")
def _softmax_fake(x):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@_fake("sdpa")
def _sdpa_fake(q, k, v, is_causal=False, scale=None, decode_max_rows=8, bias=None):
    n, hq, l, _ = q.shape
    return (q.new_empty((n, hq, l, v.shape[-1])),
            q.new_empty((n, hq, l), dtype=torch.float32))


@_fake("sdpa_decode")
def _sdpa_decode_fake(q, k, v, causal=True, scale=None):
    return q.new_empty((*q.shape[:3], v.shape[-1]))


@_fake("topk")
def _topk_fake(x, k, dim=-1, largest=True, sorted=True):
    shape = list(x.shape)
    shape[dim % x.dim()] = k
    return x.new_empty(shape), x.new_empty(shape, dtype=torch.int64)


@_fake("gather")
def _gather_fake(inp, dim, idx):
    return inp.new_empty(idx.shape)


@_fake("index")
def _index_fake(inp, dim, idx):
    dim = dim % inp.dim()
    return inp.new_empty((*inp.shape[:dim], *idx.shape, *inp.shape[dim + 1:]))


@_fake("scatter")
def _scatter_fake(inp, dim, idx, src):
    return torch.empty_like(inp, memory_format=torch.contiguous_format)


@_fake("sort")
def _sort_fake(x, dim=-1, descending=False):
    return (torch.empty_like(x, memory_format=torch.contiguous_format),
            torch.empty_like(x, dtype=torch.int64, memory_format=torch.contiguous_format))


@_fake("cumsum")
def _cumsum_fake(x, dim):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@_fake("multinomial")
def _multinomial_fake(probs, num_samples, uniforms):
    shape = (num_samples,) if probs.dim() == 1 else (probs.shape[0], num_samples)
    return probs.new_empty(shape, dtype=torch.int64)


@_fake("elementwise")
def _elementwise_fake(op, inputs, out_dtype, compute_dtype, s0=1.0, s1=0.0):
    shape = torch.broadcast_shapes(*[tuple(t.shape) for t in inputs])
    return inputs[0].new_empty(shape, dtype=out_dtype)


@_fake("mean_lastdim")
def _mean_lastdim_fake(x, keepdim=False):
    return x.new_empty((*x.shape[:-1], 1) if keepdim else tuple(x.shape[:-1]))


@_fake("cat")
def _cat_fake(tensors, dim=0):
    shape = list(tensors[0].shape)
    d = dim % len(shape)
    shape[d] = sum(int(t.shape[d]) for t in tensors)
    return tensors[0].new_empty(shape)


@_fake("index_multi")
def _index_multi_fake(inp, first, idxs):
    bshape = torch.broadcast_shapes(*[tuple(t.shape) for t in idxs])
    return inp.new_empty((*inp.shape[:first], *bshape, *inp.shape[first + len(idxs):]))
