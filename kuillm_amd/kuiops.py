"""Operator families: for each aten op, decide whether a kuiops kernel serves
the call (``supported``) and run it (``run``).

Same contract as the reference's families (kuipy/kuiops.py:27-43):

* ``supported(func, args, kwargs) -> spec | None`` is pure and cheap (no GPU
  work) and works on fake tensors too, so the Inductor pass can reuse it;
* ``run(spec, args, kwargs) -> result`` returns what the aten op returns, or
  ``None`` when the native gate refuses the call after all (the caller then
  falls through to stock PyTorch);
* ``tune_key`` / ``tune_params`` / ``tune(all)`` carry autotune parameters.

``run`` calls the ``torch.ops.kuiops`` custom operators (kuillm_amd/library.py),
the same ops the Inductor pass (kuillm_amd/inductor.py) puts into compiled
graphs.

The gates are wider than the reference's: the reference needs M, N multiples
of 64 and 2-D addmm biases (kuipy/kuiops.py:365-394, 538-540) and rejects
causal SDPA (:636-637); the kernels here take any shape, 1-D biases, causal
and grouped-query attention, and add topk / index, which the reference never
implemented (kuiops/topk/.gitkeep, kuiops/index/.gitkeep).
"""
from __future__ import annotations

import math

import torch

from . import _lib
from . import library  # noqa: F401  (defines torch.ops.kuiops)
from . import ops
from .config import log

aten = torch.ops.aten
K = torch.ops.kuiops      # the custom ops: HIP kernels behind the C ABI

_FLOAT_DTYPES = (torch.float16, torch.float32, torch.float64, torch.bfloat16)
_HALF = (torch.float16, torch.bfloat16)
_FLOATS = (torch.float16, torch.bfloat16, torch.float32, torch.float64)
_SIZE_LIMIT = 2 ** 31 - 1


def _scalar(x):
    """A Python scalar (or 0-d fp64 tensor) argument, else None
    (kuipy/kuiops.py:14-21)."""
    if isinstance(x, bool):
        return None
    if isinstance(x, (float, int)):
        return x
    if isinstance(x, torch.Tensor) and x.dim() == 0 and x.dtype == torch.float64 and not x.is_meta:
        return float(x.item())
    return None


def _norm_dim(d, rank):
    return d + rank if d < 0 else d


def _is_dev(*ts):
    return all(isinstance(t, torch.Tensor) and t.is_cuda for t in ts)


def _gemv_max_m(params) -> int:
    """The tuned decode-GEMM row limit (0 .. 64) of a GEMM family."""
    m = params.get("gemv_max_m", ops.GEMV_MAX_M) if isinstance(params, dict) else ops.GEMV_MAX_M
    return max(0, min(ops.GEMV_MAX_M, int(m)))


class _Family:
    tune_key = ""
    tune_params = ()

    def __init__(self, all_tune_params):
        self.tune_params = all_tune_params.get(self.tune_key, self.tune_params)

    def tune(self, all_tune_params):
        all_tune_params[self.tune_key] = self.tune_params
        return all_tune_params

    def __repr__(self):
        return f"{type(self).__name__}({self.tune_params!r})"


# ---------------------------------------------------------------- GEMM

class MmImpl(_Family):
    """aten.mm -> kuiops_mm (MFMA) / kuiops_gemv_splitk for M <= gemv_max_m
    (reference MmImpl kuipy/kuiops.py:397-469)."""
    tune_key = "MM"
    tune_params = {"impl": "auto", "gemv_max_m": ops.GEMV_MAX_M}

    def supported(self, func, args, kwargs):
        if len(args) != 2 or kwargs.get("alpha", 1) != 1:
            return None
        A, B = args
        if not (_is_dev(A, B) and A.dim() == 2 and B.dim() == 2 and A.dtype == B.dtype
                and A.dtype in _FLOAT_DTYPES):
            return None
        M, K = (int(x) for x in A.shape)
        K2, N = (int(x) for x in B.shape)
        if K != K2 or max(M, N, K) > _SIZE_LIMIT:
            return None
        return (A.dtype, M, N, K, [A, B])

    def run(self, spec, args, kwargs):
        _, _, _, _, (A, B) = spec
        try:
            return K.mm(A, B, _gemv_max_m(self.tune_params))
        except _lib.Unsupported:
            return None

    def tune(self, all_tune_params):
        """Measure the decode-GEMM / MFMA crossover on this GPU (when there is
        one) and keep it as ``gemv_max_m`` (the reference's tune() hook,
        kuipy/kuiops.py:38-40, which only stores the parameters)."""
        from . import tune as _tune
        params = dict(self.tune_params) if isinstance(self.tune_params, dict) else {}
        if torch.cuda.is_available():
            params["gemv_max_m"] = _tune.sweep_gemv_max_m()
        self.tune_params = params
        all_tune_params[self.tune_key] = params
        return all_tune_params


class AddmmImpl(_Family):
    """aten.addmm -> kuiops_addmm with a full or row-broadcast addend
    (reference AddmmImpl kuipy/kuiops.py:520-564, which takes 2-D C only)."""
    tune_key = "ADDMM"
    tune_params = {"splitk": "auto"}

    def supported(self, func, args, kwargs):
        if len(args) != 3:
            return None
        Cin, A, B = args
        if not (_is_dev(A, B, Cin) and A.dim() == 2 and B.dim() == 2 and Cin.dim() <= 2
                and A.dtype == B.dtype == Cin.dtype and A.dtype in _FLOAT_DTYPES):
            return None
        M, K = (int(x) for x in A.shape)
        K2, N = (int(x) for x in B.shape)
        if K != K2:
            return None
        try:
            torch.broadcast_shapes(tuple(Cin.shape), (M, N))
        except RuntimeError:
            return None
        alpha = _scalar(kwargs.get("alpha", 1))
        beta = _scalar(kwargs.get("beta", 1))
        if alpha is None or beta is None:
            return None
        return (A.dtype, M, N, K, [Cin, A, B], float(alpha), float(beta))

    def run(self, spec, args, kwargs):
        _, _, _, _, (Cin, A, B), alpha, beta = spec
        try:
            return K.addmm(Cin, A, B, beta, alpha, _gemv_max_m(self.tune_params))
        except _lib.Unsupported:
            return None


class BmmImpl(_Family):
    """aten.bmm -> kuiops_bmm (reference BmmImpl kuipy/kuiops.py:475-511)."""
    tune_key = "BMM"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) != 2:
            return None
        A, B = args
        if not (_is_dev(A, B) and A.dim() == 3 and B.dim() == 3 and A.dtype == B.dtype
                and A.dtype in _FLOAT_DTYPES):
            return None
        Bn, M, K = (int(x) for x in A.shape)
        Bn2, K2, N = (int(x) for x in B.shape)
        if Bn != Bn2 or K != K2 or Bn > 65535:
            return None
        return (A.dtype, [A, B])

    def run(self, spec, args, kwargs):
        try:
            return K.bmm(*spec[1])
        except _lib.Unsupported:
            return None


# ------------------------------------------------------------ softmax

class SoftmaxImpl(_Family):
    """aten._softmax over the last dim (reference SoftmaxImpl
    kuipy/kuiops.py:572-610)."""
    tune_key = "SOFTMAX"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) != 3:
            return None
        X, dim, half_to_float = args
        if not (_is_dev(X) and X.dtype in _FLOAT_DTYPES and not half_to_float):
            return None
        rank = X.dim()
        if rank < 1 or _norm_dim(dim, rank) != rank - 1:
            return None
        n = int(X.shape[-1])
        m = X.numel() // n if n else 0
        if m > _SIZE_LIMIT:
            return None
        return (X.dtype, m, n, [X])

    def run(self, spec, args, kwargs):
        try:
            return K.softmax(spec[3][0])
        except _lib.Unsupported:
            return None


# --------------------------------------------------------------- SDPA

class SdpaImpl(_Family):
    """aten._scaled_dot_product_efficient_attention and
    _scaled_dot_product_flash_attention -> kuiops_sdpa_fwd / kuiops_sdpa_decode.

    The reference family (kuipy/kuiops.py:621-681, disconnected at
    kuipy/registry.py:27-28,59) needs a full additive bias and rejects
    is_causal; here an additive bias (any layout broadcastable to
    (N, H, L, S), in the query dtype -- the padding mask of batched
    generation) is served, and so are causal masking, GQA head counts and
    decode shapes.  Returns the aten output tuple with an fp32 (N, H, L)
    log-sum-exp."""
    tune_key = "SDPA"
    tune_params = {"decode_max_rows": 8}

    def _parse(self, func, args, kwargs):
        q, k, v = args[0], args[1], args[2]
        if func == aten._scaled_dot_product_efficient_attention.default:
            bias = args[3] if len(args) > 3 else kwargs.get("attn_bias")
            need_lse = args[4] if len(args) > 4 else kwargs.get("compute_log_sumexp", False)
            dropout = args[5] if len(args) > 5 else kwargs.get("dropout_p", 0.0)
            causal = args[6] if len(args) > 6 else kwargs.get("is_causal", False)
            debug = False
        else:
            bias = None
            need_lse = True
            dropout = args[3] if len(args) > 3 else kwargs.get("dropout_p", 0.0)
            causal = args[4] if len(args) > 4 else kwargs.get("is_causal", False)
            debug = args[5] if len(args) > 5 else kwargs.get("return_debug_mask", False)
        return q, k, v, bias, bool(need_lse), float(dropout), bool(causal), bool(debug)

    def supported(self, func, args, kwargs):
        if len(args) < 3:
            return None
        q, k, v, bias, need_lse, dropout, causal, debug = self._parse(func, args, kwargs)
        if dropout != 0.0 or debug:
            return None
        if not (_is_dev(q, k, v) and q.dim() == 4 and k.dim() == 4 and v.dim() == 4):
            return None
        if not (q.dtype == k.dtype == v.dtype and q.dtype in _FLOATS):
            return None
        n, hq, l, e = (int(x) for x in q.shape)
        n2, hkv, s, e2 = (int(x) for x in k.shape)
        n3, hkv3, s3, ev = (int(x) for x in v.shape)
        if (n, e) != (n2, e2) or (n, hkv, s) != (n3, hkv3, s3) or hkv == 0 or hq % hkv:
            return None
        # the MFMA kernels take 16-bit e == ev <= 128; everything else up to
        # 1024 (any float dtype, e != ev) runs on kuiops_sdpa_general
        if not (0 < e <= 1024 and 0 < ev <= 1024) or n > 65535 or hq > 65535:
            return None
        if bias is not None:
            if not (_is_dev(bias) and bias.device == q.device and bias.dtype == q.dtype and bias.dim() <= 4):
                return None
            try:
                torch.broadcast_shapes(tuple(bias.shape), (n, hq, l, s))
            except RuntimeError:
                return None
        scale = kwargs.get("scale", None)
        if scale is None:
            scale = 1.0 / math.sqrt(e)
        if not scale > 0:
            return None
        return (func, float(scale), causal, need_lse, [q, k, v], bias)

    def tune(self, all_tune_params):
        """Measure, on this GPU, up to how many query rows per KV head the
        split-KV decode kernel beats the flash kernel, as ``decode_max_rows``."""
        from . import tune as _tune
        params = dict(self.tune_params) if isinstance(self.tune_params, dict) else {}
        if torch.cuda.is_available():
            params["decode_max_rows"] = _tune.sweep_decode_max_rows()
        self.tune_params = params
        all_tune_params[self.tune_key] = params
        return all_tune_params

    def run(self, spec, args, kwargs):
        func, scale, causal, need_lse, (q, k, v), bias = spec
        try:
            rows = self.tune_params.get("decode_max_rows", 8) if isinstance(self.tune_params, dict) else 8
            out, lse = K.sdpa(q, k, v, causal, scale, int(rows), bias)
        except _lib.Unsupported:
            return None
        n, hq, l = out.shape[0], out.shape[1], out.shape[2]
        empty = torch.empty([], dtype=torch.int64, device=q.device)
        if func == aten._scaled_dot_product_efficient_attention.default:
            if not need_lse:
                lse = torch.empty((n, hq, 0), dtype=torch.float32, device=q.device)
            return (out, lse, empty, empty)
        none_t = torch.empty(0, dtype=torch.int32, device=q.device)
        return (out, lse, none_t, none_t, int(l), int(k.shape[2]), empty, empty,
                torch.empty(0, dtype=q.dtype, device=q.device))


# ---------------------------------------------------- sampling: top-k

class TopkImpl(_Family):
    """aten.topk -> kuiops_topk_lastdim.  No reference kernel exists
    (kuiops/topk/.gitkeep; KERNELS.md:58): the reference falls through to
    aten.topk, which is what this matches (bit-exact on tie-free input)."""
    tune_key = "TOPK"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) < 2:
            return None
        X, k = args[0], args[1]
        dim = args[2] if len(args) > 2 else kwargs.get("dim", -1)
        largest = args[3] if len(args) > 3 else kwargs.get("largest", True)
        srt = args[4] if len(args) > 4 else kwargs.get("sorted", True)
        if not (_is_dev(X) and X.dtype in (torch.float32, torch.bfloat16, torch.float16) and X.dim() >= 1):
            return None
        dim = _norm_dim(int(dim), X.dim())
        n = int(X.shape[dim])
        k = int(k)
        if not (1 <= k <= min(n, 1024)) or n >= 2 ** 32 - 1:
            return None
        return (X, k, dim, bool(largest), bool(srt))

    def run(self, spec, args, kwargs):
        X, k, dim, largest, srt = spec
        try:
            return K.topk(X, k, dim, largest, srt)
        except _lib.Unsupported:
            return None


# ------------------------------------------------- gather / index

class GatherImpl(_Family):
    """aten.gather -> kuiops_gather (reference GatherImpl kuipy/kuiops.py:711-754;
    its ``shape_le`` gate is relaxed to aten's: only the non-gather axes of
    the index must fit the input)."""
    tune_key = "GATHER"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) < 3 or kwargs.get("sparse_grad", False):
            return None
        Inp, dim, Idx = args[0], args[1], args[2]
        if not (_is_dev(Inp, Idx) and Idx.dtype == torch.int64):
            return None
        rank = Inp.dim()
        if Idx.dim() != rank or rank < 1 or rank > 8:
            return None
        dim = _norm_dim(int(dim), rank)
        if not (0 <= dim < rank) or Inp.element_size() not in (1, 2, 4, 8):
            return None
        if any(int(Idx.shape[d]) > int(Inp.shape[d]) for d in range(rank) if d != dim):
            return None
        return (dim, [Inp, Idx])

    def run(self, spec, args, kwargs):
        dim, (Inp, Idx) = spec
        try:
            return K.gather(Inp, dim, Idx)
        except _lib.Unsupported:
            return None


class ScatterImpl(_Family):
    """aten.scatter.src -> kuiops_scatter (reference ScatterImpl
    kuipy/kuiops.py:757-807: same int64 index, dtype and rank gates; the
    reference's src-shape == index-shape requirement is relaxed to aten's
    src >= index).  Returns a scattered copy of self."""
    tune_key = "SCATTER"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) < 4 or kwargs.get("reduce") is not None:
            return None
        Self, dim, Idx, Src = args[0], args[1], args[2], args[3]
        if not all(isinstance(t, torch.Tensor) for t in (Self, Idx, Src)):
            return None
        if not (_is_dev(Self, Idx, Src) and Idx.dtype == torch.int64 and Src.dtype == Self.dtype):
            return None
        rank = Self.dim()
        if rank < 1 or rank > 8 or Idx.dim() != rank or Src.dim() != rank:
            return None
        dim = _norm_dim(int(dim), rank)
        if not (0 <= dim < rank) or Self.element_size() not in (1, 2, 4, 8):
            return None
        for d in range(rank):
            if int(Idx.shape[d]) > int(Src.shape[d]) or (d != dim and int(Idx.shape[d]) > int(Self.shape[d])):
                return None
        if Self.numel() > _SIZE_LIMIT:
            return None
        return (dim, [Self, Idx, Src])

    def run(self, spec, args, kwargs):
        dim, (Self, Idx, Src) = spec
        try:
            return K.scatter(Self, dim, Idx, Src)
        except _lib.Unsupported:
            return None


class SortImpl(_Family):
    """aten.sort (default and stable overloads) -> kuiops_sort_lastdim: a
    stable sort, a valid result for the unstable overload too.  No reference
    kernel exists (KERNELS.md row aten.sort.default): aten.sort is the
    reference's result."""
    tune_key = "SORT"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if not args or not _is_dev(args[0]):
            return None
        X = args[0]
        if func == aten.sort.stable:
            dim, desc = kwargs.get("dim", -1), kwargs.get("descending", False)
        else:
            dim = args[1] if len(args) > 1 else kwargs.get("dim", -1)
            desc = args[2] if len(args) > 2 else kwargs.get("descending", False)
        if X.dtype not in (torch.float32, torch.bfloat16, torch.float16) or X.dim() < 1:
            return None
        dim = _norm_dim(int(dim), X.dim())
        n = int(X.shape[dim])
        if n >= 2 ** 32 - 1 or (n and X.numel() // n > 65535):
            return None
        return (X, dim, bool(desc))

    def run(self, spec, args, kwargs):
        X, dim, desc = spec
        try:
            return K.sort(X, dim, desc)
        except _lib.Unsupported:
            return None


class CumsumImpl(_Family):
    """aten.cumsum (same-dtype fp32 / fp64 / int64) -> kuiops_cumsum_lastdim.
    No reference kernel (KERNELS.md rows aten.cumsum.default)."""
    tune_key = "CUMSUM"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) < 2 or not _is_dev(args[0]):
            return None
        X, dim = args[0], args[1]
        dt = kwargs.get("dtype")
        if (dt is not None and dt != X.dtype) or X.dtype not in (torch.float32, torch.float64, torch.int64):
            return None
        if X.dim() < 1:
            return None
        return (X, _norm_dim(int(dim), X.dim()))

    def run(self, spec, args, kwargs):
        X, dim = spec
        try:
            return K.cumsum(X, dim)
        except _lib.Unsupported:
            return None


class MultinomialImpl(_Family):
    """aten.multinomial -> kuiops_multinomial: inverse-CDF draws from uniforms
    that torch.rand takes from the call's generator (a different random
    stream than aten's, the same distribution).  With replacement, or one
    sample per row.  No reference kernel (KERNELS.md row
    aten.multinomial.default)."""
    tune_key = "MULTINOMIAL"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) < 2 or not _is_dev(args[0]):
            return None
        P, ns = args[0], int(args[1])
        repl = args[2] if len(args) > 2 else kwargs.get("replacement", False)
        if P.dtype not in (torch.float32, torch.float64, torch.bfloat16, torch.float16) or P.dim() not in (1, 2):
            return None
        if ns < 1 or (not repl and ns > 1) or P.shape[-1] == 0:
            return None
        return (P, ns, kwargs.get("generator"))

    def run(self, spec, args, kwargs):
        P, ns, gen = spec
        rows = 1 if P.dim() == 1 else P.shape[0]
        u = torch.rand((rows, ns), generator=gen, device=P.device, dtype=torch.float32)
        try:
            return K.multinomial(P, ns, u)
        except _lib.Unsupported:
            return None


class IndexImpl(_Family):
    """aten.index.Tensor with int64 index tensors on adjacent axes (any
    number; the reference app's call is a bool mask indexed by two int64
    tensors, KERNELS.md:67) -> kuiops_index (one index tensor, e.g. an
    embedding-row gather) or kuiops_index_multi (several, broadcast
    together).  Bool index tensors (a data-dependent result size) and
    non-adjacent index axes fall through.  No reference kernel
    (kuiops/index/.gitkeep)."""
    tune_key = "INDEX"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) != 2:
            return None
        X, indices = args
        if not _is_dev(X) or X.element_size() not in (1, 2, 4, 8):
            return None
        pos = [i for i, t in enumerate(indices) if t is not None]
        if not pos or pos != list(range(pos[0], pos[0] + len(pos))) or pos[-1] >= X.dim() or len(pos) > 8:
            return None
        idx = [indices[d] for d in pos]
        if not all(isinstance(t, torch.Tensor) and t.dtype == torch.int64 and t.is_cuda and t.device == X.device
                   for t in idx):
            return None
        try:
            torch.broadcast_shapes(*[tuple(t.shape) for t in idx])
        except RuntimeError:
            return None
        return (pos[0], [X] + idx)

    def run(self, spec, args, kwargs):
        d, (X, *idx) = spec
        try:
            return K.index(X, d, idx[0]) if len(idx) == 1 else K.index_multi(X, d, idx)
        except _lib.Unsupported:
            return None


# ------------------------------------------- elementwise / mean / cat

def _operand(x, device):
    """A tensor operand on ``device``, a python scalar (numbers and 0-d CPU
    tensors, which aten treats as wrapped scalars), or None when neither."""
    if isinstance(x, torch.Tensor):
        if x.is_complex():
            return None
        if x.device == device:
            return x
        if x.dim() == 0 and x.device.type == "cpu" and not x.is_meta:
            return x.item()
        return None
    if isinstance(x, (bool, int, float)):
        return x
    return None


def _compute_dtype(dtype):
    if dtype == torch.float64:
        return torch.float64
    if dtype.is_floating_point:
        return torch.float32
    return torch.int64


class ElementwiseImpl(_Family):
    """The reference's ElementwiseImpl (kuipy/kuiops.py:150-320): unary maps,
    binary maps with a tensor or scalar second operand, scalar comparisons,
    where and bitwise ops, over the aten overloads of kuipy/registry.py:33-53
    -> kuiops_elementwise.

    Wider than the reference's gate: operands may broadcast and be strided,
    dtypes promote as aten promotes them (bf16 * fp32 -> fp32), the Tensor
    forms of the comparisons are served, and exp / sqrt / ne / ge / gt are
    added.  Arithmetic is aten's: 16-bit floats compute in fp32, python
    scalars enter unrounded."""
    tune_key = "ELEM"
    tune_params = ()

    _UNARY = {aten.silu.default: _lib.EW_SILU, aten.neg.default: _lib.EW_NEG, aten.rsqrt.default: _lib.EW_RSQRT,
              aten.cos.default: _lib.EW_COS, aten.sin.default: _lib.EW_SIN, aten.exp.default: _lib.EW_EXP,
              aten.sqrt.default: _lib.EW_SQRT}
    _BINARY = {aten.add.Tensor: _lib.EW_ADD, aten.add.Scalar: _lib.EW_ADD, aten.sub.Tensor: _lib.EW_SUB,
               aten.sub.Scalar: _lib.EW_SUB, aten.mul.Tensor: _lib.EW_MUL, aten.mul.Scalar: _lib.EW_MUL,
               aten.div.Tensor: _lib.EW_DIV, aten.div.Scalar: _lib.EW_DIV}
    _COMPARE = {aten.eq.Scalar: _lib.EW_EQ, aten.eq.Tensor: _lib.EW_EQ, aten.ne.Scalar: _lib.EW_NE,
                aten.ne.Tensor: _lib.EW_NE, aten.le.Scalar: _lib.EW_LE, aten.le.Tensor: _lib.EW_LE,
                aten.lt.Scalar: _lib.EW_LT, aten.lt.Tensor: _lib.EW_LT, aten.ge.Scalar: _lib.EW_GE,
                aten.ge.Tensor: _lib.EW_GE, aten.gt.Scalar: _lib.EW_GT, aten.gt.Tensor: _lib.EW_GT}
    _BITWISE = {aten.bitwise_not.default: _lib.EW_BITWISE_NOT, aten.bitwise_and.Tensor: _lib.EW_BITWISE_AND,
                aten.bitwise_or.Tensor: _lib.EW_BITWISE_OR}
    OPS = (tuple(_UNARY) + tuple(_BINARY) + tuple(_COMPARE) + tuple(_BITWISE)
           + (aten.pow.Tensor_Scalar, aten.where.self))

    def supported(self, func, args, kwargs):
        if not args or not _is_dev(args[0]) or args[0].is_complex():
            return None
        A = args[0]
        dev = A.device
        if func in self._UNARY:
            if len(args) != 1 or kwargs:
                return None
            if not (A.dtype.is_floating_point or (func == aten.neg.default and A.dtype != torch.bool)):
                return None
            return (self._UNARY[func], [A], A.dtype, _compute_dtype(A.dtype), 1.0, 0.0)
        if func == aten.pow.Tensor_Scalar:
            e = args[1] if len(args) > 1 else None
            if not A.dtype.is_floating_point or isinstance(e, bool) or not isinstance(e, (int, float)):
                return None
            return (_lib.EW_POW_SCALAR, [A], A.dtype, _compute_dtype(A.dtype), float(e), 0.0)
        if func == aten.where.self:
            if len(args) != 3 or A.dtype != torch.bool:
                return None
            x, y = (_operand(t, dev) for t in args[1:])
            if x is None or y is None:
                return None
            out = torch.result_type(args[1], args[2])
            return (_lib.EW_WHERE, [A, x, y], out, _compute_dtype(out), 1.0, 0.0)
        if func in self._BITWISE:
            return None if kwargs else self._bitwise(func, args)
        if len(args) != 2:
            return None
        other = _operand(args[1], dev)
        if other is None:
            return None
        out = torch.result_type(A, args[1] if isinstance(args[1], torch.Tensor) else other)
        if func in self._COMPARE:
            if kwargs:
                return None
            return self._binary_spec(self._COMPARE[func], A, other, torch.bool, _compute_dtype(out), 1.0)
        op = self._BINARY.get(func)
        if op is None:
            return None
        alpha = 1.0
        if op in (_lib.EW_ADD, _lib.EW_SUB):
            a = kwargs.get("alpha", 1)
            if isinstance(a, bool) or not isinstance(a, (int, float)):
                return None
            alpha = float(a)
            if op == _lib.EW_SUB and out == torch.bool:
                return None
        elif kwargs.get("rounding_mode") is not None or set(kwargs) - {"rounding_mode"}:
            return None
        if op == _lib.EW_DIV and not out.is_floating_point:
            out = torch.get_default_dtype()
        return self._binary_spec(op, A, other, out, _compute_dtype(out), alpha)

    @staticmethod
    def _binary_spec(op, A, other, out, compute, alpha):
        if isinstance(other, torch.Tensor):
            return (op, [A, other], out, compute, alpha, 0.0)
        return (op, [A], out, compute, alpha, float(other))

    def _bitwise(self, func, args):
        A = args[0]
        if A.dtype.is_floating_point:
            return None
        if func == aten.bitwise_not.default:
            return (_lib.EW_BITWISE_NOT, [A], A.dtype, torch.int64, 1.0, 0.0) if len(args) == 1 else None
        if len(args) != 2 or not _is_dev(args[1]) or args[1].device != A.device or args[1].dtype.is_floating_point:
            return None
        out = torch.promote_types(A.dtype, args[1].dtype)
        return (self._BITWISE[func], [A, args[1]], out, torch.int64, 1.0, 0.0)

    def run(self, spec, args, kwargs):
        op, inputs, out, compute, s0, s1 = spec
        dev = inputs[0].device
        # where's scalar branches become 0-d device tensors (a fill kernel)
        inputs = [t if isinstance(t, torch.Tensor) else torch.full((), t, dtype=out, device=dev) for t in inputs]
        try:
            return K.elementwise(op, inputs, out, compute, s0, s1)
        except _lib.Unsupported:
            return None


class MeanImpl(_Family):
    """aten.mean.dim over the last axis -> kuiops_mean_lastdim (reference
    MeanImpl kuipy/kuiops.py:860-921, which takes keepdim=True only; both
    keepdim forms are served here)."""
    tune_key = "MEAN"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if len(args) < 2 or not _is_dev(args[0]):
            return None
        X, dim = args[0], args[1]
        keepdim = args[2] if len(args) > 2 else kwargs.get("keepdim", False)
        dt = kwargs.get("dtype")
        if (dt is not None and dt != X.dtype) or X.dtype not in _FLOAT_DTYPES or X.dim() < 1:
            return None
        if isinstance(dim, (list, tuple)):
            if len(dim) != 1:
                return None
            dim = dim[0]
        if dim is None or _norm_dim(int(dim), X.dim()) != X.dim() - 1 or X.shape[-1] == 0:
            return None
        return (X, bool(keepdim))

    def run(self, spec, args, kwargs):
        X, keepdim = spec
        try:
            return K.mean_lastdim(X, keepdim)
        except _lib.Unsupported:
            return None


class CatImpl(_Family):
    """aten.cat.default -> kuiops_cat (reference CatImpl kuipy/kuiops.py:810-857,
    two inputs only; here up to 32 inputs of one dtype and rank, strided
    inputs read in place when each row of the concatenated dims is one run)."""
    tune_key = "CAT"
    tune_params = ()

    def supported(self, func, args, kwargs):
        if not args:
            return None
        tensors = args[0]
        dim = args[1] if len(args) > 1 else kwargs.get("dim", 0)
        if not isinstance(tensors, (list, tuple)) or not 1 <= len(tensors) <= 32:
            return None
        A = tensors[0]
        if not _is_dev(*tensors) or A.dim() < 1:
            return None
        if any(t.dtype != A.dtype or t.device != A.device or t.dim() != A.dim() for t in tensors):
            return None
        d = _norm_dim(int(dim), A.dim())
        if not 0 <= d < A.dim():
            return None
        if any(t.shape[i] != A.shape[i] for t in tensors for i in range(A.dim()) if i != d):
            return None
        return (list(tensors), d)

    def run(self, spec, args, kwargs):
        tensors, d = spec
        try:
            return K.cat(tensors, d)
        except _lib.Unsupported:
            return None


ALL_FAMILIES = (MmImpl, AddmmImpl, BmmImpl, SoftmaxImpl, SdpaImpl, TopkImpl, GatherImpl, IndexImpl, ScatterImpl,
                SortImpl, CumsumImpl, MultinomialImpl, ElementwiseImpl, MeanImpl, CatImpl)
log(f"kuiops families: {[f.__name__ for f in ALL_FAMILIES]}")
