"""Tensor-level API over the kuiops C ABI (include/kuiops.h).

Each function checks shapes on the host, allocates its outputs with torch
(PyTorch-ROCm is the device-memory and stream plumbing here), and enqueues the
HIP kernels on the current torch stream through ``_lib``.  Nothing here
synchronises the device, so every function can be recorded in a HIP graph
(workspaces are allocated on first use, outside capture).

There is no fallback in this module: a shape the kernels do not cover raises
``_lib.Unsupported``; the ``kuiops`` op families decide whether to fall back to
stock PyTorch (the reference's dispatch contract, kuipy/__init__.py:53-75).
"""
from __future__ import annotations

import ctypes
import math
import os

import torch

from . import _lib
from . import compile as _compile

_DT = {
    torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16,
    torch.float64: _lib.F64, torch.int64: _lib.I64, torch.int32: _lib.I32,
    torch.int16: _lib.I16, torch.int8: _lib.I8, torch.uint8: _lib.U8, torch.bool: _lib.BOOL,
}
HALF = (torch.bfloat16, torch.float16)
CHECK_INDEX = os.environ.get("KUIOPS_CHECK_INDEX", "0") == "1"


def _lib_handle():
    return _compile.load_library()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _dt(dtype) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise _lib.Unsupported("dtype", _lib.E_UNSUPPORTED) from None


# ----------------------------------------------------------------- workspace
# One buffer per (device, stream, kind), so calls in flight on two streams
# never share split counters or partials.  "gemv" and "attn" hold split
# arrival counters (decode GEMM, decode attention), which must start at
# zero: they are zero-filled when allocated and the kernels leave the
# counters at zero.  "scratch" is plain partial-result space.
#
# A HIP graph records the raw address of the buffer it was captured with.
# Growing during capture would put the new allocation and its zero fill
# inside the graph, so it is refused: run the largest shape once eagerly
# first.  A capture stream with no buffer of its own, or one too small (the
# eager warm-up ran on another stream, as with torch.cuda.graph's default
# capture stream), takes the device's largest buffer of that kind; replays of that graph must
# then not overlap eager calls on the warm-up stream.  When a call needs more
# bytes, the old buffer is released (stream-ordered, through torch's caching
# allocator) unless a graph was captured with it: those are kept in
# _RETIRED for the life of the process, counters still zero.
_WS = {}
_RETIRED = []
_CAPTURED = set()        # data_ptr of every buffer handed out during a capture


def _stream_key(device: torch.device) -> int:
    """The stream a workspace is keyed on: torch's current stream on the device."""
    if device.type != "cuda":
        return 0
    return torch.cuda.current_stream(device).cuda_stream


def _capturing(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_current_stream_capturing()


def _ws_key(device: torch.device, kind: str):
    dev = device.index if device.index is not None else (
        torch.cuda.current_device() if device.type == "cuda" else 0)
    return dev, _stream_key(device), kind


def workspace(device: torch.device, nbytes: int, kind: str = "scratch") -> torch.Tensor:
    capturing = _capturing(device)
    key = _ws_key(device, kind)
    buf = _WS.get(key)
    if capturing and (buf is None or buf.numel() < nbytes):
        same = [b for (d, _, k), b in _WS.items() if d == key[0] and k == kind and b.numel() >= nbytes]
        if same:
            buf = max(same, key=lambda t: t.numel())
            _WS[key] = buf
    if buf is None or buf.numel() < nbytes:
        if capturing:
            raise RuntimeError(
                f"kuiops workspace '{kind}' must grow to {nbytes} bytes during HIP graph capture; "
                "run the same calls once outside capture first")
        size = max(int(nbytes), 1 << 20)
        size = (size + (1 << 20) - 1) // (1 << 20) * (1 << 20)
        if buf is not None and buf.data_ptr() in _CAPTURED:
            _RETIRED.append(buf)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _WS[key] = buf
    if capturing:
        _CAPTURED.add(buf.data_ptr())
    return buf


def workspace_buffer(device: torch.device, kind: str) -> torch.Tensor | None:
    """The current stream's workspace of ``kind`` on ``device`` (None if none yet)."""
    return _WS.get(_ws_key(device, kind))


# -------------------------------------------------------------------- layout

def _rowmajor(A: torch.Tensor) -> torch.Tensor:
    """A 2-D view with unit column stride and a row stride >= its width."""
    if A.stride(-1) != 1 or (A.size(0) > 1 and A.stride(0) < A.size(1)):
        A = A.contiguous()
    return A


def _b_operand(B: torch.Tensor):
    """(tensor, ld, layout) for a [K, N] operand: N-contiguous or K-contiguous."""
    K, N = B.shape
    if B.stride(1) == 1 and (K <= 1 or B.stride(0) >= N):
        return B, max(B.stride(0), N), _lib.B_ROW
    if B.stride(0) == 1 and (N <= 1 or B.stride(1) >= K):
        return B, max(B.stride(1), K), _lib.B_COL
    B = B.contiguous()
    return B, N, _lib.B_ROW


# ---------------------------------------------------------------------- GEMM

GEMV_MAX_M = 64


def _gemv(x, B, ldb, layout, bias, out):
    M, K = x.shape
    N = B.shape[1]
    lib = _lib_handle()
    ws_bytes = lib.kuiops_query_workspace(_lib.OP_GEMV_SPLITK, M, N, K)
    ws = workspace(x.device, ws_bytes, "gemv")
    _lib.check("kuiops_gemv_splitk", lib.kuiops_gemv_splitk(
        M, N, K, _dt(x.dtype), x.data_ptr(), x.stride(0), B.data_ptr(), ldb, layout,
        _ptr(bias), _dt(out.dtype), out.data_ptr(), out.stride(0), 0, ws.data_ptr(), ws.numel(),
        _stream(x.device)))
    return out


def mm(A: torch.Tensor, B: torch.Tensor, out_dtype=None, gemv_max_m: int | None = None) -> torch.Tensor:
    """A[M, K] @ B[K, N] with fp32 accumulation (aten.mm semantics); rows
    M <= gemv_max_m (default GEMV_MAX_M, at most 64) take the decode GEMM."""
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0] or A.dtype != B.dtype:
        raise _lib.KuiopsError("mm", _lib.E_INVALID)
    A = _rowmajor(A)
    B, ldb, layout = _b_operand(B)
    M, K = A.shape
    N = B.shape[1]
    out = torch.empty((M, N), dtype=out_dtype or A.dtype, device=A.device)
    if M == 0 or N == 0:
        return out
    if K == 0:
        return out.zero_()
    if A.dtype in HALF and M <= min(GEMV_MAX_M, GEMV_MAX_M if gemv_max_m is None else gemv_max_m):
        try:
            return _gemv(A, B, ldb, layout, None, out)
        except _lib.Unsupported:
            pass
    lib = _lib_handle()
    ws_bytes = lib.kuiops_query_workspace(_lib.OP_ADDMM, M, N, K) if A.dtype in HALF else 0
    if ws_bytes:
        # Too few output tiles to fill the GPU: the same kernels with split-K,
        # whose fp32 partials need a workspace (kuiops_mm takes none), through
        # the addmm entry point with no addend.
        ws = workspace(A.device, ws_bytes)
        _lib.check("kuiops_addmm", lib.kuiops_addmm(
            M, K, N, 1.0, 0.0, _dt(A.dtype), A.data_ptr(), A.stride(0), B.data_ptr(), ldb, layout,
            None, _lib.C_NONE, 0, _dt(out.dtype), out.data_ptr(), out.stride(0),
            0, ws.data_ptr(), ws.numel(), _stream(A.device)))
        return out
    _lib.check("kuiops_mm", lib.kuiops_mm(
        M, N, K, _dt(A.dtype), A.data_ptr(), A.stride(0), B.data_ptr(), ldb, layout,
        _dt(out.dtype), out.data_ptr(), out.stride(0), _stream(A.device)))
    return out


def addmm(C: torch.Tensor, A: torch.Tensor, B: torch.Tensor, beta=1.0, alpha=1.0,
          gemv_max_m: int | None = None) -> torch.Tensor:
    """beta * C + alpha * (A @ B) with C broadcast to [M, N] (aten.addmm); rows
    M <= gemv_max_m (default GEMV_MAX_M) take the decode GEMM."""
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise _lib.KuiopsError("addmm", _lib.E_INVALID)
    if not (A.dtype == B.dtype == C.dtype):
        raise _lib.KuiopsError("addmm", _lib.E_INVALID)
    A = _rowmajor(A)
    B, ldb, layout = _b_operand(B)
    M, K = A.shape
    N = B.shape[1]
    beta, alpha = float(beta), float(alpha)
    if beta == 0.0:
        c_kind, Cin, ldcin = _lib.C_NONE, None, 0
    elif C.dim() == 1 and C.shape[0] == N or (C.dim() == 2 and C.shape[0] == 1 and C.shape[1] == N):
        c_kind, Cin, ldcin = _lib.C_ROW, C.reshape(N).contiguous(), 0
    else:
        Cin = C.expand(M, N)
        if Cin.stride(1) != 1 or Cin.stride(0) < N:
            Cin = Cin.contiguous()
        c_kind, ldcin = _lib.C_FULL, Cin.stride(0)
    out = torch.empty((M, N), dtype=A.dtype, device=A.device)
    if M == 0 or N == 0:
        return out
    if (A.dtype in HALF and M <= min(GEMV_MAX_M, GEMV_MAX_M if gemv_max_m is None else gemv_max_m)
            and alpha == 1.0 and K > 0
            and (c_kind == _lib.C_NONE or (c_kind == _lib.C_ROW and beta == 1.0))):
        try:
            return _gemv(A, B, ldb, layout, Cin, out)
        except _lib.Unsupported:
            pass
    lib = _lib_handle()
    ws_bytes = lib.kuiops_query_workspace(_lib.OP_ADDMM, M, N, K)
    ws = workspace(A.device, ws_bytes) if ws_bytes else None
    _lib.check("kuiops_addmm", lib.kuiops_addmm(
        M, K, N, alpha, beta, _dt(A.dtype), A.data_ptr(), A.stride(0), B.data_ptr(), ldb, layout,
        _ptr(Cin), c_kind, ldcin, _dt(out.dtype), out.data_ptr(), out.stride(0),
        0, _ptr(ws), 0 if ws is None else ws.numel(), _stream(A.device)))
    return out


def linear(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x[..., K] @ W[N, K]^T (+ bias): nn.Linear with a K-contiguous weight."""
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if bias is None:
        y = mm(x2, W.t())
    else:
        y = addmm(bias, x2, W.t())
    return y.reshape(*lead, W.shape[0])


def bmm(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """C[b] = A[b] @ B[b] (aten.bmm)."""
    if A.dim() != 3 or B.dim() != 3 or A.shape[0] != B.shape[0] or A.shape[2] != B.shape[1]:
        raise _lib.KuiopsError("bmm", _lib.E_INVALID)
    if A.dtype != B.dtype:
        raise _lib.KuiopsError("bmm", _lib.E_INVALID)
    Bn, M, K = A.shape
    N = B.shape[2]
    if A.stride(2) != 1 or (M > 1 and A.stride(1) < K):
        A = A.contiguous()
    if B.stride(2) == 1 and (K <= 1 or B.stride(1) >= N):
        layout, ldb = _lib.B_ROW, max(B.stride(1), N)
    elif B.stride(1) == 1 and (N <= 1 or B.stride(2) >= K):
        layout, ldb = _lib.B_COL, max(B.stride(2), K)
    else:
        B = B.contiguous()
        layout, ldb = _lib.B_ROW, N
    out = torch.empty((Bn, M, N), dtype=A.dtype, device=A.device)
    if out.numel() == 0:
        return out
    if K == 0:
        return out.zero_()
    lib = _lib_handle()
    _lib.check("kuiops_bmm", lib.kuiops_bmm(
        Bn, M, K, N, _dt(A.dtype), A.data_ptr(), A.stride(0), A.stride(1),
        B.data_ptr(), B.stride(0), ldb, layout, _dt(out.dtype), out.data_ptr(),
        out.stride(0), out.stride(1), _stream(A.device)))
    return out


# ---------------------------------------------------------------------- SDPA

def _lastdim_contig(t):
    return t if t.stride(-1) == 1 else t.contiguous()


def _attn_prep(q, k, v):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise _lib.KuiopsError("sdpa", _lib.E_INVALID)
    q, k, v = _lastdim_contig(q), _lastdim_contig(k), _lastdim_contig(v)
    n, hq, l, e = q.shape
    _, hkv, s, _ = k.shape
    ev = v.shape[-1]
    if k.shape[0] != n or v.shape[0] != n or v.shape[1] != hkv or v.shape[2] != s or k.shape[3] != e:
        raise _lib.KuiopsError("sdpa", _lib.E_INVALID)
    if hkv == 0 or hq % hkv:
        raise _lib.KuiopsError("sdpa", _lib.E_INVALID)
    return q, k, v, (n, hq, hkv, l, s, e, ev)


def _bias_view(bias, n, hq, l, s, dtype):
    """The additive bias as an (n, hq, l, s) view with a unit key stride,
    strides that are multiples of 4 and an 8-byte aligned base (broadcast
    dims keep stride 0).  A misaligned bias is copied with its key axis padded
    to a multiple of 4 before it is broadcast, never after."""
    if bias.dtype != dtype or bias.dim() > 4:
        raise _lib.Unsupported("sdpa_fwd_bias", _lib.E_UNSUPPORTED)
    b = bias.reshape((1,) * (4 - bias.dim()) + tuple(bias.shape)) if bias.dim() < 4 else bias
    if b.shape[-1] == 1 and s > 1:
        b = b.expand(*b.shape[:-1], s)
    if s > 1 and b.stride(-1) != 1:
        b = b.contiguous()
    if any(st % 4 for sz, st in zip(b.shape[:3], b.stride()[:3]) if sz > 1) or b.data_ptr() % 8:
        b = torch.nn.functional.pad(b, (0, (-b.shape[-1]) % 4))[..., :b.shape[-1]]
    return b.expand(n, hq, l, s)


def _sdpa_general(q, k, v, is_causal, scale, return_lse, out, bias, dims):
    """kuiops_sdpa_general: fp32 / fp64 inputs, e != ev, head dims past 128."""
    n, hq, hkv, l, s, e, ev = dims
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.bfloat16, torch.float16, torch.float32,
                                                                torch.float64):
        raise _lib.Unsupported("sdpa_general", _lib.E_UNSUPPORTED)
    if out is None:
        out = torch.empty((n, hq, l, ev), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (n, hq, l, ev) or out.stride(-1) != 1 or out.dtype != q.dtype:
        raise _lib.KuiopsError("sdpa", _lib.E_INVALID)
    lse = torch.empty((n, hq, l), dtype=torch.float32, device=q.device) if return_lse else None
    if out.numel() == 0:
        if lse is not None:
            lse.fill_(-math.inf)
        return out, lse
    b = None
    if bias is not None:
        if bias.dtype != q.dtype or bias.dim() > 4:
            raise _lib.Unsupported("sdpa_general", _lib.E_UNSUPPORTED)
        b = bias.reshape((1,) * (4 - bias.dim()) + tuple(bias.shape)).expand(n, hq, l, s)
        if s > 1 and b.stride(-1) != 1:
            b = b.contiguous()
    _lib.check("kuiops_sdpa_general", _lib_handle().kuiops_sdpa_general(
        n, hq, hkv, l, s, e, ev, _dt(q.dtype), q.data_ptr(), _lib.strides3(*q.stride()[:3]), k.data_ptr(),
        _lib.strides3(*k.stride()[:3]), v.data_ptr(), _lib.strides3(*v.stride()[:3]), out.data_ptr(),
        _lib.strides3(*out.stride()[:3]), _ptr(lse), float(scale), 1 if is_causal else 0, _ptr(b),
        _lib.strides3(*b.stride()[:3]) if b is not None else None, _stream(q.device)))
    return out, lse


def _pad_head(t, e_pad):
    e = t.shape[-1]
    return t if e == e_pad else torch.nn.functional.pad(t, (0, e_pad - e))


def sdpa(q, k, v, is_causal=False, scale=None, return_lse=True, decode_max_rows=8, out=None, bias=None):
    """softmax(scale * q k^T [+ bias] [causal]) v  ->  (out, lse)   (aten SDPA
    semantics).

    q (n, hq, l, e), k / v (n, hkv, s, e) with hq % hkv == 0; causal masking is
    aten's top-left alignment (query i sees keys j <= i).  ``bias`` is an
    additive mask broadcastable to (n, hq, l, s) in q's dtype (-inf masks a
    key), as aten's efficient-attention attn_bias.  Non-causal calls without
    a bias and with few query rows per KV head use the split-KV decode kernel.
    ``out`` ([n, hq, l, ev] with a unit last stride, e.g. a transposed view of
    an [n, l, hq, ev] buffer) receives the result in place.
    """
    q, k, v, (n, hq, hkv, l, s, e, ev) = _attn_prep(q, k, v)
    if scale is None:
        scale = 1.0 / math.sqrt(e)
    if q.dtype not in HALF or e != ev or e > 128:
        return _sdpa_general(q, k, v, is_causal, scale, return_lse, out, bias, (n, hq, hkv, l, s, e, ev))
    if e == ev and e < 128 and e not in (64,) and q.dtype in HALF:
        # other head dims: zero-pad to the kernels' 64 / 128 (q k^T and the
        # kept output columns are unchanged; the scale is the caller's)
        e_pad = 64 if e < 64 else 128
        o, lse = sdpa(_pad_head(q, e_pad), _pad_head(k, e_pad), _pad_head(v, e_pad), is_causal, scale,
                      return_lse, decode_max_rows, None, bias)
        o = o[..., :e]
        if out is not None:
            out.copy_(o)
            o = out
        return o, lse
    if out is None:
        out = torch.empty((n, hq, l, ev), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (n, hq, l, ev) or out.stride(-1) != 1 or out.dtype != q.dtype:
        raise _lib.KuiopsError("sdpa", _lib.E_INVALID)
    lse = torch.empty((n, hq, l), dtype=torch.float32, device=q.device) if return_lse else None
    if out.numel() == 0:
        return out, lse
    lib = _lib_handle()
    sq = _lib.strides3(*q.stride()[:3])
    sk = _lib.strides3(*k.stride()[:3])
    sv = _lib.strides3(*v.stride()[:3])
    so = _lib.strides3(*out.stride()[:3])
    if bias is not None:
        b = _bias_view(bias, n, hq, l, s, q.dtype)
        _lib.check("kuiops_sdpa_fwd_bias", lib.kuiops_sdpa_fwd_bias(
            n, hq, hkv, l, s, e, ev, _dt(q.dtype), q.data_ptr(), sq, k.data_ptr(), sk,
            v.data_ptr(), sv, out.data_ptr(), so, _ptr(lse), float(scale), 1 if is_causal else 0,
            b.data_ptr(), _lib.strides3(*b.stride()[:3]), _stream(q.device)))
        return out, lse
    if not is_causal and (hq // hkv) * l <= decode_max_rows and s > 0:
        ws_bytes = lib.kuiops_query_workspace(_lib.OP_SDPA_DECODE, n * hq * l, s, ev)
        ws = workspace(q.device, ws_bytes, "attn")
        _lib.check("kuiops_sdpa_decode", lib.kuiops_sdpa_decode(
            n, hq, hkv, l, s, e, ev, _dt(q.dtype), q.data_ptr(), sq, k.data_ptr(), sk,
            v.data_ptr(), sv, out.data_ptr(), so, _ptr(lse), float(scale), 0, None,
            ws.data_ptr(), ws.numel(), _stream(q.device)))
        return out, lse
    _lib.check("kuiops_sdpa_fwd", lib.kuiops_sdpa_fwd(
        n, hq, hkv, l, s, e, ev, _dt(q.dtype), q.data_ptr(), sq, k.data_ptr(), sk,
        v.data_ptr(), sv, out.data_ptr(), so, _ptr(lse), float(scale), 1 if is_causal else 0,
        _stream(q.device)))
    return out, lse


def sdpa_decode(q, k, v, scale=None, causal=True, return_lse=False, kv_len=None, out=None):
    """Decode attention over a KV cache: the l queries are the LAST l positions
    of the s keys (query i sees keys j <= s - l + i when ``causal``).

    ``kv_len`` (int32 [n] on the device) limits batch entry b to its first
    kv_len[b] keys, read when the kernel runs; k / v may then be the whole
    cache (s = capacity).  ``out`` ([n, hq, l, ev], any strides with a unit
    last stride) receives the result in place."""
    q, k, v, (n, hq, hkv, l, s, e, ev) = _attn_prep(q, k, v)
    if scale is None:
        scale = 1.0 / math.sqrt(e)
    if kv_len is not None and (kv_len.dtype != torch.int32 or kv_len.numel() != n or not kv_len.is_contiguous()):
        raise _lib.KuiopsError("sdpa_decode", _lib.E_INVALID)
    if out is None:
        out = torch.empty((n, hq, l, ev), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (n, hq, l, ev) or out.stride(-1) != 1 or out.dtype != q.dtype:
        raise _lib.KuiopsError("sdpa_decode", _lib.E_INVALID)
    lse = torch.empty((n, hq, l), dtype=torch.float32, device=q.device) if return_lse else None
    if out.numel() == 0:
        return out, lse
    lib = _lib_handle()
    ws_bytes = lib.kuiops_query_workspace(_lib.OP_SDPA_DECODE, n * hq * l, s, ev)
    ws = workspace(q.device, ws_bytes, "attn")
    _lib.check("kuiops_sdpa_decode", lib.kuiops_sdpa_decode(
        n, hq, hkv, l, s, e, ev, _dt(q.dtype), q.data_ptr(), _lib.strides3(*q.stride()[:3]),
        k.data_ptr(), _lib.strides3(*k.stride()[:3]), v.data_ptr(), _lib.strides3(*v.stride()[:3]),
        out.data_ptr(), _lib.strides3(*out.stride()[:3]), _ptr(lse), float(scale), 1 if causal else 0,
        _ptr(kv_len), ws.data_ptr(), ws.numel(), _stream(q.device)))
    return out, lse


# ------------------------------------------------------------ sampling tail

def softmax(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Softmax over the last dim (aten._softmax with half_to_float=False)."""
    if x.dim() == 0 or (dim % x.dim()) != x.dim() - 1:
        raise _lib.Unsupported("softmax", _lib.E_UNSUPPORTED)
    xc = x.contiguous()
    n = xc.shape[-1] if xc.dim() else 1
    m = xc.numel() // n if n else 0
    out = torch.empty_like(xc)
    if xc.numel() == 0:
        return out
    lib = _lib_handle()
    _lib.check("kuiops_softmax_lastdim", lib.kuiops_softmax_lastdim(
        m, n, _dt(x.dtype), xc.data_ptr(), out.data_ptr(), _stream(x.device)))
    return out


def topk(x: torch.Tensor, k: int, dim: int = -1, largest: bool = True, sorted: bool = True, out=None):
    """(values, int64 indices) of the k largest / smallest along ``dim``; ties
    are ordered by ascending index and NaN is treated as the largest value.
    ``out`` = (values, indices): contiguous buffers of the result's shape
    (last dim only) written in place."""
    if x.dim() == 0:
        raise _lib.Unsupported("topk", _lib.E_UNSUPPORTED)
    dim = dim % x.dim()
    moved = dim != x.dim() - 1
    xc = (x.movedim(dim, -1) if moved else x).contiguous()
    n = xc.shape[-1]
    k = int(k)
    if k < 0 or k > n:
        raise _lib.KuiopsError("topk", _lib.E_INVALID)
    m = xc.numel() // n if n else 0
    if out is not None:
        vals, inds = out
        shape = (*xc.shape[:-1], k)
        if moved or vals.numel() != m * k or inds.numel() != m * k or vals.dtype != x.dtype or \
                inds.dtype != torch.int64 or not vals.is_contiguous() or not inds.is_contiguous():
            raise _lib.KuiopsError("topk", _lib.E_INVALID)
        vals, inds = vals.view(shape), inds.view(shape)
    else:
        vals = torch.empty((*xc.shape[:-1], k), dtype=x.dtype, device=x.device)
        inds = torch.empty((*xc.shape[:-1], k), dtype=torch.int64, device=x.device)
    if vals.numel():
        lib = _lib_handle()
        _lib.check("kuiops_topk_lastdim", lib.kuiops_topk_lastdim(
            m, n, k, _dt(x.dtype), xc.data_ptr(), vals.data_ptr(), inds.data_ptr(),
            1 if largest else 0, 1 if sorted else 0, None, 0, _stream(x.device)))
    if moved:
        vals, inds = vals.movedim(-1, dim), inds.movedim(-1, dim)
    return vals, inds


def softmax_top1(x: torch.Tensor, index_out: torch.Tensor | None = None, prob_out: torch.Tensor | None = None,
                 pos: torch.Tensor | None = None, kv_len: torch.Tensor | None = None,
                 history: torch.Tensor | None = None):
    """Greedy tail in one launch: (probability, int64 index) of the top-1 of
    softmax(x.float()) per row of x [m, n] (n <= 32768), equal to
    ``topk(softmax(x.float()), 1)``; optionally records the index in
    ``history`` [m, L] (int64) at column pos[row] and advances the device
    int32 ``pos`` / ``kv_len`` [m] by one (see kuiops_softmax_top1)."""
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    m, n = x2.shape
    if index_out is None:
        index_out = torch.empty(m, dtype=torch.int64, device=x.device)
    if index_out.numel() != m or index_out.dtype != torch.int64 or not index_out.is_contiguous():
        raise _lib.KuiopsError("softmax_top1", _lib.E_INVALID)
    for t in (prob_out, pos, kv_len):
        if t is not None and (t.numel() != m or not t.is_contiguous()):
            raise _lib.KuiopsError("softmax_top1", _lib.E_INVALID)
    if (prob_out is not None and prob_out.dtype != torch.float32) or \
            any(t is not None and t.dtype != torch.int32 for t in (pos, kv_len)):
        raise _lib.KuiopsError("softmax_top1", _lib.E_INVALID)
    if history is not None and (pos is None or history.dim() != 2 or history.shape[0] != m
                                or history.dtype != torch.int64 or not history.is_contiguous()):
        raise _lib.KuiopsError("softmax_top1", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_softmax_top1", lib.kuiops_softmax_top1(
        m, n, _dt(x.dtype), x2.data_ptr(), _ptr(prob_out), index_out.data_ptr(), _ptr(pos), _ptr(kv_len),
        _ptr(history), history.shape[1] if history is not None else 0, _stream(x.device)))
    return prob_out, index_out


def _err_flag(device):
    return torch.zeros(1, dtype=torch.int32, device=device) if CHECK_INDEX else None


def _raise_if_flagged(flag, what):
    if flag is not None and int(flag.item()) != 0:
        raise IndexError(f"{what}: index out of range")


def gather(inp: torch.Tensor, dim: int, idx: torch.Tensor, check: bool | None = None) -> torch.Tensor:
    """torch.gather(inp, dim, idx) for contiguous int64 indices (bit-exact)."""
    if idx.dtype != torch.int64 or idx.dim() != inp.dim() or inp.dim() < 1 or inp.dim() > 8:
        raise _lib.Unsupported("gather", _lib.E_UNSUPPORTED)
    dim = dim % inp.dim()
    for d in range(inp.dim()):
        if d != dim and idx.shape[d] > inp.shape[d]:
            raise _lib.KuiopsError("gather", _lib.E_INVALID)
    ic, xc = inp.contiguous(), idx.contiguous()
    out = torch.empty(idx.shape, dtype=inp.dtype, device=inp.device)
    if out.numel() == 0:
        return out
    flag = torch.zeros(1, dtype=torch.int32, device=inp.device) if (check or (check is None and CHECK_INDEX)) else None
    lib = _lib_handle()
    _lib.check("kuiops_gather", lib.kuiops_gather(
        inp.dim(), _lib.i64_array(ic.shape), _lib.i64_array(xc.shape), dim, ic.element_size(),
        ic.data_ptr(), xc.data_ptr(), out.data_ptr(), _ptr(flag), _stream(inp.device)))
    _raise_if_flagged(flag, "gather")
    return out


def index(inp: torch.Tensor, dim: int, idx: torch.Tensor, check: bool | None = None, out=None) -> torch.Tensor:
    """inp[(slice(None),) * dim + (idx,)] for one int64 index tensor
    (aten.index.Tensor with a single index); negative indices wrap.  ``out``
    (contiguous, the result's shape and dtype) receives it in place."""
    if idx.dtype != torch.int64 or inp.dim() < 1:
        raise _lib.Unsupported("index", _lib.E_UNSUPPORTED)
    dim = dim % inp.dim()
    ic, xc = inp.contiguous(), idx.contiguous()
    outer = math.prod(ic.shape[:dim])
    size = ic.shape[dim]
    inner = math.prod(ic.shape[dim + 1:])
    shape = (*ic.shape[:dim], *xc.shape, *ic.shape[dim + 1:])
    if out is None:
        out = torch.empty(shape, dtype=inp.dtype, device=inp.device)
    elif tuple(out.shape) != shape or out.dtype != inp.dtype or not out.is_contiguous():
        raise _lib.KuiopsError("index", _lib.E_INVALID)
    if out.numel() == 0:
        return out
    flag = torch.zeros(1, dtype=torch.int32, device=inp.device) if (check or (check is None and CHECK_INDEX)) else None
    lib = _lib_handle()
    _lib.check("kuiops_index", lib.kuiops_index(
        outer, size, inner, xc.numel(), ic.element_size(), ic.data_ptr(), xc.data_ptr(),
        out.data_ptr(), _ptr(flag), _stream(inp.device)))
    _raise_if_flagged(flag, "index")
    return out


def index_multi(inp: torch.Tensor, first: int, idxs, check: bool | None = None) -> torch.Tensor:
    """inp[(slice(None),) * first + tuple(idxs)] for k >= 1 int64 index tensors
    on the adjacent axes first .. first + k - 1 (aten.index.Tensor advanced
    indexing): the index tensors broadcast together, and the result is
    inp.shape[:first] + broadcast shape + inp.shape[first + k:]."""
    k = len(idxs)
    if k < 1 or k > 8 or any(t.dtype != torch.int64 for t in idxs) or first < 0 or first + k > inp.dim():
        raise _lib.Unsupported("index_multi", _lib.E_UNSUPPORTED)
    if inp.element_size() not in (1, 2, 4, 8):
        raise _lib.Unsupported("index_multi", _lib.E_UNSUPPORTED)
    bidx = [t.contiguous() for t in torch.broadcast_tensors(*idxs)]
    bshape = tuple(bidx[0].shape)
    ic = inp.contiguous()
    outer = math.prod(ic.shape[:first])
    sizes = ic.shape[first:first + k]
    inner = math.prod(ic.shape[first + k:])
    out = torch.empty((*ic.shape[:first], *bshape, *ic.shape[first + k:]), dtype=inp.dtype, device=inp.device)
    if out.numel() == 0:
        return out
    flag = torch.zeros(1, dtype=torch.int32, device=inp.device) if (check or (check is None and CHECK_INDEX)) else None
    lib = _lib_handle()
    _lib.check("kuiops_index_multi", lib.kuiops_index_multi(
        outer, k, _lib.i64_array(sizes), inner, bidx[0].numel(), (ctypes.c_void_p * k)(*[t.data_ptr() for t in bidx]),
        ic.element_size(), ic.data_ptr(), out.data_ptr(), _ptr(flag), _stream(inp.device)))
    _raise_if_flagged(flag, "index")
    return out


def scatter(inp: torch.Tensor, dim: int, idx: torch.Tensor, src: torch.Tensor, check: bool | None = None):
    """torch.scatter(inp, dim, idx, src) (aten.scatter.src): a copy of inp with
    out[x with dim <- idx[x]] = src[x] for every x of idx's shape (src sliced
    to idx's shape); int64 indices; bit-exact."""
    if idx.dtype != torch.int64 or idx.dim() != inp.dim() or src.dim() != inp.dim() or src.dtype != inp.dtype \
            or inp.dim() < 1 or inp.dim() > 8:
        raise _lib.Unsupported("scatter", _lib.E_UNSUPPORTED)
    dim = dim % inp.dim()
    for d in range(inp.dim()):
        if idx.shape[d] > src.shape[d] or (d != dim and idx.shape[d] > inp.shape[d]):
            raise _lib.KuiopsError("scatter", _lib.E_INVALID)
    out = inp.contiguous().clone()
    if idx.numel() == 0:
        return out
    xc = idx.contiguous()
    sc = src[tuple(slice(0, n) for n in idx.shape)].contiguous()
    flag = torch.zeros(1, dtype=torch.int32, device=inp.device) if (check or (check is None and CHECK_INDEX)) else None
    lib = _lib_handle()
    _lib.check("kuiops_scatter", lib.kuiops_scatter(
        inp.dim(), _lib.i64_array(out.shape), _lib.i64_array(xc.shape), dim, out.element_size(),
        sc.data_ptr(), xc.data_ptr(), out.data_ptr(), _ptr(flag), _stream(inp.device)))
    _raise_if_flagged(flag, "scatter")
    return out


def sort(x: torch.Tensor, dim: int = -1, descending: bool = False):
    """(values, int64 indices) of a stable sort along ``dim`` (aten.sort with
    stable=True): NaN counts as the largest value, -0 equals +0, equal values
    keep index order."""
    if x.dim() == 0:
        raise _lib.Unsupported("sort", _lib.E_UNSUPPORTED)
    dim = dim % x.dim()
    moved = dim != x.dim() - 1
    xc = (x.movedim(dim, -1) if moved else x).contiguous()
    n = xc.shape[-1]
    m = xc.numel() // n if n else 0
    vals = torch.empty_like(xc)
    inds = torch.empty(xc.shape, dtype=torch.int64, device=x.device)
    if vals.numel():
        lib = _lib_handle()
        ws_bytes = lib.kuiops_query_workspace(_lib.OP_SORT, m, n, 0)
        ws = workspace(x.device, ws_bytes) if ws_bytes else None
        _lib.check("kuiops_sort_lastdim", lib.kuiops_sort_lastdim(
            m, n, _dt(x.dtype), xc.data_ptr(), vals.data_ptr(), inds.data_ptr(), 1 if descending else 0,
            _ptr(ws), ws.numel() if ws is not None else 0, _stream(x.device)))
    if moved:
        vals, inds = vals.movedim(-1, dim), inds.movedim(-1, dim)
    return vals, inds


def cumsum(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Inclusive prefix sum along ``dim`` (aten.cumsum) for fp32 / fp64 / int64."""
    if x.dim() == 0:
        raise _lib.Unsupported("cumsum", _lib.E_UNSUPPORTED)
    dim = dim % x.dim()
    moved = dim != x.dim() - 1
    xc = (x.movedim(dim, -1) if moved else x).contiguous()
    n = xc.shape[-1]
    m = xc.numel() // n if n else 0
    out = torch.empty_like(xc)
    if out.numel():
        lib = _lib_handle()
        _lib.check("kuiops_cumsum_lastdim", lib.kuiops_cumsum_lastdim(
            m, n, _dt(x.dtype), xc.data_ptr(), out.data_ptr(), _stream(x.device)))
    return out.movedim(-1, dim) if moved else out


def multinomial(probs: torch.Tensor, num_samples: int, replacement: bool = False, generator=None,
                uniforms: torch.Tensor | None = None, check: bool = True) -> torch.Tensor:
    """Draws from the rows of ``probs`` ([n] or [m, n] non-negative weights) by
    inverse CDF: sample = first index whose running weight sum exceeds u *
    total, u from ``uniforms`` ([m, num_samples] fp32 on the device) or
    torch.rand(generator).  With replacement, or one sample per row (then
    replacement does not matter), as the sampling tail uses it."""
    if probs.dim() not in (1, 2) or num_samples < 1:
        raise _lib.Unsupported("multinomial", _lib.E_UNSUPPORTED)
    if not replacement and num_samples > 1:
        raise _lib.Unsupported("multinomial", _lib.E_UNSUPPORTED)
    p2 = probs.reshape(-1, probs.shape[-1]).contiguous()
    m, n = p2.shape
    if uniforms is None:
        uniforms = torch.rand((m, num_samples), generator=generator, device=probs.device, dtype=torch.float32)
    u = uniforms.reshape(m, num_samples).to(torch.float32).contiguous()
    out = torch.empty((m, num_samples), dtype=torch.int64, device=probs.device)
    flag = torch.zeros(1, dtype=torch.int32, device=probs.device) if check else None
    lib = _lib_handle()
    _lib.check("kuiops_multinomial", lib.kuiops_multinomial(
        m, n, _dt(probs.dtype), p2.data_ptr(), num_samples, u.data_ptr(), out.data_ptr(), _ptr(flag),
        _stream(probs.device)))
    if flag is not None and int(flag.item()) != 0:
        raise RuntimeError("multinomial: probability rows must be finite, non-negative and sum above 0")
    return out.view(num_samples) if probs.dim() == 1 else out


def top_p_filter(scores: torch.Tensor, top_p: float, filter_value: float = -float("inf"),
                 min_tokens_to_keep: int = 1) -> torch.Tensor:
    """transformers' TopPLogitsWarper on [m, vocab] scores: ascending sort,
    softmax, cumsum, drop the sorted prefix whose cumulative probability is
    <= 1 - top_p (keeping the last min_tokens_to_keep), scatter the mask back
    and fill the dropped scores with filter_value."""
    sorted_logits, sorted_idx = sort(scores, -1, descending=False)
    cum = cumsum(softmax(sorted_logits), -1)
    if scores.dtype == torch.float32 and scores.dim() == 2 and cum.dtype == torch.float32:
        # le / setitem / scatter / masked_fill as one scatter of the sorted values
        m, n = scores.shape
        out = torch.empty((m, n), dtype=scores.dtype, device=scores.device)
        _lib.check("kuiops_top_p_mask", _lib_handle().kuiops_top_p_mask(
            m, n, sorted_logits.contiguous().data_ptr(), sorted_idx.contiguous().data_ptr(),
            cum.contiguous().data_ptr(), float(top_p), int(min_tokens_to_keep), float(filter_value),
            out.data_ptr(), _stream(scores.device)))
        return out
    remove = cum <= (1 - top_p)
    remove[..., -min_tokens_to_keep:] = False
    mask = scatter(remove, 1, sorted_idx, remove)
    return scores.masked_fill(mask, filter_value)


def sample_top_p(scores: torch.Tensor, top_p: float, temperature: float = 1.0, generator=None,
                 uniforms: torch.Tensor | None = None, check: bool = False) -> torch.Tensor:
    """One sampled token per row of [m, vocab] fp32 scores: temperature, top-p
    filter, softmax, multinomial (the HF sampling tail) -> int64 [m].  With
    check=False nothing synchronises with the host (the call can be recorded
    in a HIP graph); the softmax rows it samples from are always valid."""
    if temperature != 1.0:
        scores = scores / temperature
    probs = softmax(top_p_filter(scores, top_p))
    return multinomial(probs, 1, generator=generator, uniforms=uniforms, check=check).view(-1)


# ------------------------------------------------------ decoder-layer glue

def _rows(x: torch.Tensor) -> torch.Tensor:
    """2-D [m, n] view with unit column stride (copy otherwise)."""
    x2 = x.reshape(-1, x.shape[-1])
    return x2 if x2.stride(-1) == 1 else x2.contiguous()


def rmsnorm(x, weight, eps, residual=None, res_out=None, out=None):
    """weight * round(h * rsqrt(mean(h^2, -1) + eps)) with h = x (+ residual).

    With ``res_out`` given, h (the updated residual stream) is stored there;
    it may be ``residual`` itself.  Shapes: x, residual, res_out, out are
    [..., n]; weight is [n]."""
    n = x.shape[-1]
    x2 = _rows(x)
    m = x2.shape[0]
    r2 = None if residual is None else residual.reshape(-1, n)
    ro2 = None if res_out is None else res_out.reshape(-1, n)
    for t in (r2, ro2):
        if t is not None and (t.shape[0] != m or t.stride(-1) != 1 or t.dtype != x.dtype):
            raise _lib.KuiopsError("rmsnorm", _lib.E_INVALID)
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    o2 = out.view(-1, n)
    if weight.shape != (n,) or weight.dtype != x.dtype or not weight.is_contiguous():
        raise _lib.KuiopsError("rmsnorm", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_rmsnorm", lib.kuiops_rmsnorm(
        m, n, _dt(x.dtype), x2.data_ptr(), x2.stride(0),
        _ptr(r2), 0 if r2 is None else r2.stride(0), _ptr(ro2), 0 if ro2 is None else ro2.stride(0),
        weight.data_ptr(), float(eps), o2.data_ptr(), o2.stride(0), _stream(x.device)))
    return out


def silu_mul(gate_up, out=None):
    """silu(gate_up[..., :n]) * gate_up[..., n:] for gate_up [..., 2n]."""
    g2 = _rows(gate_up)
    m, n2 = g2.shape
    n = n2 // 2
    if out is None:
        out = torch.empty((*gate_up.shape[:-1], n), dtype=gate_up.dtype, device=gate_up.device)
    o2 = out.view(-1, n)
    lib = _lib_handle()
    _lib.check("kuiops_silu_mul", lib.kuiops_silu_mul(
        m, n, _dt(gate_up.dtype), g2.data_ptr(), g2.stride(0), o2.data_ptr(), o2.stride(0),
        _stream(gate_up.device)))
    return out


def rope_kv_append(qkv, hq, hkv, hd, inv_freq, pos0, q_out, k_cache, v_cache):
    """Rotate q / k of the new tokens and append k / v to the cache.

    qkv [n, t, (hq + 2 hkv) hd] (rows with a unit last stride); pos0 int32 [n]
    on the device (first position of the t tokens) or None for 0; q_out
    [n, hq, t, hd]; k_cache / v_cache [n, hkv, capacity, hd]."""
    n, t, w = qkv.shape
    if w != (hq + 2 * hkv) * hd or qkv.stride(-1) != 1 or inv_freq.dtype != torch.float32:
        raise _lib.KuiopsError("rope_kv_append", _lib.E_INVALID)
    if tuple(q_out.shape) != (n, hq, t, hd) or q_out.stride(-1) != 1:
        raise _lib.KuiopsError("rope_kv_append", _lib.E_INVALID)
    for c in (k_cache, v_cache):
        if c.dim() != 4 or tuple(c.shape[:2]) != (n, hkv) or c.shape[3] != hd or c.stride(-1) != 1:
            raise _lib.KuiopsError("rope_kv_append", _lib.E_INVALID)
    if pos0 is not None and (pos0.dtype != torch.int32 or pos0.numel() != n):
        raise _lib.KuiopsError("rope_kv_append", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_rope_kv_append", lib.kuiops_rope_kv_append(
        n, t, hq, hkv, hd, _dt(qkv.dtype), qkv.data_ptr(), qkv.stride(1), qkv.stride(0),
        inv_freq.data_ptr(), _ptr(pos0), q_out.data_ptr(), _lib.strides3(*q_out.stride()[:3]),
        k_cache.data_ptr(), _lib.strides3(*k_cache.stride()[:3]),
        v_cache.data_ptr(), _lib.strides3(*v_cache.stride()[:3]), k_cache.shape[2], _stream(qkv.device)))


_X_KIND = {"plain": _lib.X_PLAIN, "rmsnorm": _lib.X_RMSNORM, "swiglu": _lib.X_SWIGLU}


def decode_linear(x, W, x_kind="plain", in_add=None, norm_w=None, eps=1e-5, h_out=None, bias=None, out=None):
    """Batch-1 decode projection out[N] = W @ f(x) with the input stage fused
    in (one launch; see kuiops_decode_linear).  W is an nn.Linear weight
    [N, K] (K contiguous).

    * ``plain``:   f(x) = x[K]
    * ``rmsnorm``: h = round(x + in_add), f = RMSNorm(h) * norm_w; h is written
                   to ``h_out`` when given
    * ``swiglu``:  x = [gate | up] (2K), f = silu(gate) * up
    """
    N, K = W.shape
    xf = x.reshape(-1)
    if x.dtype != W.dtype or W.stride(1) != 1 or not xf.is_contiguous():
        raise _lib.KuiopsError("decode_linear", _lib.E_INVALID)
    if xf.numel() != (2 * K if x_kind == "swiglu" else K):
        raise _lib.KuiopsError("decode_linear", _lib.E_INVALID)
    for t in (in_add, norm_w, h_out, bias):
        if t is not None and (t.numel() != (N if t is bias else K) or not t.is_contiguous() or t.dtype != x.dtype):
            raise _lib.KuiopsError("decode_linear", _lib.E_INVALID)
    if out is None:
        out = torch.empty(N, dtype=x.dtype, device=x.device)
    elif out.numel() != N or not out.is_contiguous() or out.dtype != x.dtype:
        raise _lib.KuiopsError("decode_linear", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_decode_linear", lib.kuiops_decode_linear(
        N, K, _dt(x.dtype), _X_KIND[x_kind], xf.data_ptr(), _ptr(in_add), _ptr(norm_w), float(eps),
        _ptr(h_out), W.data_ptr(), W.stride(0), _ptr(bias), out.data_ptr(), _stream(x.device)))
    return out


def decode_gate_up(x, W, x_kind="rmsnorm", in_add=None, norm_w=None, eps=1e-5, h_out=None, out=None):
    """Batch-1 gate/up projection with SwiGLU in the epilogue (one launch;
    see kuiops_decode_gate_up): W = [gate; up] as one nn.Linear weight
    [2 ffn, K]; returns round(silu(gate(x))) * up(x) rounded, [ffn]."""
    N2, K = W.shape
    ffn = N2 // 2
    xf = x.reshape(-1)
    if N2 % 2 or x.dtype != W.dtype or W.stride(1) != 1 or not xf.is_contiguous() or xf.numel() != K:
        raise _lib.KuiopsError("decode_gate_up", _lib.E_INVALID)
    for t in (in_add, norm_w, h_out):
        if t is not None and (t.numel() != K or not t.is_contiguous() or t.dtype != x.dtype):
            raise _lib.KuiopsError("decode_gate_up", _lib.E_INVALID)
    if out is None:
        out = torch.empty(ffn, dtype=x.dtype, device=x.device)
    elif out.numel() != ffn or not out.is_contiguous() or out.dtype != x.dtype:
        raise _lib.KuiopsError("decode_gate_up", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_decode_gate_up", lib.kuiops_decode_gate_up(
        ffn, K, _dt(x.dtype), _X_KIND[x_kind], xf.data_ptr(), _ptr(in_add), _ptr(norm_w), float(eps),
        _ptr(h_out), W.data_ptr(), W.stride(0), out.data_ptr(), _stream(x.device)))
    return out


def decode_qkv_rope(x, W, hq, hkv, hd, inv_freq, pos, q_out, k_cache, v_cache, x_kind="rmsnorm", row=None,
                    in_add=None, norm_w=None, eps=1e-5, h_out=None):
    """Batch-1 qkv projection + rotary + KV-cache append (one launch; see
    kuiops_decode_qkv_rope).  W is the fused [q; k; v] nn.Linear weight
    [(hq + 2 hkv) hd, K]; x is [K], or a [rows, K] table read at device row
    ``row`` (int64 [1], an embedding lookup); pos is int32 [1] on the device;
    q_out [hq * hd]; k_cache / v_cache [hkv, capacity, hd]."""
    N, K = W.shape
    if N != (hq + 2 * hkv) * hd or x.dtype != W.dtype or W.stride(1) != 1 or inv_freq.dtype != torch.float32:
        raise _lib.KuiopsError("decode_qkv_rope", _lib.E_INVALID)
    if row is None:
        xf, ld_in, rows = x.reshape(-1), 0, 1
        if not xf.is_contiguous() or xf.numel() != K:
            raise _lib.KuiopsError("decode_qkv_rope", _lib.E_INVALID)
    else:
        if x.dim() != 2 or x.shape[1] != K or x.stride(1) != 1 or row.dtype != torch.int64 or row.numel() < 1:
            raise _lib.KuiopsError("decode_qkv_rope", _lib.E_INVALID)
        xf, ld_in, rows = x, x.stride(0), x.shape[0]
    if pos.dtype != torch.int32 or q_out.numel() != hq * hd or not q_out.is_contiguous():
        raise _lib.KuiopsError("decode_qkv_rope", _lib.E_INVALID)
    for c in (k_cache, v_cache):
        if c.dim() != 3 or c.shape[0] != hkv or c.shape[2] != hd or c.stride(-1) != 1 or c.dtype != x.dtype:
            raise _lib.KuiopsError("decode_qkv_rope", _lib.E_INVALID)
    for t in (in_add, norm_w, h_out):
        if t is not None and (t.numel() != K or not t.is_contiguous() or t.dtype != x.dtype):
            raise _lib.KuiopsError("decode_qkv_rope", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_decode_qkv_rope", lib.kuiops_decode_qkv_rope(
        hq, hkv, hd, K, _dt(x.dtype), _X_KIND[x_kind], xf.data_ptr(), _ptr(row), ld_in, rows, _ptr(in_add),
        _ptr(norm_w), float(eps), _ptr(h_out), W.data_ptr(), W.stride(0), inv_freq.data_ptr(), pos.data_ptr(),
        q_out.data_ptr(), k_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), v_cache.data_ptr(),
        v_cache.stride(0), v_cache.stride(1), k_cache.shape[1], _stream(x.device)))
    return q_out


def decode_step_sync_bytes(n_layers: int) -> int:
    """Bytes of the counter / step-counter buffer kuiops_decode_step needs."""
    return int(_lib_handle().kuiops_decode_step_sync_bytes(n_layers))


def decode_step_scratch_bytes(n_layers: int, n_steps: int, d: int, ffn: int, hq: int, hkv: int, hd: int) -> int:
    """Bytes of the epoch-tagged vector buffer kuiops_decode_step needs for
    up to n_steps steps per call."""
    return int(_lib_handle().kuiops_decode_step_scratch_bytes(n_layers, n_steps, d, ffn, hq, hkv, hd))


def decode_step(layer_table, n_layers, d, ffn, hq, hkv, hd, vocab, eps, k_cache, v_cache, embed, final_norm,
                lm_head, inv_freq, tok, pos, kv_len, history, prob, logits, scratch, sync, n_steps=1):
    """``n_steps`` whole batch-1 greedy decode steps in one persistent launch
    (see kuiops_decode_step).  ``layer_table`` is a device int64
    [n_layers, 8] tensor of per-layer pointers (wqkv, wo, wgu, wd, ln1, ln2,
    k cache, v cache); k_cache / v_cache give the cache strides ([hkv, cap,
    hd] views of layer 0); ``logits`` [vocab] receives the last step's LM
    head output; ``scratch`` / ``sync`` are zeroed uint8 buffers of
    decode_step_scratch_bytes (for at least n_steps) /
    decode_step_sync_bytes, kept across calls."""
    if layer_table.dtype != torch.int64 or tuple(layer_table.shape) != (n_layers, 8) or not layer_table.is_contiguous():
        raise _lib.KuiopsError("decode_step", _lib.E_INVALID)
    if tok.dtype != torch.int64 or pos.dtype != torch.int32 or kv_len.dtype != torch.int32:
        raise _lib.KuiopsError("decode_step", _lib.E_INVALID)
    if history is not None and (history.dtype != torch.int64 or not history.is_contiguous()):
        raise _lib.KuiopsError("decode_step", _lib.E_INVALID)
    if prob is not None and prob.dtype != torch.float32:
        raise _lib.KuiopsError("decode_step", _lib.E_INVALID)
    for t in (logits, embed, final_norm, lm_head):
        if not t.is_contiguous() or t.dtype != embed.dtype:
            raise _lib.KuiopsError("decode_step", _lib.E_INVALID)
    for c in (k_cache, v_cache):
        if c.dim() != 3 or c.shape[0] != hkv or c.shape[2] != hd or c.stride(-1) != 1 or c.dtype != embed.dtype:
            raise _lib.KuiopsError("decode_step", _lib.E_INVALID)
    lib = _lib_handle()
    _lib.check("kuiops_decode_step", lib.kuiops_decode_step(
        n_layers, d, ffn, hq, hkv, hd, vocab, k_cache.shape[1], _dt(embed.dtype), float(eps), layer_table.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), v_cache.stride(0), v_cache.stride(1), embed.data_ptr(),
        final_norm.data_ptr(), lm_head.data_ptr(), inv_freq.data_ptr(), tok.data_ptr(), pos.data_ptr(),
        kv_len.data_ptr(), _ptr(history), history.numel() if history is not None else 0, _ptr(prob),
        logits.data_ptr(), int(n_steps), scratch.data_ptr(), scratch.numel(), sync.data_ptr(), sync.numel(),
        _stream(embed.device)))
    return logits


def decode_step_supported(n_layers, d, ffn, hq, hkv, hd, vocab, cache_cap, dtype) -> bool:
    """Whether kuiops_decode_step serves this shape on the current device:
    the host shape gate (including a cache no longer than the one-pass
    attention covers) and an occupancy query that one step work-group fits
    a CU.  False means the caller takes the per-op step."""
    return _lib_handle().kuiops_decode_step_supported(n_layers, d, ffn, hq, hkv, hd, vocab, cache_cap,
                                                      _dt(dtype)) == _lib.OK


def decode_step_error(sync, n_layers) -> bool:
    """True when a previous decode_step on ``sync`` gave up a bounded wait
    (the flag is cleared); synchronises the stream."""
    rc = _lib_handle().kuiops_decode_step_error(sync.data_ptr(), n_layers, _stream(sync.device))
    if rc < 0:
        _lib.check("kuiops_decode_step_error", rc)
    return rc == 1


# ----------------------------------------------- elementwise / mean / cat

def _compute_code(dtype) -> int:
    """Arithmetic type of an elementwise op whose operands promote to
    ``dtype``: fp64 stays fp64, other floats compute in fp32 (aten's opmath
    type), integers and bool in int64."""
    if dtype == torch.float64:
        return _lib.F64
    if dtype.is_floating_point:
        return _lib.F32
    if dtype.is_complex:
        raise _lib.Unsupported("elementwise", _lib.E_UNSUPPORTED)
    return _lib.I64


def _collapse(shape, stride_sets):
    """Drop size-1 dims and merge neighbours that every operand walks as one
    (stride[d] == stride[d+1] * shape[d+1]); returns (shape, [strides])."""
    dims = [d for d in range(len(shape)) if shape[d] != 1]
    out_shape = [shape[d] for d in dims]
    outs = [[st[d] for d in dims] for st in stride_sets]
    i = len(out_shape) - 2
    while i >= 0:
        if all(st[i] == st[i + 1] * out_shape[i + 1] for st in outs):
            out_shape[i] *= out_shape[i + 1]
            del out_shape[i + 1]
            for st in outs:
                st[i] = st[i + 1]
                del st[i + 1]
        i -= 1
    return out_shape, outs


def elementwise(op: int, inputs, out_dtype, compute_dtype=None, s0: float = 1.0, s1: float = 0.0):
    """out = op(inputs...) with broadcasting; ``op`` is a KUIOPS_EW_* code.
    Binary ops given one tensor take the python scalar ``s1`` as their second
    operand; ``s0`` is add / sub's alpha or pow's exponent.  ``compute_dtype``
    (default: promoted from the inputs) selects fp32 / fp64 / int64
    arithmetic.  Returns a new contiguous tensor of ``out_dtype``."""
    if not inputs:
        raise _lib.KuiopsError("kuiops_elementwise", _lib.E_INVALID)
    dev = inputs[0].device
    shape = list(torch.broadcast_shapes(*[tuple(t.shape) for t in inputs]))
    out = torch.empty(shape, dtype=out_dtype, device=dev)
    if out.numel() == 0:
        return out
    if compute_dtype is None:
        compute_dtype = inputs[0].dtype
        for t in inputs[1:]:
            compute_dtype = torch.promote_types(compute_dtype, t.dtype)
    strides = [list(t.expand(shape).stride()) for t in inputs]
    cshape, cstrides = _collapse(shape, strides)
    if len(cshape) > 8:
        raise _lib.Unsupported("kuiops_elementwise", _lib.E_UNSUPPORTED)
    n = len(inputs)
    rank = len(cshape)
    flat = [s for st in cstrides for s in st]
    lib = _lib_handle()
    _lib.check("kuiops_elementwise", lib.kuiops_elementwise(
        int(op), rank, _lib.i64_array(cshape), n, (ctypes.c_int * n)(*[_dt(t.dtype) for t in inputs]),
        (ctypes.c_void_p * n)(*[t.data_ptr() for t in inputs]), _lib.i64_array(flat), float(s0), float(s1),
        _compute_code(compute_dtype), _dt(out_dtype), out.data_ptr(), _stream(dev)))
    return out


def mean_lastdim(x: torch.Tensor, keepdim: bool = False) -> torch.Tensor:
    """x.mean(-1, keepdim) with fp32 accumulation (fp64 for fp64), scaled as
    aten scales its sums (by output numel / input numel)."""
    if x.dim() == 0 or x.dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        raise _lib.Unsupported("kuiops_mean_lastdim", _lib.E_UNSUPPORTED)
    n = x.shape[-1]
    rows = x.reshape(-1, n) if x.dim() != 2 else x
    if n > 0 and (rows.stride(-1) != 1 or (rows.shape[0] > 1 and rows.stride(0) < n)):
        rows = rows.contiguous()
    m = rows.shape[0]
    out_shape = (*x.shape[:-1], 1) if keepdim else tuple(x.shape[:-1])
    out = torch.empty(out_shape, dtype=x.dtype, device=x.device)
    if m == 0:
        return out
    lib = _lib_handle()
    _lib.check("kuiops_mean_lastdim", lib.kuiops_mean_lastdim(
        m, n, _dt(x.dtype), rows.data_ptr(), rows.stride(0) if m > 1 else n, out.data_ptr(), _stream(x.device)))
    return out


def _outer_stride(t: torch.Tensor, dim: int):
    """(outer rows, stride between rows) when t's dims from ``dim`` on form
    one contiguous run per row and its leading dims walk rows at one stride;
    None otherwise."""
    inner = 1
    for d in range(t.dim() - 1, dim - 1, -1):
        if t.shape[d] != 1 and t.stride(d) != inner:
            return None
        inner *= t.shape[d]
    lead = [(t.shape[d], t.stride(d)) for d in range(dim) if t.shape[d] != 1]
    if not lead:
        return 1, max(inner, 1)
    for (s0, st0), (s1, st1) in zip(lead, lead[1:]):
        if st0 != st1 * s1:
            return None
    rows = 1
    for s, _ in lead:
        rows *= s
    return rows, lead[-1][1]


def cat(tensors, dim: int = 0) -> torch.Tensor:
    """torch.cat of same-dtype, same-rank tensors along ``dim``.  Inputs whose
    rows are not single strided runs are made contiguous first."""
    if not tensors:
        raise _lib.KuiopsError("kuiops_cat", _lib.E_INVALID)
    ref = tensors[0]
    rank = ref.dim()
    if rank == 0 or any(t.dim() != rank or t.dtype != ref.dtype or t.device != ref.device for t in tensors):
        raise _lib.Unsupported("kuiops_cat", _lib.E_UNSUPPORTED)
    dim = dim % rank
    for t in tensors:
        if any(t.shape[d] != ref.shape[d] for d in range(rank) if d != dim):
            raise _lib.KuiopsError("kuiops_cat", _lib.E_INVALID)
    if len(tensors) > 32:
        raise _lib.Unsupported("kuiops_cat", _lib.E_UNSUPPORTED)
    shape = list(ref.shape)
    shape[dim] = sum(int(t.shape[dim]) for t in tensors)
    out = torch.empty(shape, dtype=ref.dtype, device=ref.device)
    if out.numel() == 0:
        return out
    outer = 1
    for d in range(dim):
        outer *= shape[d]
    inner = 1
    for d in range(dim + 1, rank):
        inner *= shape[d]
    ptrs, widths, strides, keep = [], [], [], []
    for t in tensors:
        w = int(t.shape[dim]) * inner
        if w == 0:
            continue
        rs = _outer_stride(t, dim)
        if rs is None:
            t = t.contiguous()
            rs = _outer_stride(t, dim)
        keep.append(t)
        ptrs.append(t.data_ptr())
        widths.append(w)
        strides.append(rs[1])
    n = len(ptrs)
    lib = _lib_handle()
    _lib.check("kuiops_cat", lib.kuiops_cat(
        n, (ctypes.c_void_p * max(n, 1))(*ptrs), _lib.i64_array(widths), _lib.i64_array(strides), outer,
        ref.element_size(), out.data_ptr(), _stream(ref.device)))
    return out


_OUT_KIND = {"plain": 0, "swiglu": 1, "rope": 2}


def decode_rows_batched(x, W, x_kind="plain", out_kind="plain", in_add=None, norm_w=None, eps=1e-5,
                        h_out=None, out=None, row=None, pair_off=0, hq=0, hkv=0, hd=0, inv_freq=None,
                        pos=None, k_cache=None, v_cache=None, split=True):
    """Batched (M <= 16 rows) decode projection with the fused input stage and
    epilogue of ``decode_linear`` / ``decode_gate_up`` / ``decode_qkv_rope``
    (one launch; see kuiops_decode_rows_batched).  W is an nn.Linear weight
    [N, K] (K contiguous); x is [M, K] ([M, 2K] for ``swiglu``), or a
    [rows, K] table read at the device rows ``row`` (int64 [M]).
    ``out_kind``: ``plain`` -> out [M, N]; ``swiglu`` (rows p, p + pair_off)
    -> out [M, pair_off]; ``rope`` (fused [q; k; v] heads) -> q into out
    [M, hq * hd], k / v into the caches [M, hkv, capacity, hd] at pos[m].
    ``split``: give the unstaged (17..64-row) form its workspace, so it
    splits K over work-groups (False: one pass, no workspace)."""
    N, K = W.shape
    if x.dtype != W.dtype or W.stride(1) != 1 or x.stride(-1) != 1 or x.dim() != 2:
        raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
    if row is None:
        M = x.shape[0]
        rows = M
        if x.shape[1] != (2 * K if x_kind == "swiglu" else K):
            raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
    else:
        if row.dtype != torch.int64 or row.dim() != 1 or not row.is_contiguous() or x.shape[1] != K:
            raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
        M, rows = row.numel(), x.shape[0]
    width = {"plain": N, "swiglu": N // 2, "rope": hq * hd}[out_kind]
    if out is None:
        out = torch.empty((M, width), dtype=x.dtype, device=x.device)
    elif out.dim() != 2 or tuple(out.shape) != (M, width) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
    for t in (in_add, h_out):
        if t is not None and (t.dim() != 2 or t.shape != (M, K) or t.stride(1) != 1 or t.dtype != x.dtype):
            raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
    sk = sv = None
    if out_kind == "rope":
        for c in (k_cache, v_cache):
            if c is None or c.dim() != 4 or c.shape[0] != M or c.shape[1] != hkv or c.shape[3] != hd \
                    or c.stride(-1) != 1 or c.dtype != x.dtype:
                raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
        if pos is None or pos.dtype != torch.int32 or pos.numel() != M or not pos.is_contiguous():
            raise _lib.KuiopsError("decode_rows_batched", _lib.E_INVALID)
        sk, sv = _lib.strides3(*k_cache.stride()[:3]), _lib.strides3(*v_cache.stride()[:3])
        pair_off = hd // 2
    elif out_kind == "swiglu":
        pair_off = N // 2
    lib = _lib_handle()
    ws_bytes = lib.kuiops_query_workspace(_lib.OP_DECODE_ROWS_BATCHED, M, N, K) if split else 0
    ws = workspace(x.device, ws_bytes, "decode_rows") if ws_bytes else None
    _lib.check("kuiops_decode_rows_batched", lib.kuiops_decode_rows_batched(
        M, N, K, _dt(x.dtype), _X_KIND[x_kind], _OUT_KIND[out_kind], x.data_ptr(), x.stride(0), _ptr(row), rows,
        _ptr(in_add), in_add.stride(0) if in_add is not None else 0, _ptr(norm_w), float(eps), _ptr(h_out),
        h_out.stride(0) if h_out is not None else 0, W.data_ptr(), W.stride(0), out.data_ptr(), out.stride(0),
        int(pair_off), int(hq), int(hkv), int(hd), _ptr(inv_freq), _ptr(pos),
        _ptr(k_cache), sk, _ptr(v_cache), sv, k_cache.shape[2] if k_cache is not None else 0,
        _ptr(ws), ws.numel() if ws is not None else 0, _stream(x.device)))
    return out
