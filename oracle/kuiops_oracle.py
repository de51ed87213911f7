"""CPU oracle for the kuiops hot path -- TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of what the reference computes for each hot-path
op.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU
baseline may import it, and only as the checker: nothing in ``kuillm_amd``
imports or calls this module, and the product path never routes through it.

The reference (panther03/kuiLLM) dispatches aten ops to un-vendored,
unpinned Kuiper kernels when its ``supported()`` gates accept them and to
stock aten otherwise (kuipy/__init__.py:53-75, 161-164); its own tests check
every op against stock torch (tests/test_jit_ops.py:34-43).  The oracle
therefore restates aten semantics, op by op, citing the reference's family:

  mm / addmm / bmm   kuipy/kuiops.py:403-564, kuiops/bmm/Kuiops.Bmm.fst:10-23
  _softmax           kuipy/kuiops.py:578-610
  SDPA (+ LSE)       kuipy/kuiops.py:627-681, kuiops/sdpa/Kuiops.Sdpa.fst.1:9-27
  gather             kuipy/kuiops.py:717-754, kuiops/gather/Kuiops.Gather.fst:482-486
  topk / index       no reference kernel (kuiops/topk/.gitkeep,
                     kuiops/index/.gitkeep): aten.topk / aten.index.Tensor
  scatter            kuipy/kuiops.py:757-807 (aten.scatter.src)
  elementwise /      ElementwiseImpl / MeanImpl / CatImpl, kuipy/kuiops.py:150-320,
  mean / cat         810-921 (aten semantics: opmath compute type, broadcasting)
  sort / cumsum /    no reference kernel (KERNELS.md rows aten.sort.default,
  multinomial        aten.cumsum.default, aten.multinomial.default): aten
                     semantics; multinomial as the inverse CDF of given
                     uniforms; top_p_filter restates transformers'
                     TopPLogitsWarper (the sampling tail these serve)
  verify metric      kuipy/__init__.py:193-225
  decoder glue       RMSNorm / SwiGLU / rotary + KV cache and a whole
                     Llama-style decoder: the stock
                     transformers modules the reference runs under
                     KuiperMode (infer.py:14-31), whose elementwise, mean
                     and cat ops it sends to ElementwiseImpl / MeanImpl /
                     CatImpl (kuipy/kuiops.py:150-320, 810-921)

bf16 values travel as uint16 bit patterns (numpy has no bfloat16).

How each function is pinned (tests/test_oracle.py):
  * against golden vectors written by stock aten on CPU (tests/golden/);
  * against closed forms and invariants chosen so that a dropped term, a
    wrong sign / index or a transposed operand fails (identity and one-hot
    operands, integer-valued products that are exact in fp32, softmax of a
    constant row, attention with constant V, single-key attention, causal
    row 0, brute-force sorting for topk and sort, explicit loops for
    gather / index / scatter, integer prefix sums, a CDF table lookup for
    multinomial);
  * the decoder pieces against the transformers Llama modules run on the
    CPU (RMSNorm, rotary embedding, MLP, the whole causal LM), plus closed
    forms (constant-row RMSNorm, position-0 rotation = identity, rotation
    preserves pair norms).
No function here is "parity unpinned".
"""
from __future__ import annotations

import math

import numpy as np

# ------------------------------------------------------------------- bf16


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round fp32 to bf16 (round to nearest even, NaN kept quiet) -> uint16."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """fp32 values rounded to the nearest bf16, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_dtype(x, dtype: str) -> np.ndarray:
    """Round to the storage dtype ('bf16', 'f16', 'f32', 'f64'), as fp32/fp64."""
    if dtype == "bf16":
        return round_bf16(np.asarray(x, dtype=np.float32))
    if dtype == "f16":
        return np.asarray(x, dtype=np.float16).astype(np.float32)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    return np.asarray(x, dtype=np.float64)


# ----------------------------------------------- elementwise / mean / cat
# ElementwiseImpl / MeanImpl / CatImpl (kuipy/kuiops.py:150-320, 810-921,
# registered for the aten overloads of kuipy/registry.py:33-57).  Restated
# from aten: operands broadcast, are converted to the compute type (fp32 for
# 16/32-bit floats -- aten's "opmath" type -- fp64 for fp64, int64 for
# integers and bool), scalars enter unrounded in that type, and the result is
# rounded once to the output dtype by the caller (``round_dtype``).

_UNARY_F = {
    "neg": lambda a: -a,
    "silu": lambda a: a / (a.dtype.type(1) + np.exp(-a)),
    "rsqrt": lambda a: a.dtype.type(1) / np.sqrt(a),
    "cos": np.cos,
    "sin": np.sin,
    "exp": np.exp,
    "sqrt": np.sqrt,
}


def _pow_scalar(a, e, store=None):
    # aten's special cases of pow(Tensor, Scalar); for 16-bit storage types
    # the integer powers multiply in the storage type, so the square is
    # rounded to it before the third factor / the reciprocal
    one = a.dtype.type(1)
    sq = a * a
    if store in ("bf16", "f16"):
        sq = round_dtype(sq, store).astype(a.dtype)
    if e == 2:
        return a * a
    if e == 3:
        return sq * a
    if e == 1:
        return a.copy()
    if e == 0.5:
        return np.sqrt(a)
    if e == -0.5:
        return one / np.sqrt(a)
    if e == -1:
        return one / a
    if e == -2:
        return one / sq
    return np.power(a, a.dtype.type(e))


def elementwise(op: str, *operands, alpha=1.0, exponent=None, compute="f32", store=None) -> np.ndarray:
    """op over broadcast operands in the compute type ('f32', 'f64' or
    'i64'); python scalars are operands too.  ``store`` is the output
    storage dtype where it changes an intermediate rounding (pow).  Ops: neg silu rsqrt cos sin
    exp sqrt pow add sub mul div eq ne le lt ge gt where bitwise_not
    bitwise_and bitwise_or.  Comparisons return bool, the rest the compute
    type (unrounded)."""
    ct = {"f32": np.float32, "f64": np.float64, "i64": np.int64}[compute]
    with np.errstate(all="ignore"):
        xs = [np.asarray(x).astype(ct) if not np.isscalar(x) else ct(x) for x in operands]
        xs = [np.asarray(x) for x in xs]
        if op in _UNARY_F:
            return _UNARY_F[op](xs[0])
        if op == "pow":
            return _pow_scalar(xs[0], exponent, store)
        if op == "where":
            c = np.asarray(operands[0]).astype(bool)
            return np.where(c, xs[1], xs[2])
        if op == "bitwise_not":
            b = np.asarray(operands[0])
            return ~b if b.dtype == bool else ~b.astype(np.int64)
        if op in ("bitwise_and", "bitwise_or"):
            a, b = (np.asarray(x) for x in operands[:2])
            return (a & b) if op == "bitwise_and" else (a | b)
        a, b = xs[0], xs[1]
        if op in ("add", "sub"):
            if alpha == 1:
                return a + b if op == "add" else a - b
            # aten's alpha kernels: one fused multiply-add, a + (+-alpha) * b
            al = alpha if op == "add" else -alpha
            if ct is np.int64:
                return a + np.int64(al) * b
            wide = np.float64 if ct is np.float32 else np.longdouble
            return (wide(al) * b.astype(wide) + a.astype(wide)).astype(ct)
        if op == "mul":
            return a * b
        if op == "div":
            return a / b
        cmp = {"eq": np.equal, "ne": np.not_equal, "le": np.less_equal, "lt": np.less,
               "ge": np.greater_equal, "gt": np.greater}
        if op in cmp:
            return cmp[op](a, b)
    raise ValueError(f"elementwise: unknown op {op}")


def mean_lastdim(x, keepdim=False) -> np.ndarray:
    """Mean over the last axis with a wide (fp64) sum, scaled by
    m / (m * n) as aten's mean.dim scales it (MeanImpl kuipy/kuiops.py:860-921).
    Unrounded: callers round to the storage dtype."""
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    m = x.size // n if n else 0
    factor = np.float64(m) / np.float64(m * n)
    out = x.sum(-1) * factor
    return out[..., None] if keepdim else out


def cat(tensors, dim=0) -> np.ndarray:
    """Concatenation along ``dim`` (CatImpl kuipy/kuiops.py:810-857); a copy,
    bit-exact in any dtype."""
    return np.concatenate([np.asarray(t) for t in tensors], axis=dim)


# ------------------------------------------------------------------- GEMM


def mm(A, B, acc="f64") -> np.ndarray:
    """C = A @ B for [M, K] x [K, N] with the inputs taken exactly as given
    (already rounded to their storage type) and a wide accumulator
    (aten.mm; MmImpl kuipy/kuiops.py:403-469).  The product is not rounded:
    callers round to the output dtype with ``round_dtype``."""
    A = np.asarray(A, dtype=np.float64 if acc == "f64" else np.float32)
    B = np.asarray(B, dtype=A.dtype)
    if A.ndim != 2 or B.ndim != 2 or A.shape[1] != B.shape[0]:
        raise ValueError("mm: shape mismatch")
    return A @ B


def addmm(C, A, B, alpha=1.0, beta=1.0) -> np.ndarray:
    """beta * C + alpha * (A @ B), C broadcast to [M, N] (aten.addmm;
    AddmmImpl kuipy/kuiops.py:520-564 with alpha/beta as in
    kuiops/addmm/wrapper_addmm.cu.j2:7).  beta == 0 ignores C entirely."""
    P = mm(A, B)
    out = alpha * P
    if beta != 0:
        out = out + beta * np.broadcast_to(np.asarray(C, dtype=np.float64), P.shape)
    return out


def bmm(A, B) -> np.ndarray:
    """C[b] = A[b] @ B[b], output overwritten (comb2, kuiops/bmm/Kuiops.Bmm.fst:10-23)."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    if A.ndim != 3 or B.ndim != 3 or A.shape[0] != B.shape[0] or A.shape[2] != B.shape[1]:
        raise ValueError("bmm: shape mismatch")
    return np.einsum("bmk,bkn->bmn", A, B)


def splitk_mm(A, B, splits: int) -> np.ndarray:
    """mm computed as fp32 partial products over `splits` K ranges, summed in
    split order -- the deterministic split-K contract of kuiops_addmm /
    kuiops_gemv_splitk (fixed-order reduction)."""
    A = np.asarray(A, dtype=np.float32)
    B = np.asarray(B, dtype=np.float32)
    K = A.shape[1]
    step = -(-K // splits)
    acc = np.zeros((A.shape[0], B.shape[1]), dtype=np.float32)
    for z in range(splits):
        lo, hi = z * step, min(K, (z + 1) * step)
        if lo < hi:
            acc = acc + (A[:, lo:hi].astype(np.float64) @ B[lo:hi].astype(np.float64)).astype(np.float32)
    return acc


# ---------------------------------------------------------------- softmax


def softmax(x, axis=-1) -> np.ndarray:
    """exp(x - max) / sum over `axis` in fp64 (aten._softmax;
    SoftmaxImpl kuipy/kuiops.py:572-610)."""
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(x - m)
        return e / np.sum(e, axis=axis, keepdims=True)


# ------------------------------------------------------------------- SDPA


def sdpa(q, k, v, causal=False, scale=None, bias=None, align="top_left"):
    """Attention in fp64: returns (out, lse).

    q (n, hq, l, e), k (n, hkv, s, e), v (n, hkv, s, ev); hq % hkv == 0 and
    query head h reads KV head h // (hq // hkv).  scores = scale * q k^T
    (+ bias), the softmax-over-keys weights give out = P v and
    lse = logsumexp(scores) (natural log).  Layouts (N, H, L, E) row-major
    as kuiops/sdpa/Kuiops.Sdpa.fst.1:19-27; the bias is added after scaling
    as aten does (the reference pre-divides it, kuipy/kuiops.py:673-676).
    Causal: 'top_left' is aten's is_causal (query i sees keys j <= i);
    'bottom_right' aligns the queries to the end of the keys (KV-cache
    decode).  Rows with no visible key give out = 0 and lse = -inf.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n, hq, l, e = q.shape
    hkv, s = k.shape[1], k.shape[2]
    if hq % hkv:
        raise ValueError("sdpa: hq % hkv != 0")
    g = hq // hkv
    k = np.repeat(k, g, axis=1)
    v = np.repeat(v, g, axis=1)
    if scale is None:
        scale = 1.0 / math.sqrt(e)
    sc = scale * np.matmul(q, np.swapaxes(k, -1, -2))
    if bias is not None:
        sc = sc + np.asarray(bias, dtype=np.float64)
    if causal:
        i = np.arange(l)[:, None]
        j = np.arange(s)[None, :]
        visible = j <= i if align == "top_left" else j <= (s - l + i)
        sc = np.where(visible, sc, -np.inf)
    m = np.max(sc, axis=-1, keepdims=True, initial=-np.inf)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(sc - m_safe)
    denom = np.sum(p, axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.where(denom > 0, np.matmul(p, v) / np.where(denom > 0, denom, 1), 0.0)
        lse = np.where(denom[..., 0] > 0, np.log(np.where(denom[..., 0] > 0, denom[..., 0], 1)) + m_safe[..., 0], -np.inf)
    return out, lse


# -------------------------------------------------------------------- topk


def _order_key(x: np.ndarray) -> np.ndarray:
    """Sort key with NaN above +inf (aten.topk's NaN convention)."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(np.isnan(x), np.inf, x), np.isnan(x)


def topk(x, k: int, largest=True):
    """(values, int64 indices) of the k largest (smallest) entries of each row
    of the last axis.  NaN ranks above every number; equal values are ordered
    by ascending index (lowest indices win a tie at the k-th place).
    aten.topk semantics on tie-free inputs; there is no reference kernel
    (kuiops/topk/.gitkeep)."""
    x = np.asarray(x)
    flat = x.reshape(-1, x.shape[-1])
    vals = np.empty((flat.shape[0], k), dtype=x.dtype)
    inds = np.empty((flat.shape[0], k), dtype=np.int64)
    for r in range(flat.shape[0]):
        row = flat[r]
        key, isnan = _order_key(row)
        idx = np.arange(row.shape[0])
        if largest:
            # primary: NaN first, then value descending; secondary: index ascending
            order = np.lexsort((idx, -key, ~isnan))
        else:
            order = np.lexsort((idx, key, isnan))
        sel = order[:k]
        vals[r] = row[sel]
        inds[r] = sel
    return vals.reshape(*x.shape[:-1], k), inds.reshape(*x.shape[:-1], k)


# --------------------------------------------------------- gather / index


def gather(inp, dim: int, idx) -> np.ndarray:
    """out[x] = inp[x with axis `dim` replaced by idx[x]]
    (kuiops/gather/Kuiops.Gather.fst:482-486; aten.gather)."""
    inp = np.asarray(inp)
    idx = np.asarray(idx, dtype=np.int64)
    if np.any(idx < 0) or np.any(idx >= inp.shape[dim]):
        raise IndexError("gather: index out of range")
    coords = list(np.indices(idx.shape))
    coords[dim] = idx
    return inp[tuple(coords)]


def index(inp, dim: int, idx) -> np.ndarray:
    """inp[:, ..., idx, ...] with one int64 index tensor at axis `dim`
    (aten.index.Tensor); negative indices count from the end."""
    inp = np.asarray(inp)
    idx = np.asarray(idx, dtype=np.int64)
    size = inp.shape[dim]
    if np.any(idx < -size) or np.any(idx >= size):
        raise IndexError("index: index out of range")
    idx = np.where(idx < 0, idx + size, idx)
    return np.take(inp, idx, axis=dim)


def index_multi(inp, first: int, idxs) -> np.ndarray:
    """inp[:, .., :, idxs[0], .., idxs[k-1], ...] with the k int64 index
    tensors on adjacent axes first .. first+k-1, broadcast together (aten
    advanced indexing, the reference app's mask[T(4,int64), T(4,int64)],
    KERNELS.md:67); negative indices wrap.  Written as an explicit loop over
    the broadcast index positions."""
    inp = np.asarray(inp)
    idxs = np.broadcast_arrays(*[np.asarray(t, dtype=np.int64) for t in idxs])
    k = len(idxs)
    bshape = idxs[0].shape
    lead, trail = inp.shape[:first], inp.shape[first + k:]
    out = np.empty(lead + bshape + trail, dtype=inp.dtype)
    for pos in np.ndindex(*bshape):
        sel = tuple(int(t[pos]) % inp.shape[first + d] for d, t in enumerate(idxs))
        out[(slice(None),) * first + pos] = inp[(slice(None),) * first + sel]
    return out


def scatter(inp, dim: int, idx, src) -> np.ndarray:
    """Copy of inp with out[x with axis `dim` replaced by idx[x]] = src[x] for
    every x of idx's shape (kuipy/kuiops.py:757-807; aten.scatter.src)."""
    out = np.array(inp, copy=True)
    idx = np.asarray(idx, dtype=np.int64)
    src = np.asarray(src)
    if np.any(idx < 0) or np.any(idx >= out.shape[dim]):
        raise IndexError("scatter: index out of range")
    for x in np.ndindex(*idx.shape):
        y = list(x)
        y[dim] = idx[x]
        out[tuple(y)] = src[x]
    return out


# ------------------------------------------------------- sort / cumsum / sampling


def sort(x, descending=False):
    """(values, int64 indices) of a stable sort of the last axis (aten.sort
    with stable=True): NaN ranks above every number, -0 equals +0, equal
    values keep ascending index order."""
    x = np.asarray(x)
    flat = x.reshape(-1, x.shape[-1])
    vals = np.empty_like(flat)
    inds = np.empty(flat.shape, dtype=np.int64)
    for r in range(flat.shape[0]):
        row = flat[r]
        key, isnan = _order_key(row)
        key = np.where(key == 0, 0.0, key)          # -0 == +0
        idx = np.arange(row.shape[0])
        if descending:
            order = np.lexsort((idx, -key, ~isnan))
        else:
            order = np.lexsort((idx, key, isnan))
        vals[r] = row[order]
        inds[r] = order
    return vals.reshape(x.shape), inds.reshape(x.shape)


def cumsum(x, acc="f64") -> np.ndarray:
    """Inclusive prefix sum of the last axis (aten.cumsum); floating input is
    accumulated in fp64 (the reference value), integers exactly."""
    x = np.asarray(x)
    if np.issubdtype(x.dtype, np.integer):
        return np.cumsum(x, axis=-1, dtype=np.int64)
    return np.cumsum(x.astype(np.float64), axis=-1)


def multinomial(p, u) -> np.ndarray:
    """Inverse-CDF draws: for row r and uniform u[r, s], the first index i
    whose running weight sum (fp64) exceeds u * total, never a zero weight
    (a u rounding onto the total takes the last positive weight)."""
    p = np.asarray(p, dtype=np.float64)
    p2 = p.reshape(-1, p.shape[-1])
    u2 = np.asarray(u, dtype=np.float64).reshape(p2.shape[0], -1)
    out = np.empty(u2.shape, dtype=np.int64)
    for r in range(p2.shape[0]):
        row = p2[r]
        if np.any(~np.isfinite(row)) or np.any(row < 0) or not row.sum() > 0:
            raise ValueError("multinomial: invalid probability row")
        cdf = np.cumsum(row)
        pos = np.nonzero(row > 0)[0]
        for s_ in range(u2.shape[1]):
            t = u2[r, s_] * cdf[-1]
            cand = pos[cdf[pos] > t]
            out[r, s_] = cand[0] if cand.size else pos[-1]
    return out


def top_p_filter(scores, top_p: float, filter_value=-np.inf, min_tokens_to_keep: int = 1) -> np.ndarray:
    """transformers' TopPLogitsWarper on [m, vocab] fp32 scores: ascending
    stable sort, softmax, cumulative sum, drop the sorted prefix with
    cumulative probability <= 1 - top_p (keeping the last min_tokens_to_keep),
    mask the dropped scores with filter_value."""
    scores = np.asarray(scores, dtype=np.float32)
    vals, idx = sort(scores, descending=False)
    cum = cumsum(softmax(vals), acc="f64")
    remove = cum <= (1 - top_p)
    remove[..., -min_tokens_to_keep:] = False
    mask = scatter(np.zeros_like(remove), 1, idx, remove)
    return np.where(mask, np.float32(filter_value), scores)


# ------------------------------------------------------------ verify metric


def rel_frobenius(out, ref) -> float:
    """||out - ref||_F / (||ref||_F + 1e-12) over positions finite in both
    (kuipy/__init__.py:193-225)."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    fin = np.isfinite(o) & np.isfinite(r)
    if not fin.any():
        return 0.0
    o, r = o[fin], r[fin]
    return float(np.linalg.norm(o - r) / (np.linalg.norm(r) + 1e-12))


def within(out, ref, rtol=1e-2, atol=1e-2) -> bool:
    """Elementwise |out - ref| <= atol + rtol * |ref| (the north-star bf16
    GEMM / SDPA tolerance)."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    return bool(np.all(np.abs(o - r) <= atol + rtol * np.abs(r)))


# ------------------------------------------------- decoder-layer glue
# bf16 rounding points follow the transformers Llama modules: every torch
# op on a bf16 tensor rounds its result to bf16.


def rmsnorm(x, w, eps, residual=None):
    """(y, h): h = x (+ residual, rounded), y = w * round(h * rsqrt(mean(h^2) + eps))
    (LlamaRMSNorm: variance in fp32, weight applied to the rounded value)."""
    x = np.asarray(x, dtype=np.float32)
    h = x if residual is None else round_bf16(x + np.asarray(residual, dtype=np.float32))
    var = np.mean(h.astype(np.float64) ** 2, axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    return round_bf16(np.asarray(w, dtype=np.float32) * round_bf16(h * inv)), h


def silu_mul(gate_up):
    """round(round(silu(gate)) * up) for gate_up = [gate | up] on the last axis."""
    gu = np.asarray(gate_up, dtype=np.float32)
    n = gu.shape[-1] // 2
    g, u = gu[..., :n].astype(np.float64), gu[..., n:]
    return round_bf16(round_bf16(g / (1.0 + np.exp(-g))) * u)


def rope_inv_freq(hd: int, theta: float) -> np.ndarray:
    """1 / theta^(2i / hd), i < hd / 2, in fp32 (LlamaRotaryEmbedding default init)."""
    e = (np.arange(0, hd, 2, dtype=np.int64).astype(np.float32) / np.float32(hd)).astype(np.float64)
    return (1.0 / (float(theta) ** e)).astype(np.float32)


def rope(x, pos, inv_freq):
    """Split-half rotary embedding of x[..., t, hd] at positions pos[t]:
    (x1, x2) -> (x1 c - x2 s, x2 c + x1 s), angle = fp32(pos * inv_freq),
    c / s rounded to bf16, every product and sum rounded."""
    x = np.asarray(x, dtype=np.float32)
    hd = x.shape[-1]
    half = hd // 2
    ang = (np.asarray(pos, dtype=np.float32)[:, None] * np.asarray(inv_freq, dtype=np.float32)[None, :])
    c = round_bf16(np.cos(ang.astype(np.float64)).astype(np.float32))
    s_ = round_bf16(np.sin(ang.astype(np.float64)).astype(np.float32))
    x1, x2 = x[..., :half], x[..., half:]
    o1 = round_bf16(round_bf16(x1 * c) + round_bf16(-x2 * s_))
    o2 = round_bf16(round_bf16(x2 * c) + round_bf16(x1 * s_))
    return np.concatenate([o1, o2], axis=-1)


def linear(x, W):
    """round(x @ W^T) for an nn.Linear weight W[out, in] (bf16 result)."""
    return round_bf16(mm(x, np.asarray(W, dtype=np.float32).T).astype(np.float32))


def llama_forward(p: dict, tokens, cfg: dict) -> np.ndarray:
    """Logits (bf16 values as fp32) of every position of one sequence for a
    Llama-style causal LM: embedding, cfg['layers'] x (RMSNorm, GQA attention
    with rotary q / k, residual, RMSNorm, SwiGLU MLP, residual), final
    RMSNorm, LM head.  p holds the transformers parameter names (weights as
    fp32 arrays of bf16 values)."""
    d, hq, hkv = cfg["d"], cfg["hq"], cfg["hkv"]
    hd = d // hq
    eps = cfg["eps"]
    T = len(tokens)
    inv = rope_inv_freq(hd, cfg["theta"])
    pos = np.arange(T)
    h = np.asarray(p["model.embed_tokens.weight"], dtype=np.float32)[np.asarray(tokens)]
    for i in range(cfg["layers"]):
        pre = f"model.layers.{i}."
        x, _ = rmsnorm(h, p[pre + "input_layernorm.weight"], eps)
        q = linear(x, p[pre + "self_attn.q_proj.weight"]).reshape(T, hq, hd).transpose(1, 0, 2)
        k = linear(x, p[pre + "self_attn.k_proj.weight"]).reshape(T, hkv, hd).transpose(1, 0, 2)
        v = linear(x, p[pre + "self_attn.v_proj.weight"]).reshape(T, hkv, hd).transpose(1, 0, 2)
        q, k = rope(q, pos, inv), rope(k, pos, inv)
        a, _ = sdpa(q[None], k[None], v[None], causal=True)
        a = round_bf16(a[0].transpose(1, 0, 2).reshape(T, hq * hd).astype(np.float32))
        h = round_bf16(h + linear(a, p[pre + "self_attn.o_proj.weight"]))
        x, _ = rmsnorm(h, p[pre + "post_attention_layernorm.weight"], eps)
        g = linear(x, p[pre + "mlp.gate_proj.weight"])
        u = linear(x, p[pre + "mlp.up_proj.weight"])
        h = round_bf16(h + linear(silu_mul(np.concatenate([g, u], -1)), p[pre + "mlp.down_proj.weight"]))
    x, _ = rmsnorm(h, p["model.norm.weight"], eps)
    return linear(x, p["lm_head.weight"])


def llama_greedy(p: dict, prompt, n_new: int, cfg: dict):
    """Greedy continuation: (tokens, per-step fp32 logits of the chosen
    position), recomputing the full forward each step (tiny configs only)."""
    toks = list(int(t) for t in prompt)
    steps = []
    for _ in range(n_new):
        lg = llama_forward(p, toks, cfg)[-1]
        steps.append(lg)
        probs = softmax(lg)
        toks.append(int(topk(probs, 1)[1][0]))
    return toks[len(prompt):], steps
