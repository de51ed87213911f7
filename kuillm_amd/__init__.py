"""kuillm_amd -- the kuiops hot path (GEMM, flash SDPA, sampling tail) for
MI355X / gfx950, behind the reference's ``kuipy`` operator surface.

Drop-in usage, as with the reference's ``kuipy`` (kuipy/__init__.py:135-175)::

    import kuillm_amd as kuipy
    with kuipy.KuiperMode():               # or KuiperMode(verify=True)
        model.generate(...)

Public names kept from the reference (kuipy/__init__.py:44-263):
``KuiperMode(verify, verify_tol)`` with ``dummy_print_mode``, ``is_available``,
``verify_stats`` / ``reset_verify`` / ``_verify_compare`` /
``print_verify_report(out_dev, tol)`` and ``print_profile_data(out_dev)``.
The implementation below is organised around three small pieces of state:

* the offload step (``_offload``): registry lookup + strictness policy;
* a verify ledger: per-op tallies of the relative Frobenius error between the
  kernel's result and stock PyTorch's;
* a call log: the distinct (op, signature) pairs of kernel-launching ops.
"""
from __future__ import annotations

import sys

import torch
from torch.utils._python_dispatch import TorchDispatchMode
from torch.utils._pytree import tree_leaves

from . import config as C

__all__ = ["KuiperMode", "is_available", "verify_stats", "reset_verify", "print_verify_report",
           "print_profile_data", "profile_data", "NotOffloaded"]


def is_available() -> bool:
    """True when the native library loads and a GPU is visible (the reference
    checks for its F* toolchain instead, kuipy/__init__.py:44-48)."""
    try:
        from . import compile as _compile
        _compile.load_library()
    except Exception:
        return False
    return torch.cuda.is_available()


# ------------------------------------------------------------ offload step

class NotOffloaded(RuntimeError):
    """Raised at KUIPY_JIT_STRICTNESS=2 for an op no kernel served."""


_warned_once = [False]


def _offload(func, args, kwargs):
    """The kernel result for ``func(*args, **kwargs)``, or None when stock
    PyTorch has to run it.

    Strictness levels (the reference's KUIPY_JIT_STRICTNESS,
    kuipy/config.py:42-46): 0 turns a failing kernel into one warning and a
    fallback, 1 lets the error propagate, 2 additionally refuses ops that no
    family serves."""
    from .registry import try_dispatch
    level = C.JIT_STRICTNESS
    try:
        result = try_dispatch(func, args, kwargs)
    except Exception as err:
        if level >= 1:
            raise
        if not _warned_once[0]:
            _warned_once[0] = True
            print(f"[kuipy] {func}: kernel failed ({err}); using stock PyTorch from now on "
                  "for failing calls", file=sys.stderr)
        result = None
    if result is not None:
        return result
    if C.JIT_VERBOSITY > 1:
        print(f"[kuipy] no kernel for {func} {_signature(args, kwargs)}", file=sys.stderr)
    if level >= 2:
        raise NotOffloaded(f"{func} was not offloaded (KUIPY_JIT_STRICTNESS=2)")
    return None


# ---------------------------------------------------------------- call log

def _describe(x) -> str:
    """Compact text for one argument: ``bf16[4,8]@cuda:0`` for a tensor (the
    rank only, ``bf16[2d]``, unless KUIPY_JIT_VERBOSITY > 1)."""
    if isinstance(x, torch.Tensor):
        dt = str(x.dtype).replace("torch.", "")
        dims = ",".join(str(int(s)) for s in x.shape) if C.JIT_VERBOSITY > 1 else f"{x.dim()}d"
        return f"{dt}[{dims}]@{x.device}"
    if isinstance(x, (list, tuple)):
        return "(" + " ".join(_describe(e) for e in x) + ")"
    if isinstance(x, (torch.dtype, torch.device, bool, type(None))):
        return str(x)
    return type(x).__name__


def _signature(args, kwargs, result=None) -> str:
    text = " ".join(_describe(a) for a in args)
    if kwargs:
        text += " | " + " ".join(f"{k}={_describe(v)}" for k, v in kwargs.items())
    if result is not None:
        text += " -> " + _describe(result)
    return text


# op -> set of signature strings of the calls seen with KUIPY_PRINT_PROFILING=1
profile_data: dict = {}


def _record_call(func, args, kwargs, result) -> None:
    """Log a call that runs a device kernel.  View ops (their schema returns
    aliases of an input) and calls without a tensor result launch nothing."""
    if func.is_view or not any(isinstance(t, torch.Tensor) for t in tree_leaves(result)):
        return
    profile_data.setdefault(func, set()).add(_signature(args, kwargs, result))


def print_profile_data(out_dev=sys.stdout):
    """List every kernel-launching op seen, with its distinct call
    signatures.  Ops that only decompose into other ops (no device kernel of
    their own) are marked, since their parts cannot be offloaded one by one."""
    for func in sorted(profile_data, key=str):
        try:
            direct = func.has_kernel_for_dispatch_key(torch._C.DispatchKey.CUDA)
        except Exception:
            direct = False
        note = "" if direct else "  (composite: no device kernel of its own)"
        print(f"{func}{note}", file=out_dev)
        for sig in sorted(profile_data[func]):
            print(f"    {sig}", file=out_dev)


# ----------------------------------------------------------- verify ledger

# str(op) -> {"n": checked, "fail": over tolerance, "max_rel": largest error,
#             "worst": text of the latest failure}
verify_stats: dict = {}


def reset_verify():
    verify_stats.clear()


def _rel_error(got: torch.Tensor, want: torch.Tensor):
    """||got - want|| / ||want|| over the positions finite in both, in fp64;
    None when no position is (e.g. a fully masked attention row)."""
    g = got.detach().to(torch.float64).reshape(-1)
    w = want.detach().to(torch.float64).reshape(-1)
    keep = torch.isfinite(g) & torch.isfinite(w)
    if not bool(keep.any()):
        return None
    zero = torch.zeros((), dtype=torch.float64, device=g.device)
    diff = torch.where(keep, g - w, zero)
    base = torch.where(keep, w, zero)
    return float(torch.linalg.vector_norm(diff) / (torch.linalg.vector_norm(base) + 1e-12))


def _verify_compare(func, out, ref, tol):
    """Add one comparison of a kernel's result ``out`` with stock PyTorch's
    ``ref`` to ``verify_stats[str(func)]``.  Outputs are paired in order;
    non-floating and empty ones are not compared, a shape disagreement counts
    as a failure (reference semantics, kuipy/__init__.py:193-225)."""
    entry = verify_stats.setdefault(str(func), {"n": 0, "fail": 0, "max_rel": 0.0, "worst": None})
    pairs = zip((t for t in tree_leaves(out) if isinstance(t, torch.Tensor)),
                (t for t in tree_leaves(ref) if isinstance(t, torch.Tensor)))
    for got, want in pairs:
        if not (got.is_floating_point() and want.is_floating_point()) or 0 in (got.numel(), want.numel()):
            continue
        if got.shape != want.shape:
            entry["fail"] += 1
            entry["worst"] = f"shape mismatch {tuple(got.shape)} vs {tuple(want.shape)}"
            continue
        rel = _rel_error(got, want)
        if rel is None:
            continue
        entry["n"] += 1
        entry["max_rel"] = max(entry["max_rel"], rel)
        if not rel <= tol:
            entry["fail"] += 1
            entry["worst"] = f"rel={rel:.3e} (tol {tol:.1e})"


def print_verify_report(out_dev=sys.stdout, tol=2e-2):
    """Print one line per verified op and an overall verdict.  Returns True
    when every comparison was within tolerance, False otherwise, and None
    when nothing was verified."""
    if not verify_stats:
        print("[verify] nothing was checked (no op was served by a kuiops kernel)", file=out_dev)
        return None
    width = max(len(k) for k in verify_stats)
    print(f"[verify] kuiops against stock PyTorch, relative Frobenius error, tolerance {tol:.1e}",
          file=out_dev)
    failures = 0
    for name, e in sorted(verify_stats.items()):
        failures += e["fail"]
        tag = "FAIL" if e["fail"] else "ok"
        tail = f"  last failure: {e['worst']}" if e["fail"] else ""
        print(f"  {name:<{width}}  {tag:<4} checked {e['n']:>5}  failed {e['fail']:>4}  "
              f"max_rel {e['max_rel']:.2e}{tail}", file=out_dev)
    print("[verify] " + ("PASS" if failures == 0 else f"FAIL: {failures} comparisons over tolerance"),
          file=out_dev)
    return failures == 0


# ------------------------------------------------------------- dispatch mode

class KuiperMode(TorchDispatchMode):
    """Route eligible aten calls to the kuiops HIP kernels; everything else
    runs stock PyTorch.

    ``verify=True`` also runs stock PyTorch on every non-mutating op a kernel
    served and adds the comparison to ``verify_stats``.  With
    ``dummy_print_mode`` set nothing is offloaded and only the call log is
    kept (KUIPY_PRINT_PROFILING=1)."""
    dummy_print_mode = False

    def __init__(self, verify=False, verify_tol=2e-2):
        super().__init__()
        self.verify = verify
        self.verify_tol = verify_tol

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        result = None if self.dummy_print_mode else _offload(func, args, kwargs)
        if result is None:
            result = func(*args, **kwargs)
        elif self.verify and not func._schema.is_mutable:
            _verify_compare(func, result, func(*args, **kwargs), self.verify_tol)
        if C.ENABLE_PRINT_PROFILING:
            _record_call(func, args, kwargs, result)
        return result
