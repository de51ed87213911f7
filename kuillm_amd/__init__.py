"""kuillm_amd -- the kuiops hot path (GEMM, flash SDPA, sampling tail) for
MI355X / gfx950, behind the reference's ``kuipy`` operator surface.

Drop-in usage, as with the reference's ``kuipy`` (kuipy/__init__.py:135-175)::

    import kuillm_amd as kuipy
    with kuipy.KuiperMode():               # or KuiperMode(verify=True)
        model.generate(...)

Inside the mode every aten call on the thread is looked up in the registry;
a family whose ``supported()`` accepts the call runs the HIP kernel through
the C ABI of include/kuiops.h, everything else runs stock PyTorch.
``verify=True`` also runs stock PyTorch on every offloaded op and records the
relative Frobenius error; ``KUIPY_PRINT_PROFILING=1`` records the signatures
of the kernel-launching ops seen.
"""
from __future__ import annotations

import sys

from . import config as C

__all__ = ["KuiperMode", "is_available", "verify_stats", "reset_verify", "print_verify_report",
           "print_profile_data", "profile_data"]


# ----------------------------------------------------------- call signatures

def arg_data(a):
    """Hashable summary of an argument for the profile log."""
    import torch
    if isinstance(a, torch.Tensor):
        shape = tuple(a.shape) if C.JIT_VERBOSITY > 1 else len(a.shape)
        return (shape, a.dtype, a.device)
    if isinstance(a, (list, tuple)):
        return ("list", tuple(arg_data(x) for x in a))
    if isinstance(a, (torch.dtype, torch.device, bool)):
        return a
    return type(a).__name__


def print_arg_data(a):
    if isinstance(a, tuple) and len(a) == 2 and a[0] == "list":
        return "[" + ", ".join(print_arg_data(x) for x in a[1]) + ", ]"
    if isinstance(a, tuple) and len(a) == 3:
        return f"Tensor(nshape={a[0]}, dtype={a[1]}, device={a[2]})"
    return str(a)


def print_call_data_aux(args, kwargs_keys, kwargs_values, ret):
    kw = ", ".join(f"{k}={print_arg_data(v)}" for k, v in zip(kwargs_keys, kwargs_values))
    return f"args={[print_arg_data(a) for a in args]}, kwargs={{ {kw} }} -> {print_arg_data(ret)}"


def print_call_data(args, kwargs):
    return print_call_data_aux(tuple(arg_data(a) for a in args), tuple(kwargs.keys()),
                               tuple(arg_data(v) for v in kwargs.values()), "no return captured")


def is_available() -> bool:
    """True when the native library loads and a GPU is visible (the reference
    checks for its F* toolchain instead, kuipy/__init__.py:44-48)."""
    try:
        import torch
        from . import compile as _compile
        _compile.load_library()
        return torch.cuda.is_available()
    except Exception:
        return False


# ------------------------------------------------------------------ dispatch

_jit_warned = False


class NotOffloaded(RuntimeError):
    """Raised at KUIPY_JIT_STRICTNESS=2 for an op no kernel served."""


def _jit_try(func, args, kwargs):
    """Dispatch to a kuiops kernel; None means "run stock PyTorch".

    Strictness (kuipy/config.py:42-46 semantics): 0 -- errors warn once and
    fall back; 1 -- errors raise; 2 -- additionally raise for ops the
    registry does not serve."""
    global _jit_warned
    from .registry import try_dispatch
    try:
        ret = try_dispatch(func, args, kwargs)
    except Exception as e:
        if C.JIT_STRICTNESS > 0:
            raise
        if not _jit_warned:
            _jit_warned = True
            print(f"[kuipy] kernel dispatch failed, falling back to PyTorch: {e}", file=sys.stderr)
        ret = None
    if ret is None:
        if C.JIT_VERBOSITY > 1:
            print(f"[kuipy] operator {func} ({print_call_data(args, kwargs)}) did not match",
                  file=sys.stderr)
        if C.JIT_STRICTNESS > 1:
            raise NotOffloaded(f"operator {func} was not offloaded (KUIPY_JIT_STRICTNESS=2)")
    return ret


def _tensors(x):
    import torch
    if isinstance(x, torch.Tensor):
        yield x
    elif isinstance(x, (list, tuple)):
        for e in x:
            yield from _tensors(e)


def _launches_gpu_kernel(func, args, out):
    """False for view / metadata ops whose outputs alias an input."""
    if func._schema.is_mutable:
        return True
    ins = {t.untyped_storage().data_ptr() for t in _tensors(args)}
    outs = list(_tensors(out))
    return not (outs and all(t.untyped_storage().data_ptr() in ins for t in outs))


def _has_device_kernel(func):
    """True iff the op registers a direct device kernel (not a composite)."""
    import torch
    try:
        return torch._C._dispatch_has_kernel_for_dispatch_key(func.name(), torch._C.DispatchKey.CUDA)
    except Exception:
        return False


profile_data = set()
_KuiperMode_class = None


def _KuiperMode_cls():
    global _KuiperMode_class
    if _KuiperMode_class is not None:
        return _KuiperMode_class
    from torch.utils._python_dispatch import TorchDispatchMode

    class KuiperMode(TorchDispatchMode):
        """Route eligible aten calls to the kuiops HIP kernels.

        ``verify=True`` runs stock PyTorch as well on every non-mutating op a
        kernel served and folds the relative Frobenius error into
        ``verify_stats`` (print with ``print_verify_report()``)."""
        dummy_print_mode = False   # only record profile data, never offload

        def __init__(self, verify=False, verify_tol=2e-2):
            super().__init__()
            self.verify = verify
            self.verify_tol = verify_tol

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            kwargs = kwargs or {}
            if self.dummy_print_mode:
                out = func(*args, **kwargs)
            else:
                out = _jit_try(func, args, kwargs)
                if out is None:
                    out = func(*args, **kwargs)
                elif self.verify and not func._schema.is_mutable:
                    _verify_compare(func, out, func(*args, **kwargs), self.verify_tol)
            if C.ENABLE_PRINT_PROFILING and _launches_gpu_kernel(func, args, out):
                profile_data.add((func, tuple(arg_data(a) for a in args), tuple(kwargs.keys()),
                                  tuple(arg_data(v) for v in kwargs.values()), arg_data(out)))
            return out

    _KuiperMode_class = KuiperMode
    return KuiperMode


def __getattr__(name):
    if name == "KuiperMode":
        return _KuiperMode_cls()
    raise AttributeError(name)


# -------------------------------------------------------------- verify mode

verify_stats = {}


def reset_verify():
    verify_stats.clear()


def _verify_compare(func, out, ref, tol):
    """Fold the relative Frobenius error of each floating output into
    ``verify_stats[str(func)]`` (kuipy/__init__.py:193-225 semantics):
    positions not finite in both are ignored (fully masked attention rows),
    empty references are skipped, shape mismatches count as failures."""
    name = str(func)
    st = verify_stats.setdefault(name, {"n": 0, "fail": 0, "max_rel": 0.0, "worst": None})
    for o, r in zip(_tensors(out), _tensors(ref)):
        if not (o.is_floating_point() and r.is_floating_point()):
            continue
        if r.numel() == 0 or o.numel() == 0:
            continue
        if o.shape != r.shape:
            st["fail"] += 1
            st["worst"] = f"shape mismatch {tuple(o.shape)} vs {tuple(r.shape)}"
            continue
        of, rf = o.float(), r.float()
        finite = of.isfinite() & rf.isfinite()
        if not bool(finite.any()):
            continue
        of, rf = of[finite], rf[finite]
        rel = float((of - rf).norm() / (rf.norm() + 1e-12))
        st["n"] += 1
        st["max_rel"] = max(st["max_rel"], rel)
        if rel > tol:
            st["fail"] += 1
            st["worst"] = f"rel={rel:.3e} (tol {tol:.1e})"


def print_verify_report(out_dev=sys.stdout, tol=2e-2):
    """Per-op pass / fail summary of a verify run; returns True when clean."""
    if not verify_stats:
        print("[verify] no kuiops-dispatched ops were checked.", file=out_dev)
        return None
    total_fail = sum(s["fail"] for s in verify_stats.values())
    print(f"[verify] kuiops vs stock PyTorch (relative Frobenius norm, tol {tol:.1e}):", file=out_dev)
    for name in sorted(verify_stats):
        s = verify_stats[name]
        status = "FAIL" if s["fail"] else "ok"
        line = f"  [{status:4}] {name}: {s['n']} checked, {s['fail']} fail, max_rel={s['max_rel']:.3e}"
        if s["worst"]:
            line += f", worst: {s['worst']}"
        print(line, file=out_dev)
    print(f"[verify] result: {'PASS' if total_fail == 0 else f'FAIL ({total_fail} divergences)'}",
          file=out_dev)
    return total_fail == 0


def print_profile_data(out_dev=sys.stdout):
    grouped = {}
    for func, args, kkeys, kvals, ret in profile_data:
        grouped.setdefault(func, []).append(print_call_data_aux(args, kkeys, kvals, ret))
    for func, calls in grouped.items():
        tag = "" if _has_device_kernel(func) else "  [no device kernel: composite]"
        print(f"Function {func}:{tag}", file=out_dev)
        for call in calls:
            print(f"  {call}", file=out_dev)
