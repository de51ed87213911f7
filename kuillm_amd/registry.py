"""Registry mapping aten overloads to kuiops families, and the dispatch entry.

Same hot path as the reference (kuipy/registry.py:67-84): a dict lookup, a
cheap ``supported()``, and on a hit a native call; ``None`` means "fall
through to stock PyTorch".  Tune parameters persist as JSON in
``config.TUNE_FILE`` (the reference's "LATER: load these from json",
kuipy/registry.py:71,76); ``KUIPY_RE_TUNE=1`` re-runs every family's
``tune()`` and writes the result back.
"""
from __future__ import annotations

import json
from pathlib import Path

from . import config as C
from .kuiops import (AddmmImpl, BmmImpl, CatImpl, CumsumImpl, ElementwiseImpl, GatherImpl, IndexImpl, MeanImpl,
                     MmImpl, MultinomialImpl, ScatterImpl, SdpaImpl, SoftmaxImpl, SortImpl, TopkImpl)

_REGISTRY = None
_TUNE_PARAMS = None


def load_tune_params(path=None) -> dict:
    p = path or C.TUNE_FILE
    try:
        with open(p) as f:
            data = json.load(f)
        return data if isinstance(data, dict) else {}
    except (FileNotFoundError, json.JSONDecodeError):
        return {}


def save_tune_params(params: dict, path=None) -> None:
    p = Path(path) if path else C.TUNE_FILE
    p.parent.mkdir(parents=True, exist_ok=True)
    with open(p, "w") as f:
        json.dump(params, f, indent=2, sort_keys=True, default=list)


def _build_registry(tune_params):
    import torch
    aten = torch.ops.aten
    mm, bmm, addmm = MmImpl(tune_params), BmmImpl(tune_params), AddmmImpl(tune_params)
    softmax, sdpa = SoftmaxImpl(tune_params), SdpaImpl(tune_params)
    topk, gather, index = TopkImpl(tune_params), GatherImpl(tune_params), IndexImpl(tune_params)
    scatter, sort = ScatterImpl(tune_params), SortImpl(tune_params)
    cumsum, multinomial = CumsumImpl(tune_params), MultinomialImpl(tune_params)
    elem, mean, cat = ElementwiseImpl(tune_params), MeanImpl(tune_params), CatImpl(tune_params)
    table = {op: elem for op in ElementwiseImpl.OPS}
    table.update({
        aten.mean.dim: mean,
        aten.cat.default: cat,
        aten.mm.default: mm,
        aten.bmm.default: bmm,
        aten.addmm.default: addmm,
        aten._softmax.default: softmax,
        aten._scaled_dot_product_efficient_attention.default: sdpa,
        aten._scaled_dot_product_flash_attention.default: sdpa,
        aten.topk.default: topk,
        aten.gather.default: gather,
        aten.index.Tensor: index,
        aten.scatter.src: scatter,
        aten.sort.default: sort,
        aten.sort.stable: sort,
        aten.cumsum.default: cumsum,
        aten.multinomial.default: multinomial,
    })
    return table


def _tune_impls(tune_params):
    for impl in set(_REGISTRY.values()):
        tune_params = impl.tune(tune_params)
    return tune_params


def registry():
    """The aten-op -> family map (built on first use)."""
    global _REGISTRY, _TUNE_PARAMS
    if _REGISTRY is None:
        _TUNE_PARAMS = load_tune_params()
        _REGISTRY = _build_registry(_TUNE_PARAMS)
        if C.RE_TUNE:
            _TUNE_PARAMS = _tune_impls(_TUNE_PARAMS)
            save_tune_params(_TUNE_PARAMS)
    return _REGISTRY


def reset():
    """Forget the registry (tests / re-tuning)."""
    global _REGISTRY, _TUNE_PARAMS
    _REGISTRY = None
    _TUNE_PARAMS = None


def try_dispatch(func, args, kwargs):
    """Return the result if a kuiops kernel handles ``func``, else None."""
    impl = registry().get(func)
    if impl is None:
        return None
    spec = impl.supported(func, args, kwargs)
    if spec is None:
        return None
    return impl.run(spec, args, kwargs)
