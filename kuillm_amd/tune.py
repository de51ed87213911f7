"""Autotuning of the family parameters on the GPU at hand, persisted as JSON.

The reference keeps per-family ``tune_params`` and a ``KUIPY_RE_TUNE`` switch
whose results it meant to load from and write back to JSON (the "LATER"s at
kuipy/registry.py:71,76).  Here the families' ``tune()`` measure their
parameters with the sweeps below, and the registry loads / saves them
(``registry.load_tune_params`` / ``save_tune_params``, file
``config.TUNE_FILE``).

    python -m kuillm_amd.tune [--out PATH]      # sweep every family, write the JSON

Parameters measured:

* ``MM.gemv_max_m`` (also used by ADDMM): the largest row count up to which
  the decode GEMM (``kuiops_gemv_splitk``) beats the MFMA GEMM on every
  sampled decode shape;
* ``SDPA.decode_max_rows``: the largest number of query rows per KV head up
  to which the split-KV decode kernel beats the flash kernel.
"""
from __future__ import annotations

import argparse
import json
import statistics

import torch

from . import ops


def time_us(fn, reps: int = 20, warmup: int = 3) -> float:
    """Median device time of fn() in microseconds (HIP events, current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e3)
    return statistics.median(times)


def pick_crossover(candidates, faster) -> int:
    """The largest candidate c (ascending list) such that ``faster(c')`` holds
    for c and every smaller candidate; 0 when the first already fails."""
    best = 0
    for c in candidates:
        if not faster(c):
            break
        best = c
    return best


def sweep_gemv_max_m(shapes=((4096, 11008), (2048, 2048), (4096, 4096)),
                     rows=(1, 2, 4, 8, 16, 24, 32, 48, 64), device="cuda") -> int:
    """Largest M at which the decode GEMM is at least as fast as the MFMA GEMM
    for every [K, N] weight shape in ``shapes`` (bf16, row-major W)."""
    g = torch.Generator(device=device).manual_seed(0)
    ws = [(torch.randn(K, N, device=device, generator=g) * 0.02).to(torch.bfloat16) for K, N in shapes]

    def gemv_wins(M):
        for W in ws:
            x = torch.randn(M, W.shape[0], device=device, generator=g).to(torch.bfloat16)
            t_gemv = time_us(lambda: ops.mm(x, W, gemv_max_m=ops.GEMV_MAX_M))
            t_mfma = time_us(lambda: ops.mm(x, W, gemv_max_m=0))
            if t_gemv > t_mfma:
                return False
        return True

    return pick_crossover(rows, gemv_wins)


def sweep_decode_max_rows(rows=(1, 2, 4, 8, 16, 32), s=4096, hd=128, hkv=8, device="cuda") -> int:
    """Largest number of query rows per KV head (grouped-query heads x query
    positions) at which split-KV decode attention is at least as fast as the
    flash kernel, over an s-key cache."""
    g = torch.Generator(device=device).manual_seed(0)
    k = torch.randn(1, hkv, s, hd, device=device, generator=g).to(torch.bfloat16)
    v = torch.randn(1, hkv, s, hd, device=device, generator=g).to(torch.bfloat16)

    def decode_wins(r):
        # r rows per KV head as r query heads per KV head, one position each
        q = torch.randn(1, hkv * r, 1, hd, device=device, generator=g).to(torch.bfloat16)
        t_dec = time_us(lambda: ops.sdpa(q, k, v, decode_max_rows=max(rows)))
        t_fa = time_us(lambda: ops.sdpa(q, k, v, decode_max_rows=0))
        return t_dec <= t_fa

    return pick_crossover(rows, decode_wins)


def main(argv=None):
    from . import registry
    ap = argparse.ArgumentParser(description="sweep the kuiops family parameters on this GPU")
    ap.add_argument("--out", default=None, help="JSON file (default: the registry's tune file)")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("kuillm_amd.tune: needs a GPU")
    registry.reset()
    params = registry.load_tune_params()
    impls = registry._build_registry(params)
    for impl in set(impls.values()):
        params = impl.tune(params)
    registry.save_tune_params(params, args.out)
    registry.reset()
    print(json.dumps(params, indent=2, sort_keys=True, default=list))


if __name__ == "__main__":
    main()
