#!/usr/bin/env python3
"""Benchmark of the kuiops hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu-baseline]

Headline (the JSON line's ``value``): BASELINE.json config 2, bf16 prefill
addmm  out[4096,4096] = bias[4096] + A[4096,4096] @ B[4096,4096], A~N(0,1),
B~N(0,0.02), fp32 accumulate, in bf16 TFLOP/s.  A "step" is one
``kuillm_amd.ops.addmm`` call (one MFMA kernel launch) on inputs resident in
HBM.  Ten back-to-back steps are recorded in a HIP graph and the graph is
replayed, so the timed region holds device work only and the per-replay
launch cost is spread over ten kernels; HIP events on the launch stream
bracket exactly K replays after W warm-up replays, and ``ms_per_step`` is the
time per kernel.

``workloads`` (extra keys of the same line) measures the other BASELINE.json
configs the same way: decode split-K GEMM (HBM GB/s), bmm, causal SDPA at
S=2048/4096, decode SDPA, and the softmax + top-k sampling tail.  Each
carries its own roofline fraction.

``cpu_baseline``: the reference's CPU path -- stock torch aten on the host
cores (the reference never offloads CPU tensors, kuipy/kuiops.py:531) -- on
the same addmm in fp32 (CPU bf16 is not representative), timed for a bounded
number of iterations.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
COLD_COPIES = 4               # input copies cycled by the HBM-bound workloads (> 256 MB MALL)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="run only the dominant kernel of each workload 3x plus a 256 MiB copy "
                         "(the byte-counter calibration), for rocprofv3 --pmc runs")
    return ap.parse_args()


def graph_time_ms(torch, fn, steps, warmup, reps=1):
    """Average device time of one `fn()` step: `reps` back-to-back `fn()`
    calls recorded into a HIP graph, W warm-up replays, then K replays between
    HIP events on the current (launch) stream, with device synchronisation on
    both sides; returns the time per call.  reps > 1 is for the
    microsecond-scale decode kernels, whose graph-replay overhead (a few us)
    would otherwise be timed as kernel time."""
    fn()                                    # eager run: allocates workspaces outside capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (steps * reps)


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")


def traffic_bytes(kernel):
    """HBM bytes per launch of `kernel` measured by rocprofv3 --pmc FETCH_SIZE
    and WRITE_SIZE over ``bench.py --profile-kernels``, each scaled by what
    the counter reads for a 256 MiB copy (profiles/hbm_traffic.json); None if
    not measured."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(kernel)
    if not k:
        return None
    return int(k["fetch_kib"] * 1024 * t["fetch_scale"] + k["write_kib"] * 1024 * t["write_scale"])


def roofline(bound, achieved, unit, traffic=None):
    peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def profile_kernels(torch, ops, dev):
    """The dominant kernel of each measured workload, 3 launches each, then a
    256 MiB device copy whose byte counts calibrate FETCH_SIZE / WRITE_SIZE."""
    g = torch.Generator(device=dev).manual_seed(0)
    A = torch.randn(4096, 4096, device=dev, generator=g).to(torch.bfloat16)
    B = (torch.randn(4096, 4096, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(4096, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    for _ in range(3):
        ops.addmm(bias, A, B)
    W = (torch.randn(4096, 11008, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    for M in (1, 4, 16):
        x = torch.randn(M, 4096, device=dev, generator=g).to(torch.bfloat16)
        for _ in range(3):
            ops.mm(x, W)
    q, k, v = (torch.randn(1, 32, 4096, 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    for _ in range(3):
        ops.sdpa(q, k, v, is_causal=True)
    qd = torch.randn(1, 32, 1, 128, device=dev, generator=g).to(torch.bfloat16)
    for _ in range(3):
        ops.sdpa(qd, k, v)
    A3 = torch.randn(32, 2048, 128, device=dev, generator=g).to(torch.bfloat16)
    B3 = torch.randn(32, 128, 2048, device=dev, generator=g).to(torch.bfloat16)
    for _ in range(3):
        ops.bmm(A3, B3)
    src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def cpu_baseline(torch, seconds):
    """Stock torch addmm on the host cores, fp32, same shape as the headline."""
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    A = torch.randn(4096, 4096, generator=g)
    B = torch.randn(4096, 4096, generator=g) * 0.02
    bias = torch.randn(4096, generator=g) * 0.02
    torch.addmm(bias, A, B)                      # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        torch.addmm(bias, A, B)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": round(2 * 4096 ** 3 / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "reference",
            "sample": f"stock torch {torch.__version__} CPU fp32 addmm bias[4096] + A[4096,4096] @ "
                      f"B[4096,4096], median of {len(times)} calls ({med * 1e3:.1f} ms each)"}


def extra_workloads(torch, ops, steps, warmup, dev):
    out = {}
    bf = torch.bfloat16
    torch.manual_seed(1)
    # config 1: decode split-K GEMM, HBM-bound
    # COLD copies of W (4 x 90 MB) are cycled so that every call reads its W
    # from HBM: one 90 MB W called back to back would be served largely from
    # the 256 MB MALL (memory-side cache) and overstate HBM throughput.  The
    # warm figure (one W, repeated) is reported beside it.
    Ws = [(torch.randn(4096, 11008, device=dev) * 0.02).to(bf) for _ in range(COLD_COPIES)]
    for M in (1, 4, 16):
        x = torch.randn(M, 4096, device=dev).to(bf)
        ms = graph_time_ms(torch, lambda: [ops.mm(x, W) for W in Ws], steps, warmup, reps=5) / len(Ws)
        ms_warm = graph_time_ms(torch, lambda: ops.mm(x, Ws[0]), steps, warmup, reps=20)
        nbytes = 4096 * 11008 * 2 + M * 4096 * 2 + M * 11008 * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"decode_gemm_M{M}"] = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(ms, 5),
                                    "roofline": roofline("hbm", gbs, "GB/s", traffic_bytes(f"decode_gemm_M{M}")),
                                    "warm_same_W_GBs": round(nbytes / (ms_warm * 1e-3) / 1e9, 1)}
    del Ws
    # config 2b: bmm 32 x [2048,128] @ [128,2048]
    A3 = torch.randn(32, 2048, 128, device=dev).to(bf)
    B3 = torch.randn(32, 128, 2048, device=dev).to(bf)
    ms = graph_time_ms(torch, lambda: ops.bmm(A3, B3), steps, warmup, reps=5)
    tf = 2 * 32 * 2048 * 2048 * 128 / (ms * 1e-3) / 1e12
    gbs = (2 * 32 * 2048 * 128 * 2 + 32 * 2048 * 2048 * 2) / (ms * 1e-3) / 1e9
    out["bmm_32x2048x128x2048"] = {"value": round(tf, 1), "unit": "TFLOP/s", "ms": round(ms, 5),
                                   "roofline": roofline("hbm", gbs, "GB/s", traffic_bytes("bmm_32x2048x128x2048")),
                                   "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4)}
    del A3, B3
    # config 3: causal SDPA B=1, H=32, D=128
    for S in (2048, 4096):
        q = torch.randn(1, 32, S, 128, device=dev).to(bf)
        k = torch.randn_like(q)
        v = torch.randn_like(q)
        ms = graph_time_ms(torch, lambda: ops.sdpa(q, k, v, is_causal=True), steps, warmup, reps=5)
        tf = 0.5 * 4 * 32 * S * S * 128 / (ms * 1e-3) / 1e12
        out[f"sdpa_causal_S{S}"] = {"value": round(tf, 1), "unit": "TFLOP/s", "ms": round(ms, 5),
                                    "roofline": roofline("mfma", tf, "TFLOP/s",
                                                         traffic_bytes("sdpa_causal_S4096") if S == 4096 else None)}
    # config 3b: decode SDPA, S_q = 1 over a 4096-token KV cache
    # (cold K / V caches cycled as for the decode GEMM: 5 x 67 MB > MALL)
    qd = torch.randn(1, 32, 1, 128, device=dev).to(bf)
    kvs = [(torch.randn(1, 32, 4096, 128, device=dev).to(bf), torch.randn(1, 32, 4096, 128, device=dev).to(bf))
           for _ in range(COLD_COPIES + 1)]
    ms = graph_time_ms(torch, lambda: [ops.sdpa(qd, kc, vc) for kc, vc in kvs], steps, warmup, reps=4) / len(kvs)
    ms_warm = graph_time_ms(torch, lambda: ops.sdpa(qd, *kvs[0]), steps, warmup, reps=20)
    gbs = 2 * 32 * 4096 * 128 * 2 / (ms * 1e-3) / 1e9
    out["sdpa_decode_kv4096"] = {"value": round(gbs, 1), "unit": "GB/s", "ms": round(ms, 5),
                                 "roofline": roofline("hbm", gbs, "GB/s", traffic_bytes("sdpa_decode_kv4096")),
                                 "warm_same_KV_GBs": round(2 * 32 * 4096 * 128 * 2 / (ms_warm * 1e-3) / 1e9, 1)}
    del kvs
    # sampling tail: softmax + top-1 / top-50 over a [1, 32000] fp32 logit row
    logits = torch.randn(1, 32000, device=dev)
    ms = graph_time_ms(torch, lambda: ops.topk(ops.softmax(logits), 1), steps, warmup, reps=20)
    out["sampling_softmax_top1_V32000"] = {"value": round(ms * 1e3, 2), "unit": "us"}
    ms = graph_time_ms(torch, lambda: ops.topk(ops.softmax(logits), 50), steps, warmup, reps=20)
    out["sampling_softmax_top50_V32000"] = {"value": round(ms * 1e3, 2), "unit": "us"}
    # HF top-p tail (sort, softmax, cumsum, scatter, mask, softmax, multinomial)
    # over a [1, 32000] row, uniforms resident on the device
    u = torch.rand(1, 1, device=dev)
    ms = graph_time_ms(torch, lambda: ops.sample_top_p(logits, 0.9, uniforms=u), steps, warmup, reps=10)
    out["sampling_top_p_V32000"] = {"value": round(ms * 1e3, 2), "unit": "us"}
    out["llama1b_greedy"] = llama_workload(torch, dev)
    return out


LLAMA1B = dict(vocab=32000, d=2048, ffn=5632, layers=16, hq=32, hkv=8)


def llama_state(torch, c, device, seed=0):
    """Random-init Llama-style weights (transformers parameter names):
    linear / embedding weights N(0, 0.02), norm weights 1."""
    g = torch.Generator(device=device).manual_seed(seed)
    hd = c["d"] // c["hq"]

    def w(o, i):
        return (torch.randn(o, i, device=device, generator=g) * 0.02).to(torch.bfloat16)

    st = {"model.embed_tokens.weight": w(c["vocab"], c["d"]), "lm_head.weight": w(c["vocab"], c["d"]),
          "model.norm.weight": torch.ones(c["d"], device=device, dtype=torch.bfloat16)}
    for i in range(c["layers"]):
        p = f"model.layers.{i}."
        st[p + "self_attn.q_proj.weight"] = w(c["hq"] * hd, c["d"])
        st[p + "self_attn.k_proj.weight"] = w(c["hkv"] * hd, c["d"])
        st[p + "self_attn.v_proj.weight"] = w(c["hkv"] * hd, c["d"])
        st[p + "self_attn.o_proj.weight"] = w(c["d"], c["hq"] * hd)
        st[p + "mlp.gate_proj.weight"] = w(c["ffn"], c["d"])
        st[p + "mlp.up_proj.weight"] = w(c["ffn"], c["d"])
        st[p + "mlp.down_proj.weight"] = w(c["d"], c["ffn"])
        st[p + "input_layernorm.weight"] = torch.ones(c["d"], device=device, dtype=torch.bfloat16)
        st[p + "post_attention_layernorm.weight"] = torch.ones(c["d"], device=device, dtype=torch.bfloat16)
    return st


def llama_decode_bytes(c, kv_tokens):
    """HBM bytes one decode token must read: every weight but the embedding
    table once (bf16) plus the K and V of kv_tokens cached positions."""
    hd = c["d"] // c["hq"]
    per_layer = c["d"] * (c["hq"] + 2 * c["hkv"]) * hd + c["hq"] * hd * c["d"] + 3 * c["d"] * c["ffn"]
    weights = (c["layers"] * per_layer + c["d"] * c["vocab"]) * 2
    return weights + c["layers"] * 2 * c["hkv"] * hd * 2 * kv_tokens


def llama_workload(torch, dev, prompt_len=512, n_new=128, reps=3):
    """random-init Llama-style 1B decoder (16 layers, d 2048,
    32 q / 8 kv heads, head_dim 64, FFN 5632 SwiGLU, vocab 32000), bf16; a
    512-token uniform-random prompt, then 128 greedy tokens (softmax + top-1).
    Prefill runs eagerly; each decode step is one HIP-graph replay."""
    from kuillm_amd.decoder import LlamaDecoder, LlamaShape
    c = LLAMA1B
    shape = LlamaShape(**c)
    dec = LlamaDecoder(shape, llama_state(torch, c, dev), capacity=prompt_len + n_new, device=dev)
    prompt = torch.randint(0, c["vocab"], (1, prompt_len), generator=torch.Generator().manual_seed(0))
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    dec.generate(prompt, n_new)                              # warm-up + graph capture
    pre_ms, dec_ms = [], []
    for _ in range(reps):
        torch.cuda.synchronize()
        a, b, e = ev(), ev(), ev()
        a.record()
        dec.prefill(prompt)
        b.record()
        dec.decode(n_new)
        e.record()
        torch.cuda.synchronize()
        pre_ms.append(a.elapsed_time(b))
        dec_ms.append(b.elapsed_time(e))
    pre, dms = min(pre_ms), min(dec_ms)
    step_ms = dms / (n_new - 1)
    tok_s = 1e3 / step_ms
    # bytes of the average step: KV grows from prompt_len + 1 to prompt_len + n_new - 1 keys
    step_bytes = llama_decode_bytes(c, prompt_len + n_new / 2)
    gbs = step_bytes * tok_s / 1e9
    flops_prefill = 2 * prompt_len * (llama_decode_bytes(c, 0) / 2) + \
        c["layers"] * 2 * 2 * c["hq"] * (c["d"] // c["hq"]) * prompt_len * prompt_len / 2
    del dec
    return {"value": round(tok_s, 1), "unit": "tokens/s", "decode_ms_per_token": round(step_ms, 4),
            "prefill_ms": round(pre, 3), "prefill_tokens_per_s": round(prompt_len / pre * 1e3, 1),
            "prefill_tflops": round(flops_prefill / (pre * 1e-3) / 1e12, 1),
            "end_to_end_tokens_per_s": round(n_new / ((pre + dms) * 1e-3), 1),
            "decode_bytes_per_token": int(step_bytes),
            "roofline": roofline("hbm", gbs, "GB/s"),
            "config": "random-init Llama-style 1B (16 x d2048, GQA 32/8, hd 64, FFN 5632, vocab 32000), "
                      "bf16, batch 1, 512-token prompt, 128 greedy tokens"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the kuiops hot "
              "path has no multi-GPU code -- run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from kuillm_amd import compile as _compile
    from kuillm_amd import ops
    _compile.load_library()                 # fails loudly when libkuiops.so is missing
    dev = torch.device("cuda:0")
    if args.profile_kernels:
        profile_kernels(torch, ops, dev)
        return

    # ---- headline: BASELINE config 2, bf16 addmm 4096^3 with a 1-D bias
    g = torch.Generator(device=dev).manual_seed(0)
    A = torch.randn(4096, 4096, device=dev, generator=g).to(torch.bfloat16)
    B = (torch.randn(4096, 4096, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(4096, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    ms = graph_time_ms(torch, lambda: ops.addmm(bias, A, B), args.steps, args.warmup, reps=10)
    flops = 2 * 4096 ** 3
    tflops = flops / (ms * 1e-3) / 1e12
    line = {
        "metric": "bf16 TFLOP/s (GEMM, SDPA) + decode tokens/s, % of MI355X roofline",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) / N(0,0.02) tensors, resident in HBM)",
        "config": {"workload": "prefill addmm bf16 bias[4096] + A[4096,4096] @ B[4096,4096], fp32 accumulate",
                   "M": 4096, "N": 4096, "K": 4096, "b_layout": "row-major [K,N]", "parallelism": "single GPU"},
        "roofline": roofline("mfma", tflops, "TFLOP/s", traffic_bytes("addmm_4096")),
    }
    del A, B, bias
    if not args.no_extra:
        line["workloads"] = extra_workloads(torch, ops, args.steps, args.warmup, dev)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
