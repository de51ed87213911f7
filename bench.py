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
time per kernel.  The default W = 200 (about 0.2 s of addmm) lets the GPU's
clocks settle under the load: with W = 10 the same kernel measures ~2% slower
(and causal SDPA S=2048 ~8%), the clocks still ramping from the previous,
lighter workload.

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
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/hbm_traffic.{json,md} from two rocprofv3 --pmc runs of "
                         "--profile-kernels (FETCH_SIZE, then WRITE_SIZE); no GPU needed")
    ap.add_argument("--summarize-busy", metavar="DIR",
                    help="write profiles/mfma_busy.{md,json} from a rocprofv3 --pmc run of --profile-kernels "
                         "with SQ_VALU_MFMA_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("DIR", "OUT_MD"),
                    help="write a kernel-duration table from a rocprofv3 --kernel-trace run")
    ap.add_argument("--command", default="", help="the profiling command, recorded in the summary")
    ap.add_argument("--profile-decode-step", action="store_true",
                    help="run 4 one-token persistent decode steps of BASELINE config 5 (512-token prompt), "
                         "one dispatch each, for rocprofv3 --pmc passes")
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


BUSY_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "mfma_busy.json")


def mfma_busy(segment):
    """MFMA-pipe busy fraction of the segment's longest kernel from the
    committed counter summary (profiles/mfma_busy.json), or None."""
    try:
        with open(BUSY_FILE) as f:
            return json.load(f)["segments"][segment]["mfma_busy"]
    except (OSError, ValueError, KeyError):
        return None


def roofline(bound, achieved, unit, traffic=None, segment=None):
    peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
    r = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4), "traffic": traffic}
    if bound == "mfma" and segment:
        r["mfma_busy_counter"] = mfma_busy(segment)
    return r


# Workloads of ``--profile-kernels``, in launch order.  Each segment's steps
# sit between two torch.cuda._sleep markers ("spin_kernel" dispatches) so that
# the counter summaries can split the dispatch list without knowing how many
# kernels a segment launches; every segment runs its step PROFILE_REPS times.
PROFILE_REPS = 3
PROFILE_SEGMENTS = ("addmm_4096", "decode_gemm_M1", "decode_gemm_M4", "decode_gemm_M16",
                    "sdpa_causal_S2048", "sdpa_causal_S4096", "sdpa_decode_kv4096",
                    "bmm_32x2048x128x2048", "llama1b_decode_token", "llama1b_b8_decode_step",
                    "llama1b_b64_decode_step", "copy_256MiB")
# algorithmic HBM bytes per step of each segment (the "achieved" numerators)
ALGO_BYTES = {
    "addmm_4096": 3 * 4096 * 4096 * 2 + 4096 * 2,
    "decode_gemm_M1": 4096 * 11008 * 2 + 1 * (4096 + 11008) * 2,
    "decode_gemm_M4": 4096 * 11008 * 2 + 4 * (4096 + 11008) * 2,
    "decode_gemm_M16": 4096 * 11008 * 2 + 16 * (4096 + 11008) * 2,
    "sdpa_causal_S2048": 4 * 32 * 2048 * 128 * 2,
    "sdpa_causal_S4096": 4 * 32 * 4096 * 128 * 2,
    "sdpa_decode_kv4096": 2 * 32 * 4096 * 128 * 2,
    "bmm_32x2048x128x2048": 2 * 32 * 2048 * 128 * 2 + 32 * 2048 * 2048 * 2,
    "copy_256MiB": 2 * 256 * 2 ** 20,
}
# the profiled decode step runs after a 512-token prefill: 513 cached keys
ALGO_BYTES["llama1b_decode_token"] = None     # filled in below, after llama_decode_bytes
ALGO_BYTES["llama1b_b8_decode_step"] = ALGO_BYTES["llama1b_b64_decode_step"] = None


def profile_kernels(torch, ops, dev):
    """The steps of every measured workload, PROFILE_REPS times each, one
    segment per entry of PROFILE_SEGMENTS (marker first), for rocprofv3
    --pmc runs; the last segment is a 256 MiB device copy whose byte counts
    calibrate FETCH_SIZE / WRITE_SIZE.  The Llama segment is one eager
    decode step (every kernel of one token) after a 512-token prefill."""
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16

    def segment(name, step):
        step()                               # allocations and first-touch outside the segment
        torch.cuda.synchronize()
        torch.cuda._sleep(1000)              # marker: segment starts
        for _ in range(PROFILE_REPS):
            step()
        torch.cuda._sleep(1000)              # marker: segment ends
        torch.cuda.synchronize()
        print(f"profile segment {name} done", flush=True)

    A = torch.randn(4096, 4096, device=dev, generator=g).to(bf)
    B = (torch.randn(4096, 4096, device=dev, generator=g) * 0.02).to(bf)
    bias = (torch.randn(4096, device=dev, generator=g) * 0.02).to(bf)
    segment("addmm_4096", lambda: ops.addmm(bias, A, B))
    del A, B, bias
    W = (torch.randn(4096, 11008, device=dev, generator=g) * 0.02).to(bf)
    for M in (1, 4, 16):
        x = torch.randn(M, 4096, device=dev, generator=g).to(bf)
        segment(f"decode_gemm_M{M}", lambda: ops.mm(x, W))
    del W
    for S in (2048, 4096):
        q, k, v = (torch.randn(1, 32, S, 128, device=dev, generator=g).to(bf) for _ in range(3))
        segment(f"sdpa_causal_S{S}", lambda: ops.sdpa(q, k, v, is_causal=True))
    qd = torch.randn(1, 32, 1, 128, device=dev, generator=g).to(bf)
    segment("sdpa_decode_kv4096", lambda: ops.sdpa(qd, k, v))
    del q, k, v
    A3 = torch.randn(32, 2048, 128, device=dev, generator=g).to(bf)
    B3 = torch.randn(32, 128, 2048, device=dev, generator=g).to(bf)
    segment("bmm_32x2048x128x2048", lambda: ops.bmm(A3, B3))
    del A3, B3
    from kuillm_amd.decoder import LlamaDecoder, LlamaShape
    c = LLAMA1B
    dec = LlamaDecoder(LlamaShape(**c), llama_state(torch, c, dev), capacity=512 + 128, device=dev)
    dec.prefill(torch.randint(0, c["vocab"], (1, 512), generator=torch.Generator().manual_seed(0)))
    segment("llama1b_decode_token", dec._decode_step)
    del dec
    for n in (8, 64):
        dec = LlamaDecoder(LlamaShape(**c), llama_state(torch, c, dev), capacity=512 + 128, batch=n, device=dev)
        dec.prefill(torch.randint(0, c["vocab"], (n, 512), generator=torch.Generator().manual_seed(0)))
        segment(f"llama1b_b{n}_decode_step", dec._decode_step)
        del dec
    src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    segment("copy_256MiB", lambda: dst.copy_(src))


# ------------------------------------------------ rocprofv3 output summaries

def _find_csv(directory, suffix):
    import glob
    hits = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not hits:
        raise SystemExit(f"no *{suffix} under {directory}")
    return hits[0]


def read_counter_dispatches(directory):
    """[(kernel name, {counter: value summed over the dispatch})] in dispatch
    order, from the *_counter_collection.csv of a rocprofv3 --pmc run."""
    import csv
    per = {}
    with open(_find_csv(directory, "counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            d = per.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], {}])
            name = r["Counter_Name"]
            d[1][name] = d[1].get(name, 0.0) + float(r["Counter_Value"])
    return [tuple(per[k]) for k in sorted(per)]


def split_segments(dispatches):
    """Group the dispatches of a ``--profile-kernels`` run by segment: spin_kernel
    markers come in pairs around the steps of each name of PROFILE_SEGMENTS;
    dispatches outside a pair (input set-up) belong to no segment."""
    segs, cur = {}, None
    names = iter(PROFILE_SEGMENTS)
    for kernel, counters in dispatches:
        if "spin_kernel" in kernel:
            if cur is None:
                cur = next(names)
                segs[cur] = []
            else:
                cur = None
        elif cur is not None:
            segs[cur].append((kernel, counters))
    missing = [n for n in PROFILE_SEGMENTS if n not in segs]
    if missing:
        raise SystemExit(f"profile run incomplete: segments {missing} have no marker")
    return segs


def _short(kernel, n=60):
    k = kernel.split("(")[0]
    return k if len(k) <= n else k[:n] + "..."


def summarize_traffic(fetch_dir, write_dir, out_json, out_md, command):
    """Per-step HBM bytes of every segment from a FETCH_SIZE run and a
    WRITE_SIZE run, scaled by what the counters read for the 256 MiB copy."""
    F = split_segments(read_counter_dispatches(fetch_dir))
    Wr = split_segments(read_counter_dispatches(write_dir))

    def per_step(seg, counter):
        return sum(c.get(counter, 0.0) for _, c in seg) / PROFILE_REPS

    copy_bytes_kib = 256 * 1024
    fscale = copy_bytes_kib / per_step(F["copy_256MiB"], "FETCH_SIZE")
    wscale = copy_bytes_kib / per_step(Wr["copy_256MiB"], "WRITE_SIZE")
    res = {"fetch_scale": fscale, "write_scale": wscale,
           "calibration": f"256 MiB device copy: FETCH_SIZE {copy_bytes_kib / fscale:.1f} KiB, "
                          f"WRITE_SIZE {copy_bytes_kib / wscale:.1f} KiB per dispatch",
           "command": command, "kernels": {}}
    rows = []
    for name in PROFILE_SEGMENTS[:-1]:
        fk, wk = per_step(F[name], "FETCH_SIZE"), per_step(Wr[name], "WRITE_SIZE")
        top = max(F[name], key=lambda kc: kc[1].get("FETCH_SIZE", 0.0))[0] if F[name] else ""
        res["kernels"][name] = {"kernel": top, "fetch_kib": round(fk, 3), "write_kib": round(wk, 3),
                                "dispatches_per_step": len(F[name]) // PROFILE_REPS}
        t = fk * 1024 * fscale + wk * 1024 * wscale
        alg = ALGO_BYTES.get(name)
        rows.append(f"| {name} | {len(F[name]) // PROFILE_REPS} | `{_short(top)}` | {fk:.1f} | {wk:.1f} | "
                    f"{t / 2 ** 20:.1f} MiB | " + (f"{alg / 2 ** 20:.1f} MiB | {t / alg:.2f} |" if alg else "— | — |"))
    with open(out_json, "w") as f:
        json.dump(res, f, indent=1)
    with open(out_md, "w") as f:
        f.write("# HBM traffic per step (rocprofv3 FETCH_SIZE / WRITE_SIZE)\n\nCommands (repository root):\n\n```\n"
                f"{command}\n```\n\n{res['calibration']}; scale factors fetch x{fscale:.3f}, write x{wscale:.3f}. "
                "FETCH_SIZE counts what leaves the L2, so MALL hits count as HBM traffic here.\n\n"
                "| segment | dispatches / step | largest kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic (scaled) | "
                "algorithmic bytes | ratio |\n|---|---|---|---|---|---|---|---|\n" + "\n".join(rows) + "\n")
    print("\n".join(rows))


N_XCD, N_SIMD = 8, 256 * 4      # MI355X: 8 XCDs, 256 CUs x 4 SIMDs


def summarize_busy(directory, out_md, command):
    """MFMA-pipe busy fraction and LDS bank conflicts of every segment's
    kernels from a run with SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE,
    SQ_LDS_BANK_CONFLICT and SQ_LDS_IDX_ACTIVE.  GRBM_GUI_ACTIVE is summed
    over the 8 XCDs (per-XCD cycles = value / 8) and the MFMA busy count over
    the 1024 SIMDs, so busy = (MFMA / 1024) / (GRBM / 8)."""
    segs = split_segments(read_counter_dispatches(directory))
    rows, busy_json = [], {"command": command, "segments": {}}
    for name in PROFILE_SEGMENTS[:-1]:
        kern = {}
        for k, c in segs[name]:
            a = kern.setdefault(k, {"n": 0})
            a["n"] += 1
            for ck, v in c.items():
                a[ck] = a.get(ck, 0.0) + v
        ranked = sorted(kern.items(), key=lambda kv: -kv[1].get("GRBM_GUI_ACTIVE", 0.0))
        for k, a in ranked[:2]:
            n = a["n"]
            grbm = a.get("GRBM_GUI_ACTIVE", 0.0) / n / N_XCD
            mfma = a.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / n / N_SIMD
            conf = a.get("SQ_LDS_BANK_CONFLICT", 0.0) / n
            lds = a.get("SQ_LDS_IDX_ACTIVE", 0.0) / n
            busy = mfma / grbm if grbm else 0.0
            rows.append(f"| {name} | `{_short(k)}` | {n // PROFILE_REPS} | {grbm:.0f} | {mfma:.0f} | {busy:.3f} | "
                        f"{conf:.0f} | {(conf / lds if lds else 0.0):.4f} |")
            busy_json["segments"].setdefault(name, {"kernel": k, "mfma_busy": round(busy, 4),
                                                    "lds_bank_conflict_ratio": round(conf / lds, 5) if lds else None})
    with open(out_md[:-3] + ".json" if out_md.endswith(".md") else out_md + ".json", "w") as f:
        json.dump(busy_json, f, indent=1)
    with open(out_md, "w") as f:
        f.write("# MFMA busy and LDS bank conflicts (rocprofv3 counters)\n\nCommand (repository root):\n\n```\n"
                f"{command}\n```\n\nPer dispatch: GRBM_GUI_ACTIVE / 8 XCDs = active cycles; "
                "SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs = MFMA-busy cycles per SIMD; busy = their ratio. "
                "LDS conflict ratio = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.\n\n"
                "| segment | kernel | dispatches / step | active cycles | MFMA busy cycles / SIMD | MFMA busy | "
                "LDS bank-conflict cycles | conflict ratio |\n|---|---|---|---|---|---|---|---|\n"
                + "\n".join(rows) + "\n")
    print("\n".join(rows))


def summarize_trace(directory, out_md, command, top=40):
    """Kernel durations from a rocprofv3 --kernel-trace run: per kernel and
    grid, calls / average / min / max microseconds and share of GPU time."""
    import csv
    groups = {}
    with open(_find_csv(directory, "kernel_trace.csv")) as f:
        for r in csv.DictReader(f):
            wx = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
            wy = int(r["Grid_Size_Y"]) // max(1, int(r["Workgroup_Size_Y"]))
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
            groups.setdefault((r["Kernel_Name"], wx, wy), []).append(us)
    total = sum(sum(v) for v in groups.values()) or 1.0
    items = sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]
    rows = [f"| `{_short(k, 90)}` | {wx}, {wy} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
            f"{100 * sum(v) / total:.1f} |" for (k, wx, wy), v in items]
    with open(out_md, "w") as f:
        f.write("# Kernel durations (rocprofv3 kernel trace)\n\nCommand (repository root):\n\n```\n"
                f"{command}\n```\n\n| kernel | grid x, y (work-groups) | calls | avg us | min us | max us | "
                "% of GPU time |\n|---|---|---|---|---|---|---|\n" + "\n".join(rows) + "\n")
    print("\n".join(rows[:15]))


def _cpu_median(fn, seconds, max_calls=50):
    fn()                                          # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < max_calls):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def cpu_baseline(torch, seconds):
    """The reference's CPU path -- stock torch aten on the host cores; its
    families never take CPU tensors (kuipy/kuiops.py:531) -- on the headline
    addmm shape in fp32 (``value``), and on BASELINE config 0, the
    GPT-2-small MLP up-projection x[64,768] @ W[768,3072] + bias[3072]
    (``config0``).  ``cores`` is the number of threads torch used;
    ``host_cpus`` / ``affinity_cpus`` are what the box offers."""
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    A = torch.randn(4096, 4096, generator=g)
    B = torch.randn(4096, 4096, generator=g) * 0.02
    bias = torch.randn(4096, generator=g) * 0.02
    med, n = _cpu_median(lambda: torch.addmm(bias, A, B), seconds * 0.7)
    del A, B, bias
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 768, generator=g)
    W = torch.randn(768, 3072, generator=g) * 0.02
    b0 = torch.randn(3072, generator=g) * 0.02
    med0, n0 = _cpu_median(lambda: torch.addmm(b0, x, W), seconds * 0.3, max_calls=2000)
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"value": round(2 * 4096 ** 3 / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "host_cpus": os.cpu_count(), "affinity_cpus": affinity, "kind": "reference",
            "sample": f"stock torch {torch.__version__} CPU fp32 addmm bias[4096] + A[4096,4096] @ "
                      f"B[4096,4096], median of {n} calls ({med * 1e3:.1f} ms each)",
            "config0": {"value": round(2 * 64 * 768 * 3072 / med0 / 1e9, 2), "unit": "GFLOP/s",
                        "us_per_call": round(med0 * 1e6, 1),
                        "sample": f"BASELINE config 0: fp32 addmm bias[3072] + x[64,768] @ W[768,3072], "
                                  f"seed 0, median of {n0} calls"}}


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
                                    "roofline": roofline("mfma", tf, "TFLOP/s", traffic_bytes(f"sdpa_causal_S{S}"),
                                                         f"sdpa_causal_S{S}")}
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
    out["llama1b_greedy_batch8"] = llama_workload(torch, dev, batch=8)
    out["llama1b_greedy_batch64"] = llama_workload(torch, dev, batch=64, reps=2)
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


ALGO_BYTES["llama1b_decode_token"] = llama_decode_bytes(LLAMA1B, 513)
for _n in (8, 64):      # batched steps: the weights once, every sequence's 513 keys
    ALGO_BYTES[f"llama1b_b{_n}_decode_step"] = llama_decode_bytes(LLAMA1B, 0) + _n * (
        llama_decode_bytes(LLAMA1B, 513) - llama_decode_bytes(LLAMA1B, 0))


def llama_workload(torch, dev, prompt_len=512, n_new=128, reps=3, batch=1):
    """random-init Llama-style 1B decoder (16 layers, d 2048,
    32 q / 8 kv heads, head_dim 64, FFN 5632 SwiGLU, vocab 32000), bf16; a
    512-token uniform-random prompt per sequence, then 128 greedy tokens
    (softmax + top-1).  Prefill runs eagerly; each decode step is one
    HIP-graph replay.  ``batch`` > 1 decodes that many sequences together
    (the reference app's batched generate)."""
    from kuillm_amd.decoder import LlamaDecoder, LlamaShape
    c = LLAMA1B
    shape = LlamaShape(**c)
    dec = LlamaDecoder(shape, llama_state(torch, c, dev), capacity=prompt_len + n_new, batch=batch, device=dev)
    prompt = torch.randint(0, c["vocab"], (batch, prompt_len), generator=torch.Generator().manual_seed(0))
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
    tok_s = batch * 1e3 / step_ms
    # bytes of the average step: the weights once, plus every sequence's KV
    # (growing from prompt_len + 1 to prompt_len + n_new - 1 keys)
    kv = llama_decode_bytes(c, prompt_len + n_new / 2) - llama_decode_bytes(c, 0)
    step_bytes = llama_decode_bytes(c, 0) + batch * kv
    gbs = step_bytes / (step_ms * 1e-3) / 1e9
    flops_prefill = batch * (2 * prompt_len * (llama_decode_bytes(c, 0) / 2) +
                             c["layers"] * 2 * 2 * c["hq"] * (c["d"] // c["hq"]) * prompt_len * prompt_len / 2)
    mode = (f"batch-1 persistent ({dec.steps_per_launch} steps per launch)" if dec.persistent else "batch-1 fused") if dec.fused else \
        ("batched fused (LDS-staged rows)" if dec.fused_batched else ("batched wide" if dec.fused_wide else "unfused"))
    del dec
    out = {"value": round(tok_s, 1), "unit": "tokens/s", "decode_ms_per_step": round(step_ms, 4),
           "prefill_ms": round(pre, 3), "prefill_tokens_per_s": round(batch * prompt_len / pre * 1e3, 1),
           "prefill_tflops": round(flops_prefill / (pre * 1e-3) / 1e12, 1),
           "end_to_end_tokens_per_s": round(batch * n_new / ((pre + dms) * 1e-3), 1),
           "decode_bytes_per_step": int(step_bytes), "decode_path": mode,
           "roofline": roofline("hbm", gbs, "GB/s", traffic_bytes("llama1b_decode_token" if batch == 1 else
                                                                  f"llama1b_b{batch}_decode_step")),
           "config": "random-init Llama-style 1B (16 x d2048, GQA 32/8, hd 64, FFN 5632, vocab 32000), "
                     f"bf16, batch {batch}, 512-token prompt, 128 greedy tokens"}
    if batch == 1:
        out["decode_ms_per_token"] = out["decode_ms_per_step"]
    return out


def main():
    args = parse()
    prof = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic, TRAFFIC_FILE, os.path.join(prof, "hbm_traffic.md"),
                          args.command)
        return
    if args.summarize_busy:
        summarize_busy(args.summarize_busy, os.path.join(prof, "mfma_busy.md"), args.command)
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace, args.command)
        return
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
    if args.profile_decode_step:
        from kuillm_amd.decoder import LlamaDecoder, LlamaShape
        dec = LlamaDecoder(LlamaShape(**LLAMA1B), llama_state(torch, LLAMA1B, dev), capacity=640, device=dev)
        if not dec.persistent:
            sys.exit("bench.py: the persistent decode step is not available on this device")
        dec.prefill(torch.randint(0, LLAMA1B["vocab"], (1, 512), generator=torch.Generator().manual_seed(0)))
        torch.cuda.synchronize()
        for _ in range(4):
            dec._decode_step_fused(1)
        dec.check_step_error()
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
        "roofline": roofline("mfma", tflops, "TFLOP/s", traffic_bytes("addmm_4096"), "addmm_4096"),
    }
    del A, B, bias
    if not args.no_extra:
        line["workloads"] = extra_workloads(torch, ops, args.steps, args.warmup, dev)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
