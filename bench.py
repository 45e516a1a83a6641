#!/usr/bin/env python3
"""Benchmark of the fused NF4 + multi-LoRA linear on one MI355X.

Headline (``value``): the north-star decode linear -- NF4 4096 -> 4096
(block 64, fp32 absmax), 32 rank-16 bf16 adapters, B = 64 tokens with per-token
adapter ids uniform in [0, 32) and 10 % base-only tokens -- as achieved HBM
GB/s over the algorithmic bytes of one call:
    N*K/2 (packed) + N*K/16 (fp32 absmax) + 2*B*K (x) + 2*B*N (y)
    + U * (2*r*K + 2*N*r)  (A and B of the U distinct adapters used).
One step = one call (one kernel launch). Calls are captured in a HIP graph
that cycles through 64 independent copies of the weight and the adapter set
(> 1 GB in total, four times the 256 MB Infinity Cache), so every call
streams from HBM; inputs are resident in HBM before timing starts.
Also reported: the B = 1..64 sweep (us/call, GB/s, fraction of 8 TB/s), the
same linear without adapters at B = 1 and 64 (U = 0), the c5 prefill (M=2048, K=4096, N=11008, NF4 + double quant, 8 segments of rank
32) in TFLOP/s against 2.5 PFLOP/s, and the reference's PyTorch CPU path on
the host cores (cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
N_FEAT = 4096
K_FEAT = 4096
ADAPTERS = 32
RANK = 16
LAYERS = 64


TRAFFIC_FILE = ROOT / "profiles" / "decode_hbm_traffic.json"


def measured_traffic(batch: int):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    counter runs (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter
    reads for a plain copy of known size), or None when not measured for this
    batch."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    if int(rec.get("batch", -1)) != batch:
        return None
    return int(rec["traffic_bytes_per_launch"])


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def metric_name() -> str:
    try:
        return json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    except (OSError, ValueError, KeyError):
        return "NF4+multi-LoRA linear: HBM GB/s (% peak) & us/call at B=1..64; prefill TFLOP/s"


def decode_bytes(batch: int, used: int, n: int = N_FEAT, k: int = K_FEAT, rank: int = RANK) -> int:
    return n * k // 2 + n * k // 16 + 2 * batch * k + 2 * batch * n + used * (2 * rank * k + 2 * n * rank)


class DecodeWorkload:
    """64 resident copies of an NF4 weight and of a 32-adapter table."""

    def __init__(self, device, layers: int = LAYERS, n: int = N_FEAT, k: int = K_FEAT):
        import torch

        from loraforge_amd.ops import quantize_nf4

        self.device, self.layers, self.n, self.k = device, layers, n, k
        g = torch.Generator(device="cpu").manual_seed(731)
        w = (torch.randn(n, k, generator=g) * 0.02).bfloat16().to(device)
        q, st = quantize_nf4(w)
        self.states = []
        for _ in range(layers):
            self.states.append((q.clone(), type(st)(st.absmax.clone(), st.shape, st.code, st.dtype)))
        a = (torch.randn(ADAPTERS * RANK * k, generator=g) * 0.02).bfloat16()
        b = (torch.randn(ADAPTERS * n * RANK, generator=g) * 0.02).bfloat16()
        self.a_stores = [a.to(device) for _ in range(layers)]
        self.b_stores = [b.to(device) for _ in range(layers)]
        i64 = dict(dtype=torch.int64, device=device)
        self.a_offsets = torch.arange(ADAPTERS, **i64) * (RANK * k)
        self.b_offsets = torch.arange(ADAPTERS, **i64) * (n * RANK)
        self.b_strides = torch.full((ADAPTERS,), RANK, dtype=torch.int32, device=device)
        self.ranks = torch.full((ADAPTERS,), RANK, dtype=torch.int32, device=device)
        self.scales = torch.full((ADAPTERS,), 2.0, dtype=torch.float32, device=device)
        self.slices = torch.tensor([0, n], dtype=torch.int32, device=device)
        torch.cuda.synchronize()

    def batch(self, batch: int, seed: int):
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        x = torch.randn(batch, self.k, generator=g).bfloat16().to(self.device)
        slots = torch.randint(0, ADAPTERS, (batch,), generator=g, dtype=torch.int32)
        slots[torch.rand(batch, generator=g) < 0.1] = -1
        used = int(torch.unique(slots[slots >= 0]).numel())
        return x, slots.to(self.device), used

    def lora(self, layer: int, slots):
        from loraforge_amd.ops import LoraBatch

        return LoraBatch(
            self.a_stores[layer],
            self.a_offsets,
            self.b_stores[layer],
            self.b_offsets,
            self.b_strides,
            self.ranks,
            self.scales,
            slots,
            self.slices,
            max_rank=RANK,
        )


def graph_of(calls, stream):
    """Capture ``calls`` (list of thunks) into one HIP graph on ``stream``."""
    import torch

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for fn in calls:
            fn()
    return graph


def timed_replays(graph_full, reps: int, graph_tail, stream):
    """Wall-clock and HIP-event time of ``reps`` full replays (+ optional tail)."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            graph_full.replay()
        if graph_tail is not None:
            graph_tail.replay()
        end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) / 1e3


def run_decode(work: DecodeWorkload, batch: int, steps: int, warmup: int, seed: int, lora: bool = True):
    import torch

    from loraforge_amd.ops import nf4_lora_linear

    x, slots, used = work.batch(batch, seed)
    out = torch.empty(batch, work.n, dtype=torch.bfloat16, device=work.device)
    loras = [work.lora(layer, slots) if lora else None for layer in range(work.layers)]
    used = used if lora else 0

    def call(layer):
        q, st = work.states[layer]
        return lambda: nf4_lora_linear(x, q, st, lora=loras[layer], out=out)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for layer in range(work.layers):
            call(layer)()
    torch.cuda.synchronize()
    full = graph_of([call(layer) for layer in range(work.layers)], stream)
    tail_n = steps % work.layers
    tail = graph_of([call(layer) for layer in range(tail_n)], stream) if tail_n else None
    reps = steps // work.layers
    warm_reps = max(1, -(-warmup // work.layers))
    with torch.cuda.stream(stream):
        for _ in range(warm_reps):
            full.replay()
    torch.cuda.synchronize()
    wall, gpu = timed_replays(full, reps, tail, stream)
    per_call = gpu / steps
    nbytes = decode_bytes(batch, used)
    return dict(
        batch=batch,
        adapters_used=used,
        bytes_per_call=nbytes,
        us_per_call=per_call * 1e6,
        wall_ms_per_step=wall / steps * 1e3,
        gbps=nbytes / per_call / 1e9,
        frac=nbytes / per_call / 1e9 / PEAK_HBM_GBS,
    )


def run_prefill(device, calls: int = 4, reps: int = 5):
    import torch

    from loraforge_amd.ops import LoraBatch, nf4_lora_linear, quantize_nf4

    m, n, k, rank, segs = 2048, 11008, 4096, 32, 8
    g = torch.Generator(device="cpu").manual_seed(735)
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16().to(device)
    q, st = quantize_nf4(w, compress_statistics=True)
    del w
    x = torch.randn(m, k, generator=g).bfloat16().to(device)
    cuts = torch.sort(torch.randperm(m - 1, generator=g)[: segs - 1] + 1).values
    lengths = torch.diff(torch.cat([torch.tensor([0]), cuts, torch.tensor([m])]))
    slots = torch.repeat_interleave(torch.arange(segs, dtype=torch.int32), lengths).to(device)
    a = (torch.randn(segs * rank * k, generator=g) * 0.02).bfloat16().to(device)
    b = (torch.randn(segs * n * rank, generator=g) * 0.02).bfloat16().to(device)
    i64 = dict(dtype=torch.int64, device=device)
    lora = LoraBatch(
        a,
        torch.arange(segs, **i64) * (rank * k),
        b,
        torch.arange(segs, **i64) * (n * rank),
        torch.full((segs,), rank, dtype=torch.int32, device=device),
        torch.full((segs,), rank, dtype=torch.int32, device=device),
        torch.full((segs,), 2.0, device=device),
        slots,
        torch.tensor([0, n], dtype=torch.int32, device=device),
        max_rank=rank,
    )
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    flops_base = 2 * m * n * k
    flops = flops_base + 2 * m * k * rank + 2 * m * rank * n
    results = {}
    for name, lo in (("fused", lora), ("base_only", None)):
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            nf4_lora_linear(x, q, st, lora=lo, out=out)
        torch.cuda.synchronize()
        graph = graph_of([lambda lo=lo: nf4_lora_linear(x, q, st, lora=lo, out=out)] * calls, stream)
        with torch.cuda.stream(stream):
            graph.replay()
        _, gpu = timed_replays(graph, reps, None, stream)
        per = gpu / (reps * calls)
        f = flops if lo is not None else flops_base
        results[name] = dict(us_per_call=per * 1e6, tflops=f / per / 1e12, frac=f / per / 1e12 / PEAK_BF16_TFLOPS)
    return dict(
        config=dict(m=m, n=n, k=k, segments=segs, rank=rank, double_quant=True, segment_lengths=lengths.tolist()),
        flops=flops,
        **results,
    )


def cpu_baseline(batch: int, budget_s: float):
    """The reference chain on the host cores (PyTorch CPU), bounded sample."""
    import torch

    from oracle import cpu_path

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    out = {}
    for name, b, adapters, share in (("headline", batch, ADAPTERS, 0.7), ("c1", 1, 1, 0.3)):
        inp = cpu_path.make_inputs(b, N_FEAT, K_FEAT, adapters, RANK, seed=731 + b)
        used = int(torch.unique(inp["slots"][inp["slots"] >= 0]).numel())
        cpu_path.reference_call(**inp)
        times = []
        t_end = time.perf_counter() + budget_s * share
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 500):
            t = time.perf_counter()
            cpu_path.reference_call(**inp)
            times.append(time.perf_counter() - t)
        med = statistics.median(times)
        out[name] = dict(batch=b, adapters_used=used, calls=len(times), us_per_call=med * 1e6, gbps=decode_bytes(b, used) / med / 1e9)
    return out, cores, model


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=640)
    parser.add_argument("--warmup", type=int, default=64)
    parser.add_argument("--batch", type=int, default=64)
    parser.add_argument("--only", action="store_true", help="headline decode only (no sweep/prefill/CPU)")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-prefill", action="store_true")
    parser.add_argument("--prefill-only", action="store_true", help="c5 prefill only (JSON of its timings)")
    parser.add_argument("--cpu-seconds", type=float, default=12.0)
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    import torch

    device = torch.device("cuda:0")
    if args.prefill_only:
        pre = run_prefill(device)
        log(f"prefill c5: {pre['fused']['us_per_call']:.1f} us/call, {pre['fused']['tflops']:.1f} TFLOP/s ({pre['fused']['frac']:.1%})")
        print(json.dumps(pre), flush=True)
        return 0
    log(f"device {torch.cuda.get_device_name(0)}; building {LAYERS} weight/adapter copies")
    work = DecodeWorkload(device)
    log(f"headline decode B={args.batch}: warmup {args.warmup}, steps {args.steps}")
    t0 = time.perf_counter()
    head = run_decode(work, args.batch, args.steps, args.warmup, seed=731 + args.batch)
    timed_wall = time.perf_counter() - t0
    log(f"headline {head['us_per_call']:.2f} us/call, {head['gbps']:.0f} GB/s ({head['frac']:.1%} of peak)")
    result = {
        "metric": metric_name(),
        "value": round(head["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["wall_ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"fused NF4+multi-LoRA decode linear {N_FEAT}->{K_FEAT}, B={args.batch}, "
            f"{ADAPTERS} rank-{RANK} adapters, 10% base-only tokens",
            "batch": args.batch,
            "n": N_FEAT,
            "k": K_FEAT,
            "adapters": ADAPTERS,
            "rank": RANK,
            "adapters_used": head["adapters_used"],
            "weight_copies": LAYERS,
            "timing": "HIP graph of 64 calls over 64 weight/adapter copies; HIP events on the replay stream",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(head["gbps"], 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(head["frac"], 4),
            "traffic": measured_traffic(args.batch),
            "kernel": "nf4_gemv_kernel",
            "bytes_per_launch": head["bytes_per_call"],
            "us_per_launch": round(head["us_per_call"], 3),
            "timing": "HIP events on the graph-replay stream over the timed calls (includes the graph's "
            "inter-kernel dispatch gap; rocprofv3 kernel durations are in profiles/)",
        },
    }
    if not args.only:
        sweep = {}
        for b in (1, 2, 4, 8, 16, 32, 64):
            r = run_decode(work, b, 640, 64, seed=731 + b)
            sweep[str(b)] = {key: round(r[key], 4) for key in ("us_per_call", "gbps", "frac")} | {"adapters_used": r["adapters_used"]}
            log(f"sweep B={b}: {r['us_per_call']:.2f} us/call, {r['gbps']:.0f} GB/s ({r['frac']:.1%})")
        result["sweep"] = sweep
        base = {}
        for b in (1, 64):
            r = run_decode(work, b, 640, 64, seed=731 + b, lora=False)
            base[str(b)] = {key: round(r[key], 4) for key in ("us_per_call", "gbps", "frac")}
            log(f"base only B={b}: {r['us_per_call']:.2f} us/call, {r['gbps']:.0f} GB/s ({r['frac']:.1%})")
        result["sweep_base_only"] = base
    del work
    torch.cuda.empty_cache()
    if not args.only and not args.no_prefill:
        pre = run_prefill(device)
        result["prefill"] = pre
        log(f"prefill c5: {pre['fused']['us_per_call']:.1f} us/call, {pre['fused']['tflops']:.1f} TFLOP/s ({pre['fused']['frac']:.1%})")
    if not args.only and not args.no_cpu:
        log("cpu baseline (PyTorch CPU restatement of the reference path)")
        cpu, cores, model = cpu_baseline(args.batch, args.cpu_seconds)
        result["cpu_baseline"] = {
            "value": round(cpu["headline"]["gbps"], 4),
            "unit": "GB/s",
            "cores": cores,
            "kind": "port",
            "sample": f"{cpu['headline']['calls']} calls of the B={args.batch} headline workload "
            f"({cpu['headline']['us_per_call']:.0f} us/call median) and {cpu['c1']['calls']} calls of c1 "
            f"(B=1, one rank-16 adapter: {cpu['c1']['us_per_call']:.0f} us/call) on {model or platform.processor()}",
            "c1_us_per_call": round(cpu["c1"]["us_per_call"], 1),
        }
    result["timed_wall_s"] = round(timed_wall, 3)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
