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
streams from HBM; inputs are resident in HBM before timing starts. The
headline times exactly --steps calls after --warmup untimed ones.

``configs`` (unless --only) holds every BASELINE.json configuration, each
timed the same way (graph replays over enough copies to defeat the Infinity
Cache, HIP events on the replay stream) and reported as the median of three
rounds run in shuffled order (the reference's protocol,
benchmarks/check_qwen35_nf4_ops.py:11-41):
  c1          NF4 4096^2, B = 1, one rank-16 adapter;
  north_star  B = 1, 2, 4, ..., 64 (32 rank-16 adapters), also base only and
              with the exact-weights decode arithmetic;
  c2          BF16 row_shrink + row_expand, 64 tokens, 32 x rank 16 (c2_fused:
              the same update by lora_apply in one launch);
  c3          NF4 + double-quant SwiGLU MLP 4096 / 12288 (gate/up, SwiGLU,
              down), 16 rank-8 adapters, B = 1 / 8 / 64; c3_fused_* runs the
              SwiGLU in the gate/up kernel's epilogue (two launches), c3_nested_*
              the same with the kernels reading the double-quant state itself
              (scales="nested") instead of cached fp32 scales;
  c4          NF4 4096^2, 256 tokens, 128 retained-rank adapters
              (ranks {4..64}), Zipf(1.1) routing;
  c5          prefill M = 2048, K = 4096, N = 11008, NF4 + double quant,
              8 segments of rank 32 (TFLOP/s against 2.5 PFLOP/s); c5_swiglu
              reads the weight as a merged gate/up projection (two rank-32
              slices) with the SwiGLU in the GEMM's epilogue, against the
              linear followed by silu_mul (c5_swiglu_two_launches);
  fleet       the Fleet row_expand at the reference's row-tile study shapes
              (docs/qwen35.md:379-386): 32 tokens over four mixed-rank
              adapters, 1024 output columns and QKV 4096/512/512 (warm: the
              same tensors every call, as there);
  dequant     standalone NF4 dequantisation 8192 x 1024 (the reference's
              published operator screen).
``cpu_baseline`` is the reference's chain in PyTorch on the host cores.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import random
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
ROUNDS = 3

TRAFFIC_FILE = ROOT / "profiles" / "decode_hbm_traffic.json"
# The kernel that runs a decode batch of the headline shape (N = K = 4096): 1..8
# tokens the narrow decode kernel, 9..64 the wide one (32 rows x 32 tokens per
# workgroup).
NARROW_SOURCE = ROOT / "loraforge_amd" / "csrc" / "nf4_gemv.hip"
WIDE_SOURCE = ROOT / "loraforge_amd" / "csrc" / "nf4_decode_wide.hip"


def decode_kernel(batch: int) -> tuple[str, Path]:
    # The library's routing at N = K = 4096: the wide kernel above 8 tokens.
    return ("nf4_decode_wide_kernel", WIDE_SOURCE) if batch > 8 else ("nf4_gemv_kernel", NARROW_SOURCE)


def source_digest(path: Path) -> str:
    try:
        return hashlib.sha256(path.read_bytes()).hexdigest()[:16]
    except OSError:
        return ""


def measured_traffic(batch: int):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    counter runs (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter
    reads for a plain copy of known size), or None when they were not taken
    for this batch or for the kernel source being measured now."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    if int(rec.get("batch", -1)) != batch or rec.get("source_sha256_16") != source_digest(decode_kernel(batch)[1]):
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


class Timed:
    """A graph of ``len(calls)`` calls (one per resident copy), replayed ``reps`` times per round."""

    def __init__(self, name, calls, reps, work, unit="GB/s"):
        import torch

        self.name, self.calls, self.reps, self.work, self.unit = name, len(calls), reps, work, unit
        # The graph addresses every tensor the calls touch but holds no reference to
        # them: the thunks (and so their tensors) live as long as the graph.
        self.fns = list(calls)
        self.stream = torch.cuda.Stream()
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            for fn in calls:  # eager warm-up: workspaces and prepared scales exist before capture
                fn()
        torch.cuda.synchronize()
        self.graph = graph_of(calls, self.stream)
        with torch.cuda.stream(self.stream):
            self.graph.replay()
        torch.cuda.synchronize()
        self.samples = []

    def round(self):
        _, gpu = timed_replays(self.graph, self.reps, None, self.stream)
        self.samples.append(gpu / (self.reps * self.calls))

    def result(self):
        per = statistics.median(self.samples)
        rate = self.work / per / (1e9 if self.unit == "GB/s" else 1e12)
        peak = PEAK_HBM_GBS if self.unit == "GB/s" else PEAK_BF16_TFLOPS
        out = {
            "us_per_call": round(per * 1e6, 3),
            "rounds_us": [round(s * 1e6, 3) for s in self.samples],
            ("bytes_per_call" if self.unit == "GB/s" else "flops_per_call"): int(self.work),
            ("gbps" if self.unit == "GB/s" else "tflops"): round(rate, 2),
            "frac": round(rate / peak, 4),
        }
        return out


def run_rounds(items, rounds: int = ROUNDS, seed: int = 0):
    rng = random.Random(seed)
    for r in range(rounds):
        order = list(items)
        rng.shuffle(order)
        for item in order:
            item.round()
        log(f"round {r + 1}/{rounds} done ({len(order)} items)")
    return {item.name: item.result() for item in items}


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

    def batch(self, batch: int, seed: int, null_frac: float = 0.1, adapters: int = ADAPTERS):
        import torch

        g = torch.Generator(device="cpu").manual_seed(seed)
        x = torch.randn(batch, self.k, generator=g).bfloat16().to(self.device)
        slots = torch.randint(0, adapters, (batch,), generator=g, dtype=torch.int32)
        slots[torch.rand(batch, generator=g) < null_frac] = -1
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

    def calls(self, x, slots, out, *, lora=True, exact=False):
        from loraforge_amd.ops import nf4_lora_linear

        loras = [self.lora(layer, slots) if lora else None for layer in range(self.layers)]

        def call(layer):
            q, st = self.states[layer]
            return lambda: nf4_lora_linear(x, q, st, lora=loras[layer], out=out, exact=exact)

        return [call(layer) for layer in range(self.layers)]


def run_headline(work: DecodeWorkload, batch: int, steps: int, warmup: int, seed: int):
    """The driver's contract: ``warmup`` untimed calls, then exactly ``steps`` timed calls."""
    import torch

    x, slots, used = work.batch(batch, seed)
    out = torch.empty(batch, work.n, dtype=torch.bfloat16, device=work.device)
    calls = work.calls(x, slots, out)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for fn in calls:
            fn()
    torch.cuda.synchronize()
    full = graph_of(calls, stream)
    tail_n = steps % work.layers
    tail = graph_of(calls[:tail_n], stream) if tail_n else None
    reps = steps // work.layers
    warm_full, warm_tail = divmod(warmup, work.layers)
    with torch.cuda.stream(stream):
        for _ in range(warm_full):
            full.replay()
        if warm_tail:
            warm = graph_of(calls[:warm_tail], stream)
            warm.replay()
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


def segments_of(routes, max_rows: int = 16):
    """Tokens grouped by slot into row_expand segments of at most 16 rows."""
    import numpy as np

    indptr, seg_slots, order = [0], [], []
    for g in sorted(set(routes) - {-1}):
        tokens = [t for t, r in enumerate(routes) if r == g]
        for i in range(0, len(tokens), max_rows):
            chunk = tokens[i : i + max_rows]
            order += chunk
            seg_slots.append(g)
            indptr.append(indptr[-1] + len(chunk))
    return np.array(indptr, np.int32), np.array(seg_slots, np.int32), np.array(order, np.int32)


def decode_items(work: DecodeWorkload, reps: int, wanted=("c1", "north_star", "c2")):
    """c1, the north-star sweep (with LoRA, base only, exact weights) and c2 (those in ``wanted``)."""
    import torch

    from loraforge_amd.ops import row_expand, row_shrink

    items, meta = [], {}

    def add(name, batch, seed, *, lora=True, exact=False, null_frac=0.1, adapters=ADAPTERS):
        if (name if name == "c1" else "north_star") not in wanted:
            return
        x, slots, used = work.batch(batch, seed, null_frac=null_frac, adapters=adapters)
        used = used if lora else 0
        out = torch.empty(batch, work.n, dtype=torch.bfloat16, device=work.device)
        items.append(Timed(name, work.calls(x, slots, out, lora=lora, exact=exact), reps, decode_bytes(batch, used)))
        meta[name] = dict(batch=batch, adapters_used=used, exact=exact)

    add("c1", 1, 732, null_frac=0.0, adapters=1)
    for b in (1, 2, 4, 8, 16, 32, 64):
        add(f"north_star_b{b}", b, 731 + b)
    for b in (1, 64):
        add(f"base_only_b{b}", b, 731 + b, lora=False)
        add(f"exact_b{b}", b, 731 + b, exact=True)

    if "c2" not in wanted:
        return items, meta
    # c2: the row operators alone on the same 64 adapter copies (A as [32, 16, K]).
    x, slots, used = work.batch(64, 733)
    indptr, seg_slots, order = segments_of(slots.cpu().tolist())
    dev = work.device
    seg = dict(
        segment_indptr=torch.from_numpy(indptr).to(dev),
        segment_slots=torch.from_numpy(seg_slots).to(dev),
        token_indices=torch.from_numpy(order).to(dev),
        segment_count=torch.tensor([len(seg_slots)], dtype=torch.int32, device=dev),
    )
    y = torch.randn(64, work.n, device=dev).bfloat16()
    z = torch.zeros(64, RANK, dtype=torch.bfloat16, device=dev)

    def rows_call(layer):
        a = work.a_stores[layer].view(ADAPTERS, RANK, work.k)

        def fn():
            row_shrink(x, a, z, slots, work.ranks, max_rank=RANK)
            row_expand(
                z, work.b_stores[layer], y, b_offsets=work.b_offsets, b_strides=work.b_strides, ranks=work.ranks,
                scales=work.scales, slice_offsets=work.slices, **seg,
            )

        return fn

    c2_bytes = 262144 * used + 2 * 64 * work.k + 2 * 2 * 64 * work.n
    items.append(Timed("c2", [rows_call(layer) for layer in range(work.layers)], reps, c2_bytes))
    meta["c2"] = dict(batch=64, adapters_used=used, launches_per_call=2, segments=len(seg_slots))

    # The same update in one launch (lora_apply: shrink + expand, z kept on chip).
    from loraforge_amd.ops import lora_apply

    y2 = y.clone()

    def fused_call(layer):
        batch = work.lora(layer, slots)
        return lambda: lora_apply(x, y2, batch)

    items.append(Timed("c2_fused", [fused_call(layer) for layer in range(work.layers)], reps, c2_bytes))
    meta["c2_fused"] = dict(batch=64, adapters_used=used, launches_per_call=1, op="lora_apply")
    return items, meta


def c3_items(device, reps: int, copies: int = 6):
    """NF4 + double-quant SwiGLU MLP 4096 / 12288 with 16 rank-8 adapters on gate/up (two slices) and down."""
    import torch

    from loraforge_amd.ops import LoraBatch, nf4_lora_linear, quantize_nf4
    from loraforge_amd.ops.activation import silu_mul

    hidden, inter, adapters, rank = 4096, 12288, 16, 8
    g = torch.Generator(device="cpu").manual_seed(734)
    mlps = []
    i64 = dict(dtype=torch.int64, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    for _ in range(copies):
        gu_w = (torch.randn(2 * inter, hidden, generator=g) * 0.02).bfloat16().to(device)
        dn_w = (torch.randn(hidden, inter, generator=g) * 0.02).bfloat16().to(device)
        gu = quantize_nf4(gu_w, compress_statistics=True)
        dn = quantize_nf4(dn_w, compress_statistics=True)
        del gu_w, dn_w
        a1 = (torch.randn(adapters * 2 * rank * hidden, generator=g) * 0.02).bfloat16().to(device)
        b1 = (torch.randn(adapters * 2 * inter * rank, generator=g) * 0.02).bfloat16().to(device)
        a2 = (torch.randn(adapters * rank * inter, generator=g) * 0.02).bfloat16().to(device)
        b2 = (torch.randn(adapters * hidden * rank, generator=g) * 0.02).bfloat16().to(device)
        mlps.append((gu, dn, a1, b1, a2, b2))
    common = dict(
        b_strides=torch.full((adapters,), rank, **i32),
        ranks=torch.full((adapters,), rank, **i32),
        scales=torch.full((adapters,), 2.0, device=device),
    )
    items, meta = [], {}

    def per_batch(batch):
        # One scope per batch: the thunks captured for a graph must keep their own
        # tensors (a loop variable rebound for the next batch would free them).
        x = torch.randn(batch, hidden, generator=g).bfloat16().to(device)
        slots = torch.randint(0, adapters, (batch,), generator=g, dtype=torch.int32)
        used = int(torch.unique(slots).numel())
        slots = slots.to(device)
        gu_out = torch.empty(batch, 2 * inter, dtype=torch.bfloat16, device=device)
        h = torch.empty(batch, inter, dtype=torch.bfloat16, device=device)
        y = torch.empty(batch, hidden, dtype=torch.bfloat16, device=device)

        def chain(mlp):
            (q1, s1), (q2, s2), a1, b1, a2, b2 = mlp
            l1 = LoraBatch(
                a1, torch.arange(adapters, **i64) * (2 * rank * hidden), b1, torch.arange(adapters, **i64) * (2 * inter * rank),
                token_slots=slots, slice_offsets=torch.tensor([0, inter, 2 * inter], **i32), max_rank=rank, **common,
            )
            l2 = LoraBatch(
                a2, torch.arange(adapters, **i64) * (rank * inter), b2, torch.arange(adapters, **i64) * (hidden * rank),
                token_slots=slots, slice_offsets=torch.tensor([0, hidden], **i32), max_rank=rank, **common,
            )

            def fn():
                nf4_lora_linear(x, q1, s1, lora=l1, out=gu_out)
                silu_mul(gu_out, out=h)
                nf4_lora_linear(h, q2, s2, lora=l2, out=y)

            def fused():
                # The SwiGLU in the gate/up epilogue (decode batches): two launches.
                nf4_lora_linear(x, q1, s1, lora=l1, out=h, swiglu=True)
                nf4_lora_linear(h, q2, s2, lora=l2, out=y)

            def nested():
                # The same two launches reading the double-quant state itself (no
                # fp32 scales resident; codes converted in LDS by each workgroup).
                nf4_lora_linear(x, q1, s1, scales="nested", lora=l1, out=h, swiglu=True)
                nf4_lora_linear(h, q2, s2, scales="nested", lora=l2, out=y)

            return fn, fused, nested

        # Algorithmic bytes: packed weights, uint8 absmax codes, fp32 second-level
        # scales and code2 of both weights, the adapters used, and the activations
        # (x in, y out, h written and read once).
        q_bytes = (2 * inter * hidden + hidden * inter) // 2
        nblocks = (2 * inter * hidden + hidden * inter) // 64
        absmax2 = 4 * (-(-(2 * inter * hidden // 64) // 256) + -(-(hidden * inter // 64) // 256))
        base = q_bytes + nblocks + absmax2 + 2 * 256 * 4
        act = batch * (hidden * 2 * 2 + inter * 2 * 2)
        work = base + 786432 * used + act
        chains = [chain(m) for m in mlps]
        name = f"c3_b{batch}"
        items.append(Timed(name, [c[0] for c in chains], reps, work))
        meta[name] = dict(batch=batch, adapters_used=used, launches_per_call=3)
        items.append(Timed(f"c3_fused_b{batch}", [c[1] for c in chains], reps, work))
        meta[f"c3_fused_b{batch}"] = dict(batch=batch, adapters_used=used, launches_per_call=2, swiglu="gate/up epilogue")
        items.append(Timed(f"c3_nested_b{batch}", [c[2] for c in chains], reps, work))
        meta[f"c3_nested_b{batch}"] = dict(batch=batch, adapters_used=used, launches_per_call=2, swiglu="gate/up epilogue",
                                           scales="nested state read in-kernel")

    for batch in (1, 8, 64):
        per_batch(batch)
    return items, meta


def c4_items(device, reps: int, copies: int = 8):
    """NF4 4096^2 + 128 retained-rank adapters (ranks {4..64}, ragged), 256 tokens, Zipf(1.1) routes."""
    import numpy as np
    import torch

    from loraforge_amd.ops import LoraBatch, nf4_lora_linear, quantize_nf4

    n = k = 4096
    tokens, adapters = 256, 128
    rng = np.random.default_rng(737)
    ranks = rng.choice([4, 8, 16, 32, 64], size=adapters)
    p = 1.0 / np.arange(1, adapters + 1) ** 1.1
    routes = rng.choice(adapters, size=tokens, p=p / p.sum()).astype(np.int32)
    used = np.unique(routes)
    a_off = np.concatenate([[0], np.cumsum(ranks * k)[:-1]]).astype(np.int64)
    b_off = np.concatenate([[0], np.cumsum(ranks * n)[:-1]]).astype(np.int64)
    total_a, total_b = int((ranks * k).sum()), int((ranks * n).sum())
    g = torch.Generator(device="cpu").manual_seed(738)
    i32 = dict(dtype=torch.int32, device=device)
    meta_t = dict(
        a_offsets=torch.from_numpy(a_off).to(device),
        b_offsets=torch.from_numpy(b_off).to(device),
        b_strides=torch.from_numpy(ranks.astype(np.int32)).to(device),
        ranks=torch.from_numpy(ranks.astype(np.int32)).to(device),
        scales=torch.full((adapters,), 2.0, device=device),
        token_slots=torch.from_numpy(routes).to(device),
        slice_offsets=torch.tensor([0, n], **i32),
    )
    x = torch.randn(tokens, k, generator=g).bfloat16().to(device)
    out = torch.empty(tokens, n, dtype=torch.bfloat16, device=device)
    calls = []
    for _ in range(copies):
        w = (torch.randn(n, k, generator=g) * 0.02).bfloat16().to(device)
        q, st = quantize_nf4(w)
        del w
        a = (torch.randn(total_a, generator=g) * 0.02).bfloat16().to(device)
        b = (torch.randn(total_b, generator=g) * 0.02).bfloat16().to(device)
        lora = LoraBatch(a_store=a, b_store=b, max_rank=64, **meta_t)
        calls.append((q, st, lora))
    work = n * k // 2 + n * k // 16 + int(sum(16384 * int(ranks[i]) for i in used)) + tokens * k * 2 * 2
    flops = 2 * tokens * n * k + int(sum(2 * int((routes == i).sum()) * int(ranks[i]) * (k + n) for i in used))

    def thunks(plan):
        return [lambda q=q, st=st, lora=lora: nf4_lora_linear(x, q, st, lora=lora, out=out, plan=plan) for q, st, lora in calls]

    # The library's plan (the chunked decode at this shape) and the prefill GEMM forced, on the same copies.
    items = [Timed("c4", thunks(None), reps, work), Timed("c4_prefill", thunks("prefill"), reps, work)]
    info = dict(tokens=tokens, adapters_used=int(used.size), flops_per_call=flops)
    return items, {"c4": dict(info, plan="library choice"), "c4_prefill": dict(info, plan="prefill GEMM (forced)")}


def c5_items(device, reps: int):
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
    # The same weight read as a merged gate/up projection (5504 + 5504 rows) with two
    # rank-32 slices per segment: the SwiGLU output in the GEMM's epilogue, against the
    # linear followed by silu_mul.
    from loraforge_amd.ops.activation import silu_mul

    lora2 = LoraBatch(
        (torch.randn(segs * 2 * rank * k, generator=g) * 0.02).bfloat16().to(device),
        torch.arange(segs, **i64) * (2 * rank * k),
        b,
        torch.arange(segs, **i64) * (n * rank),
        torch.full((segs,), rank, dtype=torch.int32, device=device),
        torch.full((segs,), rank, dtype=torch.int32, device=device),
        torch.full((segs,), 2.0, device=device),
        slots,
        torch.tensor([0, n // 2, n], dtype=torch.int32, device=device),
        max_rank=rank,
    )
    h = torch.empty(m, n // 2, dtype=torch.bfloat16, device=device)

    def two_launches():
        nf4_lora_linear(x, q, st, lora=lora2, out=out)
        silu_mul(out, out=h)

    flops_swiglu = flops_base + 2 * m * k * 2 * rank + 2 * m * rank * n
    items = [
        Timed("c5", [lambda: nf4_lora_linear(x, q, st, lora=lora, out=out)] * 4, reps, flops, unit="TFLOP/s"),
        Timed("c5_base_only", [lambda: nf4_lora_linear(x, q, st, out=out)] * 4, reps, flops_base, unit="TFLOP/s"),
        Timed("c5_swiglu", [lambda: nf4_lora_linear(x, q, st, lora=lora2, out=h, swiglu=True)] * 4, reps, flops_swiglu,
              unit="TFLOP/s"),
        Timed("c5_swiglu_two_launches", [two_launches] * 4, reps, flops_swiglu, unit="TFLOP/s"),
    ]
    meta = dict(m=m, n=n, k=k, segments=segs, rank=rank, double_quant=True, segment_lengths=lengths.tolist())
    sw = dict(meta, gate_up=[n // 2, n // 2], slices=2, swiglu=True)
    return items, {"c5": meta, "c5_base_only": dict(meta, lora=False), "c5_swiglu": dict(sw, launches=1),
                   "c5_swiglu_two_launches": dict(sw, launches=2)}


FLEET_SHAPES = (
    # (name, slice widths, retained ranks of slots 1..4): the reference's row-tile study
    # (docs/qwen35.md:379-386, benchmarks/rowexpand_tiles.py:38-42), 32 tokens routed 1,2,3,4,1,...
    ("fleet_out_proj_1024", (1024,), (8, 16, 32, 64)),
    ("fleet_qkv_4096_512_512", (4096, 512, 512), (32, 64, 64, 64)),
)


def fleet_items(device, reps: int, tokens: int = 32, capacity: int = 64):
    """The Fleet ``row_expand`` at the reference's published shapes (warm: the same tensors every call)."""
    import numpy as np
    import torch

    from loraforge_amd.ops import rowexpand

    items, meta = [], {}
    g = torch.Generator(device="cpu").manual_seed(411)
    routes = [1 + t % 4 for t in range(tokens)]
    indptr, seg_slots, order = segments_of(routes)
    i32 = dict(dtype=torch.int32, device=device)
    for name, widths, retained in FLEET_SHAPES:
        n, slices = sum(widths), len(widths)
        ranks = np.array((0,) + retained, np.int32)
        sizes = n * ranks
        offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
        store = (torch.randn(int(sizes.sum()) + 8, generator=g) / 20).bfloat16().to(device)
        z = (torch.randn(tokens, slices * capacity, generator=g) / 10).bfloat16().to(device)
        y = (torch.randn(tokens, n, generator=g) / 10).bfloat16().to(device)
        args = (
            z, store, torch.from_numpy(offsets).to(device), torch.from_numpy(ranks).to(device), y,
            torch.from_numpy(indptr).to(device), torch.from_numpy(seg_slots).to(device),
            torch.from_numpy(order).to(device), torch.from_numpy(ranks).to(device),
            torch.tensor([0.0, 1.0, 0.75, 1.25, 0.5], device=device),
            torch.tensor(np.concatenate([[0], np.cumsum(widths)]), **i32),
            torch.tensor([len(seg_slots)], **i32), capacity,
        )
        used = [int(ranks[s]) for s in routes]
        work = sum(2 * n * int(r) for r in retained) + sum(2 * slices * r for r in used) + 2 * 2 * tokens * n
        items.append(Timed(name, [lambda a=args: rowexpand.row_expand(*a)] * 8, reps, work))
        meta[name] = dict(tokens=tokens, widths=list(widths), ranks=list(retained), segments=len(seg_slots), op="row_expand")
    return items, meta


def dequant_items(device, reps: int, copies: int = 64):
    """Standalone NF4 dequantisation of an 8192 x 1024 weight (bf16 out), over 64 weight copies."""
    import torch

    from loraforge_amd.ops import dequantize_nf4, quantize_nf4

    n, k = 8192, 1024
    g = torch.Generator(device="cpu").manual_seed(739)
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16().to(device)
    q, st = quantize_nf4(w)
    copies_ = [(q.clone(), st.absmax.clone()) for _ in range(copies)]
    out = torch.empty(n, k, dtype=torch.bfloat16, device=device)
    calls = [lambda q=qq, s=ss: dequantize_nf4(q, s, st.code, (n, k), out=out) for qq, ss in copies_]
    work = n * k // 2 + n * k // 16 + n * k * 2
    return [Timed("dequant_8192x1024", calls, reps, work)], {"dequant_8192x1024": dict(n=n, k=k)}


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
    parser.add_argument("--only", action="store_true", help="headline decode only (no configs/CPU)")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--configs", default="all", help="comma list of c1,north_star,c2,c3,c4,c5,fleet,dequant (default all)")
    parser.add_argument("--reps", type=int, default=10, help="graph replays per round for each config")
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
    log(f"device {torch.cuda.get_device_name(0)}; building {LAYERS} weight/adapter copies")
    work = DecodeWorkload(device)
    log(f"headline decode B={args.batch}: warmup {args.warmup}, steps {args.steps}")
    t0 = time.perf_counter()
    head = run_headline(work, args.batch, args.steps, args.warmup, seed=731 + args.batch)
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
            "kernel": decode_kernel(args.batch)[0],
            "bytes_per_launch": head["bytes_per_call"],
            "us_per_launch": round(head["us_per_call"], 3),
            "timing": "HIP events on the graph-replay stream over the timed calls (includes the graph's "
            "inter-kernel dispatch gap; rocprofv3 kernel durations are in profiles/)",
        },
    }
    if not args.only:
        wanted = set(args.configs.split(",")) if args.configs != "all" else {"c1", "north_star", "c2", "c3", "c4", "c5", "fleet", "dequant"}
        items, meta = [], {}
        if wanted & {"c1", "north_star", "c2"}:
            it, me = decode_items(work, args.reps, wanted)
            items += it
            meta.update(me)
        if "c3" in wanted:
            it, me = c3_items(device, args.reps)
            items += it
            meta.update(me)
        if "c4" in wanted:
            it, me = c4_items(device, args.reps)
            items += it
            meta.update(me)
        if "c5" in wanted:
            it, me = c5_items(device, max(2, args.reps // 2))
            items += it
            meta.update(me)
        if "fleet" in wanted:
            it, me = fleet_items(device, args.reps)
            items += it
            meta.update(me)
        if "dequant" in wanted:
            it, me = dequant_items(device, args.reps)
            items += it
            meta.update(me)
        log(f"configs: {', '.join(i.name for i in items)} ({ROUNDS} shuffled rounds)")
        res = run_rounds(items)
        configs = {}
        for name, r in res.items():
            configs[name] = {**meta.get(name, {}), **r}
            rate = r.get("gbps", r.get("tflops"))
            log(f"{name}: {r['us_per_call']:.2f} us/call, {rate} {'GB/s' if 'gbps' in r else 'TFLOP/s'} ({r['frac']:.1%})")
        result["configs"] = configs
        del items
    del work
    torch.cuda.empty_cache()
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
    rc = main()
    # The JSON line is out: end the process at once instead of tearing down
    # torch's HIP state and the resident copies (which leaves it running for a
    # while after the result is printed).
    sys.stdout.flush()
    sys.stderr.flush()
    try:
        import torch

        if torch.cuda.is_initialized():
            torch.cuda.synchronize()
    except Exception:  # noqa: BLE001 - best effort before exiting
        pass
    # Under a profiler (rocprofv3 preloads its tool library and writes its
    # results from exit hooks) the process ends normally.
    if any(k.startswith("ROCPROF") for k in os.environ) or "rocprofiler" in os.environ.get("LD_PRELOAD", ""):
        sys.exit(rc)
    os._exit(rc)
