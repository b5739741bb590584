"""MoE expert-layer benchmark on one MI355X.

Headline (the JSON `value`): T=8 speculative-verify MoE layer with Zipf(1.1)
expert popularity -- HBM GB/s on the unique expert weight bytes a step
touches.  A step is one sparse MoE block over 8 tokens: softmax/top-k on the
drawn logits, bucketing, routed SwiGLU experts, shared expert, ordered
combine.  Steps rotate over the resident layers so the touched experts are
not Infinity-Cache resident; the steps run as HIP-graph replays.

Also reported under "configs": T=1 decode layer with the router (latency and
GB/s), the raw expert gather at T in {1,4,8,16}, the 40-layer decode chain
with RMSNorm + residual at T=1 and T=16 (one persistent launch, and for
comparison one launch per layer in a graph), and the T=2048 prefill
(TFLOPS).

`roofline` is for moe_decode, the one kernel of the headline step, timed
with HIP events stamped by its own dispatches; `cpu_baseline` is the reference CPU expert
kernel (edge35b/cpu_experts.c built from source into oracle/_ref) on the
host's cores over a bounded sample of the same routes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from lightreason_amd import _native  # noqa: E402
from lightreason_amd.moe import (CODEC_DN_BASES, CODEC_GU_BASES, EXPERT_BYTES, EXPERT_ELEMENTS,  # noqa: E402
                                 GATE_UP_ELEMENTS, HIDDEN, INNER, CodecBank, LayerWeights, Workspace, gather,
                                 moe_chain, moe_layer)
from lightreason_amd.synthetic import SyntheticModel  # noqa: E402

METRIC = "MoE layer µs + HBM GB/s vs peak at T=1,8; prefill BF16 TFLOPS at T=2048"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PAIR_FLOP = 2 * 3 * INNER * HIDDEN  # one (token, expert) SwiGLU pair
SHARED_BYTES = EXPERT_BYTES + 2 * HIDDEN
ROUTER_BYTES = 256 * HIDDEN * 2
COPY_BYTES = 256 * 2**20


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def bf16_from_f64(values: np.ndarray, device) -> torch.Tensor:
    f32 = np.ascontiguousarray(values, dtype=np.float32)
    bits = f32.view(np.uint32).astype(np.uint64)
    b = (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(device)


def zipf_logits(tokens: int, seed: int, s: float = 1.1) -> np.ndarray:
    """L[t, e] = -s ln(rank_e) + Gumbel[t, e]: top-8 of a row is a Zipf(s)
    draw of 8 distinct experts (Gumbel-top-k)."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(256) + 1
    return -s * np.log(ranks)[None, :] + rng.gumbel(size=(tokens, 256))


def timed_replays(graph, replays: int) -> float:
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


def replay_percentiles(graph, replays: int, layers: int) -> dict:
    """p10/p50/p90 of the per-layer time over single replays, each bracketed
    by its own events (a separate pass from the timed one)."""
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    torch.cuda.synchronize()
    for start, stop in events:
        start.record()
        graph.replay()
        stop.record()
    torch.cuda.synchronize()
    us = np.array([start.elapsed_time(stop) * 1e3 / layers for start, stop in events])
    return {f"p{q}": round(float(np.percentile(us, q)), 2) for q in (10, 50, 90)}


def copy_peak_gbs(device, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Achievable HBM bandwidth of a plain device copy (read + write bytes
    per second, best of `reps`), to report fractions against a measured peak
    beside the spec one."""
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=device).fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        dst.copy_(src)
        stop.record()
        torch.cuda.synchronize()
        best = min(best, start.elapsed_time(stop))
    del src, dst
    return 2 * nbytes / (best * 1e-3) / 1e9


def capture(fn):
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


class Case:
    """One workload: per-layer static inputs and outputs, run as one graph
    that steps through the layers in order."""

    def __init__(self, model, tokens, *, logits=None, norm=False, chain=False, layers=None, one_launch=False,
                 codec=None):
        self.model = model
        self.tokens = tokens
        self.layer_ids = list(range(len(model.layers))) if layers is None else layers
        device = model.device
        self.ws = Workspace(device, tokens)
        self.x = [model.hidden(tokens, step=100 + i) for i in self.layer_ids]
        self.out = [torch.empty((tokens, HIDDEN), dtype=torch.bfloat16, device=device) for _ in self.layer_ids]
        self.idx_all = torch.empty((len(self.layer_ids), tokens, 8), dtype=torch.int64, device=device)
        self.idx = list(self.idx_all)
        self.logits = logits
        self.chain = chain
        self.one_launch = one_launch
        self.layers = []
        for i in self.layer_ids:
            base = model.layers[i]
            self.layers.append(LayerWeights(**{**base.__dict__, "norm_weight": base.norm_weight if norm else None,
                                               "codec": None if codec is None else codec.table(i)}))

    def run(self):
        if self.one_launch:
            # The whole stack as persistent chain launches (48 layers each).
            moe_chain(self.x[0], self.layers, out=self.out[-1], indices=self.idx_all, workspace=self.ws)
            return
        for j, layer in enumerate(self.layers):
            x = self.out[j - 1] if (self.chain and j > 0) else self.x[j]
            moe_layer(x, layer, out=self.out[j], indices=self.idx[j],
                      logits_in=None if self.logits is None else self.logits[j], workspace=self.ws)

    def unique_counts(self) -> list[int]:
        self.run()
        torch.cuda.synchronize()
        return [len(set(i.cpu().numpy().ravel().tolist())) for i in self.idx]


class GatherCase:
    """C1: per layer, gather its selected experts (packed 6 MiB rows) into
    one contiguous staging buffer."""

    def __init__(self, ptrs, per_layer, staging, device):
        self.descs = [torch.stack([ptrs[l][:, 0], torch.full((256,), -1), torch.zeros(256, dtype=torch.int64)], 1)[None]
                      .contiguous().to(device) for l in range(len(per_layer))]
        self.srcs = [torch.tensor(sel + [0] * (128 - len(sel)), dtype=torch.int32, device=device) for sel in per_layer]
        self.dst = torch.arange(128, dtype=torch.int32, device=device)
        self.counts = [torch.tensor([len(sel)], device=device) for sel in per_layer]
        self.dests = torch.tensor([staging.data_ptr()], device=device)
        self.sizes = torch.tensor([EXPERT_BYTES], device=device)
        self.max_copies = max(len(sel) for sel in per_layer)

    def run(self):
        for l in range(len(self.descs)):
            gather(self.descs[l], self.dests, self.sizes, self.srcs[l], self.dst, self.counts[l],
                   max_copies=self.max_copies, experts=256, stripes=48)


class CodecGatherCase:
    """C1 with codec rows: per layer, gather its selected experts' 6 MiB rows
    from the tile codec ("cpu-tiles": lrmoe_gather_tiles) or the escape codec
    (lrmoe_gather), packed on the device from the resident experts."""

    def __init__(self, model, per_layer, staging, device, codec: str):
        from lightreason_amd.moe import pack_escape_row, pack_tiles_reference_order

        self.codec = codec
        self.keep = []
        self.descs = []
        self.read_bytes = 0
        for l, sel in enumerate(per_layer):
            ptrs = model.bank.tables[l][:, 0].cpu()
            desc = torch.zeros((1, 256, 3), dtype=torch.int64)
            desc[0, :, 2 if codec == "tile" else 0] = ptrs
            if codec == "escape":
                desc[0, :, 1] = -1
            for e in sel:
                row = model.bank.bank[l, e]
                if codec == "tile":
                    packed, bases, _ = pack_tiles_reference_order(row.view(-1, 256))
                    self.keep += [packed, bases]
                    desc[0, e, 0], desc[0, e, 1] = packed.data_ptr(), bases.data_ptr()
                    self.read_bytes += packed.numel() + bases.numel()
                else:
                    packed, base, escapes = pack_escape_row(row)
                    self.keep.append(packed)
                    desc[0, e] = torch.tensor([packed.data_ptr(), base, escapes])
                    self.read_bytes += packed.numel()
            self.descs.append(desc.to(device))
        self.read_bytes /= len(per_layer)
        self.srcs = [torch.tensor(sel + [0] * (128 - len(sel)), dtype=torch.int32, device=device) for sel in per_layer]
        self.dst = torch.arange(128, dtype=torch.int32, device=device)
        self.counts = [torch.tensor([len(sel)], device=device) for sel in per_layer]
        self.dests = torch.tensor([staging.data_ptr()], device=device)
        self.sizes = torch.tensor([EXPERT_BYTES], device=device)
        self.max_copies = max(len(sel) for sel in per_layer)
        self.stream = torch.cuda.current_stream(device).cuda_stream

    def run(self):
        for l in range(len(self.descs)):
            if self.codec == "tile":
                _native.call("lrmoe_gather_tiles", self.descs[l].data_ptr(), self.dests.data_ptr(),
                             self.sizes.data_ptr(), self.srcs[l].data_ptr(), self.dst.data_ptr(),
                             self.counts[l].data_ptr(), 256, 1, self.max_copies, 48, 256, 0,
                             torch.cuda.current_stream().cuda_stream)
            else:
                gather(self.descs[l], self.dests, self.sizes, self.srcs[l], self.dst, self.counts[l],
                       max_copies=self.max_copies, experts=256, stripes=48)


def bench_case(case: Case, replays: int, warmup: int, spread: dict | None = None) -> float:
    """Milliseconds per graph replay (one pass over the case's layers).  With
    `spread`, also fills it with per-layer percentiles from a separate pass."""
    graph = capture(case.run)
    for _ in range(warmup):
        graph.replay()
    ms = timed_replays(graph, replays) / replays
    if spread is not None:
        spread.update(replay_percentiles(graph, max(replays, 10), len(case.layers)))
    return ms


def kernel_time(case: Case, stage: int, passes: int) -> tuple[float, int]:
    """Average duration (ms) of one stage's launches over eager passes."""
    case.run()
    torch.cuda.synchronize()
    _native.timing_enable(stage, passes * len(case.layers) + 8)
    for _ in range(passes):
        case.run()
    total, launches = _native.timing_collect(stage)
    _native.timing_enable(0)
    return total / max(launches, 1), launches


def measured_traffic(kernel: str) -> dict | None:
    """HBM bytes per dispatch of ``kernel`` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE passes, scaled by a 256 MiB copy)."""
    path = ROOT / "profiles" / "moe_decode_t8_zipf_hbm_traffic.md"
    if not path.exists():
        return None
    text = path.read_text()
    start = text.find("```json")
    if start < 0:
        return None
    block = json.loads(text[start + 7:text.index("```", start + 7)])
    if block.get("kernel") != kernel:
        return None
    return {"bytes": int(block["read_bytes"]) + int(block["write_bytes"]),
            "source": f"profiles/{path.name}"}


def cpu_workers_t1(model, case: Case, budget_s: float = 5.0) -> dict | None:
    """The reference's persistent CPU expert workers (oracle/_ref/
    libpacked_workers.so, built from edge35b/packed_workers.cpp) on T=1
    decode routes: one submit/wait of the 8 routed experts per layer, cycling
    over 8 layers' host copies.  GB/s on the 8 x 6 MiB expert bytes."""
    import ctypes as C

    from oracle import oracle as O

    ref = O.reference_workers()
    if ref is None:
        return None
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    calls = []
    for j in range(min(len(case.layer_ids), 8)):
        layer = case.layer_ids[j]
        experts = case.idx[j][0].cpu().tolist()
        rows = [model.bank.bank[layer, e].cpu().view(torch.int16).numpy().view(np.uint16) for e in experts]
        gates = (C.c_void_p * 8)(*[r.ctypes.data for r in rows])
        downs = (C.c_void_p * 8)(*[r.ctypes.data + 2 * GATE_UP_ELEMENTS for r in rows])
        x = case.x[j].cpu().view(torch.int16).numpy().view(np.uint16)
        calls.append((gates, downs, x, rows))
    out = np.empty((8, HIDDEN), dtype=np.uint16)
    workers = ref.packed_workers_create(threads)
    try:
        for gates, downs, x, _ in calls:
            ref.packed_workers_submit(workers, gates, downs, x.ctypes.data, out.ctypes.data, 8)
            ref.packed_workers_wait(workers)
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            gates, downs, x, _ = calls[n % len(calls)]
            ref.packed_workers_submit(workers, gates, downs, x.ctypes.data, out.ctypes.data, 8)
            ref.packed_workers_wait(workers)
            n += 1
        dt = time.perf_counter() - t0
    finally:
        ref.packed_workers_destroy(workers)
    return {"value": round(n * 8 * EXPERT_BYTES / dt / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "reference", "us_per_layer": round(1e6 * dt / n, 1),
            "sample": f"{n} submit/wait calls of 8 routed experts (T=1), cycling over {len(calls)} layers, "
                      f"packed_workers with {threads} threads"}


def cpu_baseline(model, case: Case, uniques, budget_s: float = 15.0) -> dict:
    """The reference CPU expert kernel (oracle/_ref/libcpu_experts.so, built
    from edge35b/cpu_experts.c) on the headline routes: expert_block_rows over
    the 64 (token, expert) rows of a layer, with the threads of this process's
    CPU share.  The sample holds several layers' experts in host memory and
    cycles through them call by call, so no call finds its weights in the host
    caches.  GB/s on the same unique-expert bytes as the GPU figure."""
    from oracle import oracle as O

    ref = O.reference()
    kind = "reference"
    if ref is None:
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": kind,
                "sample": "reference CPU kernel not built (oracle/Makefile needs the reference source)"}
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    sample_layers = min(len(case.layer_ids), 8)
    calls = []
    for j in range(sample_layers):
        layer = case.layer_ids[j]
        idx = case.idx[j].cpu().numpy()
        x = case.x[j].cpu().view(torch.int16).numpy().view(np.uint16)
        host = {}
        for e in sorted(set(idx.ravel().tolist())):
            row = model.bank.bank[layer, e].cpu().view(torch.int16).numpy().view(np.uint16)
            host[e] = (np.ascontiguousarray(row[:2 * INNER * HIDDEN]), np.ascontiguousarray(row[2 * INNER * HIDDEN:]))
        gu = [host[e][0] for e in idx.ravel().tolist()]
        dn = [host[e][1] for e in idx.ravel().tolist()]
        tok = np.repeat(np.arange(idx.shape[0], dtype=np.int32), idx.shape[1])
        calls.append((gu, dn, x, tok, uniques[j] * EXPERT_BYTES, host))
    for gu, dn, x, tok, _, _ in calls:  # first touch of every page
        O.reference_expert_block_rows(gu, dn, x, tok, threads)
    total_bytes, n = 0, 0
    t0 = time.perf_counter()
    while n < 3 * sample_layers or time.perf_counter() - t0 < budget_s:
        gu, dn, x, tok, nbytes, _ = calls[n % sample_layers]
        O.reference_expert_block_rows(gu, dn, x, tok, threads)
        total_bytes += nbytes
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    gbs = total_bytes / dt / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": kind,
            "ms_per_layer": round(1e3 * dt / n, 3),
            "sample": f"{n} calls cycling over {sample_layers} layers' T=8 Zipf routes "
                      f"({sum(c[4] for c in calls) / 2**20:.0f} MiB of unique experts), expert_block_rows with "
                      f"{threads} OpenMP threads, 64 rows per call; routed experts only (the reference CPU path "
                      "has no router, combine or shared expert)"}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=400, help="timed headline steps (layer calls)")
    parser.add_argument("--warmup", type=int, default=40)
    parser.add_argument("--layers", type=int, default=40, help="resident layers (40 = the whole model)")
    parser.add_argument("--seed", type=int, default=2026)
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--skip-prefill", action="store_true")
    parser.add_argument("--only", default="", help="comma list of c0,c1,c2,c3,c4,c5 to run (default all)")
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="also run a plain 256 MiB device copy (untimed) so that HBM byte counters "
                             "of a profiler run can be scaled by a kernel of known traffic")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(multi-GPU sharding is a design note only)", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    _native.device_check()
    t0 = time.perf_counter()
    model = SyntheticModel(layers=args.layers, device=device, seed=args.seed, shared=True, norm="normal")
    torch.cuda.synchronize()
    log(f"[bench] {args.layers} layers resident ({model.bank.nbytes / 2**30:.1f} GiB experts) "
        f"in {time.perf_counter() - t0:.1f}s")
    L = args.layers
    replays = max(1, args.steps // L)
    warm = max(1, args.warmup // L)
    only = set(filter(None, args.only.split(","))) or {"c0", "c1", "c2", "c3", "c4", "c5"}
    if args.skip_prefill:
        only.discard("c4")
    configs = {}
    if args.calibrate_copy:
        src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- headline: T=8 Zipf verify ----
    logits = [bf16_from_f64(zipf_logits(8, args.seed * 1000 + l), device) for l in range(L)]
    c2 = Case(model, 8, logits=logits)
    uniques = c2.unique_counts()
    spread = {}
    ms = bench_case(c2, replays, warm, spread)
    ms_step = ms / L
    bytes_step = (np.mean(uniques) * EXPERT_BYTES + SHARED_BYTES)
    gbs = bytes_step / (ms_step * 1e-3) / 1e9
    log(f"[bench] C2 T=8 zipf: {ms_step * 1e3:.1f} us/layer, U={np.mean(uniques):.1f}, {gbs:.0f} GB/s, "
        f"per-replay us/layer {spread}")
    # The T <= 16 layer is one kernel (moe_decode): its launches are timed
    # with start/stop events stamped by the dispatch itself.
    layer_ms, layer_launches = kernel_time(c2, _native.STAGE_LAYER, passes=max(2, replays))
    stage_us = {"moe_decode": round(layer_ms * 1e3, 2)}
    # Algorithmic bytes of one launch: the unique routed experts and the
    # shared expert (6 MiB each), the shared-expert gate row, and per token
    # the hidden row in, the logits row in and the output row out.
    layer_bytes = (np.mean(uniques) + 1) * EXPERT_BYTES + 2 * HIDDEN + 8 * (2 * HIDDEN + 2 * 256 + 2 * HIDDEN)
    layer_gbs = layer_bytes / (layer_ms * 1e-3) / 1e9
    log(f"[bench] C2 moe_decode kernel (event-bracketed): {stage_us['moe_decode']} us, {layer_gbs:.0f} GB/s")
    configs["c2_verify_t8_zipf"] = dict(us_per_layer=round(ms_step * 1e3, 2),
                                        unique_experts=round(float(np.mean(uniques)), 2), gbs=round(gbs, 1),
                                        frac_hbm=round(gbs / HBM_PEAK_GBS, 4), stage_us=stage_us,
                                        us_per_layer_spread=spread)

    # ---- C0: T=1 decode layer with the router ----
    if "c0" in only:
        c0 = Case(model, 1)
        ms0 = bench_case(c0, replays, warm) / L
        b0 = 8 * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES
        st0 = {"moe_decode": round(kernel_time(c0, _native.STAGE_LAYER, passes=2)[0] * 1e3, 2)}
        configs["c0_decode_t1"] = dict(us_per_layer=round(ms0 * 1e3, 2), gbs=round(b0 / (ms0 * 1e-3) / 1e9, 1),
                                       frac_hbm=round(b0 / (ms0 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), stage_us=st0)
        if not args.skip_cpu:
            configs["c0_decode_t1"]["cpu_reference_workers"] = cpu_workers_t1(model, c0)
        log(f"[bench] C0 T=1: {ms0 * 1e3:.1f} us/layer, {configs['c0_decode_t1']['gbs']} GB/s, stages {st0}")

    # ---- C1: raw expert gather ----
    if "c1" in only:
        gather_res = {}
        ptrs = model.bank.tables.cpu()
        staging = torch.empty((128, EXPERT_ELEMENTS), dtype=torch.bfloat16, device=device)
        for T in (1, 4, 8, 16):
            rng = np.random.default_rng(T)
            per_layer = [sorted(set(np.concatenate([rng.choice(256, 8, replace=False) for _ in range(T)]).tolist()))
                         for _ in range(L)]
            gcase = GatherCase(ptrs, per_layer, staging, device)
            msg = bench_case(gcase, replays, warm) / L
            u = float(np.mean([len(sel) for sel in per_layer]))
            moved = 2 * u * EXPERT_BYTES
            gather_res[f"t{T}"] = dict(unique=round(u, 1), us=round(msg * 1e3, 2),
                                       gbs_moved=round(moved / (msg * 1e-3) / 1e9, 1))
            if T == 8:
                t8_layers = per_layer
        # Codec rows, T=8 selections of the first 8 layers: raw-equivalent
        # GB/s (6 MiB read + 6 MiB written per row) and the bytes read.
        for codec in ("tile", "escape"):
            sel8 = t8_layers[:min(L, 8)]
            ccase = CodecGatherCase(model, sel8, staging, device, codec)
            msc = bench_case(ccase, replays, warm) / len(sel8)
            u = float(np.mean([len(sel) for sel in sel8]))
            gather_res[f"t8_{codec}_codec"] = dict(
                unique=round(u, 1), us=round(msc * 1e3, 2),
                gbs_raw_equivalent=round(2 * u * EXPERT_BYTES / (msc * 1e-3) / 1e9, 1),
                read_fraction=round(ccase.read_bytes / (u * EXPERT_BYTES), 4),
                gbs_moved=round((ccase.read_bytes + u * EXPERT_BYTES) / (msc * 1e-3) / 1e9, 1))
            del ccase
        configs["c1_gather"] = gather_res
        log(f"[bench] C1 gather: {gather_res}")
        del staging

    # ---- C3: 40-layer chain with RMSNorm + residual ----
    if "c3" in only:
        for T in (1, 16):
            for one_launch in (True, False):
                c3 = Case(model, T, norm=True, chain=True, one_launch=one_launch)
                u3 = c3.unique_counts()
                ms3 = bench_case(c3, max(2, replays // 2), 1)
                b3 = sum(u * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES + 2 * HIDDEN for u in u3)
                key = f"c3_chain_t{T}" if one_launch else f"c3_layer_graph_t{T}"
                configs[key] = dict(layers=L, ms_per_step=round(ms3, 4), gbs=round(b3 / (ms3 * 1e-3) / 1e9, 1),
                                    frac_hbm=round(b3 / (ms3 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                    mean_unique=round(float(np.mean(u3)), 1),
                                    launches="one persistent launch" if one_launch else "one per layer, in a graph")
                log(f"[bench] C3 T={T} {'chain' if one_launch else 'per-layer'}: {ms3:.3f} ms/step over {L} layers, "
                    f"{configs[key]['gbs']} GB/s")

    # ---- C5: the decode layers reading tile-codec experts ----
    if "c5" in only:
        t0 = time.perf_counter()
        bank = CodecBank(model.bank, [(ly.shared_gate_proj, ly.shared_up_proj, ly.shared_down_proj)
                                      for ly in model.layers])
        torch.cuda.synchronize()
        misfit_tiles = float(bank.misfit.sum()) / (bank.misfit.numel() * (CODEC_GU_BASES + CODEC_DN_BASES))
        # Weight bytes read per raw byte: a fitting tile is 384 bytes and its
        # base byte instead of 512; a tile that does not fit is read raw.  (A
        # workgroup's first item is read raw, its second with the
        # per-(item, wave) flags: units_packed of them pack.)
        read_frac = (1 - misfit_tiles) * 385 / 512 + misfit_tiles
        log(f"[bench] C5 codec bank in {time.perf_counter() - t0:.1f}s: {bank.nbytes / 2**30:.1f} GiB, "
            f"tiles misfit {misfit_tiles:.4f}, weight bytes read x{read_frac:.3f}")
        res = dict(tiles_misfit=round(misfit_tiles, 5), weight_bytes_read_frac=round(read_frac, 4),
                   units_packed=round(bank.packed_fraction, 4), bank_gib=round(bank.nbytes / 2**30, 1))
        c5 = Case(model, 8, logits=logits, codec=bank)
        assert c5.unique_counts() == uniques
        ms5 = bench_case(c5, replays, warm) / L
        res["c2_verify_t8_zipf"] = dict(us_per_layer=round(ms5 * 1e3, 2),
                                        raw_equivalent_gbs=round(bytes_step / (ms5 * 1e-3) / 1e9, 1),
                                        speedup_vs_raw=round(ms_step / ms5, 3))
        log(f"[bench] C5 T=8 zipf codec: {ms5 * 1e3:.1f} us/layer (raw {ms_step * 1e3:.1f})")
        for T in (1, 16):
            c5 = Case(model, T, norm=True, chain=True, one_launch=True, codec=bank)
            u5 = c5.unique_counts()
            ms5 = bench_case(c5, max(2, replays // 2), 1)
            b5 = sum(u * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES + 2 * HIDDEN for u in u5)
            res[f"c3_chain_t{T}"] = dict(ms_per_step=round(ms5, 4),
                                         raw_equivalent_gbs=round(b5 / (ms5 * 1e-3) / 1e9, 1))
            raw = configs.get(f"c3_chain_t{T}")
            if raw is not None:
                res[f"c3_chain_t{T}"]["speedup_vs_raw"] = round(raw["ms_per_step"] / ms5, 3)
            log(f"[bench] C5 T={T} chain codec: {ms5:.3f} ms/step")
        configs["c5_codec"] = res
        del bank

    # ---- C4: T=2048 prefill with skewed routing ----
    if "c4" in only:
        T = 2048
        sigma_bias = 0.25
        rng = np.random.default_rng(args.seed + 4)
        layer_ids = list(range(min(L, 4)))
        lg = []
        for l in layer_ids:
            x = model.hidden(T, step=100 + l).float()
            base = (x @ model.layers[l].router.float().T).cpu().numpy()
            lg.append(bf16_from_f64(base + rng.normal(0, sigma_bias, size=(1, 256)), device))
        c4 = Case(model, T, logits=lg, layers=layer_ids)
        c4.run()
        torch.cuda.synchronize()
        idx_counts = [np.bincount(i.cpu().numpy().ravel(), minlength=256) for i in c4.idx]
        ms4 = bench_case(c4, 3, 1) / len(layer_ids)
        flops = (T * 8 + T) * PAIR_FLOP
        hit = float(np.mean([(c > 0).sum() for c in idx_counts]))
        skew = float(np.mean([c.max() / c.mean() for c in idx_counts]))
        tflops = flops / (ms4 * 1e-3) / 1e12
        configs["c4_prefill_t2048"] = dict(ms_per_layer=round(ms4, 3), tflops=round(tflops, 2),
                                           frac_mfma=round(tflops / BF16_PEAK_TFLOPS, 4), experts_hit=hit,
                                           max_over_mean=round(skew, 2), bias_sigma=sigma_bias,
                                           flop_per_layer=flops, note="router GEMV excluded (logits given)")
        log(f"[bench] C4 T=2048: {ms4:.3f} ms/layer, {tflops:.1f} TFLOPS, hit {hit}, max/mean {skew:.2f}")

    cpu = {"value": None, "unit": "GB/s", "cores": 0, "kind": "reference", "sample": "skipped"}
    if not args.skip_cpu:
        cpu = cpu_baseline(model, c2, uniques)
        log(f"[bench] CPU baseline: {cpu}")

    traffic = measured_traffic("moe_decode")
    copy_gbs = copy_peak_gbs(device)
    log(f"[bench] measured copy peak {copy_gbs:.0f} GB/s (read + write)")
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": replays * L,
        "warmup": warm * L,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded counter-based generator; Zipf(1.1) Gumbel-top-k logits)",
        "config": {"workload": "T=8 speculative-verify MoE layer, 256 experts top-8, Zipf(1.1) routing, "
                               "shared expert, HBM GB/s on unique expert bytes; steps rotate over resident layers",
                   "tokens": 8, "hidden": HIDDEN, "experts": 256, "topk": 8, "inner": INNER,
                   "layers_rotated": L, "mean_unique_experts": round(float(np.mean(uniques)), 2)},
        "roofline": {"bound": "hbm", "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else traffic["bytes"],
                     "traffic_source": None if traffic is None else traffic["source"],
                     "measured_peak": round(copy_gbs, 1), "frac_of_measured": round(layer_gbs / copy_gbs, 4),
                     "kernel": "moe_decode", "avg_us": round(layer_ms * 1e3, 3), "launches": layer_launches,
                     "algorithmic_bytes": int(layer_bytes)},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
