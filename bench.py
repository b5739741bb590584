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
comparison one launch per layer in a graph), the T=2048 prefill (TFLOPS),
(C7) the Gated DeltaNet mixer step of the 30 linear-attention layers at
T=1 and T=16 (µs and GB/s on its weight and state bytes, per-kernel times,
a torch gate, and the oracle's C step timed on one core beside it), and (C8)
the full-attention decode step of the 10 full-attention layers at a
4096-position context, T=1 and T=16 (the same figures on its weight and
key/value bytes), and (C9) the whole 40-layer decoder step -- input RMSNorm,
Gated DeltaNet mixer or full attention, residual add, MoE block -- as one
captured graph per verify width 1/4/8/16 (ms per verify pass, and GB/s on
every weight, state and cached byte the pass touches).

`roofline` is for moe_decode, the one kernel of the headline step, timed
with HIP events stamped by its own dispatches, against the 8 TB/s spec and,
beside it, a measured read-only stream peak.  `cpu_baseline` is the reference
CPU expert kernel (edge35b/cpu_experts.c built from source into oracle/_ref)
on the headline's routes, run by oracle/cpu_baseline.py in a child process
pinned one thread per physical core; C0, C3 and C4 carry their own CPU legs
(`cpu_reference`).  The headline and C4 pass an fp32 torch parity gate on
sampled tokens before their numbers are reported, and every timed case
reports the workspace status word (0 = valid routes, no expired wait).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L]

A headline step is one T=8 layer call; the K timed steps (after W untimed
ones) cycle over the L resident layers and run as one captured graph.
"""

from __future__ import annotations

import argparse
import json
import os
import shutil
import subprocess
import sys
import tempfile
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
        self.wts_all = torch.empty((len(self.layer_ids), tokens, 8), dtype=torch.bfloat16, device=device)
        self.wts = list(self.wts_all)
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
            moe_chain(self.x[0], self.layers, out=self.out[-1], indices=self.idx_all, weights=self.wts_all,
                      workspace=self.ws)
            return
        for j, layer in enumerate(self.layers):
            x = self.out[j - 1] if (self.chain and j > 0) else self.x[j]
            moe_layer(x, layer, out=self.out[j], indices=self.idx[j], weights=self.wts[j],
                      logits_in=None if self.logits is None else self.logits[j], workspace=self.ws)

    def run_steps(self, steps: int):
        """`steps` single-layer calls, cycling over the case's layers (layer
        i % L for call i); for cases without a chain."""
        for i in range(steps):
            j = i % len(self.layers)
            moe_layer(self.x[j], self.layers[j], out=self.out[j], indices=self.idx[j], weights=self.wts[j],
                      logits_in=None if self.logits is None else self.logits[j], workspace=self.ws)

    def unique_counts(self) -> list[int]:
        self.run()
        torch.cuda.synchronize()
        self.ws.check("bench case")
        return [len(set(i.cpu().numpy().ravel().tolist())) for i in self.idx]

    def status(self) -> int:
        """The workspace status word after the case's last call (0: routes
        valid and no bounded wait expired)."""
        torch.cuda.synchronize()
        return self.ws.status()


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


def read_peak_gbs(device, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Achievable HBM read rate: best of `reps` launches of liblrmoe's
    read-only stream kernel over `nbytes` (the bound of a weight-streaming
    kernel, which reads far more than it writes)."""
    import ctypes as C

    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=device).fill_(1.0)
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    best = C.c_double(0.0)
    _native.call("lrmoe_read_bandwidth", src.data_ptr(), nbytes, reps, sink.data_ptr(), C.byref(best),
                 torch.cuda.current_stream(device).cuda_stream)
    del src
    return nbytes / (best.value * 1e-3) / 1e9


# ---- fp32 parity gates (torch on the GPU; no oracle in the timed legs) -----------

def torch_block_rows(model, layer: int, x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, rows) -> torch.Tensor:
    """The sparse MoE block without RMSNorm for the tokens `rows`, given its
    routes (indices and bf16 weights), in torch on the GPU with the rounding
    points of the reference's CPU expert kernel and ordered combine: gate,
    up, SiLU and their product rounded to bf16, the down projection to bf16,
    then per token over its routes in ascending expert order
    acc = bf16(acc + bf16(y * w)), plus bf16(sigmoid(bf16(x . w_sg))) times
    the shared expert.  Matrix-vector products in fp32."""
    f = torch.nn.functional
    ly = model.layers[layer]

    def r(t):
        return t.to(torch.bfloat16).float()

    def expert(gate, up, down, xf):
        g, u = r(torch.mv(gate.float(), xf)), r(torch.mv(up.float(), xf))
        return r(torch.mv(down.float(), r(r(f.silu(g)) * u)))

    out = []
    for t in rows:
        xf = x[t].float()
        acc = torch.zeros(HIDDEN, dtype=torch.float32, device=x.device)
        for k in sorted(range(8), key=lambda k: int(idx[t, k])):
            gu, dn = model.bank.expert(layer, int(idx[t, k]))
            acc = r(acc + r(expert(gu[:INNER], gu[INNER:], dn, xf) * w[t, k].float()))
        shared = expert(ly.shared_gate_proj, ly.shared_up_proj, ly.shared_down_proj, xf)
        gate = r(torch.sigmoid(r(torch.dot(ly.shared_expert_gate.float(), xf))))
        out.append(r(acc + r(gate * shared)))
    return torch.stack(out)


def parity_gate(model, layer: int, x, out, idx, w, rows, rel: float = 1e-2) -> dict:
    """The bench's own correctness gate for a timed case: sampled output
    rows against torch_block_rows, with the tests' output bar (bf16 storage,
    fp32 accumulation): max |got - ref| <= rel * max |ref| over the sample,
    and every row's L2 error <= rel of the row's norm."""
    want = torch_block_rows(model, layer, x, idx, w, rows)
    got = out[list(rows)].float()
    tensor_rel = float((got - want).abs().max() / want.abs().max().clamp_min(1e-30))
    row_l2 = float(((got - want).norm(dim=1) / want.norm(dim=1).clamp_min(1e-30)).max())
    return {"tokens_checked": len(rows), "max_rel": round(tensor_rel, 5), "worst_row_l2_rel": round(row_l2, 5),
            "tolerance": rel, "ok": bool(tensor_rel <= rel and row_l2 <= rel and torch.isfinite(got).all())}


def torch_mixer_step(m, x, conv, state):
    """The Gated DeltaNet mixer step in torch on the GPU, fp32 arithmetic with
    the Transformers forward's bf16 rounding points ([HF]
    Qwen3_5MoeGatedDeltaNet.forward 430-543, causal_conv1d_update,
    torch_recurrent_gated_delta_rule, Qwen3_5MoeRMSNormGated): the bench's
    gate for the mixer case.  x [T, 2048] bf16, conv [8192, 4] bf16, state
    [32, 128, 128] fp32 (not modified).  Returns out [T, 2048] fp32."""
    r = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    xf = x.float()
    mixed = r(xf @ m.in_proj_qkv.float().T)                       # [T, 8192]
    z = r(xf @ m.in_proj_z.float().T)
    b = r(xf @ m.in_proj_b.float().T)
    a = r(xf @ m.in_proj_a.float().T)
    T = x.shape[0]
    seq = torch.cat([conv.float(), mixed.T], dim=1)                # [8192, 4 + T]
    w = m.conv1d.float()
    act = torch.empty_like(mixed)
    for t in range(T):
        acc = torch.zeros(seq.shape[0], device=x.device)
        for j in range(4):
            acc = torch.addcmul(acc, w[:, j], seq[:, t + 1 + j])
        act[t] = r(torch.nn.functional.silu(r(acc)))
    beta = r(torch.sigmoid(b))
    g = -m.A_log.float().exp() * torch.nn.functional.softplus(a + m.dt_bias.float())
    G = g.exp()

    def l2(v):  # torch l2norm on bf16 tensors: every step rounded
        vb = v.to(torch.bfloat16)
        inv = torch.rsqrt((vb * vb).sum(-1, keepdim=True) + 1e-6)
        return (vb * inv).float()

    S = state.float().clone()
    core = torch.empty(T, 32, 128, device=x.device)
    for t in range(T):
        q = l2(act[t, :2048].view(16, 128)).repeat_interleave(2, 0) * (128 ** -0.5)
        k = l2(act[t, 2048:4096].view(16, 128)).repeat_interleave(2, 0)
        v = act[t, 4096:].view(32, 128)
        S = S * G[t][:, None, None]
        mem = (S * k[:, :, None]).sum(1)
        delta = (v - mem) * beta[t][:, None]
        S = S + k[:, :, None] * delta[:, None, :]
        core[t] = r((S * q[:, :, None]).sum(1))
    var = (core * core).mean(-1, keepdim=True)
    n = r(core * torch.rsqrt(var + m.eps))
    normed = r(r(m.norm.float() * n) * torch.nn.functional.silu(z.view(T, 32, 128)))
    return normed.view(T, 4096) @ m.out_proj.float().T


# ---- CPU baseline: the reference kernel in a pinned child process ---------------

def cpu_placement(limit: int = 16) -> tuple[list[int], int]:
    """One CPU per physical core among those this process may run on (SMT
    siblings dropped), at most `limit` (the box's CPU share for one GPU).
    Returns (cpus, number of CPUs available)."""
    allowed = sorted(os.sched_getaffinity(0))
    first = {}
    for cpu in allowed:
        try:
            key = Path(f"/sys/devices/system/cpu/cpu{cpu}/topology/thread_siblings_list").read_text().strip()
        except OSError:
            key = str(cpu)
        first.setdefault(key, cpu)
    return sorted(first.values())[:limit], len(allowed)


def cpu_leg(model, calls, kernel: str, budget_s: float, min_calls: int) -> dict | None:
    """Time the reference CPU expert kernel (oracle/_ref/libcpu_experts.so,
    built from edge35b/cpu_experts.c) on `calls` = [(layer, experts [R],
    tokens [R], hidden bits [T, 2048])], one kernel call each, round-robin.
    The expert rows are staged in /dev/shm; oracle/cpu_baseline.py runs the
    calls in a child process pinned one thread per physical core (taskset,
    OMP_PLACES=cores, OMP_PROC_BIND=close, OMP_WAIT_POLICY=PASSIVE)."""
    from numpy.lib.format import open_memmap

    if not (ROOT / "oracle" / "_ref" / "libcpu_experts.so").exists():
        return None
    keys = sorted({(l, int(e)) for l, es, _, _ in calls for e in es})
    index = {k: i for i, k in enumerate(keys)}
    shm = Path("/dev/shm")
    with tempfile.TemporaryDirectory(dir=shm if shm.is_dir() else None, prefix="lrmoe_cpu_") as tmp:
        d = Path(tmp)
        gu = open_memmap(d / "gate_up.npy", mode="w+", dtype=np.uint16, shape=(len(keys), GATE_UP_ELEMENTS))
        dn = open_memmap(d / "down.npy", mode="w+", dtype=np.uint16,
                         shape=(len(keys), EXPERT_ELEMENTS - GATE_UP_ELEMENTS))
        for i, (l, e) in enumerate(keys):
            row = model.bank.bank[l, e].cpu().view(torch.int16).numpy().view(np.uint16)
            gu[i] = row[:GATE_UP_ELEMENTS]
            dn[i] = row[GATE_UP_ELEMENTS:]
        gu.flush()
        dn.flush()
        del gu, dn
        width = max(len(es) for _, es, _, _ in calls)
        tokens = max(x.shape[0] for *_, x in calls)
        rows = np.full((len(calls), width), -1, dtype=np.int32)
        toks = np.zeros((len(calls), width), dtype=np.int32)
        hidden = np.zeros((len(calls), tokens, HIDDEN), dtype=np.uint16)
        for c, (l, es, ts, x) in enumerate(calls):
            rows[c, :len(es)] = [index[(l, int(e))] for e in es]
            toks[c, :len(ts)] = ts
            hidden[c, :x.shape[0]] = x
        np.save(d / "rows.npy", rows)
        np.save(d / "tokens.npy", toks)
        np.save(d / "nrows.npy", np.array([len(es) for _, es, _, _ in calls], dtype=np.int32))
        np.save(d / "hidden.npy", hidden)
        (d / "meta.json").write_text(json.dumps({"kernel": kernel, "budget_s": budget_s, "min_calls": min_calls}))
        cpus, available = cpu_placement()
        cpu_list = ",".join(map(str, cpus))
        cmd = [sys.executable, "-m", "oracle.cpu_baseline", str(d), cpu_list]
        pinned = "sched_setaffinity"
        if shutil.which("taskset"):
            cmd = ["taskset", "-c", cpu_list, *cmd]
            pinned = "taskset + sched_setaffinity"
        env = {**os.environ, "OMP_WAIT_POLICY": "PASSIVE", "OMP_PROC_BIND": "close", "OMP_PLACES": "cores"}
        res = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=4 * budget_s + 300)
        if res.returncode != 0:
            log(f"[bench] CPU leg failed ({res.returncode}): {res.stderr[-2000:]}")
            return None
        out = json.loads(res.stdout.strip().splitlines()[-1])
    out.update(cores=len(cpus), cpus_available=available, pinned=pinned, staged_experts=len(keys))
    return out


def cpu_legs(model, legs: dict, budget: float) -> dict:
    """The reference CPU kernel on each measured workload's own routes."""
    res = {}
    if "t1" in legs:
        calls = [(l, idx[0].tolist(), [0] * 8, x) for l, idx, x in legs["t1"]]
        r = cpu_leg(model, calls, "expert_rows", 3.0 * budget, 3 * len(calls))
        if r:
            us = 1e6 * r["sec_per_call"]
            res["c0_decode_t1"] = dict(us_per_layer=round(us, 1), gbs=round(8 * EXPERT_BYTES / us / 1e3, 2),
                                       cores=r["cores"], kind="reference",
                                       sample=f"expert_rows, 8 routed experts (T=1), {r['calls']} calls cycling over "
                                              f"{len(calls)} layers' routes, {r['cores']} threads pinned "
                                              f"({r['pinned']}) of {r['cpus_available']} CPUs")
            res["c3_chain_t1"] = dict(ms_per_step=round(40 * us / 1e3, 3), cores=r["cores"], kind="reference",
                                      sample=f"scaled: 40 x the per-layer expert_rows time above ({len(calls)}-layer "
                                             "sample); routed experts only")
    if "c2" in legs:
        calls, nbytes = [], []
        for l, idx, x in legs["c2"]:
            es = idx.ravel().tolist()
            calls.append((l, es, np.repeat(np.arange(idx.shape[0]), idx.shape[1]).tolist(), x))
            nbytes.append(len(set(es)) * EXPERT_BYTES)
        r = cpu_leg(model, calls, "expert_block_rows", 8.0 * budget, 3 * len(calls))
        if r:
            moved = sum(nbytes[i % len(nbytes)] for i in range(r["calls"]))
            res["c2_verify_t8_zipf"] = dict(
                value=round(moved / r["seconds"] / 1e9, 2), unit="GB/s", cores=r["cores"], kind="reference",
                ms_per_layer=round(1e3 * r["sec_per_call"], 3),
                sample=f"{r['calls']} calls cycling over {len(calls)} layers' T=8 Zipf routes "
                       f"({sum(nbytes) / 2**20:.0f} MiB of unique experts), expert_block_rows with {r['cores']} "
                       f"OpenMP threads pinned one per physical core ({r['pinned']}; {r['cpus_available']} CPUs "
                       "available, at most 16 used), 64 rows per call; routed experts only (the reference CPU path "
                       "has no router, combine or shared expert)")
    if "c3_t16" in legs:
        calls, nbytes = [], []
        for l, idx, x in legs["c3_t16"]:
            es = idx.ravel().tolist()
            calls.append((l, es, np.repeat(np.arange(idx.shape[0]), idx.shape[1]).tolist(), x))
            nbytes.append(len(set(es)) * EXPERT_BYTES)
        r = cpu_leg(model, calls, "expert_block_rows", 4.0 * budget, 2 * len(calls))
        if r:
            ms = 1e3 * r["sec_per_call"]
            res["c3_chain_t16"] = dict(ms_per_step=round(40 * ms, 3), ms_per_layer=round(ms, 3),
                                       gbs=round(np.mean(nbytes) / (ms * 1e-3) / 1e9, 2), cores=r["cores"],
                                       kind="reference",
                                       sample=f"scaled: 40 x the per-layer time of expert_block_rows with 128 rows over "
                                              f"16 tokens, {r['calls']} calls cycling over {len(calls)} layers' "
                                              f"routes; {r['cores']} threads pinned; routed experts only")
    if "c4" in legs:
        l, idx, x = legs["c4"]
        calls = []
        for c in range(0, idx.shape[0], 16):
            chunk = idx[c:c + 16]
            calls.append((l, chunk.ravel().tolist(), np.repeat(np.arange(chunk.shape[0]), 8).tolist(), x[c:c + 16]))
        r = cpu_leg(model, calls, "expert_block_rows", 2.0 * budget, len(calls))
        if r:
            ms_layer = 1e3 * r["sec_per_call"] * len(calls)
            flops = idx.size * PAIR_FLOP
            res["c4_prefill_t2048"] = dict(ms_per_layer=round(ms_layer, 2),
                                           gflops=round(flops / (ms_layer * 1e-3) / 1e9, 1), cores=r["cores"],
                                           kind="reference",
                                           sample=f"{len(calls)} chunks of 16 tokens (128 rows each) of one layer's "
                                                  f"T=2048 routes, {r['calls']} calls, {r['cores']} threads pinned; "
                                                  "routed experts only")
    return res


def cpu_workers_t1(model, legs_t1, budget_s: float = 3.0) -> dict | None:
    """The reference's persistent CPU expert workers (oracle/_ref/
    libpacked_workers.so, built from edge35b/packed_workers.cpp) on T=1
    decode routes: one submit/wait of the 8 routed experts per layer, cycling
    over the sample layers' host copies.  GB/s on the 8 x 6 MiB expert
    bytes.  Its own std::thread pool, one thread per physical core."""
    import ctypes as C

    from oracle import oracle as O

    ref = O.reference_workers()
    if ref is None:
        return None
    threads = len(cpu_placement()[0])
    calls = []
    for layer, idx, x in legs_t1:
        rows = [model.bank.bank[layer, e].cpu().view(torch.int16).numpy().view(np.uint16) for e in idx[0].tolist()]
        gates = (C.c_void_p * 8)(*[r.ctypes.data for r in rows])
        downs = (C.c_void_p * 8)(*[r.ctypes.data + 2 * GATE_UP_ELEMENTS for r in rows])
        calls.append((gates, downs, np.ascontiguousarray(x[0]), rows))
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


MIXER_LAYERS = 30  # linear-attention layers of the 35B model
MIXER_WEIGHT_BYTES = ((8192 + 4096 + 2 * 32) * HIDDEN + HIDDEN * 4096) * 2


def mixer_bytes(tokens: int) -> int:
    """Algorithmic HBM bytes of one mixer step: the weights once, the fp32
    recurrent state and the conv state read and written, per token the
    hidden row in and the output row out."""
    return MIXER_WEIGHT_BYTES + 2 * (32 * 128 * 128 * 4) + 2 * (8192 * 4 * 2) + tokens * 2 * HIDDEN * 2


def bench_mixers(device, seed: int, passes: int, skip_cpu: bool) -> dict:
    """C7: one cached Gated DeltaNet mixer step (lrmoe_delta_mixer: in_proj +
    conv, the delta rule, the gated RMSNorm, out_proj) at T = 1 (decode) and
    T = 16 (a verify block, no state records), rotating over 30 resident
    layers (1.9 GiB of weights, so no step finds its weights in the Infinity
    Cache), as graph replays; per-kernel times from event pairs stamped by the
    kernels' own dispatches; a torch gate on layer 0 before timing."""
    from lightreason_amd.delta import mixer_status
    from lightreason_amd.synthetic import SyntheticMixers

    mix = SyntheticMixers(MIXER_LAYERS, device, seed)
    out = {}
    for T in (1, 16):
        xs = [mix.hidden(T, step=l) for l in range(MIXER_LAYERS)]
        outs = [torch.empty(T, HIDDEN, dtype=torch.bfloat16, device=device) for _ in range(MIXER_LAYERS)]
        conv0, state0 = mix.conv[0].clone(), mix.state[0].clone()
        want = torch_mixer_step(mix.mixers[0], xs[0], conv0, state0)
        got = mix.mixers[0].step(xs[0], conv0, state0).float()
        tensor_rel = float((got - want).abs().max() / want.abs().max().clamp_min(1e-30))
        row_l2 = float(((got - want).norm(dim=1) / want.norm(dim=1).clamp_min(1e-30)).max())
        gate = {"tokens_checked": T, "max_rel": round(tensor_rel, 5), "worst_row_l2_rel": round(row_l2, 5),
                "tolerance": 1e-2, "ok": bool(tensor_rel <= 1e-2 and row_l2 <= 1e-2 and torch.isfinite(got).all())}

        def run(n, T=T, xs=xs, outs=outs):
            for i in range(n):
                l = i % MIXER_LAYERS
                mix.mixers[l].step(xs[l], mix.conv[l], mix.state[l], out=outs[l])

        steps = MIXER_LAYERS * passes
        graph = capture(lambda: run(steps))
        graph.replay()
        ms = timed_replays(graph, 1) / steps
        del graph
        torch.cuda.synchronize()
        _native.timing_enable(_native.STAGE_DELTA_MIXER, 2 * MIXER_LAYERS + 8)
        run(2 * MIXER_LAYERS)
        total, n = _native.timing_collect(_native.STAGE_DELTA_MIXER)
        _native.timing_enable(0)
        kernel_us = total / max(n, 1) * 1e3
        nbytes = mixer_bytes(T)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"t{T}"] = dict(us_per_layer=round(ms * 1e3, 2), algorithmic_bytes=nbytes, gbs=round(gbs, 1),
                            frac_hbm=round(gbs / HBM_PEAK_GBS, 4), dn_mixer_us=round(kernel_us, 2),
                            dn_mixer_gbs=round(nbytes / (kernel_us * 1e-6) / 1e9, 1), parity=gate,
                            status=mixer_status(device))
    if not skip_cpu:
        out["cpu_reference"] = mixer_cpu_leg(mix)
    return out


def mixer_cpu_leg(mix, budget_s: float = 3.0) -> dict:
    """The oracle's C mixer step (oracle/lro.c lro_delta_mixer, one thread:
    the reference has no CPU implementation of this step) at T = 1 on layer
    0's weights, as many calls as fit in `budget_s`."""
    from oracle import oracle as O

    m = mix.mixers[0]
    w = {name: bits(getattr(m, name)) for name in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "conv1d",
                                                   "A_log", "dt_bias", "norm", "out_proj")}
    x, conv, state = bits(mix.hidden(1, step=0)), bits(mix.conv[0]), mix.state[0].cpu().numpy()
    calls, t0 = 0, time.perf_counter()
    while calls < 2 or time.perf_counter() - t0 < budget_s:
        O.delta_mixer(x, w, conv, state, eps=m.eps)
        calls += 1
    sec = (time.perf_counter() - t0) / calls
    return {"value": round(sec * 1e6, 1), "unit": "us per T=1 mixer step", "cores": 1, "kind": "port",
            "sample": f"{calls} calls of the oracle's C mixer step on one layer"}


ATTN_LAYERS = 10     # full-attention layers of the 35B model
ATTN_CONTEXT = 4096  # cached positions before each C8 step
ATTN_WEIGHT_BYTES = ((8192 + 512 + 512) * HIDDEN + HIDDEN * 4096) * 2


def attn_bytes(tokens: int, length: int) -> int:
    """Algorithmic HBM bytes of one full-attention step: the weights once,
    the key and value rows of every position read (2 heads x 256 x 2 B
    each), the new rows written, per token the hidden row in and out."""
    return ATTN_WEIGHT_BYTES + (length + tokens) * 2 * 2 * 256 * 2 + tokens * 2 * 2 * 256 * 2 + tokens * 2 * HIDDEN * 2


def torch_attn_step(a, x, cos, sin, k_cache, v_cache, length):
    """The full-attention step in torch on the GPU, fp32 arithmetic with the
    Transformers eager forward's bf16 rounding points ([HF]
    Qwen3_5MoeAttention.forward, Qwen3_5MoeRMSNorm, apply_rotary_pos_emb,
    eager_attention_forward): the bench's gate for C8.  Caches are read, not
    modified.  Returns out [T, 2048] fp32."""
    r = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    T = x.shape[0]
    xf = x.float()
    qg = r(xf @ a.q_proj.float().T).view(T, 16, 512)
    q, gate = qg[..., :256], qg[..., 256:]
    k = r(xf @ a.k_proj.float().T).view(T, 2, 256)
    v = r(xf @ a.v_proj.float().T).view(T, 2, 256)

    def norm_rope(h, w):
        n = r((h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + a.eps)) * (1.0 + w.float()))
        c, s_ = cos.float()[:, None, :], sin.float()[:, None, :]
        rot = torch.cat([-n[..., 32:64], n[..., :32]], dim=-1)
        return torch.cat([r(r(n[..., :64] * c) + r(rot * s_)), n[..., 64:]], dim=-1)

    q, k = norm_rope(q, a.q_norm), norm_rope(k, a.k_norm)
    keys = torch.cat([k_cache[:, :length].float(), k.transpose(0, 1)], dim=1)     # [2, L + T, 256]
    vals = torch.cat([v_cache[:, :length].float(), v.transpose(0, 1)], dim=1)
    kk, vv = keys.repeat_interleave(8, 0), vals.repeat_interleave(8, 0)          # [16, L + T, 256]
    s = r(torch.einsum("thd,hpd->htp", q, kk)) * 0.0625
    mask = torch.arange(length + T, device=x.device)[None, :] > (length + torch.arange(T, device=x.device))[:, None]
    s = s.masked_fill(mask[None], float("-inf"))
    p = r(torch.softmax(s, dim=-1))
    o = r(torch.einsum("htp,hpd->thd", p, vv))
    att = r(o * r(torch.sigmoid(gate))).reshape(T, 4096)
    return r(att @ a.o_proj.float().T)


def bench_attention(device, seed: int, passes: int, skip_cpu: bool) -> dict:
    """C8: one cached full-attention decode step (lrmoe_attn_decode) at T = 1
    (decode) and T = 16 (a verify block) after 4096 cached positions,
    rotating over 10 resident layers (0.55 GB of weights: no step finds its
    weights in the Infinity Cache), as graph replays; the step's kernel time
    from the event pair stamped by its first and last dispatches; a torch
    gate on layer 0 before timing.  Random weights ~N(0, 0.02), norms
    ~N(0, 0.1), cached rows ~N(0, 1)."""
    from lightreason_amd.attention import AttentionDecode

    g = torch.Generator(device=device).manual_seed(seed + 8)
    rnd = lambda *shape, s=0.02: (torch.randn(*shape, generator=g, device=device) * s).to(torch.bfloat16)  # noqa: E731
    layers = [AttentionDecode(q_proj=rnd(8192, HIDDEN), k_proj=rnd(512, HIDDEN), v_proj=rnd(512, HIDDEN),
                              o_proj=rnd(HIDDEN, 4096), q_norm=rnd(256, s=0.1), k_norm=rnd(256, s=0.1))
              for _ in range(ATTN_LAYERS)]
    L = ATTN_CONTEXT
    caches = [(rnd(2, L + 16, 256, s=1.0), rnd(2, L + 16, 256, s=1.0)) for _ in range(ATTN_LAYERS)]
    pos = torch.arange(L, L + 16, device=device, dtype=torch.float32)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, device=device, dtype=torch.float32) / 64))
    ang = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=1)
    cos_all, sin_all = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    out = {}
    for T in (1, 16):
        xs = [(torch.randn(T, HIDDEN, generator=g, device=device)).to(torch.bfloat16) for _ in range(ATTN_LAYERS)]
        outs = [torch.empty(T, HIDDEN, dtype=torch.bfloat16, device=device) for _ in range(ATTN_LAYERS)]
        cos, sin = cos_all[:T].contiguous(), sin_all[:T].contiguous()
        a0, (k0, v0) = layers[0], caches[0]
        want = torch_attn_step(a0, xs[0], cos, sin, k0, v0, L)
        got = a0.step(xs[0], cos, sin, k0, v0, L).float()
        tensor_rel = float((got - want).abs().max() / want.abs().max().clamp_min(1e-30))
        row_l2 = float(((got - want).norm(dim=1) / want.norm(dim=1).clamp_min(1e-30)).max())
        gate = {"tokens_checked": T, "max_rel": round(tensor_rel, 5), "worst_row_l2_rel": round(row_l2, 5),
                "tolerance": 1e-2, "ok": bool(tensor_rel <= 1e-2 and row_l2 <= 1e-2 and torch.isfinite(got).all())}

        def run(n, T=T, xs=xs, outs=outs, cos=cos, sin=sin):
            for i in range(n):
                l = i % ATTN_LAYERS
                layers[l].step(xs[l], cos, sin, caches[l][0], caches[l][1], L, out=outs[l])

        steps = ATTN_LAYERS * passes * 3
        graph = capture(lambda: run(steps))
        graph.replay()
        ms = timed_replays(graph, 1) / steps
        del graph
        torch.cuda.synchronize()
        _native.timing_enable(_native.STAGE_ATTENTION, 2 * ATTN_LAYERS + 8)
        run(2 * ATTN_LAYERS)
        total, n = _native.timing_collect(_native.STAGE_ATTENTION)
        _native.timing_enable(0)
        kernel_us = total / max(n, 1) * 1e3
        nbytes = attn_bytes(T, L)
        gbs = nbytes / (ms * 1e-3) / 1e9
        # (the event pair spans an eager step: from the first kernel's start
        # to the last one's end, host launch gaps between them included)
        out[f"t{T}"] = dict(us_per_layer=round(ms * 1e3, 2), context=L, algorithmic_bytes=nbytes, gbs=round(gbs, 1),
                            frac_hbm=round(gbs / HBM_PEAK_GBS, 4), eager_step_span_us=round(kernel_us, 2),
                            parity=gate)
    if not skip_cpu:
        out["cpu_reference"] = attn_cpu_leg(layers[0], caches[0], cos_all[:1], sin_all[:1], L)
    return out


DECODER_WIDTHS = (1, 4, 8, 16)


def bench_decoder(model, device, seed: int, reps: int) -> dict:
    """C9: the whole 35B decoder step (per layer the input RMSNorm, the Gated
    DeltaNet mixer or the full attention, the residual add, the MoE block;
    30 + 10 layers over the resident MoE blocks of `model`) as one captured
    graph per verify width (lightreason_amd.decoder.VerifyPass) after 4096
    cached positions, fp32 mixer states; ms per verify pass, and HBM bytes
    touched per pass: every layer's unique routed experts, shared expert,
    router and norm rows; every mixer's weights and state read and written;
    every attention layer's weights and cached rows."""
    from lightreason_amd.decoder import VerifyPass, is_full_attention
    from lightreason_amd.synthetic import SyntheticDecoder

    L = len(model.layers)
    t0 = time.perf_counter()
    dec = SyntheticDecoder(L, device, seed, context=ATTN_CONTEXT, moe=model)
    vp = VerifyPass(dec.stack, DECODER_WIDTHS, ATTN_CONTEXT)
    torch.cuda.synchronize()
    log(f"[bench] C9 decoder stack ({sum(not is_full_attention(l) for l in range(L))} Gated DeltaNet + "
        f"{sum(is_full_attention(l) for l in range(L))} attention layers) captured in {time.perf_counter() - t0:.1f}s")
    out = {}
    for W in DECODER_WIDTHS:
        x = dec.hidden(W, step=900 + W)
        cos, sin = dec.rope(W, ATTN_CONTEXT)
        vp.verify(x, cos, sin)  # warm, and the status words checked
        graph, static = vp.graphs[W]
        ms = timed_replays(graph, reps) / reps
        dec.stack.check_status()
        uniques = [len(set(i.ravel().tolist())) for i in static["buffers"].indices.cpu().numpy()]
        nbytes = 0
        for l in range(L):
            nbytes += uniques[l] * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES + 4 * HIDDEN  # norm rows in, h out
            nbytes += attn_bytes(W, ATTN_CONTEXT) if is_full_attention(l) else mixer_bytes(W)
            nbytes += HIDDEN * 2  # the input RMSNorm weight
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"t{W}"] = dict(ms_per_pass=round(ms, 4), positions_per_s=round(W / (ms * 1e-3), 1),
                            bytes_per_pass=nbytes, gbs=round(gbs, 1), frac_hbm=round(gbs / HBM_PEAK_GBS, 4),
                            mean_unique=round(float(np.mean(uniques)), 1))
    del vp, dec
    torch.cuda.empty_cache()
    out["note"] = ("one replay = one verify pass of the 40-layer decoder (embedding and lm_head omitted) after "
                   f"{ATTN_CONTEXT} cached positions, router-driven routes; status words checked after timing")
    return out


def attn_cpu_leg(a, cache, cos, sin, length, budget_s: float = 3.0) -> dict:
    """The oracle's C attention step (oracle/lro.c lro_attn_decode, one
    thread: the reference runs this step in Transformers) at T = 1 after
    `length` cached positions, as many calls as fit in `budget_s`."""
    from oracle import oracle as O

    w = {name: bits(getattr(a, name)) for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")}
    x = bits(torch.randn(1, HIDDEN, device=cos.device).to(torch.bfloat16))
    kc, vc = bits(cache[0]), bits(cache[1])
    c, s_ = bits(cos), bits(sin)
    calls, t0 = 0, time.perf_counter()
    while calls < 2 or time.perf_counter() - t0 < budget_s:
        O.attn_decode(x, w, c, s_, kc, vc, length, eps=a.eps)
        calls += 1
    sec = (time.perf_counter() - t0) / calls
    return {"value": round(sec * 1e6, 1), "unit": "us per T=1 attention step", "cores": 1, "kind": "port",
            "sample": f"{calls} calls of the oracle's C attention step on one layer, {length} cached positions"}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=400, help="timed headline steps (T=8 layer calls)")
    parser.add_argument("--warmup", type=int, default=40, help="untimed headline steps before the timed ones")
    parser.add_argument("--layers", type=int, default=40, help="resident layers (40 = the whole model)")
    parser.add_argument("--seed", type=int, default=2026)
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--skip-prefill", action="store_true")
    parser.add_argument("--cpu-budget", type=float, default=1.0, help="scale of the CPU legs' time budgets")
    parser.add_argument("--only", default="", help="comma list of c0,c1,c3,c4,c5,c6,c7,c8,c9 to run besides the headline "
                                                   "(default all)")
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="also run a plain 256 MiB device copy (untimed) so that HBM byte counters "
                             "of a profiler run can be scaled by a kernel of known traffic")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(multi-GPU sharding is a design note only)", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    _native.device_check()
    t0 = time.perf_counter()
    model = SyntheticModel(layers=args.layers, device=device, seed=args.seed, shared=True, norm="normal")
    torch.cuda.synchronize()
    log(f"[bench] {args.layers} layers resident ({model.bank.nbytes / 2**30:.1f} GiB experts) "
        f"in {time.perf_counter() - t0:.1f}s")
    L = args.layers
    aux = max(2, min(10, args.steps // L))  # graph replays of the secondary configs
    only = set(filter(None, args.only.split(","))) or {"c0", "c1", "c3", "c4", "c5", "c6", "c7", "c8", "c9"}
    if args.skip_prefill:
        only.discard("c4")
    configs = {}
    cpu_routes = {}
    statuses = {}
    if args.calibrate_copy:
        src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- headline: T=8 Zipf verify; a step = one layer call ----
    logits = [bf16_from_f64(zipf_logits(8, args.seed * 1000 + l), device) for l in range(L)]
    c2 = Case(model, 8, logits=logits)
    uniques = c2.unique_counts()
    gate2 = parity_gate(model, 0, c2.x[0], c2.out[0], c2.idx[0], c2.wts[0], range(8))
    log(f"[bench] C2 parity gate (fp32 torch, layer 0, 8 tokens): {gate2}")
    warm_graph = capture(lambda: c2.run_steps(args.warmup)) if args.warmup else None
    step_graph = capture(lambda: c2.run_steps(args.steps))
    if warm_graph is not None:
        warm_graph.replay()
    ms = timed_replays(step_graph, 1)
    statuses["c2"] = c2.status()
    ms_step = ms / args.steps
    step_uniques = [uniques[i % L] for i in range(args.steps)]
    bytes_step = float(np.mean(step_uniques)) * EXPERT_BYTES + SHARED_BYTES
    gbs = bytes_step / (ms_step * 1e-3) / 1e9
    spread = {}
    bench_case(c2, aux, 1, spread)
    log(f"[bench] C2 T=8 zipf: {args.steps} steps after {args.warmup} warmup: {ms_step * 1e3:.2f} us/layer, "
        f"U={np.mean(step_uniques):.1f}, {gbs:.0f} GB/s, per-replay us/layer {spread}")
    del warm_graph, step_graph
    # The T <= 16 layer is one kernel (moe_decode): its launches are timed
    # with start/stop events stamped by the dispatch itself.
    layer_ms, layer_launches = kernel_time(c2, _native.STAGE_LAYER, passes=aux)
    stage_us = {"moe_decode": round(layer_ms * 1e3, 2)}
    # Algorithmic bytes of one launch: the unique routed experts and the
    # shared expert (6 MiB each), the shared-expert gate row, and per token
    # the hidden row in, the logits row in and the output row out.
    layer_bytes = (np.mean(uniques) + 1) * EXPERT_BYTES + 2 * HIDDEN + 8 * (2 * HIDDEN + 2 * 256 + 2 * HIDDEN)
    layer_gbs = layer_bytes / (layer_ms * 1e-3) / 1e9
    log(f"[bench] C2 moe_decode kernel (event-bracketed): {stage_us['moe_decode']} us, {layer_gbs:.0f} GB/s")
    configs["c2_verify_t8_zipf"] = dict(us_per_layer=round(ms_step * 1e3, 2),
                                        unique_experts=round(float(np.mean(step_uniques)), 2), gbs=round(gbs, 1),
                                        frac_hbm=round(gbs / HBM_PEAK_GBS, 4), stage_us=stage_us,
                                        us_per_layer_spread=spread, parity=gate2, status=statuses["c2"])
    cpu_routes["c2"] = [(c2.layer_ids[j], c2.idx[j].cpu().numpy(), bits(c2.x[j])) for j in range(min(L, 8))]

    # ---- C0: T=1 decode layer with the router ----
    if "c0" in only:
        c0 = Case(model, 1)
        c0.unique_counts()
        ms0 = bench_case(c0, aux, 1) / L
        statuses["c0"] = c0.status()
        b0 = 8 * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES
        st0 = {"moe_decode": round(kernel_time(c0, _native.STAGE_LAYER, passes=2)[0] * 1e3, 2)}
        configs["c0_decode_t1"] = dict(us_per_layer=round(ms0 * 1e3, 2), gbs=round(b0 / (ms0 * 1e-3) / 1e9, 1),
                                       frac_hbm=round(b0 / (ms0 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), stage_us=st0,
                                       status=statuses["c0"])
        cpu_routes["t1"] = [(c0.layer_ids[j], c0.idx[j].cpu().numpy(), bits(c0.x[j])) for j in range(min(L, 8))]
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
            msg = bench_case(gcase, aux, 1) / L
            u = float(np.mean([len(sel) for sel in per_layer]))
            moved = 2 * u * EXPERT_BYTES
            gather_res[f"t{T}"] = dict(unique=round(u, 1), us=round(msg * 1e3, 2),
                                       gbs_moved=round(moved / (msg * 1e-3) / 1e9, 1))
            # Bytes check of the last layer's copies (the graph ran it last).
            last = per_layer[-1]
            torch.cuda.synchronize()
            ok = all(torch.equal(staging[i].view(torch.int16), model.bank.bank[L - 1, e].view(torch.int16))
                     for i, e in enumerate(last))
            gather_res[f"t{T}"]["bytes_equal"] = ok
            if T == 8:
                t8_layers = per_layer
        for codec in ("tile", "escape"):
            sel8 = t8_layers[:min(L, 8)]
            ccase = CodecGatherCase(model, sel8, staging, device, codec)
            msc = bench_case(ccase, aux, 1) / len(sel8)
            u = float(np.mean([len(sel) for sel in sel8]))
            torch.cuda.synchronize()
            ok = all(torch.equal(staging[i].view(torch.int16), model.bank.bank[len(sel8) - 1, e].view(torch.int16))
                     for i, e in enumerate(sel8[-1]))
            gather_res[f"t8_{codec}_codec"] = dict(
                unique=round(u, 1), us=round(msc * 1e3, 2),
                gbs_raw_equivalent=round(2 * u * EXPERT_BYTES / (msc * 1e-3) / 1e9, 1),
                read_fraction=round(ccase.read_bytes / (u * EXPERT_BYTES), 4),
                gbs_moved=round((ccase.read_bytes + u * EXPERT_BYTES) / (msc * 1e-3) / 1e9, 1), bytes_equal=ok)
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
                ms3 = bench_case(c3, max(2, aux // 2), 1)
                key = f"c3_chain_t{T}" if one_launch else f"c3_layer_graph_t{T}"
                statuses[key] = c3.status()
                b3 = sum(u * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES + 2 * HIDDEN for u in u3)
                configs[key] = dict(layers=L, ms_per_step=round(ms3, 4), gbs=round(b3 / (ms3 * 1e-3) / 1e9, 1),
                                    frac_hbm=round(b3 / (ms3 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                    mean_unique=round(float(np.mean(u3)), 1), status=statuses[key],
                                    launches="one persistent launch" if one_launch else "one per layer, in a graph")
                if T == 16 and one_launch:
                    cpu_routes["c3_t16"] = [(c3.layer_ids[j], c3.idx[j].cpu().numpy(), bits(c3.x[j]))
                                            for j in range(min(L, 4))]
                log(f"[bench] C3 T={T} {'chain' if one_launch else 'per-layer'}: {ms3:.3f} ms/step over {L} layers, "
                    f"{configs[key]['gbs']} GB/s")

    # ---- C6: verify widths (speculative-verify blocks of 1-16 positions) ----
    if "c6" in only:
        from lightreason_amd.verify import VerifyGraphs

        sweep = {}
        for W in (1, 2, 4, 6, 8, 10, 12, 14, 16):
            lgw = [bf16_from_f64(zipf_logits(W, args.seed * 1000 + 500 + l), device) for l in range(L)]
            cw = Case(model, W, logits=lgw)
            uw = cw.unique_counts()
            msw = bench_case(cw, aux, 1) / L
            bw = float(np.mean(uw)) * EXPERT_BYTES + SHARED_BYTES
            sweep[f"t{W}"] = dict(us_per_layer=round(msw * 1e3, 2), unique_experts=round(float(np.mean(uw)), 1),
                                  gbs=round(bw / (msw * 1e-3) / 1e9, 1), status=cw.status())
            del cw
        stacks = {}
        layers_n = [LayerWeights(**ly.__dict__) for ly in model.layers]
        vg = VerifyGraphs(layers_n, widths=(4, 8, 12, 16))
        for W in (4, 8, 12, 16):
            xw = model.hidden(W, step=700 + W)
            vg.verify(xw)
            torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = max(3, aux)
            start.record()
            for _ in range(reps):
                vg.verify(xw)
            stop.record()
            torch.cuda.synchronize()
            msv = start.elapsed_time(stop) / reps
            idx_v, _ = vg.routes(W)
            uv = [len(set(i.ravel().tolist())) for i in idx_v.cpu().numpy()]
            bv = sum(u * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES + 2 * HIDDEN for u in uv)
            stacks[f"t{W}"] = dict(ms_per_pass=round(msv, 4), positions_per_s=round(W / (msv * 1e-3), 1),
                                   gbs=round(bv / (msv * 1e-3) / 1e9, 1), mean_unique=round(float(np.mean(uv)), 1),
                                   status=vg.status())
        del vg
        configs["c6_verify_widths"] = dict(
            layer_zipf=sweep, stack_40_graphs=stacks,
            note="layer_zipf: one decode layer per width with Zipf(1.1) Gumbel logits, graph replays rotating over "
                 "the resident layers; stack_40_graphs: the 40-layer stack (router, RMSNorm, residual) as one "
                 "captured graph per width (lightreason_amd.verify.VerifyGraphs), one replay per verify pass")
        log(f"[bench] C6 verify widths: {sweep}; 40-layer graphs {stacks}")

    # ---- C5: the decode layers reading tile-codec experts ----
    if "c5" in only:
        t0 = time.perf_counter()
        bank = CodecBank(model.bank, [(ly.shared_gate_proj, ly.shared_up_proj, ly.shared_down_proj)
                                      for ly in model.layers])
        torch.cuda.synchronize()
        misfit_tiles = float(bank.misfit.sum()) / (bank.misfit.numel() * (CODEC_GU_BASES + CODEC_DN_BASES))
        # Weight bytes read per raw byte: a fitting tile is 384 bytes and its
        # base byte instead of 512; a tile that does not fit is read raw.
        read_frac = (1 - misfit_tiles) * 385 / 512 + misfit_tiles
        log(f"[bench] C5 codec bank in {time.perf_counter() - t0:.1f}s: {bank.nbytes / 2**30:.1f} GiB, "
            f"tiles misfit {misfit_tiles:.4f}, weight bytes read x{read_frac:.3f}")
        res = dict(tiles_misfit=round(misfit_tiles, 5), weight_bytes_read_frac=round(read_frac, 4),
                   units_packed=round(bank.packed_fraction, 4), bank_gib=round(bank.nbytes / 2**30, 1))
        c5 = Case(model, 8, logits=logits, codec=bank)
        assert c5.unique_counts() == uniques
        ms5 = bench_case(c5, aux, 1) / L
        same = all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(c5.out, c2.out))
        res["c2_verify_t8_zipf"] = dict(us_per_layer=round(ms5 * 1e3, 2),
                                        raw_equivalent_gbs=round(bytes_step / (ms5 * 1e-3) / 1e9, 1),
                                        speedup_vs_raw=round(ms_step / ms5, 3), outputs_equal_raw=same,
                                        status=c5.status())
        log(f"[bench] C5 T=8 zipf codec: {ms5 * 1e3:.1f} us/layer (raw {ms_step * 1e3:.1f}), equal to raw: {same}")
        for T in (1, 16):
            c5 = Case(model, T, norm=True, chain=True, one_launch=True, codec=bank)
            u5 = c5.unique_counts()
            ms5 = bench_case(c5, max(2, aux // 2), 1)
            b5 = sum(u * EXPERT_BYTES + ROUTER_BYTES + SHARED_BYTES + 2 * HIDDEN for u in u5)
            res[f"c3_chain_t{T}"] = dict(ms_per_step=round(ms5, 4),
                                         raw_equivalent_gbs=round(b5 / (ms5 * 1e-3) / 1e9, 1), status=c5.status())
            raw = configs.get(f"c3_chain_t{T}")
            if raw is not None:
                res[f"c3_chain_t{T}"]["speedup_vs_raw"] = round(raw["ms_per_step"] / ms5, 3)
            log(f"[bench] C5 T={T} chain codec: {ms5:.3f} ms/step")
        configs["c5_codec"] = res
        del bank, c5

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
        c4.ws.check("C4 prefill")
        idx0 = c4.idx[0].cpu().numpy()
        idx_counts = [np.bincount(i.cpu().numpy().ravel(), minlength=256) for i in c4.idx]
        # Gate sample: the unit boundaries of the hottest expert (pairs
        # 127/128, 255/256, ... of its token list) and of the shared expert
        # (tokens 127/128, ...), plus tokens 63-65 of the first units.
        hot = int(np.argmax(idx_counts[0]))
        hot_tokens = np.nonzero((idx0 == hot).any(axis=1))[0]
        sample = {63, 64, 65, T - 1}
        for start in range(128, T, 128):
            sample |= {start - 1, start}
        for start in range(0, len(hot_tokens), 128):
            sample |= {int(hot_tokens[p]) for p in (start - 1, start, start + 64) if 0 <= p < len(hot_tokens)}
        rows = sorted(sample)
        gate4 = parity_gate(model, 0, c4.x[0], c4.out[0], c4.idx[0], c4.wts[0], rows)
        log(f"[bench] C4 parity gate (fp32 torch, {len(rows)} tokens): {gate4}")
        ms4 = bench_case(c4, 3, 1) / len(layer_ids)
        statuses["c4"] = c4.status()
        flops = (T * 8 + T) * PAIR_FLOP
        hit = float(np.mean([(c > 0).sum() for c in idx_counts]))
        skew = float(np.mean([c.max() / c.mean() for c in idx_counts]))
        tflops = flops / (ms4 * 1e-3) / 1e12
        # The roofline of this shape: every hit expert's weights and the
        # shared expert's read once, the token rows in and out once; the
        # ceiling is min(dense bf16 MFMA peak, HBM peak x FLOP per byte).
        c4_bytes = (hit + 1) * EXPERT_BYTES + 2 * T * HIDDEN * 2
        intensity = flops / c4_bytes
        ceiling = min(BF16_PEAK_TFLOPS, HBM_PEAK_GBS * 1e9 * intensity / 1e12)
        configs["c4_prefill_t2048"] = dict(ms_per_layer=round(ms4, 3), tflops=round(tflops, 2) if gate4["ok"] else None,
                                           frac_mfma=round(tflops / BF16_PEAK_TFLOPS, 4) if gate4["ok"] else None,
                                           flop_per_byte=round(intensity, 1), ceiling_tflops=round(ceiling, 1),
                                           frac_of_ceiling=round(tflops / ceiling, 4) if gate4["ok"] else None,
                                           experts_hit=hit, max_over_mean=round(skew, 2), bias_sigma=sigma_bias,
                                           flop_per_layer=flops, parity=gate4, status=statuses["c4"],
                                           note="router GEMV excluded (logits given)")
        cpu_routes["c4"] = (0, idx0, bits(c4.x[0]))
        log(f"[bench] C4 T=2048: {ms4:.3f} ms/layer, {tflops:.1f} TFLOPS, hit {hit}, max/mean {skew:.2f}")
        del c4

    # ---- C7: Gated DeltaNet mixer step (the 30 linear-attention layers) ----
    if "c7" in only:
        configs["c7_delta_mixer"] = bench_mixers(device, args.seed, aux, args.skip_cpu)
        log(f"[bench] C7 mixer: {configs['c7_delta_mixer']}")
    # ---- C9: the whole decoder step per verify width ----
    if "c9" in only:
        configs["c9_decoder_verify"] = bench_decoder(model, device, args.seed, max(5, 2 * aux))
        log(f"[bench] C9 decoder verify pass: {configs['c9_decoder_verify']}")

    # ---- C8: full-attention decode step (the 10 full-attention layers) ----
    if "c8" in only:
        configs["c8_attention"] = bench_attention(device, args.seed, aux, args.skip_cpu)
        log(f"[bench] C8 attention: {configs['c8_attention']}")

    cpu = {"value": None, "unit": "GB/s", "cores": 0, "kind": "reference", "sample": "skipped"}
    if not args.skip_cpu:
        t0 = time.perf_counter()
        legs = cpu_legs(model, cpu_routes, args.cpu_budget)
        if "c2_verify_t8_zipf" in legs:
            cpu = legs.pop("c2_verify_t8_zipf")
        for key, leg in legs.items():
            configs.setdefault(key, {})["cpu_reference"] = leg
        if "t1" in cpu_routes:
            configs["c0_decode_t1"]["cpu_reference_workers"] = cpu_workers_t1(model, cpu_routes["t1"])
        log(f"[bench] CPU legs in {time.perf_counter() - t0:.1f}s: headline {cpu}")

    traffic = measured_traffic("moe_decode")
    copy_gbs = copy_peak_gbs(device)
    read_gbs = read_peak_gbs(device)
    log(f"[bench] measured copy peak {copy_gbs:.0f} GB/s (read + write), read-only stream {read_gbs:.0f} GB/s")
    bad = {k: v for k, v in statuses.items() if v != 0}
    if bad:
        log(f"[bench] WARNING: non-zero workspace status after timed cases: {bad}")
    line = {
        "metric": METRIC,
        "value": round(gbs, 1) if gate2["ok"] and statuses["c2"] == 0 else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded counter-based generator; Zipf(1.1) Gumbel-top-k logits)",
        "config": {"workload": "T=8 speculative-verify MoE layer, 256 experts top-8, Zipf(1.1) routing, "
                               "shared expert, HBM GB/s on unique expert bytes; steps rotate over resident layers",
                   "tokens": 8, "hidden": HIDDEN, "experts": 256, "topk": 8, "inner": INNER,
                   "layers_rotated": L, "mean_unique_experts": round(float(np.mean(step_uniques)), 2)},
        "roofline": {"bound": "hbm", "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else traffic["bytes"],
                     "traffic_source": None if traffic is None else traffic["source"],
                     "measured_read_peak": round(read_gbs, 1), "frac_of_read_peak": round(layer_gbs / read_gbs, 4),
                     "measured_copy_peak": round(copy_gbs, 1),
                     "kernel": "moe_decode", "avg_us": round(layer_ms * 1e3, 3), "launches": layer_launches,
                     "algorithmic_bytes": int(layer_bytes)},
        "cpu_baseline": cpu,
        "status": statuses,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
