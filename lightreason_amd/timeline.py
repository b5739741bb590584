"""Per-workgroup timeline of one decode layer (lrmoe_moe_layer, T <= 16),
with --mixer of one Gated DeltaNet mixer step (lrmoe_delta_mixer), or with
--attention of one full-attention step (lrmoe_attn_decode), from the
timeline build of the library (`python -m lightreason_amd.build
--timeline`: liblrmoe_timeline.so, whose decode, mixer and attention
kernels stamp the wall clock at their phases).

Runs the workload the benchmark times -- 40 resident seeded layers (seed
2026), T tokens, with Zipf(1.1) Gumbel logits (T > 1) or the router (T = 1)
-- twice over the layers so that no call finds its experts in the Infinity
Cache, stamps every 5th call of the second pass, and prints, per stamped
call, the median and maximum over workgroups of each phase (microseconds
from the first workgroup's entry) and per item step the median start, wait
for the step's weights, wait for its inputs, and end.

The mixer run steps 30 resident seeded mixers of the 35B shape (seed 7)
three times over, stamps every call of the last two passes, and prints per
phase the median over calls of the per-workgroup median and maximum.

The attention run replays a graph of one step on each of 10 resident
seeded layers of the 35B shape (4096 cached positions) and reads the
stamps of its last step after each replay: per launch (q/gate/k/v
projection, attention partials, merge, o_proj) the entry and end, and the
partial kernel's phases, as the median over replays of the per-workgroup
median and maximum, in us from the projection's first entry.

Usage: python -m lightreason_amd.timeline [--tokens T] [--layers L] [--mixer | --attention]
"""

from __future__ import annotations

import argparse
import ctypes as C
import sys

import numpy as np
import torch

from . import _native

WORDS = 128  # stamps per workgroup (kTimelineWords)
PHASES = (("entry", 0), ("counters", 7), ("top8_w0", 118), ("top8", 1), ("first_issued_w0", 2),
          ("first_issued_w7", 5), ("rows_staged", 6), ("rows_staged_w7", 121), ("masks", 119), ("slots", 120),
          ("plan", 3), ("router_rows", 122), ("published", 123), ("logits_seen", 124), ("half1_w0", 125), ("end", 4))
STEPS = 22  # item steps stamped (words 8 + 5 n .. 8 + 5 n + 4; words 118 and up hold phases)


MIXER_PHASES = (("unit 0 multiplied", 1), ("unit 0 epilogue", 2), ("unit 1 + beta/G", 3), ("phase A end", 4),
                ("barrier 1", 5), ("rule inputs staged", 11), ("q, k l2norm'd", 13), ("token loop done", 14), ("rule done", 6), ("z done, counted in", 7), ("gated norm done", 8),
                ("barrier 2", 9), ("out_proj done", 10))


def mixer_timeline(lib, tokens: int, layers: int, seed: int) -> int:
    from .delta import mixer_status
    from .synthetic import SyntheticMixers

    lib.lrmoe_mixer_timeline_set.argtypes = [C.c_void_p]
    lib.lrmoe_mixer_timeline_set.restype = C.c_int
    device = torch.device("cuda:0")
    mix = SyntheticMixers(layers, device, seed)
    stamps = torch.zeros(256 * 16, dtype=torch.int64, device=device)
    if lib.lrmoe_mixer_timeline_set(C.c_void_p(stamps.data_ptr())) != 0:
        raise RuntimeError("lrmoe_mixer_timeline_set failed")
    x = mix.hidden(tokens, 1)
    outs = [torch.empty(tokens, x.shape[1], dtype=torch.bfloat16, device=device) for _ in range(layers)]
    calls = []
    for rep in range(3):
        for l in range(layers):
            stamps.zero_()
            mix.mixers[l].step(x, mix.conv[l], mix.state[l], out=outs[l])
            torch.cuda.synchronize()
            if rep > 0:
                calls.append(stamps.view(256, 16).cpu().numpy().astype(np.int64))
    if mixer_status(device) != 0:
        raise RuntimeError(f"mixer status {mixer_status(device)}")
    st = np.stack(calls)
    rel = (st[:, :, :15] - st[:, :, 0].min(1)[:, None, None]) / 100.0
    last = st[:, :, 12] == 1
    print(f"Gated DeltaNet mixer step T={tokens}, {len(calls)} calls over {layers} layers, 256 workgroups; "
          "us from the first workgroup's entry, median over calls of the per-workgroup median / max")
    print(f"  {'entry':20s} {np.median(np.median(rel[:, :, 0], 1)):6.2f} / {np.median(rel[:, :, 0].max(1)):6.2f}")
    for name, i in MIXER_PHASES:
        v = rel[:, :, i]
        if i == 8:  # the gated norm runs on each head's last workgroup only
            med = np.median([np.median(v[c][last[c]]) for c in range(len(calls))])
            mx = np.median([v[c][last[c]].max() for c in range(len(calls))])
        else:
            med, mx = np.median(np.median(v, 1)), np.median(v.max(1))
        print(f"  {name:20s} {med:6.2f} / {mx:6.2f}")
    return 0


ATTN_PHASES = (("first barrier", 1), ("queries normed", 2), ("new positions", 3), ("sub-block 0", 4),
               ("sub-block 1", 5), ("sub-block 2", 6), ("partials stored", 7))


def attention_timeline(lib, tokens: int, layers: int, seed: int, replays: int = 20) -> int:
    from .attention import AttentionDecode

    lib.lrmoe_attn_timeline_set.argtypes = [C.c_void_p]
    lib.lrmoe_attn_timeline_set.restype = C.c_int
    device = torch.device("cuda:0")
    g = torch.Generator(device=device).manual_seed(seed)
    rnd = lambda *shape, s=0.02: (torch.randn(*shape, generator=g, device=device) * s).to(torch.bfloat16)  # noqa: E731
    hidden, context = 2048, 4096
    mods = [AttentionDecode(q_proj=rnd(8192, hidden), k_proj=rnd(512, hidden), v_proj=rnd(512, hidden),
                            o_proj=rnd(hidden, 4096), q_norm=rnd(256, s=0.1), k_norm=rnd(256, s=0.1))
            for _ in range(layers)]
    caches = [(rnd(2, context + 16, 256, s=1.0), rnd(2, context + 16, 256, s=1.0)) for _ in range(layers)]
    pos = torch.arange(context, context + tokens, device=device, dtype=torch.float32)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, device=device, dtype=torch.float32) / 64))
    ang = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=1)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    xs = [torch.randn(tokens, hidden, generator=g, device=device).to(torch.bfloat16) for _ in range(layers)]
    outs = [torch.empty(tokens, hidden, dtype=torch.bfloat16, device=device) for _ in range(layers)]
    stamps = torch.zeros(4 * 8192, dtype=torch.int64, device=device)
    if lib.lrmoe_attn_timeline_set(C.c_void_p(stamps.data_ptr())) != 0:
        raise RuntimeError("lrmoe_attn_timeline_set failed")

    def run():
        for l in range(layers):
            mods[l].step(xs[l], cos, sin, caches[l][0], caches[l][1], context, out=outs[l])

    run()  # (workspaces allocated before capture)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    calls = []
    for _ in range(replays):
        stamps.zero_()
        graph.replay()
        torch.cuda.synchronize()
        calls.append(stamps.view(4, 8192).cpu().numpy().astype(np.int64))
    del graph
    st = np.stack(calls)  # [replay][launch][word]
    t0 = np.array([c[1][c[1] > 0].min() for c in st])[:, None]  # the projection's first entry
    rel = lambda a: np.where(a > 0, (a - t0) / 100.0, np.nan)  # noqa: E731

    def row(name, v):
        med = np.nanmedian(np.nanmedian(v, 1))
        mx = np.nanmedian(np.nanmax(v, 1))
        print(f"  {name:28s} {med:6.2f} / {mx:6.2f}")

    print(f"full-attention step T={tokens}, {context} cached positions, {replays} replays of {layers} layers; "
          "us from the projection's first entry, median over replays of the per-workgroup median / max")
    # the chunk of each at_attend workgroup (the launch geometry of attention.hip)
    S = (context + tokens + 31) // 32
    halves = 2 if tokens > 8 else 1
    cap = 128 // halves
    floor_per = 1 if tokens <= 4 or 2 * halves * S <= 128 else 2
    per = max(floor_per, (S + cap) // (cap + 1))
    chunks = min((S + per - 1) // per, cap)
    b = np.arange(512)
    chunk_of = ((b >> 4) * 8 + (b & 7)) % chunks if tokens > 8 else b % chunks
    for launch, name, stride in ((1, "q/gate/k/v projection", 4), (0, "attention partials", 16),
                                 (2, "merge", 4), (3, "o_proj", 4)):
        words = st[:, launch, :].reshape(len(calls), -1, stride)
        live = (words[:, :, 0] > 0).any(0)
        if not live.any():  # (one token: the merge and o_proj are one launch, stamped as the merge)
            continue
        words = words[:, live, :]
        row(f"{name}: entry", rel(words[:, :, 0]))
        if launch == 0:
            last = chunk_of[:live.size][live] == chunks - 1
            for pname, i in ATTN_PHASES:
                v = rel(words[:, :, i])
                if not np.isnan(v).all():
                    row(f"  {pname}", v)
                    if (~np.isnan(v[:, ~last])).any():
                        row(f"    (all but the last chunk)", v[:, ~last])
                    row(f"    (the last chunk)", v[:, last])
            row(f"{name}: end", rel(words[:, :, 7]))
        else:
            row(f"{name}: end", rel(words[:, :, 1]))
    return 0


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--tokens", type=int, default=8)
    parser.add_argument("--layers", type=int, default=None, help="40 decode layers, 30 mixers")
    parser.add_argument("--seed", type=int, default=None, help="2026 decode, 7 mixers")
    parser.add_argument("--mixer", action="store_true", help="time the Gated DeltaNet mixer step instead")
    parser.add_argument("--attention", action="store_true", help="time the full-attention step instead")
    args = parser.parse_args(argv)
    from .build import TIMELINE_LIBRARY
    if not TIMELINE_LIBRARY.exists():
        print(f"{TIMELINE_LIBRARY} is missing: python -m lightreason_amd.build --timeline", file=sys.stderr)
        return 2
    _native.LIBRARY = TIMELINE_LIBRARY
    lib = _native.library()
    if args.mixer:
        return mixer_timeline(lib, args.tokens, args.layers or 30, 7 if args.seed is None else args.seed)
    if args.attention:
        return attention_timeline(lib, args.tokens, args.layers or 10, 8 if args.seed is None else args.seed)
    args.layers = args.layers or 40
    args.seed = 2026 if args.seed is None else args.seed
    lib.lrmoe_timeline_set.argtypes = [C.c_void_p]
    lib.lrmoe_timeline_set.restype = C.c_int

    from .moe import Workspace, moe_layer
    from .synthetic import SyntheticModel

    T, L = args.tokens, args.layers
    device = torch.device("cuda:0")
    model = SyntheticModel(layers=L, device=device, seed=args.seed, shared=True, norm="normal")
    G = torch.cuda.get_device_properties(0).multi_processor_count
    stamps = torch.zeros(256 * WORDS, dtype=torch.int64, device=device)
    if lib.lrmoe_timeline_set(C.c_void_p(stamps.data_ptr())) != 0:
        raise RuntimeError("lrmoe_timeline_set failed")
    rng_logits = []
    for l in range(L):
        if T == 1:
            rng_logits.append(None)
            continue
        rng = np.random.default_rng(args.seed * 1000 + l)
        ranks = rng.permutation(256) + 1
        raw = (-1.1 * np.log(ranks)[None, :] + rng.gumbel(size=(T, 256))).astype(np.float32)
        bits = raw.view(np.uint32).astype(np.uint64)
        b16 = (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)
        rng_logits.append(torch.from_numpy(b16.view(np.int16)).view(torch.bfloat16).to(device))
    xs = [model.hidden(T, step=100 + l) for l in range(L)]
    idx = [torch.empty((T, 8), dtype=torch.int64, device=device) for _ in range(L)]
    ws = Workspace(device, T)
    traces = []
    for rep in range(2):
        for l in range(L):
            stamps.zero_()
            moe_layer(xs[l], model.layers[l], logits_in=rng_logits[l], indices=idx[l], workspace=ws)
            if rep == 1 and l % 5 == 0:
                torch.cuda.synchronize()
                traces.append((l, stamps.view(256, WORDS)[:G].cpu().numpy().astype(np.int64)))
    torch.cuda.synchronize()
    ws.check("timeline run")
    print(f"decode layer T={T} ({'router' if T == 1 else 'Zipf(1.1) logits'}), {G} workgroups; "
          "times in us from the first workgroup's entry (wall clock, 10 ns)")
    for l, t in traces:
        t0 = t[:, 0].min()
        f = lambda a: np.where(a > 0, (a - t0) / 100.0, np.nan)  # noqa: E731
        unique = len(set(idx[l].cpu().numpy().ravel().tolist()))
        print(f"\nlayer {l}: {unique} unique experts")
        cells = []
        for name, i in PHASES:
            v = f(t[:, i])
            cells.append(f"{name} {np.nanmedian(v):.2f}/{np.nanmax(v):.2f}" if (~np.isnan(v)).any() else f"{name} -")
        print("  " + " | ".join(cells) + "   (median/max)")
        for name, i in (("counters", 7), ("logits_seen", 124), ("plan", 3), ("end", 4)):
            v = f(t[:, i])
            if (~np.isnan(v)).any():
                late = np.argsort(np.nan_to_num(v, nan=-1.0))[::-1][:6]
                print(f"  latest at {name}: " + ", ".join(f"wg {w} {v[w]:.2f}" for w in late))
        for n in range(STEPS):
            b = 8 + 5 * n
            s0, s1, s2, s3 = (f(t[:, b + i]) for i in range(4))
            ok = ~np.isnan(s0)
            if not ok.any():
                break
            kinds = (t[ok, b + 4] // 1000000).tolist()
            names = {1: "A", 2: "B", 3: "C", 0: "-"}
            mix = ", ".join(f"{names[k]}:{kinds.count(k)}" for k in sorted(set(kinds)))
            print(f"  step {n:2d}: {int(ok.sum()):3d} wgs  start {np.nanmedian(s0):6.2f}  weights-wait "
                  f"{np.nanmedian(s1 - s0):5.2f}  input-wait {np.nanmedian(s2 - s1):5.2f} (max {np.nanmax(s2 - s1):5.2f})"
                  f"  end {np.nanmedian(s3):6.2f} (max {np.nanmax(s3):6.2f})  items {mix}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
