"""Times the reference CPU expert kernel (edge35b/cpu_experts.c, built from
source into oracle/_ref/libcpu_experts.so by oracle/Makefile) on a staged
sample of expert rows.  TEST/BENCH INFRASTRUCTURE ONLY: bench.py's
CPU-baseline leg runs it as a child process, so that OpenMP starts in a
process of its own under the thread placement the parent chose (taskset,
OMP_PLACES=cores, OMP_PROC_BIND=close, OMP_WAIT_POLICY=PASSIVE); a process
that has imported torch already holds torch's OpenMP runtime, whose settings
were fixed at import.

Input: a directory of .npy files written by bench.py:
  gate_up.npy  uint16 [N, 1024 * 2048]   staged expert rows (gate then up)
  down.npy     uint16 [N, 2048 * 512]
  rows.npy     int32  [C, R]   per call, the staged expert row of each
                               (token, expert) output row (-1 = unused)
  tokens.npy   int32  [C, R]   per call, the token of each output row
  nrows.npy    int32  [C]      output rows per call
  hidden.npy   uint16 [C, T, 2048]  per call, its tokens' hidden rows
  meta.json    {"kernel": "expert_rows" | "expert_block_rows", "budget_s": s,
                "min_calls": n}
Calls run round-robin (one call's experts are not the next call's) until the
budget is spent and at least min_calls have run.  Prints one JSON line:
{"calls", "seconds", "threads", "sec_per_call"}.

Usage: python -m oracle.cpu_baseline DIR CPUS   (CPUS: comma list, one
thread per listed CPU; the process pins itself to them before OpenMP starts)
"""

from __future__ import annotations

import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = HERE / "_ref" / "libcpu_experts.so"


def main() -> int:
    folder = Path(sys.argv[1])
    cpus = [int(c) for c in sys.argv[2].split(",")]
    os.sched_setaffinity(0, cpus)
    threads = len(cpus)
    meta = json.loads((folder / "meta.json").read_text())
    so = C.CDLL(str(REF))
    so.expert_rows.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_int]
    so.expert_rows.restype = None
    so.expert_block_rows.argtypes = [C.c_void_p] * 5 + [C.c_int, C.c_int, C.c_int]
    so.expert_block_rows.restype = None
    gate_up = np.load(folder / "gate_up.npy", mmap_mode="r")
    down = np.load(folder / "down.npy", mmap_mode="r")
    rows = np.load(folder / "rows.npy")
    tokens = np.load(folder / "tokens.npy")
    nrows = np.load(folder / "nrows.npy")
    hidden = np.load(folder / "hidden.npy")
    gu_base, dn_base = gate_up.ctypes.data, down.ctypes.data
    gu_stride, dn_stride = gate_up.strides[0], down.strides[0]
    calls = []
    for c in range(len(nrows)):
        n = int(nrows[c])
        ids = rows[c, :n]
        gps = (C.c_void_p * n)(*[gu_base + int(i) * gu_stride for i in ids])
        dps = (C.c_void_p * n)(*[dn_base + int(i) * dn_stride for i in ids])
        x = np.ascontiguousarray(hidden[c])
        tok = np.ascontiguousarray(tokens[c, :n], dtype=np.int32)
        out = np.empty((n, 2048), dtype=np.uint16)
        calls.append((gps, dps, x, tok, out, n))
    block = meta["kernel"] == "expert_block_rows"

    def run(call):
        gps, dps, x, tok, out, n = call
        if block:
            so.expert_block_rows(gps, dps, x.ctypes.data, tok.ctypes.data, out.ctypes.data, x.shape[0], n, threads)
        else:
            so.expert_rows(gps, dps, x.ctypes.data, out.ctypes.data, n, threads)

    for call in calls:  # first touch of every staged page
        run(call)
    budget, least = float(meta["budget_s"]), int(meta["min_calls"])
    n = 0
    t0 = time.perf_counter()
    while n < least or time.perf_counter() - t0 < budget:
        run(calls[n % len(calls)])
        n += 1
    dt = time.perf_counter() - t0
    print(json.dumps({"calls": n, "seconds": dt, "threads": threads, "sec_per_call": dt / n}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
