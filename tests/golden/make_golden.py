"""Write the expert-arithmetic golden vectors from the reference CPU kernel.

Runs edge35b/cpu_experts.c -- compiled from /root/reference by
oracle/Makefile into oracle/_ref/libcpu_experts.so -- on inputs drawn from the
counter-based generator, and stores the inputs' generator spec, their SHA-256
and the reference outputs in tests/golden/cpu_experts_golden.npz.

Cases:
  rows8    expert_rows, 8 experts, one token (the T=1 decode shape)
  rows3    expert_rows, 3 experts (a partial route list)
  block16  expert_block_rows, 16 rows over 4 tokens (a verify block)
  special  expert_rows, 2 experts, with a hidden state holding signed zeros,
           large magnitudes and a few exact zeros in the weights

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

SEED = 20261201
OUT = Path(__file__).resolve().parent / "cpu_experts_golden.npz"


def expert_inputs(count: int, stream0: int):
    gate_up = [O.normal_bf16((2 * O.INNER, O.HIDDEN), SEED, stream0 + 2 * e, 0.02) for e in range(count)]
    down = [O.normal_bf16((O.HIDDEN, O.INNER), SEED, stream0 + 2 * e + 1, 0.02) for e in range(count)]
    return gate_up, down


def digest(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main() -> None:
    if O.reference() is None:
        raise SystemExit("reference kernel unavailable: needs /root/reference/edge35b/cpu_experts.c")
    out = {}

    gate_up, down = expert_inputs(8, 100)
    hidden = O.normal_bf16((O.HIDDEN,), SEED, 1, 1.0)
    out["rows8_output"] = O.reference_expert_rows(gate_up, down, hidden, threads=1)
    out["rows8_sha256"] = np.frombuffer(digest([*gate_up, *down, hidden]).encode(), dtype=np.uint8)

    out["rows3_output"] = O.reference_expert_rows(gate_up[2:5], down[2:5], hidden, threads=1)

    block_gu, block_down = expert_inputs(16, 300)
    tokens = O.normal_bf16((4, O.HIDDEN), SEED, 2, 1.0)
    token_ids = np.array([0, 0, 1, 3, 2, 1, 0, 3, 3, 2, 1, 0, 2, 2, 1, 3], dtype=np.int32)
    out["block16_token_ids"] = token_ids
    out["block16_output"] = O.reference_expert_block_rows(block_gu, block_down, tokens, token_ids, threads=1)
    out["block16_sha256"] = np.frombuffer(digest([*block_gu, *block_down, tokens]).encode(), dtype=np.uint8)

    special_gu, special_down = expert_inputs(2, 500)
    special_gu[0][:, :64] = 0
    special_gu[1][5] = 0x8000
    hidden_special = O.normal_bf16((O.HIDDEN,), SEED, 3, 4.0)
    hidden_special[:16] = 0x8000
    hidden_special[16:32] = 0
    hidden_special[32] = 0x4300  # 128.0
    hidden_special[33] = 0xC300  # -128.0
    out["special_hidden"] = hidden_special
    out["special_output"] = O.reference_expert_rows(special_gu, special_down, hidden_special, threads=1)
    np.savez_compressed(OUT, seed=np.array([SEED], dtype=np.int64), **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
