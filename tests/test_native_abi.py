"""liblrmoe.so loads on the CPU host and exports every symbol include/lrmoe.h
declares; host-side argument checks reject misuse without touching a GPU."""

from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lrmoe.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(lrmoe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from lightreason_amd import _native

    if not _native.LIBRARY.exists():
        pytest.fail("liblrmoe.so is not built: run `python -m lightreason_amd.build` (or __graft_entry__.build())")
    return _native.library()


def test_every_declared_symbol_is_exported(lib):
    declared = _declared()
    assert len(declared) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "lightreason_amd" / "liblrmoe.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(lrmoe_\w+)", out))
    missing = [name for name in declared if name not in exported]
    assert not missing, missing
    from lightreason_amd import _native

    assert sorted(_native.symbols()) == declared


def test_host_side_queries(lib):
    assert lib.lrmoe_version().decode().startswith("lrmoe")
    assert lib.lrmoe_error_string(-1).decode().startswith("lrmoe: invalid argument")
    assert lib.lrmoe_error_string(-2).decode().startswith("lrmoe: workspace")
    small, big = lib.lrmoe_workspace_bytes(1), lib.lrmoe_workspace_bytes(2048)
    assert 0 < small < big
    # the workspace holds at least the expert intermediates: (8T + T) rows of 512 and 2048 bf16
    assert big >= 9 * 2048 * (512 + 2048) * 2


def test_argument_errors_are_reported_before_any_launch(lib):
    null = None
    # the no-allocation decode layer: sizes beyond its maximum and missing
    # pointers are rejected on the host
    assert lib.lrmoe_moe_layer_static(null, 17, null, null, null, null, null, null, null, null, null, 1e-6, null,
                                      null, null, null, null) == -1
    assert lib.lrmoe_moe_layer_static(null, 1, null, null, null, null, null, null, null, null, null, 1e-6, null,
                                      null, null, null, null) == -1
    assert lib.lrmoe_moe_layer_static(null, 0, null, null, null, null, null, null, null, null, null, 1e-6, null,
                                      null, null, null, null) == 0
    assert lib.lrmoe_route_topk(null, 1, null, null, null, 1e-6, null, null, null, null, null, null, null, 0,
                                null) == -1
    assert lib.lrmoe_moe_layer(null, 1, null, null, null, null, null, null, null, null, null, 1e-6, null, null, null,
                               null,
                               0, null) == -1
    dummy = C.c_void_p(16)
    # both a router and logits: refused
    assert lib.lrmoe_route_topk(dummy, 1, dummy, dummy, null, 1e-6, null, null, dummy, dummy, null, null, dummy,
                                1 << 30, null) == -1
    assert lib.lrmoe_moe_experts(null, -1, null, null, null, null, null, 0, null) == -1
    dummy = C.c_void_p(16)
    # a workspace that is too small is refused
    assert lib.lrmoe_moe_experts(dummy, 4, dummy, dummy, dummy, dummy, dummy, 8, null) == -2
    assert lib.lrmoe_matvec(dummy, dummy, dummy, 100, 8, 0, 1, 3, 8, null) == -1  # K not a multiple of 512
    assert lib.lrmoe_ordered_sum(dummy, dummy, null, dummy, dummy, 5, null) == -1
    assert lib.lrmoe_project(dummy, dummy, dummy, dummy, 2048, 1000, 0, 4, null) == -1
    assert lib.lrmoe_gather(dummy, dummy, dummy, dummy, dummy, dummy, 0, 2, 8, 64, 256, 0, null, null) == -1
    assert lib.lrmoe_gather(dummy, dummy, dummy, dummy, dummy, dummy, 8, 2, 8, 64, 100, 0, null, null) == -1
    # chain: more than 16 tokens, more than 48 layers per call, a layer
    # without a router, or only some of the shared-expert tensors: refused
    big = 1 << 30
    table = (C.c_int64 * 8)(16, 16, 16, 16, 16, 16, 0, 0)
    for tokens, layers, entry in ((17, 1, None), (1, 49, None), (1, 1, (0, 0)), (1, 1, (4, 0))):
        t = (C.c_int64 * (8 * max(layers, 1)))()
        for l in range(layers):
            for i in range(8):
                t[8 * l + i] = table[i]
        if entry is not None:
            t[entry[0]] = entry[1]
        assert lib.lrmoe_moe_chain(dummy, tokens, layers, t, C.c_float(1e-6), dummy, null, null, dummy, big,
                                   null) == -1, (tokens, layers, entry)
    assert lib.lrmoe_moe_chain(dummy, 1, 1, table, C.c_float(1e-6), dummy, null, null, dummy, 8, null) == -2
    assert lib.lrmoe_moe_chain(dummy, 1, 0, table, C.c_float(1e-6), dummy, null, null, dummy, 8, null) == 0
    # zero tokens is a successful no-op
    assert lib.lrmoe_moe_experts(dummy, 0, dummy, dummy, dummy, dummy, dummy, 0, null) == 0
    # attention decode: more than 16 tokens, a cache too short for the new
    # positions, missing pointers, a short workspace; zero tokens is a no-op
    w8 = dummy
    aligned = C.c_void_p(256)  # the workspace must be 256-byte aligned
    args = lambda tokens, cap, length, ws: (w8, tokens, w8, w8, w8, w8, w8, w8, C.c_float(1e-6), w8, w8, w8, w8,
                                            cap, length, w8, aligned, ws, null)
    assert lib.lrmoe_attn_workspace_bytes(17) == 0 and lib.lrmoe_attn_workspace_bytes(16) > 0
    assert lib.lrmoe_attn_decode(*args(17, 100, 0, big)) == -1
    assert lib.lrmoe_attn_decode(*args(4, 100, 97, big)) == -1
    assert lib.lrmoe_attn_decode(*args(4, (1 << 22) + 1, 0, big)) == -1
    assert lib.lrmoe_attn_decode(null, 1, *args(1, 100, 0, big)[2:]) == -1
    assert lib.lrmoe_attn_decode(*args(1, 100, 0, 8)) == -2
    assert lib.lrmoe_attn_decode(*args(0, 100, 0, 0)) == 0
    # the device-length variant: no length pointer, or one not 4-byte aligned
    args_at = lambda tokens, cap, length: (w8, tokens, w8, w8, w8, w8, w8, w8, C.c_float(1e-6), w8, w8, w8, w8,
                                           cap, length, w8, aligned, big, null)
    assert lib.lrmoe_attn_decode_at(*args_at(4, 100, null)) == -1
    assert lib.lrmoe_attn_decode_at(*args_at(4, 100, C.c_void_p(258))) == -1
    assert lib.lrmoe_attn_decode_at(*args_at(17, 100, aligned)) == -1
    # the fused layer steps: no input norm, or no residual output
    mix_step = lambda norm, sum_out, tokens=1: lib.lrmoe_delta_mixer_step(
        aligned, tokens, norm, C.c_float(1e-6), *([aligned] * 8), C.c_float(1e-6), aligned, aligned, aligned, 0, null,
        null, aligned, sum_out, null, aligned, big, null)
    assert mix_step(null, aligned) == -1
    assert mix_step(aligned, null) == -1
    assert mix_step(C.c_void_p(258), aligned) == -1
    assert mix_step(null, null, tokens=0) == 0
    att_step = lambda norm, sum_out, tokens=1: lib.lrmoe_attn_decode_step(
        aligned, tokens, norm, C.c_float(1e-6), *([aligned] * 6), C.c_float(1e-6), aligned, aligned, aligned, aligned,
        100, 0, null, aligned, sum_out, null, aligned, big, null)
    assert att_step(null, aligned) == -1
    assert att_step(aligned, null) == -1
    assert att_step(null, null, tokens=0) == 0
    # decoder glue: nothing to write, a sum without an addend, a norm weight
    # without its output (or the reverse), a misaligned row, a negative count
    eps = C.c_float(1e-6)
    assert lib.lrmoe_add_rmsnorm(aligned, null, 1, null, eps, null, null, null) == -1
    assert lib.lrmoe_add_rmsnorm(aligned, null, 1, null, eps, aligned, null, null) == -1
    assert lib.lrmoe_add_rmsnorm(aligned, null, 1, aligned, eps, null, null, null) == -1
    assert lib.lrmoe_add_rmsnorm(aligned, null, 1, null, eps, null, aligned, null) == -1
    assert lib.lrmoe_add_rmsnorm(C.c_void_p(8), null, 1, aligned, eps, null, aligned, null) == -1
    assert lib.lrmoe_add_rmsnorm(aligned, null, -1, aligned, eps, null, aligned, null) == -1
    assert lib.lrmoe_add_rmsnorm(aligned, null, 0, aligned, eps, null, aligned, null) == 0
    from lightreason_amd import _native

    with pytest.raises(ValueError):
        _native.call("lrmoe_fill_normal_bf16", None, 4, 0, 0, 1.0, 0, None)


def test_product_does_not_reach_the_oracle():
    """Nothing under lightreason_amd/ imports, loads or names oracle code."""
    for path in (ROOT / "lightreason_amd").rglob("*"):
        if path.suffix in {".py", ".hip", ".h", ".cpp"}:
            text = path.read_text()
            assert "import oracle" not in text and "from oracle" not in text, path
            assert "liblro" not in text and "lro_" not in text, path


def test_header_constants_match_the_bindings():
    from lightreason_amd import _native

    text = (ROOT / "include" / "lrmoe.h").read_text()
    defines = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define LRMOE_(\w+) \(?(-?\d+)\)?", text)}
    pairs = {"OK": _native.LRMOE_OK, "E_ARG": _native.LRMOE_E_ARG, "E_WORKSPACE": _native.LRMOE_E_WORKSPACE,
             "E_DEVICE": _native.LRMOE_E_DEVICE, "WS_STATUS_OFFSET": _native.WS_STATUS_OFFSET,
             "STATUS_BAD_EXPERT": _native.STATUS_BAD_EXPERT,
             "STATUS_REPEATED_EXPERT": _native.STATUS_REPEATED_EXPERT,
             "STATUS_CODEC_ROW": _native.STATUS_CODEC_ROW, "CHAIN_PTRS": _native.CHAIN_PTRS,
             "CHAIN_MAX_LAYERS": _native.CHAIN_MAX_LAYERS, "CODEC_TABLE_COLUMNS": _native.CODEC_TABLE_COLUMNS}
    for name, value in pairs.items():
        assert defines.get(name) == value, name
