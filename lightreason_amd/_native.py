"""ctypes binding of liblrmoe.so (include/lrmoe.h).

The library is the only compute path: when it is missing or the device is
not gfx950 every entry point raises; there is no fallback.
"""

from __future__ import annotations

import ctypes as C
from functools import lru_cache
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "liblrmoe.so"

LRMOE_OK = 0
LRMOE_E_ARG = -1
LRMOE_E_WORKSPACE = -2
LRMOE_E_DEVICE = -3
WS_STATUS_OFFSET = 4
STATUS_BAD_EXPERT = 1
STATUS_REPEATED_EXPERT = 2
STATUS_CODEC_ROW = 4
STATUS_TIMEOUT = 8       # a bounded cross-workgroup wait of the decode kernel expired: outputs invalid

STATIC_MAX_TOKENS = 16  # tokens per lrmoe_moe_layer_static call
CHAIN_PTRS = 8           # int64 addresses per layer in a chain's layer table
CHAIN_MAX_LAYERS = 48    # layers per lrmoe_moe_chain call
CODEC_TABLE_COLUMNS = 10  # int64 per expert in a decode codec table (4 addresses, 48 flag bytes)

_P = C.c_void_p
_I = C.c_int
_SIGNATURES = {
    "lrmoe_version": ([], C.c_char_p),
    "lrmoe_error_string": ([_I], C.c_char_p),
    "lrmoe_device_check": ([], _I),
    "lrmoe_workspace_bytes": ([_I], C.c_size_t),
    "lrmoe_route_topk": ([_P, _I, _P, _P, _P, C.c_float, _P, _P, _P, _P, _P, _P, _P, C.c_size_t, _P], _I),
    "lrmoe_bucket": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, C.c_size_t, _P], _I),
    "lrmoe_moe_experts": ([_P, _I, _P, _P, _P, _P, _P, C.c_size_t, _P], _I),
    "lrmoe_moe_layer": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P, C.c_size_t, _P], _I),
    "lrmoe_gather_tiles": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "lrmoe_moe_layer_static": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P, _P], _I),
    "lrmoe_moe_chain": ([_P, _I, _I, _P, C.c_float, _P, _P, _P, _P, C.c_size_t, _P], _I),
    "lrmoe_codec_pack": ([_P, C.c_int64, _I, _P, _P, _P, _P], _I),
    "lrmoe_codec_unpack": ([_P, _P, C.c_int64, _I, _P, _P], _I),
    "lrmoe_gather": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P], _I),
    "lrmoe_matvec": ([_P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "lrmoe_ordered_sum": ([_P, _P, _P, _P, _P, _I, _P], _I),
    "lrmoe_gate_silu": ([_P, _P, _P, _I, _I, _P], _I),
    "lrmoe_project": ([_P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "lrmoe_swiglu_rows": ([_P, _P, _I, _P], _I),
    "lrmoe_add_rmsnorm": ([_P, _P, _I, _P, C.c_float, _P, _P, _P], _I),
    "lrmoe_block_combine": ([_P, _P, _P, _P, _P, _I, _I, _P], _I),
    "lrmoe_fill_normal_bf16": ([_P, C.c_int64, C.c_uint64, C.c_uint64, C.c_double, C.c_int64, _P], _I),
    "lrmoe_timing_enable": ([_I, _I], _I),
    "lrmoe_timing_collect": ([_I, C.POINTER(C.c_double), C.POINTER(_I)], _I),
    "lrmoe_read_bandwidth": ([_P, C.c_int64, _I, _P, C.POINTER(C.c_double), _P], _I),
    "lrmoe_delta_workspace_bytes": ([_I], C.c_size_t),
    "lrmoe_delta_rule": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P], _I),
    "lrmoe_delta_mixer": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _I, _P, _P, _P, _P,
                           C.c_size_t, _P], _I),
    "lrmoe_delta_mixer_step": ([_P, _I, _P, C.c_float, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _I,
                                _P, _P, _P, _P, _P, _P, C.c_size_t, _P], _I),
    "lrmoe_attn_workspace_bytes": ([_I], C.c_size_t),
    "lrmoe_attn_decode": ([_P, _I, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P, _I, _I, _P, _P, C.c_size_t,
                           _P], _I),
    "lrmoe_attn_decode_at": ([_P, _I, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P, _I, _P, _P, _P,
                              C.c_size_t, _P], _I),
    "lrmoe_attn_decode_step": ([_P, _I, _P, C.c_float, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P, _I, _I,
                                _P, _P, _P, _P, _P, C.c_size_t, _P], _I),
}

STAGE_ROUTE = 1
STAGE_GATE_UP = 2
STAGE_DOWN = 4
STAGE_COMBINE = 8
STAGE_GATHER = 16
STAGE_LAYER = 32
STAGE_DELTA_MIXER = 64
STAGE_DELTA_RULE = 128
DELTA_WS_STATUS_OFFSET = 0  # int32 status word of a mixer workspace
DELTA_MAX_TOKENS = 16    # tokens per lrmoe_delta_mixer call
STAGE_ATTENTION = 256
ATTN_MAX_TOKENS = 16     # tokens per lrmoe_attn_decode call


class NativeError(RuntimeError):
    """A liblrmoe call returned a non-zero status."""

    def __init__(self, name: str, code: int, text: str):
        super().__init__(f"{name} failed ({code}): {text}")
        self.code = code


@lru_cache(maxsize=1)
def library() -> C.CDLL:
    if not LIBRARY.exists():
        raise RuntimeError(
            f"{LIBRARY} is missing: build it with `python -m lightreason_amd.build` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    lib = C.CDLL(str(LIBRARY))
    for name, (argtypes, restype) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


def symbols() -> list[str]:
    return list(_SIGNATURES)


def call(name: str, *args) -> None:
    lib = library()
    code = getattr(lib, name)(*args)
    if code != LRMOE_OK:
        text = lib.lrmoe_error_string(code).decode()
        if code == LRMOE_E_ARG:
            raise ValueError(f"{name}: {text}")
        raise NativeError(name, code, text)


def workspace_bytes(tokens: int) -> int:
    return int(library().lrmoe_workspace_bytes(tokens))


def device_check() -> None:
    code = library().lrmoe_device_check()
    if code != LRMOE_OK:
        raise NativeError("lrmoe_device_check", code, library().lrmoe_error_string(code).decode())


def timing_enable(mask: int, launches: int = 4096) -> None:
    call("lrmoe_timing_enable", int(mask), int(launches))


def timing_collect(stage: int) -> tuple[float, int]:
    """(summed milliseconds, launches) of the timed launches of ``stage``."""
    ms, n = C.c_double(0.0), C.c_int(0)
    call("lrmoe_timing_collect", int(stage), C.byref(ms), C.byref(n))
    return ms.value, n.value
