"""ctypes view of the CPU oracle (lro.c) and of the reference CPU kernel.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this module, and only to check or time
against it; the product package never does.

Arrays are numpy: bf16 values travel as uint16 bit patterns.  ``reference()``
loads ``_ref/libcpu_experts.so``, which oracle/Makefile compiles from the
reference's own edge35b/cpu_experts.c; it is absent where the reference tree
is absent, and callers must treat that as "not available", never as a pass.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liblro.so"
REF = HERE / "_ref" / "libcpu_experts.so"
REF_WORKERS = HERE / "_ref" / "libpacked_workers.so"
REF_TILE_CODEC = HERE / "_ref" / "libref_tile_codec.so"
HIDDEN, INNER, EXPERTS, TOPK = 2048, 512, 256, 8
EXPERT_ELEMENTS = 3 * INNER * HIDDEN

_P = C.c_void_p


def build(ref: bool | None = None) -> None:
    """Compile liblro.so, and the reference kernel when its source exists."""
    targets = ["oracle"]
    if ref or (ref is None and Path("/root/reference/edge35b/cpu_experts.c").exists()):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True)


def _ptr(array: np.ndarray | None) -> int | None:
    if array is None:
        return None
    if not array.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arrays must be C-contiguous")
    return array.ctypes.data


@lru_cache(maxsize=1)
def lib() -> C.CDLL:
    if not LIB.exists():
        build(ref=False)
    so = C.CDLL(str(LIB))
    so.lro_bf16_value.argtypes = [C.c_uint16]
    so.lro_bf16_value.restype = C.c_float
    so.lro_bf16_round.argtypes = [C.c_float]
    so.lro_bf16_round.restype = C.c_uint16
    so.lro_exp.argtypes = [C.c_float]
    so.lro_exp.restype = C.c_float
    so.lro_fill_normal_bf16.argtypes = [_P, C.c_int64, C.c_uint64, C.c_uint64, C.c_double, C.c_int64]
    so.lro_expert_dot.argtypes = [_P, _P, C.c_int]
    so.lro_expert_dot.restype = C.c_float
    so.lro_canon_dot.argtypes = [_P, _P, C.c_int]
    so.lro_canon_dot.restype = C.c_float
    so.lro_expert_pair.argtypes = [_P, _P, _P, _P, _P]
    so.lro_expert_rows.argtypes = [_P, _P, _P, _P, C.c_int]
    so.lro_expert_block_rows.argtypes = [_P, _P, _P, _P, _P, C.c_int, C.c_int]
    so.lro_route.argtypes = [_P, _P, C.c_int, _P, _P, _P]
    so.lro_route_logits.argtypes = [_P, C.c_int, _P, _P]
    so.lro_shared_gate.argtypes = [_P, _P, C.c_int, _P]
    so.lro_rmsnorm.argtypes = [_P, _P, C.c_int, C.c_float, _P]
    so.lro_bucket.argtypes = [_P, C.c_int, _P, _P, _P, _P, _P]
    so.lro_bucket.restype = C.c_int
    so.lro_combine.argtypes = [_P, _P, _P, _P, _P, _P, _P, C.c_int, _P]
    so.lro_moe_layer.argtypes = [_P, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P]
    so.lro_delta_rule.argtypes = [_P, _P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_int, _P, _P]
    so.lro_delta_rule.restype = None
    so.lro_delta_mixer.argtypes = [_P, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, C.c_int, _P, _P]
    so.lro_delta_mixer.restype = None
    so.lro_attn_decode.argtypes = [_P, C.c_int, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P, C.c_int, C.c_int, _P]
    so.lro_attn_decode.restype = None
    so.lro_codec_pack.argtypes = [_P, C.c_int64, C.c_int, _P, _P]
    so.lro_codec_pack.restype = C.c_int64
    so.lro_codec_unpack.argtypes = [_P, _P, C.c_int64, C.c_int, _P]
    so.lro_codec_unpack.restype = None
    for name in ("lro_fill_normal_bf16", "lro_expert_pair", "lro_expert_rows", "lro_expert_block_rows",
                 "lro_route", "lro_route_logits", "lro_shared_gate", "lro_rmsnorm", "lro_combine", "lro_moe_layer"):
        getattr(so, name).restype = None
    return so


@lru_cache(maxsize=1)
def reference() -> C.CDLL | None:
    """The reference's cpu_experts.c as compiled by oracle/Makefile, or None."""
    if not REF.exists():
        if Path("/root/reference/edge35b/cpu_experts.c").exists():
            build(ref=True)
        else:
            return None
    so = C.CDLL(str(REF))
    so.expert_rows.argtypes = [_P, _P, _P, _P, C.c_int, C.c_int]
    so.expert_rows.restype = None
    so.expert_block_rows.argtypes = [_P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int]
    so.expert_block_rows.restype = None
    return so


@lru_cache(maxsize=1)
def reference_workers() -> C.CDLL | None:
    """The reference's packed_workers.cpp (persistent CPU expert workers,
    packed_workers.cpp:14-122) as compiled by oracle/Makefile, or None."""
    if not REF_WORKERS.exists():
        if Path("/root/reference/edge35b/packed_workers.cpp").exists():
            build(ref=True)
        else:
            return None
    so = C.CDLL(str(REF_WORKERS))
    so.packed_workers_create.argtypes = [C.c_int]
    so.packed_workers_create.restype = _P
    so.packed_workers_destroy.argtypes = [_P]
    so.packed_workers_destroy.restype = None
    so.packed_workers_submit.argtypes = [_P, _P, _P, _P, _P, C.c_int]
    so.packed_workers_submit.restype = None
    so.packed_workers_wait.argtypes = [_P]
    so.packed_workers_wait.restype = None
    so.packed_plan.argtypes = [_P, _P, _P, C.c_int, _P, _P]
    so.packed_plan.restype = None
    return so


# ---- scalar helpers -------------------------------------------------------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """cpu_experts.c:18-22 rounding (RNE, no NaN special case), vectorised."""
    bits = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)


def exp(x: float) -> float:
    return lib().lro_exp(float(x))


# ---- generator ------------------------------------------------------------

def normal_bf16(shape, seed: int, stream: int, sigma: float, first: int = 0) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().lro_fill_normal_bf16(_ptr(out), out.size, seed & (2**64 - 1), stream & (2**64 - 1), float(sigma), first)
    return out


# ---- expert arithmetic (cpu_experts.c restatement) -------------------------

def _pointer_array(arrays):
    return (C.c_void_p * len(arrays))(*[_ptr(a) for a in arrays])


def expert_rows(gate_up: list[np.ndarray], down: list[np.ndarray], hidden: np.ndarray) -> np.ndarray:
    out = np.empty((len(gate_up), HIDDEN), dtype=np.uint16)
    lib().lro_expert_rows(_pointer_array(gate_up), _pointer_array(down), _ptr(hidden), _ptr(out), len(gate_up))
    return out


def expert_block_rows(gate_up, down, hidden: np.ndarray, token_ids: np.ndarray) -> np.ndarray:
    token_ids = np.ascontiguousarray(token_ids, dtype=np.int32)
    out = np.empty((len(gate_up), HIDDEN), dtype=np.uint16)
    lib().lro_expert_block_rows(_pointer_array(gate_up), _pointer_array(down), _ptr(hidden), _ptr(token_ids),
                                _ptr(out), hidden.shape[0], len(gate_up))
    return out


def expert_pair(gate: np.ndarray, up: np.ndarray, down: np.ndarray, x_bf16: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(bf16_to_f32(x_bf16))
    y = np.empty(HIDDEN, dtype=np.uint16)
    lib().lro_expert_pair(_ptr(gate), _ptr(up), _ptr(down), _ptr(x), _ptr(y))
    return y


def reference_expert_rows(gate_up, down, hidden, threads: int = 1) -> np.ndarray:
    ref = reference()
    if ref is None:
        raise FileNotFoundError("reference CPU kernel not built")
    out = np.empty((len(gate_up), HIDDEN), dtype=np.uint16)
    ref.expert_rows(_pointer_array(gate_up), _pointer_array(down), _ptr(hidden), _ptr(out), len(gate_up), threads)
    return out


def reference_expert_block_rows(gate_up, down, hidden, token_ids, threads: int = 1) -> np.ndarray:
    ref = reference()
    if ref is None:
        raise FileNotFoundError("reference CPU kernel not built")
    token_ids = np.ascontiguousarray(token_ids, dtype=np.int32)
    out = np.empty((len(gate_up), HIDDEN), dtype=np.uint16)
    ref.expert_block_rows(_pointer_array(gate_up), _pointer_array(down), _ptr(hidden), _ptr(token_ids), _ptr(out),
                          hidden.shape[0], len(gate_up), threads)
    return out


# ---- router, shared gate, RMSNorm, bucketing, combine ---------------------

def canon_dot(weights: np.ndarray, x_f32: np.ndarray) -> float:
    return lib().lro_canon_dot(_ptr(weights), _ptr(np.ascontiguousarray(x_f32, dtype=np.float32)), weights.size)


def route(x: np.ndarray, router: np.ndarray):
    tokens = x.shape[0]
    logits = np.empty((tokens, EXPERTS), dtype=np.uint16)
    indices = np.empty((tokens, TOPK), dtype=np.int64)
    weights = np.empty((tokens, TOPK), dtype=np.uint16)
    lib().lro_route(_ptr(x), _ptr(router), tokens, _ptr(logits), _ptr(indices), _ptr(weights))
    return logits, indices, weights


def route_logits(logits: np.ndarray):
    """Top-8 with softmax renormalisation of given bf16 logits [T, 256]
    ([HF] Qwen3_5MoeTopKRouter.forward 768-777 after the GEMV): (indices
    [T, 8] int64 in rank order, weights [T, 8] bf16 bits)."""
    logits = np.ascontiguousarray(logits, dtype=np.uint16)
    tokens = logits.shape[0]
    indices = np.empty((tokens, TOPK), dtype=np.int64)
    weights = np.empty((tokens, TOPK), dtype=np.uint16)
    lib().lro_route_logits(_ptr(logits), tokens, _ptr(indices), _ptr(weights))
    return indices, weights


def shared_gate(x: np.ndarray, gate_weight: np.ndarray) -> np.ndarray:
    out = np.empty(x.shape[0], dtype=np.uint16)
    lib().lro_shared_gate(_ptr(x), _ptr(gate_weight), x.shape[0], _ptr(out))
    return out


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    out = np.empty_like(x)
    lib().lro_rmsnorm(_ptr(x), _ptr(weight), x.shape[0], float(eps), _ptr(out))
    return out


def bucket(indices: np.ndarray):
    indices = np.ascontiguousarray(indices, dtype=np.int64)
    tokens = indices.shape[0]
    expert = np.full(EXPERTS, -1, dtype=np.int32)
    offset = np.zeros(EXPERTS + 1, dtype=np.int32)
    pair_token = np.empty(tokens * TOPK, dtype=np.int32)
    pair_slot = np.empty(tokens * TOPK, dtype=np.int32)
    route_pair = np.empty(tokens * TOPK, dtype=np.int32)
    unique = lib().lro_bucket(_ptr(indices), tokens, _ptr(expert), _ptr(offset), _ptr(pair_token),
                              _ptr(pair_slot), _ptr(route_pair))
    if unique < 0:
        raise ValueError("invalid routes" if unique == -1 else "repeated expert in a token")
    return dict(unique=unique, expert=expert[:unique], offset=offset[:unique + 1], pair_token=pair_token,
                pair_slot=pair_slot, route_pair=route_pair.reshape(tokens, TOPK))


def combine(y, route_pair, pair_slot, weights, y_shared=None, sg=None, residual=None) -> np.ndarray:
    tokens = weights.shape[0]
    out = np.empty((tokens, HIDDEN), dtype=np.uint16)
    lib().lro_combine(_ptr(np.ascontiguousarray(y)), _ptr(np.ascontiguousarray(route_pair, dtype=np.int32)),
                      _ptr(np.ascontiguousarray(pair_slot, dtype=np.int32)), _ptr(np.ascontiguousarray(weights)),
                      _ptr(y_shared), _ptr(sg), _ptr(residual), tokens, _ptr(out))
    return out


def moe_layer(x, router, gate_up, down, shared=None, norm_weight=None, eps: float = 1e-6):
    """Whole layer for ``x`` [T, 2048].  ``gate_up``/``down`` are 256-entry lists
    of per-expert arrays (entries for unrouted experts may be any array).
    ``shared`` = (gate_proj, up_proj, down_proj, shared_expert_gate) or None."""
    tokens = x.shape[0]
    out = np.empty((tokens, HIDDEN), dtype=np.uint16)
    indices = np.empty((tokens, TOPK), dtype=np.int64)
    weights = np.empty((tokens, TOPK), dtype=np.uint16)
    sg_proj, su_proj, sd_proj, sgate = shared if shared is not None else (None, None, None, None)
    lib().lro_moe_layer(_ptr(x), tokens, _ptr(router), _pointer_array(gate_up), _pointer_array(down),
                        _ptr(sg_proj), _ptr(su_proj), _ptr(sd_proj), _ptr(sgate), _ptr(norm_weight), float(eps),
                        _ptr(out), _ptr(indices), _ptr(weights))
    return out, indices, weights


# ---- Gated DeltaNet decode (linear-attention mixer) ------------------------

DN_KEY_HEADS, DN_VALUE_HEADS, DN_WIDTH, DN_CONV_K = 16, 32, 128, 4
DN_CONV = 2 * DN_KEY_HEADS * DN_WIDTH + DN_VALUE_HEADS * DN_WIDTH   # 8192 channels


def delta_rule(q, k, v, G, beta, state, *, normalize: bool, record: bool):
    """edge35b/delta_decode.py:11-55 restated (lro_delta_rule): q, k [T, H, D]
    and v [T, H, E] bf16 bits, G [T, H] float32 (= exp(g)), beta [T, H] bf16
    bits, state [H, D, E] float32 or bf16 bits (uint16).  Returns (out [T, H,
    E] bf16 bits, states [T or 1, H, D, E] in the state's dtype)."""
    q, k, v, beta = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v, beta))
    G = np.ascontiguousarray(G, dtype=np.float32)
    state = np.ascontiguousarray(state)
    bf16_state = state.dtype == np.uint16
    if not bf16_state and state.dtype != np.float32:
        raise ValueError("state must be float32 or bf16 bits")
    T, H, D = q.shape
    E = v.shape[-1]
    out = np.empty((T, H, E), dtype=np.uint16)
    states = np.empty((T if record else 1, H, D, E), dtype=state.dtype)
    lib().lro_delta_rule(_ptr(q), _ptr(k), _ptr(v), _ptr(G), _ptr(beta), _ptr(state), int(bf16_state), T, H, D, E,
                         int(normalize), int(record), _ptr(out), _ptr(states))
    return out, states


def delta_mixer(x, weights: dict, conv_state, state, eps: float = 1e-6, record: bool = False):
    """The Gated DeltaNet mixer step for x [T, 2048] (lro_delta_mixer).
    weights: in_proj_qkv [8192, 2048], in_proj_z [4096, 2048], in_proj_b and
    in_proj_a [32, 2048], conv1d [8192, 4], A_log [32], dt_bias [32], norm
    [128], out_proj [2048, 4096], all bf16 bits.  conv_state [8192, 4] bf16
    bits and state [32, 128, 128] (float32 or bf16 bits) are copied; returns
    (out [T, 2048], new conv_state, new state, per-token states or None)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    T = x.shape[0]
    w = {name: np.ascontiguousarray(weights[name], dtype=np.uint16)
         for name in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "conv1d", "A_log", "dt_bias", "norm",
                      "out_proj")}
    conv = np.array(conv_state, dtype=np.uint16, copy=True, order="C")
    st = np.array(state, copy=True, order="C")
    bf16_state = st.dtype == np.uint16
    rec = np.empty((T, DN_VALUE_HEADS, DN_WIDTH, DN_WIDTH), dtype=st.dtype) if record else None
    out = np.empty((T, HIDDEN), dtype=np.uint16)
    lib().lro_delta_mixer(_ptr(x), T, _ptr(w["in_proj_qkv"]), _ptr(w["in_proj_z"]), _ptr(w["in_proj_b"]),
                          _ptr(w["in_proj_a"]), _ptr(w["conv1d"]), _ptr(w["A_log"]), _ptr(w["dt_bias"]),
                          _ptr(w["norm"]), float(eps), _ptr(w["out_proj"]), _ptr(conv), _ptr(st), int(bf16_state),
                          _ptr(rec), _ptr(out))
    return out, conv, st, rec


AT_HEADS, AT_KV, AT_D, AT_ROT = 16, 2, 256, 64


def attn_decode(x, weights: dict, cos, sin, k_cache, v_cache, length: int, eps: float = 1e-6):
    """The full-attention decode step for x [T, 2048] after `length` cached
    positions (lro_attn_decode).  weights: q_proj [8192, 2048], k_proj and
    v_proj [512, 2048], o_proj [2048, 4096], q_norm and k_norm [256], all
    bf16 bits; cos, sin [T, 64] bf16 bits; k_cache, v_cache [2, capacity,
    256] bf16 bits are copied.  Returns (out [T, 2048], new k_cache, new
    v_cache)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    T = x.shape[0]
    w = {name: np.ascontiguousarray(weights[name], dtype=np.uint16)
         for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")}
    cos = np.ascontiguousarray(cos, dtype=np.uint16)
    sin = np.ascontiguousarray(sin, dtype=np.uint16)
    kc = np.array(k_cache, dtype=np.uint16, copy=True, order="C")
    vc = np.array(v_cache, dtype=np.uint16, copy=True, order="C")
    capacity = kc.shape[1]
    if kc.shape != (AT_KV, capacity, AT_D) or vc.shape != kc.shape or length + T > capacity:
        raise ValueError(f"caches must be [{AT_KV}, capacity >= {length + T}, {AT_D}], got {kc.shape}, {vc.shape}")
    if cos.shape != (T, AT_ROT) or sin.shape != (T, AT_ROT):
        raise ValueError(f"cos and sin must be [{T}, {AT_ROT}]")
    out = np.empty((T, HIDDEN), dtype=np.uint16)
    lib().lro_attn_decode(_ptr(x), T, _ptr(w["q_proj"]), _ptr(w["k_proj"]), _ptr(w["v_proj"]), _ptr(w["o_proj"]),
                          _ptr(w["q_norm"]), _ptr(w["k_norm"]), float(eps), _ptr(cos), _ptr(sin), _ptr(kc), _ptr(vc),
                          capacity, int(length), _ptr(out))
    return out, kc, vc


CODEC_TILE = 256
CODEC_TILE_BYTES = 384


def codec_pack(w: np.ndarray):
    """Tile-codec packing of a [rows, cols] bf16-bit array (cols a multiple of
    256) in the decode kernel's byte order.  Returns (packed [rows, tiles,
    384] u8, bases [rows, tiles] u8, number of tiles that do not fit)."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    rows, cols = w.shape
    tiles = cols // CODEC_TILE
    packed = np.empty((rows, tiles, CODEC_TILE_BYTES), dtype=np.uint8)
    bases = np.empty((rows, tiles), dtype=np.uint8)
    misfit = lib().lro_codec_pack(_ptr(w), rows, cols, _ptr(packed), _ptr(bases))
    return packed, bases, int(misfit)


def codec_unpack(packed: np.ndarray, bases: np.ndarray) -> np.ndarray:
    rows, tiles, _ = packed.shape
    out = np.empty((rows, tiles * CODEC_TILE), dtype=np.uint16)
    lib().lro_codec_unpack(_ptr(np.ascontiguousarray(packed)), _ptr(np.ascontiguousarray(bases)), rows,
                           tiles * CODEC_TILE, _ptr(out))
    return out


def _reference_order():
    """Byte positions in codec_pack's tile of the reference's bytes: value k's
    low byte (reference byte k) and the byte and nibble holding its code
    (reference nibble k of bytes 256..383)."""
    k = np.arange(CODEC_TILE)
    g, s, j = (k >> 3) & 3, k >> 5, k & 7
    low_at = 64 * (s >> 1) + 16 * g + 8 * (s & 1) + j
    code_at = 256 + 64 * (s >> 2) + 16 * g + 4 * (s & 3) + (j & 3)
    return k, low_at, code_at, 4 * (j >> 2)


def codec_pack_reference_order(w: np.ndarray):
    """Tile-codec packing in the reference's byte order
    (edge35b/cpu_bf16_reads.h:16-52, pack_cpu_read_tiles): per tile value k's
    low byte at byte k and its code in nibble k (low nibble first) of bytes
    256..383; tiles that do not fit (base 255) are all zero.  The bytes of
    codec_pack, rearranged.  Returns (packed [rows, tiles, 384], bases [rows,
    tiles], number of tiles that do not fit)."""
    ours, bases, misfit = codec_pack(w)
    k, low_at, code_at, shift = _reference_order()
    out = np.zeros_like(ours)
    out[..., :CODEC_TILE] = ours[..., low_at]
    codes = (ours[..., code_at] >> shift) & 15
    out[..., CODEC_TILE:] = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return out, bases, misfit


def compact_rows(w: np.ndarray):
    """The reference's compact resident row (edge35b/gpu_resident_experts.py:
    22-45, encode) of the tiles of a bf16-bit array, in reading order: a
    fitting tile's 384 packed bytes (reference order) or a raw tile's 512
    bytes, and per tile the header (raw tiles before it) << 8 | base.
    Returns (data u8, headers u32, tiles encoded, tiles raw); data is the raw
    bytes and headers None when the compact form would not be smaller."""
    raw = np.ascontiguousarray(w, dtype=np.uint16).reshape(-1, CODEC_TILE)
    packed, bases, _ = codec_pack_reference_order(raw)
    packed, bases = packed[:, 0], bases[:, 0]
    fits = bases != 255
    raw_before = np.cumsum(~fits, dtype=np.uint32) - (~fits)
    headers = (raw_before << 8) | bases.astype(np.uint32)
    raw_bytes = raw.view(np.uint8).reshape(len(raw), 2 * CODEC_TILE)
    if int(np.where(fits, CODEC_TILE_BYTES, 2 * CODEC_TILE).sum()) + headers.nbytes >= raw_bytes.nbytes:
        return raw_bytes.reshape(-1), None, 0, len(raw)
    parts = [packed[t] if fits[t] else raw_bytes[t] for t in range(len(raw))]
    return np.concatenate(parts), headers, int(fits.sum()), int((~fits).sum())


def decode_compact_rows(data: np.ndarray, headers: np.ndarray) -> np.ndarray:
    """Inverse of compact_rows (bf16 bits, tiles in order), in plain numpy
    from the reference layout: a check of the encoder independent of the
    device decoder."""
    out = np.empty((len(headers), CODEC_TILE), dtype=np.uint16)
    k = np.arange(CODEC_TILE)
    for t, h in enumerate(headers.tolist()):
        base, before = h & 255, h >> 8
        at = t * CODEC_TILE_BYTES + before * 128
        if base == 255:
            out[t] = data[at:at + 2 * CODEC_TILE].view(np.uint16)
            continue
        tile = data[at:at + CODEC_TILE_BYTES].astype(np.uint16)
        code = (tile[CODEC_TILE + k // 2] >> (4 * (k & 1))) & 15
        out[t] = (((base + (code & 7)) | ((code & 8) << 4)) << 8) | tile[k]
    return out


# ---- the escape codec of the gather (edge35b/bf16_expert_codec.py:27-78) ----

ESCAPE_WINDOW = 16


def escape_window(bits: np.ndarray):
    """(base, escapes) of a flat row of bf16 bits (bf16_expert_codec.py:27-35):
    base starts the window of 16 consecutive 8-bit exponents (bits 14..7)
    that holds the most values, the first such window on ties; escapes =
    values outside it."""
    bits = np.asarray(bits, dtype=np.uint16)
    if bits.ndim != 1 or bits.size % 8 or not 0 < bits.size < 2**31:
        raise ValueError("Expected a flat, aligned BF16 bit array")
    counts = np.bincount((bits >> 7) & 255, minlength=256).astype(np.int64)
    upto = np.concatenate([[0], np.cumsum(counts)])
    inside = upto[ESCAPE_WINDOW:] - upto[:-ESCAPE_WINDOW]   # window b covers exponents b .. b+15
    base = int(np.argmax(inside))
    return base, int(bits.size - inside[base])


def escape_row_bytes(n: int, escapes: int) -> int:
    """n sign|fraction bytes, n/2 delta bytes, 4 + 2 bytes per escape."""
    return 3 * n // 2 + 6 * escapes


def escape_pack(bits: np.ndarray, base: int, escapes: int) -> np.ndarray:
    """Packed row (bf16_expert_codec.py:42-55): per value its sign and
    fraction in one byte (sign at bit 7), its exponent - base in a nibble
    (value 2i in the low nibble of byte i; escaped values keep the low four
    bits), then the escapes' int32 indices in order and their raw bits."""
    bits = np.asarray(bits, dtype=np.uint16)
    n = bits.size
    delta = ((bits >> 7) & 255).astype(np.int32) - base
    escaped = np.flatnonzero((delta < 0) | (delta >= ESCAPE_WINDOW))
    if escaped.size != escapes:
        raise ValueError("escape count disagrees with the row")
    out = np.zeros(escape_row_bytes(n, escapes), dtype=np.uint8)
    out[:n] = ((bits & 0x7F) | ((bits >> 8) & 0x80)).astype(np.uint8)
    nib = (delta & 15).astype(np.uint8)
    out[n:3 * n // 2] = nib[0::2] | (nib[1::2] << 4)
    tail = 3 * n // 2
    out[tail:tail + 4 * escapes] = escaped.astype("<i4").view(np.uint8)
    out[tail + 4 * escapes:] = bits[escaped].astype("<u2").view(np.uint8)
    return out


def escape_restore(packed: np.ndarray, n: int, base: int, escapes: int) -> np.ndarray:
    """Inverse of escape_pack (bf16_expert_codec.py:58-67)."""
    packed = np.asarray(packed, dtype=np.uint8)
    sf = packed[:n].astype(np.uint16)
    nib = packed[n:3 * n // 2]
    delta = np.empty(n, dtype=np.uint16)
    delta[0::2] = nib & 15
    delta[1::2] = nib >> 4
    bits = ((sf & 0x80) << 8) | (sf & 0x7F) | ((delta + base) << 7)
    tail = 3 * n // 2
    idx = packed[tail:tail + 4 * escapes].view("<i4")
    bits[idx] = packed[tail + 4 * escapes:tail + 6 * escapes].view("<u2")
    return bits.astype(np.uint16)


def escape_plan(rows: np.ndarray):
    """Layout of a bank of packed rows (bf16_expert_codec.py:70-81): per row
    (offset, base, escapes), or None where more than 1% of its values escape
    (that row stays raw); offsets 16-byte aligned.  Returns (plans, bytes)."""
    plans, size = [], 0
    for row in rows:
        base, escapes = escape_window(row)
        if escapes * 100 > row.size:
            plans.append(None)
            continue
        plans.append((size, base, escapes))
        size = (size + escape_row_bytes(row.size, escapes) + 15) & ~15
    return plans, size


@lru_cache(maxsize=1)
def reference_tile_codec() -> C.CDLL | None:
    """The reference's own tile packer (edge35b/cpu_bf16_reads.h:16-52), built
    into oracle/_ref by oracle/Makefile where /root/reference is present."""
    if not REF_TILE_CODEC.exists():
        if Path("/root/reference/edge35b/cpu_bf16_reads.h").exists():
            build(ref=True)
        else:
            return None
    so = C.CDLL(str(REF_TILE_CODEC))
    so.ref_pack_cpu_read_tiles.argtypes = [_P, _P, _P, C.c_size_t]
    so.ref_pack_cpu_read_tiles.restype = C.c_int64
    return so


def physical_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
