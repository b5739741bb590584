"""Expert-row gather (edge35b/native_bf16_gather.py) on liblrmoe.

The reference compiles its gather with NVRTC for sm_89 and copies expert rows
from pinned host memory into device cache slots (native_bf16_gather.py:32-93,
bf16_gather_ada.cu).  Here the rows are resident in HBM and the copy is
HBM -> HBM; the launch protocol is unchanged: descriptors int64
[banks, experts, 3] = (address, base, escapes), destinations int64[banks],
sizes int64[banks], src/dst int32[max_copies], count int64[1] on the
device, grid (stripes, banks, max_copies), torch's current stream, no host
synchronisation (graph-capturable; a replay picks up new counts and
descriptors).

Policies "default" and "l2" copy raw BF16 rows (base < 0) bit for bit and
decode escape-codec rows (base >= 0, bf16_expert_codec.py; flagged in
``status`` as STATUS_CODEC_ROW) with lrmoe_gather.
Policies "cpu-tiles" and "resident" decode the tile codec (descriptors
(packed, bases, raw), "resident" also compact rows with raw = -1;
lrmoe_gather_tiles), like bf16_gather_ada.cu:127-201.  ``stage_primary`` and
``copy_compact_tail`` (the reference's host-cache staging) raise
NotImplementedError.
"""

from __future__ import annotations

import torch

from .. import _native, moe
from ._grid import pointer, stream_of

NATIVE_GEOMETRIES = (
    (4, 256, "default"), (8, 128, "default"), (8, 256, "default"), (16, 128, "default"),
    (8, 256, "l2"), (16, 128, "l2"),
)
CPU_TILE_GEOMETRIES = ((4, 256, "cpu-tiles"), (8, 128, "cpu-tiles"), (16, 128, "cpu-tiles"))
_LEGACY_PREFIX = "cuda-"


def name(geometry) -> str:
    return "hip-" + "-".join(map(str, geometry))


def select_geometry(tag, *, shared=False):
    """Geometry for a tag; the reference's ``cuda-...`` tags are accepted
    as aliases of the same geometry."""
    for geometry in CPU_TILE_GEOMETRIES if shared else NATIVE_GEOMETRIES:
        if tag in (name(geometry), _LEGACY_PREFIX + "-".join(map(str, geometry))):
            return geometry
    raise ValueError(f"Unknown gather geometry {tag!r}.")


class NativeBf16Gather:
    def __init__(self):
        if not torch.cuda.is_available():
            raise ValueError("The native gather requires an MI355X (gfx950) GPU.")
        torch.empty(1, device="cuda")
        try:
            _native.device_check()
        except _native.NativeError as exc:
            if exc.code == _native.LRMOE_E_DEVICE:
                raise ValueError("The native gather requires an MI355X (gfx950) GPU.") from exc
            raise RuntimeError(str(exc)) from exc
        self.status = torch.zeros(1, dtype=torch.int32, device="cuda")

    def copy(self, descriptors, destinations, sizes, src, dst, count, *, max_copies, experts, geometry):
        stripes, threads, policy = geometry
        if policy not in ("default", "l2", "cpu-tiles", "resident"):
            raise ValueError(f"Unknown gather policy {policy!r}.")
        banks = destinations.numel()
        if descriptors.numel() < banks * int(experts) * 3 or sizes.numel() < banks:
            raise ValueError("descriptors must be [banks, experts, 3] and sizes [banks]")
        if src.numel() < int(max_copies) or dst.numel() < int(max_copies) or count.numel() < 1:
            raise ValueError("src and dst need max_copies entries and count one")
        if self.status.device != destinations.device:
            self.status = torch.zeros(1, dtype=torch.int32, device=destinations.device)
        else:
            # Per-copy flag: cleared by a fill kernel on the device's current
            # stream, the copy's stream (stream-ordered, graph-capturable).
            self.status.zero_()
        try:
            if policy in ("cpu-tiles", "resident"):
                _native.call("lrmoe_gather_tiles", pointer(descriptors, torch.int64, "descriptors"),
                             pointer(destinations, torch.int64, "destinations"), pointer(sizes, torch.int64, "sizes"),
                             pointer(src, torch.int32, "src"), pointer(dst, torch.int32, "dst"),
                             pointer(count, torch.int64, "count"), int(experts), banks, int(max_copies),
                             int(stripes), int(threads), int(policy == "resident"), stream_of(destinations))
                return
            _native.call("lrmoe_gather", pointer(descriptors, torch.int64, "descriptors"),
                         pointer(destinations, torch.int64, "destinations"), pointer(sizes, torch.int64, "sizes"),
                         pointer(src, torch.int32, "src"), pointer(dst, torch.int32, "dst"),
                         pointer(count, torch.int64, "count"), int(experts), banks, int(max_copies), int(stripes),
                         int(threads), int(policy == "l2"), self.status.data_ptr(), stream_of(destinations))
        except _native.NativeError as exc:
            raise RuntimeError(str(exc)) from exc

    def codec_rows_seen(self) -> bool:
        """True when the last copy decoded an escape-codec row (reads the
        device).  Copies on the "cpu-tiles"/"resident" policies leave it
        False."""
        return bool(int(self.status.item()) & _native.STATUS_CODEC_ROW)

    def stage_primary(self, *args, **kwargs):
        raise NotImplementedError("stage_primary fills the reference's host-side expert caches; experts are "
                                  "resident in HBM here (tile-codec rows: copy() with 'cpu-tiles'/'resident')")

    def copy_compact_tail(self, *args, **kwargs):
        raise NotImplementedError("copy_compact_tail fills the reference's host-side expert caches; experts are "
                                  "resident in HBM here (tile-codec rows: copy() with 'cpu-tiles'/'resident')")


def expert_descriptors(expert_ptrs: torch.Tensor) -> torch.Tensor:
    """Raw-row descriptors [2, 256, 3] (gate_up bank, down bank) for a layer's
    device expert table [256, 2]: (address, -1, 0)."""
    if expert_ptrs.shape != (moe.EXPERTS, 2) or expert_ptrs.dtype != torch.int64:
        raise ValueError("expert_ptrs must be int64 [256, 2]")
    desc = torch.zeros((2, moe.EXPERTS, 3), dtype=torch.int64, device=expert_ptrs.device)
    desc[:, :, 0] = expert_ptrs.t()
    desc[:, :, 1] = -1
    return desc
