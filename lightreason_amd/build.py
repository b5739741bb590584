"""Build liblrmoe.so in-tree with hipcc for gfx950.

Every source is compiled with -ffp-contract=off (rounding points must match
the reference's, so only explicit fmaf contracts) and with packed fp32 math
disabled.  Objects go to lightreason_amd/_build/, the library to
lightreason_amd/liblrmoe.so.  `--timeline` builds the measurement variant
liblrmoe_timeline.so instead (-DLRMOE_TIMELINE: the decode kernel stamps the
wall clock at its phases; read by lightreason_amd.timeline).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "liblrmoe.so"
TIMELINE_LIBRARY = PACKAGE / "liblrmoe_timeline.so"
INCLUDE = PACKAGE.parent / "include"
ARCH = os.environ.get("LRMOE_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise FileNotFoundError("hipcc not found (ROCm is required to build liblrmoe.so)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(source: Path, build_dir: Path = BUILD, extra=()) -> Path:
    obj = build_dir / (source.stem + ".o")
    cmd = [hipcc(), *FLAGS, *extra, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)
    return obj


def build(jobs: int = 4, timeline: bool = False) -> Path:
    build_dir = BUILD if not timeline else PACKAGE / "_build_timeline"
    library = LIBRARY if not timeline else TIMELINE_LIBRARY
    extra = ("-DLRMOE_TIMELINE",) if timeline else ()
    build_dir.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda src: _compile(src, build_dir, extra), sources()))
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, library)
    return library


if __name__ == "__main__":
    print(build(timeline="--timeline" in sys.argv[1:]))
