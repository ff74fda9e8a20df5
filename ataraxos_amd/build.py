"""Build recipe for ``libataraxos_attn.so``, the gfx950 attention library.

Each ``csrc/*.hip`` translation unit is compiled by ``hipcc`` for gfx950 in
parallel, then linked into one shared library next to this file.  The library
has no libtorch dependency; Python reaches it through ``ctypes``
(:mod:`ataraxos_amd._lib`).

Run ``python -m ataraxos_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = PKG_DIR.parent / "include"
LIB_NAME = "libataraxos_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"

# Packed-FP32 VALU instructions are switched off for every HIP source.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the gfx950 attention library cannot be built")
    return exe


def _compile(src: Path, extra: list[str]) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and os.environ.get("ATX_BUILD_VERBOSE"):
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every ``csrc/*.hip`` file and link ``libataraxos_attn.so``.

    Always recompiles (the caller asked for a build).  Returns the library path.
    """
    extra = list(extra_flags or [])
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    workers = min(len(sources), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, extra), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {LIB_NAME} failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
