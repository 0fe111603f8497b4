"""Build recipe of the gfx950 HIP library ``ebr_amd/_lib/libebr_attn.so`` (in-tree, so it travels with the repo).

``python -m ebr_amd.build`` compiles it; ``__graft_entry__.build()`` calls :func:`build`. hipcc cross-compiles for
gfx950 without a GPU. Packed-fp32 instruction selection is disabled (``-packed-fp32-ops``) for every HIP source.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libebr_attn.so"
ARCH = "gfx950"

SOURCES = [CSRC / "ebr_attn.hip", CSRC / "ebr_rope.hip", CSRC / "ebr_descent.hip", CSRC / "ebr_block.hip",
           CSRC / "ebr_noalloc.hip"]
HEADERS = [
    CSRC / "attn_tiles.hpp",
    CSRC / "attn_resident.hpp",
    CSRC / "attn_long.hpp",
    ROOT / "include" / "ebr_attn.h",
    ROOT / "include" / "ebr_rope.h",
    ROOT / "include" / "ebr_descent.h",
    ROOT / "include" / "ebr_block.h",
    CSRC / "attn_f64.hpp",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def compile_flags(arch: str = ARCH) -> list:
    """Flags of every HIP translation unit (compiled to an object each, then linked into the shared library)."""
    return [
        f"--offload-arch={arch}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        f"-I{ROOT / 'include'}",
    ]


def link_flags(arch: str = ARCH, extra_flags: tuple = ()) -> list:
    """Flags of the link step: the target, and every extra flag except those that only steer preprocessing (-I, -D,
    -U), so that flags that matter at link time too (-fgpu-rdc, -g, host-side instrumentation) reach it."""
    pre = ("-I", "-D", "-U")
    return [f"--offload-arch={arch}", "-shared", "-fPIC", *(f for f in extra_flags if not f.startswith(pre))]


def _run(cmd: list, verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}: {' '.join(cmd[-3:])}")
    return proc.stderr


def build(verbose: bool = False, extra_flags: tuple = (), jobs: int = 0, arch: str = ARCH) -> Path:
    """Compile every HIP source (in parallel, one object each) and link the in-tree shared library; return its path.
    ``extra_flags`` go to every compile and, bar preprocessor flags, to the link."""
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    flags = [*compile_flags(arch), *extra_flags]
    objs = [obj_dir / (src.stem + ".o") for src in SOURCES]
    t0 = time.time()
    workers = jobs or min(len(SOURCES), max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        logs = list(pool.map(lambda so: _run([cc, *flags, "-c", str(so[0]), "-o", str(so[1])], verbose),
                             zip(SOURCES, objs)))
    _run([cc, *link_flags(arch, tuple(extra_flags)), *map(str, objs), "-o", str(tmp)], verbose)
    if verbose:
        noise = "is not a recognized feature for this target"
        for log in logs:
            lines = [ln for ln in log.splitlines() if noise not in ln]
            if lines:
                sys.stderr.write("\n".join(lines) + "\n")
        print(f"built in {time.time() - t0:.1f} s", flush=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
