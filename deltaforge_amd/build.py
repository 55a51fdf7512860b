"""Build the gfx950 HIP library ``deltaforge_amd/_lib/libdeltaforge_hip.so`` in-tree.

    python -m deltaforge_amd.build          # compile every csrc/*.hip, link one .so

hipcc cross-compiles for gfx950 without a GPU. Packed-FP32 codegen is disabled
(``-packed-fp32-ops``); the host pass warns that it does not know the feature, which is
harmless. Objects are rebuilt every call (the driver's build check expects a real compile).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libdeltaforge_hip.so"
ARCH = os.environ.get("DF_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-inline-asm",  # m0 is clobbered by the persistent kernel's LDS-DMA asm (nothing else uses it)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return found


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{errs}")
    if errs.strip():
        print(errs, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    objdir = OUT_DIR / "obj"
    objdir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in sources]
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        list(pool.map(lambda pair: _compile(*pair), zip(sources, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(sources)} sources for {ARCH}")
    return LIB


if __name__ == "__main__":
    build()
