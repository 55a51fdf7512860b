"""Build the gfx950 HIP library ``deltaforge_amd/_lib/libdeltaforge_hip.so`` in-tree.

    python -m deltaforge_amd.build          # compile every csrc/*.hip, link one .so
    python -m deltaforge_amd.build --trace  # the same with the persistent kernel's phase stamps
                                            # (DF_TRACE), as _lib/libdeltaforge_hip_trace.so

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


TRACE_LIB = OUT_DIR / "libdeltaforge_hip_trace.so"


def _compile(src: Path, obj: Path, extra: tuple[str, ...] = ()) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{errs}")
    if errs.strip():
        print(errs, file=sys.stderr)


def build(verbose: bool = True, trace: bool = False) -> Path:
    """Compile and link the library; ``trace`` builds the phase-stamping variant
    (``PersistentDecoder.trace_decode`` needs it) beside the product library."""
    OUT_DIR.mkdir(exist_ok=True)
    objdir = OUT_DIR / ("obj_trace" if trace else "obj")
    objdir.mkdir(exist_ok=True)
    out = TRACE_LIB if trace else LIB
    extra = ("-DDF_TRACE",) if trace else ()
    sources = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in sources]
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        list(pool.map(lambda pair: _compile(*pair, extra), zip(sources, objs)))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    tmp.replace(out)
    if verbose:
        print(f"built {out.relative_to(ROOT)} from {len(sources)} sources for {ARCH}")
    return out


if __name__ == "__main__":
    build(trace="--trace" in sys.argv[1:])
