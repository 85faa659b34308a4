"""Build the gfx950 HIP library ``polylora_amd/_lib/libpolylora_hip.so``.

Run ``python -m polylora_amd.build``.  Every source under ``csrc/`` is
compiled with ``hipcc --offload-arch=gfx950`` into an object under
``polylora_amd/_build/`` and the objects are linked into one shared library
with a plain C ABI (``include/polylora_hip.h``); nothing links against
libtorch, so the library binds to whichever HIP runtime the process already
loaded (torch's, when torch is imported first).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libpolylora_hip.so"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"

ARCH = "gfx950"
SOURCES = ("capi.hip", "plan.hip", "sgmv_tiled.hip", "sgmv_fused.hip", "sgmv_rows.hip", "sgmv_refop.hip")
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    "-Wall",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # The only global atomics are the decode hand-off's single-lane counter
    # updates; left alone, the atomic optimizer rewrites each into a wave-wide
    # form that waits for the atomic's result at once, where the kernel means
    # to check it only at the end of the workgroup.
    "-mllvm",
    "-amdgpu-atomic-optimizer-strategy=None",
)


def _hipcc() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    candidate = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    raise RuntimeError("hipcc not found; the polylora_amd HIP library cannot be built")


def _run(cmd: list[str]) -> subprocess.Popen:
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    procs = []
    objects = []
    for name in SOURCES:
        src = CSRC_DIR / name
        obj = BUILD_DIR / (src.stem + ".o")
        objects.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-c", str(src), "-o", str(obj)]
        procs.append((name, cmd, _run(cmd)))
    failed = []
    for name, cmd, proc in procs:
        out, _ = proc.communicate()
        lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
        if proc.returncode != 0:
            failed.append((name, " ".join(cmd), "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        msg = "\n\n".join(f"[{n}] {c}\n{o}" for n, c, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp_lib = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_lib), *map(str, objects)]
    proc = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(link)}\n{proc.stdout}")
    os.replace(tmp_lib, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
