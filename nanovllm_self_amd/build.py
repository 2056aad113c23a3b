"""Build libnvs_attention.so (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` translation unit is compiled to an object under
``nanovllm_self_amd/_build/`` and linked into
``nanovllm_self_amd/libnvs_attention.so``.  Run ``python -m
nanovllm_self_amd.build`` (or call :func:`build`) after changing a source.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libnvs_attention.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"
# Packed-fp32 VALU ops are disabled for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]
# The MFMA prefill kernel runs compiled decode code beside its asm statement
# at one wave per SIMD, where the compiler would otherwise keep the decode
# accumulators in AGPRs and copy them to and from VGPRs every tile.
FILE_FLAGS = {"paged_prefill_mx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build")
    return exe


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the device-only feature; drop that warning.
    noise = "-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def generate() -> None:
    """Regenerate the prefill kernel's tile loop (csrc/prefill_mx_asm.inc),
    check that every register it writes is declared to the compiler, and run
    the loop on the CPU over a few random batches for its LDS waits and
    barriers and the tiles its MFMAs read."""
    for script in ("gen_prefill_mx.py", "check_prefill_mx.py", "check_prefill_lds.py"):
        res = subprocess.run([sys.executable, str(CSRC / script)], capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"{script} failed:\n{res.stdout}{res.stderr}")


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    generate()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
