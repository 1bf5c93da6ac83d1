"""Build recipe for libmtp_glora_amd.so (gfx950), in-tree.

``python -m`` is not needed: ``build_library()`` runs hipcc on every
``csrc/*.hip`` file and links them into ``lib/libmtp_glora_amd.so`` next to
this file. hipcc cross-compiles for gfx950 without a GPU present.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_NAME = "libmtp_glora_amd.so"
ARCH = os.environ.get("MGA_OFFLOAD_ARCH", "gfx950")

# Packed fp32 VALU ops are disabled for every device pass (hipcc's host pass
# reports the feature as unknown; that warning is harmless).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
                "-Wno-unused-function", "-Wno-unused-variable", "-munsafe-fp-atomics"]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmtp_glora_amd.so")
    return cand


COMPILE_TIMEOUT_S = 900


def lib_path() -> Path:
    return LIB_DIR / LIB_NAME


def build_library(verbose: bool = False, jobs: int = 4, src_dir=None, out_path=None) -> Path:
    """Compile every csrc/*.hip to an object and link the shared library.

    src_dir / out_path build another source tree (with the same file set) into
    another library file, e.g. a variant to time against the in-tree build;
    the default is csrc/ -> lib/libmtp_glora_amd.so."""
    cc = hipcc()
    src = Path(src_dir) if src_dir is not None else CSRC
    out = Path(out_path) if out_path is not None else lib_path()
    objdir = out.parent / ("obj" if out_path is None else out.stem + "_obj")
    objdir.mkdir(parents=True, exist_ok=True)
    sources = sorted(src.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {src}")

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [cc, *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
        try:
            # a compiler that loops (it has, on some unrolled kernels) fails
            # the build instead of holding it forever
            res = subprocess.run(cmd, capture_output=True, text=True, timeout=COMPILE_TIMEOUT_S)
        except subprocess.TimeoutExpired:
            raise RuntimeError(f"hipcc did not finish {src.name} within {COMPILE_TIMEOUT_S} s") from None
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
        if verbose:
            print(" ".join(cmd))
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = out.with_suffix(".so.tmp")
    # --no-undefined: a kernel template whose host launch stub the compiler
    # dropped must fail here, not when the library is loaded on a GPU box
    cmd = [cc, "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp),
           "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,--no-undefined"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
