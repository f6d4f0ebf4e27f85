"""Build recipe for the gfx950 MHSEA library (``libhz_mhsea.so``).

Compiles every ``csrc/*.hip`` file with ``hipcc --offload-arch=gfx950`` into object
files under ``_build/`` and links them into ``hamiltonzero_amd/_lib/libhz_mhsea.so``.
The library is built in-tree so that it travels with the source tree; nothing is
installed.  Run ``python -m hamiltonzero_amd.build`` or call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libhz_mhsea.so"
LIB_PATH = LIB_DIR / LIB_NAME
REPO_ROOT = PKG_DIR.parent

ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU instructions
# (v_pk_fma_f32 and friends). The host pass does not know the feature and says so once
# per file; that warning is filtered below.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]

# Per-file additions. The large-N bf16 kernel runs with every VGPR in use (two waves per
# SIMD); LLVM's memory-clause scheduling strategy groups its LDS operand reads ahead of the
# products without spilling (no scratch in any instantiation) and gives bit-identical
# results ~2% faster at [128, 1024, 16, 64], T = 2 (3264 vs 3326 us on MI355X).
EXTRA_FLAGS = {
    "mhsea_fwd_bf16_large.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
}

_HOST_FEATURE_WARNING = "'-packed-fp32-ops' is not a recognized feature for this target"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc and PATH)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = [
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if line.strip() and _HOST_FEATURE_WARNING not in line
    ]
    if proc.returncode != 0:
        raise RuntimeError(
            "command failed (%d): %s\n%s" % (proc.returncode, " ".join(cmd), "\n".join(noise))
        )
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link ``libhz_mhsea.so``. Always rebuilds."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    include = ["-I", str(REPO_ROOT / "include"), "-I", str(CSRC)]

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), *include, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
