"""Build ``libgptq2d.so``, the HIP/C-ABI library of the GPTQ-2D engine, for gfx950.

Every ``csrc/*.hip`` file is compiled with hipcc (in parallel) and linked into one shared
library next to this file.  Run as a script or call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE.parent / "_build"
LIB = HERE / "libgptq2d.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32, which are not trusted on these boxes.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{HERE.parent / 'include'}",
    f"-I{CSRC}",
]

# No libraries beyond the HIP runtime hipcc links by itself.
LINK_LIBS: list[str] = []

# Per-file extra flags.  The trellis search must not contract a*b+c into fma: its costs are
# compared for exact ties and must equal the reference's unfused sums.  The register-staged MFMA kernels
# (the strided GEMMs, the cell-masked block flush, the fp32 strip Cholesky panel) keep their accumulators
# in VGPRs: by default the compiler put them in AGPRs and copied all of them out and back around every
# k-block (64 to 192 v_accvgpr moves, the read-out waiting for the MFMA chain).  In these files the flag
# changes no other kernel's code.
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
EXTRA_FLAGS = {
    "viterbi.hip": ["-ffp-contract=off"],
    "gemm.hip": VGPR_MFMA,
    "flush.hip": VGPR_MFMA,
    "ldl.hip": VGPR_MFMA,
}


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source and link ``libgptq2d.so``; returns its path."""
    if not pathlib.Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), *LINK_LIBS, "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
