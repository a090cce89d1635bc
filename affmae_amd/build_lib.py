"""Compile the gfx950 HIP sources under affmae_amd/csrc into affmae_amd/libaffmae.so.

Every ``*.hip`` file is compiled to an object with hipcc and the objects are
linked into one shared library that exports the C ABI declared in
include/affmae.h.  Run ``python -m affmae_amd.build_lib`` or call ``build()``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB_PATH = PKG / "libaffmae.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 ops (v_pk_fma_f32 and relatives) stay off on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# Per-file extra flags.
EXTRA_FLAGS = {
    # Distances must be the un-fused fp32 value; the kernel also pins this
    # with a scoped pragma.
    "knn.hip": ["-ffp-contract=off"],
    "knn_brute.hip": ["-ffp-contract=off"],
    # The curve and anchor keys reproduce torch's separately rounded products and sums.
    "sfc.hip": ["-ffp-contract=off"],
    # MFMA results in VGPRs: the attention kernels read every S element with VALU
    # ops, which an AGPR destination would precede with a copy.
    "nbhd_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


# Hot kernels that must compile without scratch (register spills): a spill in the
# attention kernel once added 18.8 MB of HBM writes per launch.  The compiler's
# resource-usage remarks are checked for every kernel whose name contains the string.
NO_SCRATCH = {
    "nbhd_attn.hip": "nbhd_attn_wave_kernel",
    "knn.hip": "knn_win_kernel",
}


def _scratch_kernels(remarks: str, name_part: str) -> list:
    """(kernel, bytes per lane) of every kernel containing name_part with scratch > 0."""
    bad, cur = [], None
    for line in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            continue
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and cur and name_part in cur and int(m.group(1)) > 0:
            bad.append((cur, int(m.group(1))))
    return bad


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    check = NO_SCRATCH.get(src.name)
    remarks = ["-Rpass-analysis=kernel-resource-usage"] if check else []
    cmd = [HIPCC, *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), *remarks, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    if check:
        bad = _scratch_kernels(proc.stderr, check)
        if bad:
            raise RuntimeError(f"{src.name}: kernels compiled with scratch (register spills): " +
                               ", ".join(f"{k} {n} B/lane" for k, n in bad[:4]))
    return obj


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every HIP source and link libaffmae.so (always rebuilds)."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    if verbose:
        print(f"[affmae build] hipcc {ARCH}: {', '.join(s.name for s in sources)}", flush=True)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[affmae build] wrote {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
