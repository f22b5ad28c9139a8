"""Builds ``libeagle4_amd.so``, the gfx950 kernels behind the ``eagle_harness`` host modules of this directory.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 into ``_build/`` (in parallel), then linked into
``eagle_harness/kernels/libeagle4_amd.so``, where the host binding loads it. Runs offline: hipcc cross-compiles without
a GPU. ``python eagle-4_amd/build.py`` builds from the command line.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIBRARY = ROOT / "eagle_harness" / "kernels" / "libeagle4_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc would otherwise pair fp32 adds / multiplies / FMAs into v_pk_*_f32 on its own.
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
]


# Per-file additions. The streamed attention, tree-chunk and tree-replay kernels keep their MFMA accumulators in VGPRs (the default
# AGPR form makes LLVM shuttle them between the two register files: every iteration in the attention kernel, for every
# accumulator the chunk and replay kernels' VALU math reads).
EXTRA_FLAGS = {"verify_attention_stream.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
               "gdn_tree_chunk.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
               "gdn_tree_replay.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 kernels)")


def _spills(stderr: str) -> list[str]:
    """Kernels whose resource-usage remarks report spilled vector registers or scratch memory, as "name: what".
    (Scalar registers spill into vector-register lanes, not memory, and are left alone.)"""
    found, name = [], None
    for line in stderr.splitlines():
        if "remark: Function Name:" in line:
            name = line.split("Function Name:")[1].split("[")[0].strip()
        for key in ("VGPRs Spill:", "ScratchSize [bytes/lane]:"):
            if key in line and name is not None:
                value = int(line.split(key)[1].split("[")[0].strip())
                if value > 0:
                    found.append(f"{name}: {key} {value}")
    return found


def _compile(hipcc: str, src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-Rpass-analysis=kernel-resource-usage", "-c",
           str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    # a kernel that spills vector registers to scratch runs its inner loops through memory: refuse the build
    spilled = _spills(proc.stderr)
    if spilled:
        raise RuntimeError(f"{src.name}: kernels spill vector registers (the hot loops would go through scratch):\n  "
                           + "\n  ".join(spilled))
    return obj


def build(jobs: int | None = None) -> Path:
    """Compiles every kernel source and links the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(lambda s: _compile(hipcc, s), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
    sys.exit(0)
