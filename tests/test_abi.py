"""The C-ABI boundary on the CPU: the built library loads, exports exactly the entry points include/eagle4_amd.h
declares, agrees with the ctypes binding on every argument struct's size, and the host binding covers every compute
entry point. No kernel is launched (no GPU here)."""

import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "eagle4_amd.h")


def _declared() -> set:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(eagle4_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib_path():
    from eagle_harness.kernels import _native

    path = str(_native.LIBRARY)
    if not os.path.exists(path):  # build it (hipcc cross-compiles gfx950 without a GPU)
        sys.path.insert(0, os.path.join(ROOT, "eagle-4_amd"))
        import build

        build.build()
    return path


def test_header_declares_the_entry_points():
    names = _declared()
    assert "eagle4_verify_attention" in names and "eagle4_gdn_tree_recurrent_update" in names
    assert len(names) >= 15


def test_library_exports_exactly_the_declared_symbols(lib_path):
    lib = ctypes.CDLL(lib_path)
    declared = _declared()
    missing = sorted(n for n in declared if not hasattr(lib, n))
    assert not missing, f"declared in eagle4_amd.h but not exported: {missing}"
    nm = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if line.split() and line.split()[-1].startswith("eagle4_")}
    assert exported == declared, f"exported but undeclared: {sorted(exported - declared)}"


def test_binding_struct_sizes_and_version(lib_path):
    from eagle_harness.kernels import _native

    lib = _native.library()  # checks every args struct against eagle4_args_size
    assert b"gfx950" in lib.eagle4_version()
    bound = set(_native.ENTRIES) | set(_native.EXTRA_SYMBOLS)
    assert bound == _declared(), f"declared but not bound by the host module: {sorted(_declared() - bound)}"
    assert lib.eagle4_args_size(len(_native.ENTRIES)) < 0  # past the last struct: an error, not a size


def test_launch_refuses_cpu_tensors():
    """No CPU fallback: a host tensor is an error before anything is launched."""
    import torch

    from eagle_harness.kernels import _native

    with pytest.raises(RuntimeError, match="ROCm GPU"):
        _native.launch("eagle4_stage_tree", _native.StageTreeArgs(), torch.device("cpu"))
