"""Which GPU can run which kernel: the single place that reads a device's architecture (kernels/arch.py).

The kernels here are built for one target, gfx950 (MI355X). Importing this module never initialises the GPU and never
raises; :func:`unsupported_reason` says why a device is not covered and :func:`require_supported` raises
:class:`UnsupportedHardware` with that message. The feature predicates keep the reference's names (kernels/arch.py:
122-171) so callers read them unchanged: PDL, clusters and the Gluon GDN twin are NVIDIA features and are off; the
records-replay commit is on (the AMD default of the reference).
"""

from __future__ import annotations

import functools
from dataclasses import dataclass
from typing import Optional, Union

import torch

TARGET_ARCH = "gfx950"
AMD_ARCHS = (TARGET_ARCH,)

DeviceLike = Union[None, int, str, torch.device]


class UnsupportedHardware(RuntimeError):
    """The visible GPU (or the software stack) is outside what the kernels cover."""


@dataclass(frozen=True)
class Gpu:
    """One visible GPU: index, name, vendor and architecture."""

    index: int
    name: str
    vendor: str
    arch: str
    sm: int = 0

    @property
    def nvidia(self) -> bool:
        return self.vendor == "nvidia"


def _index(device: DeviceLike) -> Optional[int]:
    if isinstance(device, int):
        return device
    dev = torch.device("cuda" if device is None else device)
    if dev.type != "cuda":
        return None
    return torch.cuda.current_device() if dev.index is None else dev.index


@functools.lru_cache(maxsize=None)
def _probe(index: int) -> Gpu:
    props = torch.cuda.get_device_properties(index)
    if torch.version.hip:
        return Gpu(index, props.name, "amd", props.gcnArchName.split(":")[0], 0)
    return Gpu(index, props.name, "nvidia", f"sm_{props.major}{props.minor}", props.major * 10 + props.minor)


def gpu(device: DeviceLike = None) -> Optional[Gpu]:
    """The GPU behind ``device`` (default: the current one), None without one."""
    if not torch.cuda.is_available():
        return None
    index = _index(device)
    return _probe(index) if index is not None else None


def unsupported_reason(device: DeviceLike = None) -> Optional[str]:
    """None when the kernels run on ``device``, else a one-line reason."""
    g = gpu(device)
    if g is None:
        return "no ROCm device is visible to torch"
    if g.nvidia or g.arch not in AMD_ARCHS:
        return f"{g.name} ({g.arch}) is not {TARGET_ARCH} (MI355X); the kernels are built for {TARGET_ARCH} only"
    return None


def require_supported(device: DeviceLike = None) -> Gpu:
    """The GPU behind ``device``; raises :class:`UnsupportedHardware` where the kernels do not run."""
    if (reason := unsupported_reason(device)) is not None:
        raise UnsupportedHardware(f"eagle4_amd kernels are off: {reason}.")
    return gpu(device)  # type: ignore[return-value]


def _ours(device: DeviceLike) -> bool:
    return unsupported_reason(device) is None


def native_candidate_tail(device: DeviceLike = None) -> bool:
    """The CUDA candidate-tail kernel: NVIDIA only."""
    return False


def clusters(device: DeviceLike = None) -> bool:
    """Thread-block clusters: NVIDIA only."""
    return False


def pdl(device: DeviceLike = None) -> bool:
    """Programmatic dependent launch: NVIDIA only; the HIP kernels here run in stream order."""
    return False


def gluon_gdn(device: DeviceLike = None) -> bool:
    """The Gluon GDN twin: NVIDIA sm_103 only."""
    return False


def draftmk(device: DeviceLike = None) -> bool:
    """The draft-round megakernel: NVIDIA B300 only."""
    return False


def gdn_records_replay(device: DeviceLike = None) -> bool:
    """Replay records plus an accepted-path commit instead of per-node snapshots (the reference's AMD default)."""
    return _ours(device)


def side_stream_prelaunch(device: DeviceLike = None) -> bool:
    """Draft prelaunch on a side stream: off on AMD, as in the reference."""
    return False


def report() -> str:
    """One line per visible device."""
    if not torch.cuda.is_available():
        return f"no GPU visible: {unsupported_reason()}"
    lines = []
    for i in range(torch.cuda.device_count()):
        g = _probe(i)
        reason = unsupported_reason(i)
        lines.append(f"cuda:{i} {g.name} ({g.arch}): " + (f"OFF, {reason}" if reason else "supported"))
    return "\n".join(lines)


if __name__ == "__main__":
    print(report())
