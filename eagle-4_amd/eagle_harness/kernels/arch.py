"""Device gate of the gfx950 library: which visible GPU the kernels run on, and the launch features callers ask about.

``libeagle4_amd.so`` carries code objects for a single ISA, gfx950 (MI355X, CDNA4). A device is covered exactly when
the ISA part of its target name (``gcnArchName`` up to the first ``:``, e.g. ``gfx950`` of
``gfx950:sramecc+:xnack-``) is that ISA; nothing else about the device changes which kernel runs. Looking a device
up goes through torch's device properties only, so importing this module does not touch the GPU, and asking about a
machine without one returns a reason instead of raising.

The feature predicates are the names the reference's launchers call (kernels/arch.py:122-171). Each is a fixed answer
for a covered gfx950 device, listed in :data:`FEATURES` with the reason, and False for any device that is not
covered.
"""

from __future__ import annotations

import functools
from dataclasses import dataclass
from typing import Callable, Optional, Union

import torch

TARGET_ARCH = "gfx950"
AMD_ARCHS = (TARGET_ARCH,)

DeviceLike = Union[None, int, str, torch.device]


class UnsupportedHardware(RuntimeError):
    """Raised by :func:`require_supported` when the device cannot run the gfx950 code objects."""


@dataclass(frozen=True)
class Gpu:
    """What the gate knows about one visible device."""

    index: int
    name: str
    vendor: str  # "amd" on a ROCm build of torch, "nvidia" on a CUDA build
    arch: str  # ISA name: "gfx950"; "sm_90" style on NVIDIA
    sm: int = 0  # NVIDIA compute capability (major * 10 + minor); 0 on AMD
    target: str = ""  # the full target string with its feature flags, e.g. "gfx950:sramecc+:xnack-"
    compute_units: int = 0

    @property
    def nvidia(self) -> bool:
        return self.vendor == "nvidia"


def _device_index(device: DeviceLike) -> Optional[int]:
    """Index of a GPU device spec; None for anything that names a non-GPU device."""
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    spec = torch.device(device)
    if spec.type != "cuda":
        return None
    return spec.index if spec.index is not None else torch.cuda.current_device()


@functools.lru_cache(maxsize=None)
def _describe(index: int) -> Gpu:
    props = torch.cuda.get_device_properties(index)
    cus = int(getattr(props, "multi_processor_count", 0))
    if torch.version.hip is None:
        cc = props.major * 10 + props.minor
        return Gpu(index, props.name, "nvidia", f"sm_{cc}", cc, "", cus)
    target = str(props.gcnArchName)
    return Gpu(index, props.name, "amd", target.partition(":")[0], 0, target, cus)


def gpu(device: DeviceLike = None) -> Optional[Gpu]:
    """Description of the device behind ``device`` (the current one by default); None when there is no GPU."""
    if not torch.cuda.is_available():
        return None
    index = _device_index(device)
    return None if index is None else _describe(index)


def unsupported_reason(device: DeviceLike = None) -> Optional[str]:
    """Why the kernels cannot run on ``device``, in one line; None when they can."""
    found = gpu(device)
    if found is None:
        return "torch sees no ROCm GPU"
    if found.arch != TARGET_ARCH:
        return (f"{found.name} is {found.arch or 'an unknown ISA'}, and libeagle4_amd.so holds {TARGET_ARCH} "
                f"(MI355X) code objects only")
    return None


def require_supported(device: DeviceLike = None) -> Gpu:
    """The covered device behind ``device``; :class:`UnsupportedHardware` otherwise."""
    reason = unsupported_reason(device)
    if reason is not None:
        raise UnsupportedHardware(f"eagle4_amd: the gfx950 kernels cannot run here: {reason}")
    return gpu(device)  # type: ignore[return-value]


# Launch features, as the reference's launchers name them: the answer on a covered gfx950 device, and why.
FEATURES: dict[str, tuple[bool, str]] = {
    "native_candidate_tail": (False, "the candidate tail is a CUDA kernel; its HIP counterpart is not on this path"),
    "clusters": (False, "thread-block clusters are a CUDA launch attribute; CDNA4 has no counterpart"),
    "pdl": (False, "programmatic dependent launch is CUDA-only; these kernels follow plain stream order"),
    "gluon_gdn": (False, "the Gluon GDN walk targets NVIDIA sm_103; the HIP walk serves every shape here"),
    "draftmk": (False, "the draft-round megakernel ships as sm_103a code only"),
    "gdn_records_replay": (True, "GDN verify keeps replay records and commits the accepted path, the AMD default"),
    "side_stream_prelaunch": (False, "the next round's draft work stays on the caller's stream on AMD"),
}


def _feature(name: str) -> Callable[[DeviceLike], bool]:
    on, why = FEATURES[name]

    def predicate(device: DeviceLike = None) -> bool:
        return on and unsupported_reason(device) is None

    predicate.__name__ = predicate.__qualname__ = name
    predicate.__doc__ = f"{'On' if on else 'Off'} for gfx950: {why}."
    return predicate


native_candidate_tail = _feature("native_candidate_tail")
clusters = _feature("clusters")
pdl = _feature("pdl")
gluon_gdn = _feature("gluon_gdn")
draftmk = _feature("draftmk")
gdn_records_replay = _feature("gdn_records_replay")
side_stream_prelaunch = _feature("side_stream_prelaunch")


def report() -> str:
    """Every visible device with its verdict, and the feature answers when it is covered."""
    if not torch.cuda.is_available():
        return f"no device: {unsupported_reason()}"
    out = []
    for index in range(torch.cuda.device_count()):
        found = _describe(index)
        reason = unsupported_reason(index)
        head = f"cuda:{index} {found.name} [{found.target or found.arch}, {found.compute_units} CUs]"
        if reason is not None:
            out.append(f"{head}: not covered ({reason})")
            continue
        flags = " ".join(f"{name}={'on' if on else 'off'}" for name, (on, _) in FEATURES.items())
        out.append(f"{head}: covered; {flags}")
    return "\n".join(out)


if __name__ == "__main__":
    print(report())
