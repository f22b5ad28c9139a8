"""Reaching the installed eagle-harness's own module behind one of this overlay's modules.

Two of the modules this package provides under the reference's names also carry engine glue that is not part of the
verify kernels: vLLM's ``TreeRejectionSampler`` (a subclass of vLLM's rejection sampler that applies the engine's
sampling parameters, then calls the tree walk) lives in the reference's ``vllm/tree_accept.py``. This overlay does not
rewrite that glue; :func:`engine_module` runs the installed package's own file for such a module under a private name
and rebinds the kernel entry points it calls (``accept_tree``, ...) to this package's, so the glue's launches land in
``libeagle4_amd.so``.
"""

from __future__ import annotations

import importlib.util
import os
import sys
from types import ModuleType
from typing import Any, Optional


def shadowed_file(fullname: str) -> Optional[str]:
    """The installed package's source file of module ``fullname``, which this overlay's module of that name shadows:
    the first ``<portion>/<leaf>.py`` among the parent package's ``__path__`` portions other than this overlay's own
    directory; None when no installed package provides it."""
    parent, _, leaf = fullname.rpartition(".")
    own = os.path.dirname(os.path.realpath(sys.modules[fullname].__file__))
    for portion in sys.modules[parent].__path__:
        if os.path.realpath(portion) == own:
            continue
        path = os.path.join(portion, leaf + ".py")
        if os.path.isfile(path):
            return path
    return None


def engine_module(fullname: str, **rebind: Any) -> ModuleType:
    """The installed package's own ``fullname``, executed once as ``<parent>._installed_<leaf>`` with the names in
    ``rebind`` then pointed at this overlay's objects. Its imports of other ``eagle_harness`` modules resolve as any
    caller's do (to this overlay's modules where they exist). Raises ImportError when no installed package provides
    the module."""
    parent, _, leaf = fullname.rpartition(".")
    alias = f"{parent}._installed_{leaf}"
    module = sys.modules.get(alias)
    if module is not None:
        return module
    path = shadowed_file(fullname)
    if path is None:
        raise ImportError(
            f"{fullname}: the engine glue of this module is the installed eagle-harness's, and none is installed "
            "behind this overlay (put the overlay ahead of an eagle-harness installation on sys.path)", name=alias)
    spec = importlib.util.spec_from_file_location(alias, path)
    module = importlib.util.module_from_spec(spec)
    module.__package__ = parent
    sys.modules[alias] = module
    try:
        spec.loader.exec_module(module)
    except BaseException:
        del sys.modules[alias]
        raise
    for name, value in rebind.items():
        if not hasattr(module, name):
            raise ImportError(f"{path} defines no {name} to rebind to this overlay's kernels", name=alias)
        setattr(module, name, value)
    return module
