"""MI355X-native kernels of EAGLE-4's draft-tree verify hot path, as an overlay on the reference package.

This ``eagle_harness`` holds only the verify path of eagle-harness 0.1.5, with the reference's module names and call
signatures:

- ``eagle_harness.kernels``: ``gdn_tree`` (tree tables), ``gdn_tree_conv``, ``gdn_tree_recurrence``,
  ``gdn_tree_records``, ``accept_tail``, ``verify_prep``, ``row_attention``, ``mamba2_tree``;
- ``eagle_harness.vllm``: ``verify_attention``, ``verify_layout`` (the verify stage), ``tree_attention`` (the CUSTOM
  backend), ``tree_accept`` (the greedy walk), ``gdn_tree_verify`` (the layer hook and the accepted-path state
  commit) and ``round_commit``.

Every launch of these modules goes to hand-written gfx950 HIP kernels in ``kernels/libeagle4_amd.so`` through a plain
C ABI; nothing here falls back to another implementation.

Placed ahead of an installed eagle-harness on ``sys.path``, the package and its ``kernels`` / ``vllm`` subpackages
extend their ``__path__`` with the installed package's directories (:func:`pkgutil.extend_path`): a module built
here is found here first, every other module (the engines' plugins, the draft side, ``kernels.arch``, the cost model)
is the installed one, unchanged. The plugins' own imports of the verify path then land on this package's modules.
"""

from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)


def _reference_version() -> str:
    """The installed eagle-harness distribution's version (``compat`` reports it); the version whose interface this
    overlay serves when none is installed."""
    import importlib.metadata

    try:
        return importlib.metadata.version("eagle-harness")
    except importlib.metadata.PackageNotFoundError:
        return "0.1.5"


__version__ = _reference_version()
__amd_version__ = "0.3.0"  # this overlay's own version
