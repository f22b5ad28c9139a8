"""Kernels of the EAGLE-4 verify round on MI355X (gfx950). Raw tensors in, raw tensors out; no engine imports.

==================  =====================================================================================
module              what
==================  =====================================================================================
``gdn_tree``        GDN tree tables: links -> parents, conv window codes, path table
``gdn_tree_conv``   width-4 tree causal conv1d
``gdn_tree_recurrence``  gated delta rule over the tree, per-node state snapshots
``gdn_tree_records``     replay records and the accepted-path commit (records contract)
``accept_tail``     bs1 greedy accept tail and row compaction
``verify_prep``     tail-mask words
``row_attention``   draft-side row attention (sliding window + tree ancestors)
``mamba2_tree``     Mamba2 tree selective state update
``_native``         the ctypes binding of ``libeagle4_amd.so`` and its device gate
==================  =====================================================================================

The kernels are compiled ahead of time into ``libeagle4_amd.so`` (``python eagle-4_amd/build.py``). Modules not
built here (``arch``, the candidate head, the draft-side kernels) come from the installed eagle-harness: this
package's ``__path__`` continues into it.
"""

from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
