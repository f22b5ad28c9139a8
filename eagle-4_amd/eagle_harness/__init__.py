"""MI355X-native kernels of EAGLE-4's draft-tree verify hot path, under the reference package's module names.

This ``eagle_harness`` holds only the verify path of eagle-harness 0.1.5, with the reference's call signatures, so its
callers drop in unchanged:

- ``eagle_harness.kernels``: ``gdn_tree`` (tree tables), ``gdn_tree_conv``, ``gdn_tree_recurrence``,
  ``gdn_tree_records``, ``accept_tail``, ``verify_prep``, ``row_attention``, ``mamba2_tree``, ``arch``
  (the reference's ``online_softmax`` is a Triton helper inlined into its attention kernels; its step lives inside
  the HIP attention kernels here, so there is no module for it);
- ``eagle_harness.vllm``: ``verify_attention``, ``verify_layout`` (the verify stage), ``tree_accept`` (the walk) and
  ``gdn_tree_verify`` (the accepted-path state commit), all engine-free.

Every launch goes to hand-written gfx950 HIP kernels in ``kernels/libeagle4_amd.so`` through a plain C ABI; nothing
here falls back to another implementation.
"""

__version__ = "0.1.0"
