"""GDN tree verify tables (kernels/gdn_tree.py): the tree of every request derived once per forward.

:func:`gdn_tree_ancestors` replays sglang's parent derivation from the first-child / next-sibling links, records the
three conv-window ancestors of every node (code ``v >= 0`` is node ``v``; ``-1 / -2 / -3`` are conv-state columns
``2 / 1 / 0``) and, with ``paths``, the path table of the replay kernels (one row per leaf: ``[length, write_from,
root path...]``). One gfx950 workgroup per request (``csrc/tree_tables.hip``).
"""

from __future__ import annotations

from typing import Optional

import torch

from eagle_harness.kernels import _native

PAD_SLOT_ID = -1  # a padded request row of a batch (sglang's causal_conv1d PAD_SLOT_ID)


def gdn_tree_ancestors(
    retrieve_next_token: torch.Tensor,
    retrieve_next_sibling: torch.Tensor,
    retrieve_parent_token: torch.Tensor,
    conv_state_indices: torch.Tensor,
    width: int,
    ancestors: torch.Tensor,
    query_start_loc: Optional[torch.Tensor] = None,
    paths: Optional[torch.Tensor] = None,
    pad_slot_id: int = PAD_SLOT_ID,
) -> None:
    """Derive the tree of every request from the first ``width`` columns of the links (kernels/gdn_tree.py:189-237).

    Writes ``retrieve_parent_token[:, :width]`` and ``ancestors`` (batch, 3, width), and with ``paths`` (batch, width,
    2 + width) the path table (each request's node count from ``query_start_loc``). Rows whose
    ``conv_state_indices`` entry is ``pad_slot_id`` keep their parents and ancestors; their paths follow their current
    parents.
    """
    batch = ancestors.shape[0]
    assert tuple(ancestors.shape) == (batch, 3, width) and ancestors.dtype == torch.int32
    assert ancestors.is_contiguous()
    build_paths = paths is not None
    if build_paths:
        assert query_start_loc is not None and width < 256
        assert tuple(paths.shape) == (batch, width, 2 + width) and paths.dtype == torch.int32
        assert paths.stride(2) == 1
    args = _native.AncestorsArgs(
        next_token=_native.itab(retrieve_next_token),
        next_sibling=_native.itab(retrieve_next_sibling),
        parent_token=_native.itab(retrieve_parent_token),
        conv_state_indices=_native.itab(conv_state_indices),
        query_start_loc=_native.itab(query_start_loc if build_paths else None),
        ancestors=ancestors.data_ptr(),
        paths=_native.ptr(paths),
        stride_paths_seq=paths.stride(0) if build_paths else 0,
        stride_paths_path=paths.stride(1) if build_paths else 0,
        batch=batch,
        width=width,
        pad_slot_id=pad_slot_id,
    )
    _native.launch("eagle4_gdn_tree_ancestors", args, ancestors.device)


def gdn_tree_paths_buffer(batch: int, width: int, device) -> torch.Tensor:
    """A path table for ``gdn_tree_ancestors(paths=...)`` (kernels/gdn_tree.py:240-242)."""
    return torch.zeros((batch, width, 2 + width), dtype=torch.int32, device=device)
