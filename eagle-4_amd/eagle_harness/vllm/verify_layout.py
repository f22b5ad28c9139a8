"""Verify-round tree tables kept in fixed buffers, so a captured HIP graph sees the current round's trees
(the role of vllm/verify_layout.py).

Two holders. :class:`TreeStore` is indexed by request state slot and outlives a round: the drafter writes each
request's parent rows into it, the accept walk writes the accepted rows back. :class:`VerifyStage` is indexed by the
row of the current batch: :meth:`VerifyStage.stage` copies the batch's trees out of the store, derives the tables the
verify kernels read (masks, window codes, context lengths, slot-indexed parents and depths) and moves each draft
row's position from its place in the flattened chain to ``context + depth``. One gfx950 launch does all of it
(``csrc/tree_tables.hip``). Rows of a tree are ordered so a parent precedes its children; a prefix of the rows is a
tree of its own.
"""

from __future__ import annotations

import torch

from eagle_harness.kernels import _native

# Negative window codes name the columns of the request's saved conv history: the root's parent is -1 (the newest
# saved input), its grandparent -2, and -3 is the oldest of the three.
WINDOW_CODES = (-1, -2, -3)


def stage_tree(
    parents: torch.Tensor,
    idx_mapping: torch.Tensor,
    query_start_loc: torch.Tensor,
    cu_num_logits: torch.Tensor,
    positions: torch.Tensor,
    stage_parents: torch.Tensor,
    stage_anc: torch.Tensor,
    stage_mask: torch.Tensor,
    context_lens: torch.Tensor,
    slot_parents: torch.Tensor,
    slot_depths: torch.Tensor,
    num_reqs: int,
    *,
    tree: bool,
    chain_positions: torch.Tensor | None = None,
    num_tokens: int = 0,
) -> None:
    """The engine-free form of ``_stage_tree_kernel`` (vllm/verify_layout.py:31-86): per request, depth, the three
    window codes, the ancestor-or-self int64 mask, ``context_lens = positions[start]`` and, for a tree, positions
    rewritten to ``context + depth``; chains for anything that is not a tree. With ``chain_positions``, the same
    launch first saves ``positions[:num_tokens]`` into it (VerifyStage.stage's copy, :159)."""
    width = stage_parents.shape[1]
    if width > 64:
        raise ValueError(f"a verify tree has at most 64 rows, got {width}")
    for t, name in ((stage_parents, "stage_parents"), (stage_anc, "stage_anc"), (stage_mask, "stage_mask"),
                    (slot_parents, "slot_parents"), (slot_depths, "slot_depths")):
        assert t.is_contiguous(), f"{name} must be contiguous"
    assert positions.dtype == torch.int64 and stage_mask.dtype == torch.int64
    if chain_positions is not None:
        assert chain_positions.dtype == torch.int64 and chain_positions.is_contiguous()
        assert chain_positions.numel() >= num_tokens and positions.numel() >= num_tokens
    args = _native.StageTreeArgs(
        parents=_native.itab(parents),
        idx_mapping=_native.itab(idx_mapping),
        query_start_loc=_native.itab(query_start_loc),
        cu_num_logits=_native.itab(cu_num_logits),
        positions=positions.data_ptr(),
        stage_parents=stage_parents.data_ptr(),
        stage_anc=stage_anc.data_ptr(),
        stage_mask=stage_mask.data_ptr(),
        context_lens=context_lens.data_ptr(),
        slot_parents=slot_parents.data_ptr(),
        slot_depths=slot_depths.data_ptr(),
        chain_positions=_native.ptr(chain_positions),
        num_reqs=num_reqs,
        width=width,
        tree=int(tree),
        num_tokens=num_tokens if chain_positions is not None else 0,
    )
    _native.launch("eagle4_stage_tree", args, positions.device)


class TreeStore:
    """Per request state slot (vllm/verify_layout.py:89-97): ``parents`` [slots, W] int32 as the drafter leaves them
    (row 0 holds -1), and the accept walk's result, ``path`` [slots, W] (accepted rows from the root) with
    ``path_len`` [slots] valid entries."""

    def __init__(self, max_reqs: int, width: int, device: torch.device):
        self.width = width
        self.parents = torch.full((max_reqs, width), -1, dtype=torch.int32, device=device)
        self.path = torch.zeros(max_reqs, width, dtype=torch.int32, device=device)
        self.path_len = torch.ones(max_reqs, dtype=torch.int32, device=device)


class VerifyStage:
    """Per batch row (vllm/verify_layout.py:100-190): the tables the verify layers read during one forward, plus
    ``state_slots``, the GDN slot rows a linear-attention layer copies in during the forward so that a graph replay
    refreshes them as well."""

    def __init__(self, max_reqs: int, max_tokens: int, width: int, device: torch.device):
        if width > 64:
            raise ValueError(f"a verify tree has at most 64 rows, got {width}")
        self.width = width
        self.parents = torch.zeros(max_reqs, width, dtype=torch.int32, device=device)
        self.ancestors = torch.zeros(max_reqs, 3, width, dtype=torch.int32, device=device)
        self.masks = torch.ones(max_reqs, width, dtype=torch.int64, device=device)
        self.context_lens = torch.zeros(max_reqs, dtype=torch.int32, device=device)
        self.slot_parents = torch.zeros(max_reqs, width, dtype=torch.int32, device=device)
        self.slot_depths = torch.zeros(max_reqs, width, dtype=torch.int32, device=device)
        self.chain_positions = torch.zeros(max_tokens, dtype=torch.int64, device=device)
        self.max_reqs, self.device = max_reqs, device
        self.state_slots: dict[str, torch.Tensor] = {}
        self.active = True

    @property
    def verifying(self) -> bool:
        """True when the layers must run their tree kernels: after a tree was staged, and always while the current
        stream captures a graph (a capture records only the kernels it runs, and the verify graphs are captured
        with no batch staged)."""
        return self.active or torch.cuda.is_current_stream_capturing()

    def publish_slots_of(self, layer_name: str) -> torch.Tensor:
        """Allocates (or replaces) the [max_reqs, W] int32 table into which the layer ``layer_name``, the one chosen
        per KV cache group, copies its group's state slots."""
        buf = self.state_slots[layer_name] = torch.zeros(self.max_reqs, self.width, dtype=torch.int32, device=self.device)
        return buf

    def stage(
        self,
        store: TreeStore,
        idx_mapping: torch.Tensor,
        query_start_loc: torch.Tensor,
        cu_num_logits: torch.Tensor,
        positions: torch.Tensor,
        num_reqs: int,
        num_tokens: int,
        *,
        tree: bool,
        model_positions: torch.Tensor | None = None,
    ) -> None:
        """Fills this stage from ``store`` for the batch described by ``idx_mapping`` / ``query_start_loc`` /
        ``cu_num_logits`` and rewrites ``positions`` in place to tree positions; the chain positions are kept for
        :meth:`restore_positions`. With ``tree=False`` every request is staged as a chain and ``positions`` keep
        their values. ``model_positions``, when the model reads positions from a separate (e.g. multi-row)
        tensor, is shifted by the same per-token amounts."""
        stage_tree(
            store.parents,
            idx_mapping,
            query_start_loc,
            cu_num_logits,
            positions,
            self.parents,
            self.ancestors,
            self.masks,
            self.context_lens,
            self.slot_parents,
            self.slot_depths,
            num_reqs,
            tree=tree,
            chain_positions=self.chain_positions,
            num_tokens=num_tokens,
        )
        self.active = tree
        if model_positions is not None:
            model_positions[:, :num_tokens] += positions[:num_tokens] - self.chain_positions[:num_tokens]

    def restore_positions(self, positions: torch.Tensor, num_tokens: int) -> None:
        """Writes the saved chain positions back into ``positions`` (a no-op when chains were staged)."""
        if self.active:
            positions[:num_tokens].copy_(self.chain_positions[:num_tokens])


_STAGE: VerifyStage | None = None


def set_stage(stage: VerifyStage | None) -> None:
    global _STAGE
    _STAGE = stage


def get_stage() -> VerifyStage | None:
    """The stage registered by :func:`set_stage`, or ``None``."""
    return _STAGE
