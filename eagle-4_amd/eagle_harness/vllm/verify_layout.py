"""The tree of the current verify forward, in buffers that graphs replay (vllm/verify_layout.py).

``propose`` stores the parent row of every verify row of a request (:class:`TreeStore`, by request state slot).
Before each target forward :meth:`VerifyStage.stage` gathers the batch's rows into :class:`VerifyStage` (by batch
row) and rewrites the forward's positions from chain positions to depths, in one gfx950 launch
(``csrc/tree_tables.hip``). Row 0 of a request is the root; rows are parent first, so any prefix of the rows is a
tree too.
"""

from __future__ import annotations

import torch

from eagle_harness.kernels import _native

# The conv window of the root reads the request's conv state: codes -1, -2, -3 are the last, second to last and
# third to last entry of the window before the root.
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
) -> None:
    """The engine-free form of ``_stage_tree_kernel`` (vllm/verify_layout.py:31-86): per request, depth, the three
    window codes, the ancestor-or-self int64 mask, ``context_lens = positions[start]`` and, for a tree, positions
    rewritten to ``context + depth``; chains for anything that is not a tree."""
    width = stage_parents.shape[1]
    if width > 64:
        raise ValueError(f"a verify tree has at most 64 rows, got {width}")
    for t, name in ((stage_parents, "stage_parents"), (stage_anc, "stage_anc"), (stage_mask, "stage_mask"),
                    (slot_parents, "slot_parents"), (slot_depths, "slot_depths")):
        assert t.is_contiguous(), f"{name} must be contiguous"
    assert positions.dtype == torch.int64 and stage_mask.dtype == torch.int64
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
        num_reqs=num_reqs,
        width=width,
        tree=int(tree),
    )
    _native.launch("eagle4_stage_tree", args, positions.device)


class TreeStore:
    """The tree of each request by request state slot: ``parents`` (written by the drafter) and the accepted
    ``path`` (root first, ``path_len`` rows) the walk writes (vllm/verify_layout.py:89-97)."""

    def __init__(self, max_reqs: int, width: int, device: torch.device):
        self.width = width
        self.parents = torch.full((max_reqs, width), -1, dtype=torch.int32, device=device)
        self.path = torch.zeros(max_reqs, width, dtype=torch.int32, device=device)
        self.path_len = torch.ones(max_reqs, dtype=torch.int32, device=device)


class VerifyStage:
    """The batch's trees, by batch row (vllm/verify_layout.py:100-190)."""

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
        """Whether the target's layers take the tree path now: a tree is staged, or a graph is being captured."""
        return self.active or torch.cuda.is_current_stream_capturing()

    def publish_slots_of(self, layer_name: str) -> torch.Tensor:
        """The buffer a linear-attention layer (one per KV cache group) publishes its group's slots to."""
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
        """Gather the batch's trees from ``store`` and turn ``positions`` from chain to depth positions
        (``tree=False``: stage chains and leave the positions)."""
        self.chain_positions[:num_tokens].copy_(positions[:num_tokens])
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
        )
        self.active = tree
        if model_positions is not None:
            model_positions[:, :num_tokens] += positions[:num_tokens] - self.chain_positions[:num_tokens]

    def restore_positions(self, positions: torch.Tensor, num_tokens: int) -> None:
        """Put the chain positions back after the verify forward."""
        if self.active:
            positions[:num_tokens].copy_(self.chain_positions[:num_tokens])


_STAGE: VerifyStage | None = None


def set_stage(stage: VerifyStage | None) -> None:
    global _STAGE
    _STAGE = stage


def get_stage() -> VerifyStage | None:
    """The process's verify stage; ``None`` while no speculator is running."""
    return _STAGE
