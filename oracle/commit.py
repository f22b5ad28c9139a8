"""vLLM's accepted-path commit of the linear-attention state, restated on the CPU (oracle; test infrastructure only).

Follows ``LinearStateCommit.commit`` with ``_compact_window_kernel`` and ``_move_state_kernel``
(vllm/gdn_tree_verify.py:186-245, 289-322): the window columns of the accepted rows move next to each other
(column ``2 + path[j]`` to ``2 + j``, ascending) and the recurrent state of the last accepted row moves into the slot
of row ``path_len - 1``, where the next round resumes. Slots ``<= 0`` (vLLM's null block) are skipped.
"""

from __future__ import annotations

import torch

NULL_BLOCK_ID = 0


def linear_state_commit(
    conv_states: list[torch.Tensor],
    ssm_states: list[torch.Tensor],
    slots: list[torch.Tensor],
    idx_mapping: torch.Tensor,
    path: torch.Tensor,
    path_len: torch.Tensor,
) -> None:
    """In place on every layer's window cache ``conv_states[l]`` ([slots, dim, state_len] view) and state pool
    ``ssm_states[l]`` ([slots, ...]); ``slots[l]`` [reqs, S] int32 is the layer's slot table."""
    num_reqs = idx_mapping.shape[0]
    for layer in range(len(conv_states)):
        conv, ssm, tab = conv_states[layer], ssm_states[layer], slots[layer]
        for b in range(num_reqs):
            state = int(idx_mapping[b])
            n = int(path_len[state])
            # _compact_window_kernel (:201-215)
            wslot = int(tab[b, 0])
            if wslot > NULL_BLOCK_ID:
                for j in range(1, n):
                    src = 2 + int(path[state, j])
                    if src != 2 + j:
                        conv[wslot, :, 2 + j] = conv[wslot, :, src]
            # _move_state_kernel (:232-245)
            last = int(path[state, n - 1])
            src_slot = int(tab[b, last])
            dst_slot = int(tab[b, n - 1])
            if last != n - 1 and src_slot > NULL_BLOCK_ID and dst_slot > NULL_BLOCK_ID:
                ssm[dst_slot] = ssm[src_slot]
