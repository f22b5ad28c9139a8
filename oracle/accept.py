"""Greedy tree acceptance, restated on the CPU (oracle; test infrastructure only)."""

from __future__ import annotations

from typing import Optional

import torch


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """The greedy target token of every row: ``torch.argmax`` (first index on ties), int64. The reference takes it
    from vLLM's sampler with temperature 0 (vllm/tree_accept.py:195-216)."""
    return logits.float().argmax(-1)


def accept_tree(
    target: torch.Tensor,
    drafted: torch.Tensor,
    cu_num_logits: torch.Tensor,
    idx_mapping: torch.Tensor,
    parents: torch.Tensor,
    path: torch.Tensor,
    path_len: torch.Tensor,
    width: int,
):
    """``_tree_accept_kernel`` / ``accept_tree`` (vllm/tree_accept.py:45-115): from the root, emit the target token of
    the current node and move to the lowest-index row whose parent is the node and whose drafted token equals it.

    Returns (sampled [R, W] int64 with only the walked steps written (others 0), num_sampled [R] int32); writes
    ``path[slot, :count]`` and ``path_len[slot]``."""
    num_reqs = cu_num_logits.shape[0] - 1
    sampled = torch.zeros(num_reqs, width, dtype=torch.int64)
    num_sampled = torch.zeros(num_reqs, dtype=torch.int32)
    for b in range(num_reqs):
        slot = int(idx_mapping[b])
        start = int(cu_num_logits[b])
        rows = int(cu_num_logits[b + 1]) - start
        par = [int(parents[slot, r]) for r in range(width)]
        node, alive, count = 0, rows > 0, 0
        for step in range(width):
            token = int(target[start + node]) if 0 <= node < rows else 0
            if alive:
                sampled[b, step] = token
                path[slot, step] = node
                count += 1
            child = None
            for r in range(1, min(rows, width)):
                if par[r] == node and int(drafted[start + r]) == token:
                    child = r
                    break
            alive = alive and child is not None
            if alive:
                node = child
        num_sampled[b] = count
        path_len[slot] = count
    return sampled, num_sampled


def accept_tail(target_predict, candidates, retrieve_index, retrieve_next_token, retrieve_next_sibling, seq_lens,
                out_cache_loc, req_to_token, req_pool_indices, depth: int):
    """``_accept_tail_kernel`` / ``accept_tail`` (kernels/accept_tail.py:56-187), batch size 1.

    Returns a dict with the fields of the reference's ``Accepted`` (:37-46)."""
    width = target_predict.numel()
    tp = [int(x) for x in target_predict.reshape(-1)]
    cand = [int(x) for x in candidates.reshape(-1)]
    ridx = [int(x) for x in retrieve_index.reshape(-1)]
    nxt = [int(x) for x in retrieve_next_token.reshape(-1)]
    sib = [int(x) for x in retrieve_next_sibling.reshape(-1)]
    accept_index = [-1] * depth  # :79-80
    last = ridx[0]
    if depth > 0:
        accept_index[0] = last  # :85-86
    cur, num, active = 0, 0, True
    for _level in range(1, depth):  # :90-106
        if not active:
            continue
        cur = nxt[cur]
        target_token = tp[last]
        found = 0
        for _sibling in range(width):
            if found != 0:
                continue
            valid = cur != -1
            safe = cur if valid else 0
            node = ridx[safe]
            match = valid and cand[safe] == target_token
            if match:
                accept_index[num + 1] = node
                num += 1
                last = node
            elif valid:
                cur = sib[safe]
            found = 1 if match else (0 if valid else -1)
        active = found == 1
    seq_len = int(seq_lens.reshape(-1)[0])
    # :115-123: predictions, the accepted path moved to the front (padding reads node 0's target)
    accepted = set(accept_index[d] for d in range(depth) if d <= num)
    predict = []
    for node in range(width):
        if node < depth:
            predict.append(tp[max(accept_index[node], 0)])
        else:
            predict.append(tp[node] if node in accepted else 0)
    row = int(req_pool_indices.reshape(-1)[0])
    committed, accepted_slots = [], []
    for d in range(depth):  # :126-132
        keep = d <= num
        committed.append(int(req_to_token[row, seq_len + d]) if keep else 0)
        accepted_slots.append(int(out_cache_loc.reshape(-1)[accept_index[d]]) if keep else 0)
    return dict(
        predict=torch.tensor(predict, dtype=torch.int32),
        accept_index=torch.tensor([accept_index], dtype=torch.int32),
        accept_lens=torch.tensor([num + 1], dtype=torch.int32),
        new_seq_lens=torch.tensor([seq_len + num + 1], dtype=seq_lens.dtype),
        bonus_tokens=torch.tensor([tp[last]], dtype=torch.int32),
        committed_slots=torch.tensor(committed, dtype=torch.int64),
        accepted_slots=torch.tensor(accepted_slots, dtype=torch.int64),
    )


def compact_rows(rows: torch.Tensor, accept_index: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``_compact_rows_kernel`` / ``compact_rows`` (kernels/accept_tail.py:190-224): row ``i < depth`` takes row
    ``max(accept_index[0, i], 0)``, the others keep their own."""
    width = rows.shape[0]
    depth = accept_index.shape[1]
    if out is None:
        out = torch.empty_like(rows)
    for r in range(width):
        src = max(int(accept_index[0, min(r, depth - 1)]), 0) if r < depth else r
        out[r] = rows[src]
    return out


def accepted_rows_first(expanded_idx_mapping, expanded_local_pos, path, path_len) -> torch.Tensor:
    """``accepted_rows_first`` (vllm/tree_accept.py:118-126)."""
    rows = torch.arange(expanded_local_pos.shape[0])
    slots, k = expanded_idx_mapping.long(), expanded_local_pos.long()
    accepted = rows - k + path[slots, k].long()
    return torch.where(k < path_len[slots], accepted, rows)
