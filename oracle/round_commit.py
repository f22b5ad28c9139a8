"""vLLM's round commit, restated on the CPU (oracle; test infrastructure only).

Follows vllm/round_commit.py: ``KvCompactor.compact`` with ``_compact_kv_kernel`` (:33-83, :117-143) copies the KV of
the accepted rows of every verified tree to the chain slots ``context + j`` in path order; ``chainize`` with
``_chainize_kernel`` (:146-215) rewrites the round's rows for the draft's prefill. A request is a verified tree when
its query width is above 1 and equals its logits count (``_is_tree``, :26-29).
"""

from __future__ import annotations

import torch


def _is_tree(query_start_loc: torch.Tensor, cu_num_logits: torch.Tensor, b: int) -> bool:
    width = int(query_start_loc[b + 1]) - int(query_start_loc[b])
    return width > 1 and width == int(cu_num_logits[b + 1]) - int(cu_num_logits[b])


def compact_kv(
    kv_caches: list[torch.Tensor],
    block_tables: list[torch.Tensor],
    table_block_sizes: list[int],
    idx_mapping: torch.Tensor,
    query_start_loc: torch.Tensor,
    cu_num_logits: torch.Tensor,
    seq_lens: torch.Tensor,
    path: torch.Tensor,
    path_len: torch.Tensor,
) -> None:
    """In place on every layer's cache ``kv_caches[l]`` as the backend views it: (blocks, heads, slots in a block,
    2 * head_dim). Rows move one at a time in path order (:58-82)."""
    for layer, cache in enumerate(kv_caches):
        table, tbs = block_tables[layer], int(table_block_sizes[layer])
        block_size = cache.shape[2]
        for b in range(idx_mapping.shape[0]):
            if not _is_tree(query_start_loc, cu_num_logits, b):
                continue
            slot = int(idx_mapping[b])
            width = int(query_start_loc[b + 1]) - int(query_start_loc[b])
            context = int(seq_lens[b]) - width

            def where(pos: int) -> tuple[int, int]:  # (cache block, slot in the block) of a token position
                token = int(table[b, pos // tbs]) * tbs + pos % tbs
                return token // block_size, token % block_size

            for j in range(1, int(path_len[slot])):
                src, dst = context + int(path[slot, j]), context + j
                if src != dst:
                    (sb, ss), (db, ds) = where(src), where(dst)
                    cache[db, :, ds] = cache[sb, :, ss]


def chainize(
    input_ids: torch.Tensor,
    positions: torch.Tensor,
    src_rows: torch.Tensor,
    *,
    idx_mapping: torch.Tensor,
    query_start_loc: torch.Tensor,
    cu_num_logits: torch.Tensor,
    seq_lens: torch.Tensor,
    path: torch.Tensor,
    path_len: torch.Tensor,
    sampled: torch.Tensor,
    width: int,
) -> None:
    """In place: for every verified tree, row r (r < the power of two >= ``width``, inside the query) takes the
    hidden state of accepted row path[r] (its own past the path), chain position context + r, and rows
    1 .. accepted - 1 the sampled token r - 1 (:160-179)."""
    rows = 1 << max(int(width) - 1, 0).bit_length()
    for b in range(idx_mapping.shape[0]):
        start = int(query_start_loc[b])
        w = int(query_start_loc[b + 1]) - start
        if not _is_tree(query_start_loc, cu_num_logits, b):
            continue
        slot = int(idx_mapping[b])
        accepted = min(int(path_len[slot]), w)
        context = int(seq_lens[b]) - w
        for r in range(min(rows, w)):
            src_rows[start + r] = start + (int(path[slot, r]) if r < accepted else r)
            positions[start + r] = context + r
            if 1 <= r < accepted:
                input_ids[start + r] = int(sampled[b, r - 1])
