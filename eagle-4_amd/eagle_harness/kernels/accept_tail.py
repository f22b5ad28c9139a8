"""The greedy tree acceptance and everything that follows it, for one request (kernels/accept_tail.py).

:func:`accept_tail` is the walk over sglang's first-child / next-sibling links and all of the index and token
bookkeeping (accept lengths, bonus token, predictions with the accepted path moved to the front, the KV slots to
move) in one gfx950 launch; :func:`compact_rows` moves the accepted rows of a node-indexed tensor to the front.
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from eagle_harness.kernels import _native

# The reference sizes its index vectors to one warp (kernels/accept_tail.py:29-30); kept for callers that read it.
LANES = 32


class Accepted(NamedTuple):
    """Result of :func:`accept_tail` for one request (the fields of kernels/accept_tail.py:37-46). ``W`` is the
    tree width, ``depth`` the caller's maximum number of accepted tokens; ``n`` below is ``accept_lens[0]``."""

    predict: torch.Tensor  # [W] int32; entries 0..n-1: the target's token at each accepted node, root first
    accept_index: torch.Tensor  # [1, depth] int32; the accepted nodes' rows, then -1
    accept_lens: torch.Tensor  # [1] int32; n = accepted draft tokens + 1 (the target's own token at the end)
    new_seq_lens: torch.Tensor  # [1], dtype of seq_lens; seq_lens + n
    bonus_tokens: torch.Tensor  # [1] int32; predict[n - 1]
    committed_slots: torch.Tensor  # [depth] int64; KV slot where accepted token i belongs after the round, then 0
    accepted_slots: torch.Tensor  # [depth] int64; KV slot the verify forward wrote accepted token i to, then 0


def accept_tail(
    target_predict: torch.Tensor,
    candidates: torch.Tensor,
    retrieve_index: torch.Tensor,
    retrieve_next_token: torch.Tensor,
    retrieve_next_sibling: torch.Tensor,
    seq_lens: torch.Tensor,
    out_cache_loc: torch.Tensor,
    req_to_token: torch.Tensor,
    req_pool_indices: torch.Tensor,
    depth: int,
) -> Accepted:
    """Greedy-accept one request's verify tree against ``target_predict`` (the target's argmax per node;
    kernels/accept_tail.py:135-187). ``depth`` is the width of ``accept_index``."""
    width = target_predict.numel()
    device = target_predict.device
    out = Accepted(
        torch.empty(width, dtype=torch.int32, device=device),
        torch.empty((1, depth), dtype=torch.int32, device=device),
        torch.empty(1, dtype=torch.int32, device=device),
        torch.empty(1, dtype=seq_lens.dtype, device=device),
        torch.empty(1, dtype=torch.int32, device=device),
        torch.empty(depth, dtype=torch.int64, device=device),
        torch.empty(depth, dtype=torch.int64, device=device),
    )
    flat = lambda t: t.reshape(-1)  # noqa: E731  (1-D views of the [1, W] tables)
    args = _native.AcceptTailArgs(
        target_predict=_native.itab(flat(target_predict)),
        candidates=_native.itab(flat(candidates)),
        retrieve_index=_native.itab(flat(retrieve_index)),
        retrieve_next_token=_native.itab(flat(retrieve_next_token)),
        retrieve_next_sibling=_native.itab(flat(retrieve_next_sibling)),
        seq_lens=_native.itab(flat(seq_lens)),
        out_cache_loc=_native.itab(flat(out_cache_loc)),
        req_to_token=_native.itab(req_to_token),
        req_pool_indices=_native.itab(flat(req_pool_indices)),
        predict=out.predict.data_ptr(),
        accept_index=out.accept_index.data_ptr(),
        accept_lens=out.accept_lens.data_ptr(),
        new_seq_lens=out.new_seq_lens.data_ptr(),
        bonus=out.bonus_tokens.data_ptr(),
        committed_slots=out.committed_slots.data_ptr(),
        accepted_slots=out.accepted_slots.data_ptr(),
        width=width,
        depth=depth,
    )
    _native.launch("eagle4_accept_tail", args, device)
    return out


def compact_rows(
    rows: torch.Tensor, accept_index: torch.Tensor, block: int = 2048, out: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """Gathers the accepted rows of ``rows`` [W, cols] (indexed by tree node) to the front: row ``i`` of the result
    is ``rows[accept_index[0, i]]`` for ``i < accept_index.shape[1]`` (an index of -1 reads node 0) and ``rows[i]``
    after that (kernels/accept_tail.py:209-224). The result goes to ``out`` when given (``rows``' shape, unit column
    stride, another buffer), else to a new tensor. ``block`` only keeps the reference's signature."""
    width, cols = rows.shape
    if rows.stride(1) != 1:
        raise ValueError("compact_rows needs rows with a unit column stride")
    if out is None:
        out = torch.empty_like(rows, memory_format=torch.contiguous_format)
    elif out.shape != rows.shape or out.stride(1) != 1 or out.data_ptr() == rows.data_ptr():
        raise ValueError("compact_rows needs an out of the rows' shape, unit column stride, not the rows")
    es = rows.element_size()
    args = _native.CompactRowsArgs(
        src=rows.data_ptr(),
        dst=out.data_ptr(),
        accept_index=_native.itab(accept_index),
        src_stride=rows.stride(0) * es,
        dst_stride=out.stride(0) * es,
        row_bytes=cols * es,
        width=width,
        depth=accept_index.shape[1],
    )
    _native.launch("eagle4_compact_rows", args, rows.device)
    return out


def warm_up(hidden_rows: torch.Tensor, hidden_dtype: torch.dtype) -> None:
    """Launch check before serving (kernels/accept_tail.py:227-249). The reference compiles its two kernels here;
    these are compiled ahead of time, so one launch of each on ``hidden_rows``' device is what is left to do: it
    loads the library there and surfaces a launch failure before the first request. The tree is a lone root (always
    accepted); row 0 of ``hidden_rows`` receives zeros of ``hidden_dtype``, the dtype the served compaction copies."""
    device = hidden_rows.device
    one = lambda value: torch.full((1, 1), value, dtype=torch.int64, device=device)  # noqa: E731
    got = accept_tail(one(0), one(0), one(0), one(-1), one(-1), one(1), one(0),
                      torch.zeros(1, 2, dtype=torch.int32, device=device), one(0), 1)
    compact_rows(torch.zeros(1, hidden_rows.shape[1], dtype=hidden_dtype, device=device), got.accept_index,
                 out=hidden_rows[:1])
