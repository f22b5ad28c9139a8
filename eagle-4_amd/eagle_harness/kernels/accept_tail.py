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
    """What a greedy tree verify of one request accepted (kernels/accept_tail.py:37-46)."""

    predict: torch.Tensor  # int32 [width]: target token of each accepted node, the accepted path moved to the front
    accept_index: torch.Tensor  # int32 [1, depth]: node of each accepted token, -1 padded
    accept_lens: torch.Tensor  # int32 [1]: accepted drafts + the bonus token
    new_seq_lens: torch.Tensor  # [1], seq_lens + accept_lens
    bonus_tokens: torch.Tensor  # int32 [1]: the last accepted token
    committed_slots: torch.Tensor  # int64 [depth]: KV slots the accepted tokens move to (0 past accept_lens)
    accepted_slots: torch.Tensor  # int64 [depth]: KV slots they were written to by the verify (0 past accept_lens)


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
    """A copy of the node-indexed ``rows`` [width, cols] whose first ``accept_index.shape[1]`` rows are the accepted
    path (padding: row 0), the other rows unchanged; into ``out`` (same shape, not ``rows``) if given
    (kernels/accept_tail.py:209-224). ``block`` is accepted for signature compatibility."""
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
    """Runs :func:`accept_tail` and :func:`compact_rows` once before serving (kernels/accept_tail.py:227-249). The
    kernels are compiled ahead of time, so this only exercises the launch path; its first two rows are overwritten."""
    long = dict(dtype=torch.int64, device=hidden_rows.device)
    tokens = torch.zeros(2, **long)
    tables = torch.tensor([[1, -1]], **long)
    accepted = accept_tail(
        tokens,
        tokens,
        torch.arange(2, **long).reshape(1, 2),
        tables,
        tables,
        torch.ones(1, **long),
        tokens,
        torch.zeros(1, 4, dtype=torch.int32, device=hidden_rows.device),
        torch.zeros(1, **long),
        2,
    )
    compact_rows(torch.zeros_like(hidden_rows[:2], dtype=hidden_dtype), accepted.accept_index, out=hidden_rows[:2])
