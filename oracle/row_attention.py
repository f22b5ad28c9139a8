"""Draft-row attention restated on the CPU (oracle; test infrastructure only).

Follows kernels/row_attention.py: a draft step's rows (``step > 0``) see the committed keys of the window frozen at
the last committed position — positions ``[window_start(seq_len - 1), seq_len - 1]`` (:75-81, :144-146) — plus their
own ``step`` ancestors (KV slots, :171-178); extend rows (``step == 0``, row ``j`` at ``seq_len + j``) see
``[window_start(pos), pos]`` (:126-131). A position ``p`` of request ``b`` is slot
``table[table_rows[b], p // table_page] * table_page + p % table_page`` (:146-153), at ``(slot // cache_page,
slot % cache_page, kv head)`` of the caches (:84-97). Softmax over the visible keys, scores scaled; computed in
float64 (the reference's fp32 sums agree to well inside the kernels' tolerance).
"""

from __future__ import annotations

import torch


def window_start(pos: int, window: int) -> int:
    return max(pos - window + 1, 0) if window > 0 else 0


def visible_slots(table: torch.Tensor, table_row: int, seq_len: int, t: int, step: int, window: int,
                  ancestors: torch.Tensor | None, b: int, table_page: int = 1) -> list[int]:
    """The KV slots row ``t`` of request ``b`` attends to, in key order."""
    if step == 0:
        pos = seq_len + t
        positions = range(window_start(pos, window), pos + 1)
    else:
        positions = range(window_start(seq_len - 1, window), seq_len)
    slots = [int(table[table_row, p // table_page]) * table_page + p % table_page for p in positions]
    if step > 0:
        slots += [int(s) for s in ancestors[b, t, :step]]
    return slots


def _rows(cache: torch.Tensor, slots: list[int], kv_head: int, cache_page: int, lo: int, hi: int) -> torch.Tensor:
    idx = torch.tensor(slots, dtype=torch.int64)
    if cache.dim() == 3:
        return cache[idx, kv_head, lo:hi].double()
    return cache[idx // cache_page, idx % cache_page, kv_head, lo:hi].double()


def rows_attention(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor | None,
    table: torch.Tensor,
    seq_lens: torch.Tensor,
    ancestors: torch.Tensor | None,
    *,
    rows_per_request: int,
    step: int,
    window: int,
    scale: float,
    table_rows: torch.Tensor | None = None,
    table_page: int = 1,
) -> torch.Tensor:
    """``out`` like ``q`` ``[bs * rows_per_request, heads, D]`` (q's dtype); caches as the kernel takes them
    (``values=None``: K then V packed in ``keys``' last dim)."""
    rows, heads, D = q.shape
    kv_heads = keys.shape[-2]
    G = heads // kv_heads
    cache_page = 1 if keys.dim() == 3 else keys.shape[1]
    out = torch.empty(rows, heads, D, dtype=torch.float64)
    for row in range(rows):
        b, t = divmod(row, rows_per_request)
        trow = int(table_rows[b]) if table_rows is not None else b
        slots = visible_slots(table, trow, int(seq_lens[b]), t, step, window, ancestors, b, table_page)
        for h in range(heads):
            kvh = h // G
            k = _rows(keys, slots, kvh, cache_page, 0, D)
            v = _rows(keys, slots, kvh, cache_page, D, 2 * D) if values is None else _rows(values, slots, kvh,
                                                                                              cache_page, 0, D)
            p = torch.softmax((k @ q[row, h].double()) * scale, dim=0)
            out[row, h] = p @ v
    return out.to(q.dtype)
