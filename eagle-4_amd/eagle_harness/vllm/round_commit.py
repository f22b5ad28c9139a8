"""What a tree round leaves behind, turned back into what vLLM expects after a chain round (vllm/round_commit.py).

After the tree walk the accepted rows are not a prefix of the verify rows. :class:`KvCompactor` copies the KV of the
accepted rows of the target's full-attention layers to the chain slots ``context + j`` (all layers in one gfx950
launch, ``csrc/round_commit.hip``), and :func:`chainize` rewrites the round's ``input_ids`` / ``positions`` for the
draft's prefill and says which row's hidden state each draft input takes. Rows of requests that are not a verified
tree (one row, or one logit per request) are left alone.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from eagle_harness.kernels import _native


class KvCompactor:
    """Moves the KV of the accepted rows of a tree round to the chain slots, in every given layer
    (vllm/round_commit.py:86-143).

    ``kv_caches[i]``: layer ``i``'s cache as the attention backend views it, (blocks, heads, slots in a block,
    2 * head_dim) with K then V of a token and head adjacent; ``block_tables[i]`` and ``table_block_sizes[i]``: that
    layer's KV cache group's persistent [num_reqs, max_blocks] int32 block table (the batch's rows, as the forward got
    them) and its tokens per block.
    """

    def __init__(
        self,
        kv_caches: Sequence[torch.Tensor],
        block_tables: Sequence[torch.Tensor],
        table_block_sizes: Sequence[int],
        device: torch.device,
    ):
        first = kv_caches[0]
        view = first.transpose(1, 2)  # (blocks, slots in a block, heads, 2 * head_dim)
        if any(c.transpose(1, 2).stride() != view.stride() or c.dtype != first.dtype for c in kv_caches):
            raise ValueError("the target's full-attention layers must share one KV cache layout")
        if view.stride(3) != 1:
            raise ValueError("KV cache rows must be contiguous")
        self.strides = (view.stride(0), view.stride(2), view.stride(1))  # block, head, slot
        self.num_heads, self.dim, self.dtype = view.shape[2], view.shape[3], first.dtype
        self.block_size = view.shape[1]
        self.device = device
        self.layer_ptrs = torch.tensor([c.data_ptr() for c in kv_caches], dtype=torch.uint64, device=device)
        self.table_ptrs = torch.tensor([t.data_ptr() for t in block_tables], dtype=torch.uint64, device=device)
        self.table_strides = torch.tensor([t.stride(0) for t in block_tables], dtype=torch.int64, device=device)
        self.table_block_sizes = torch.tensor(list(table_block_sizes), dtype=torch.int32, device=device)
        if any(t.dtype != torch.int32 for t in block_tables):
            raise ValueError("block tables must be int32")
        self._keep = (list(kv_caches), list(block_tables))

    def compact(
        self,
        idx_mapping: torch.Tensor,
        query_start_loc: torch.Tensor,
        cu_num_logits: torch.Tensor,
        seq_lens: torch.Tensor,
        path: torch.Tensor,
        path_len: torch.Tensor,
    ) -> None:
        """``path [state slots, W]`` / ``path_len [state slots]``: the accepted rows of each request, root first;
        ``seq_lens`` counts the round's rows (context = seq_len - query width)."""
        args = _native.CompactKvArgs(
            layer_ptrs=self.layer_ptrs.data_ptr(),
            table_ptrs=self.table_ptrs.data_ptr(),
            table_strides=self.table_strides.data_ptr(),
            table_block_sizes=self.table_block_sizes.data_ptr(),
            idx_mapping=_native.itab(idx_mapping),
            query_start_loc=_native.itab(query_start_loc),
            cu_num_logits=_native.itab(cu_num_logits),
            seq_lens=_native.itab(seq_lens),
            path=_native.itab(path),
            path_len=_native.itab(path_len),
            stride_block=self.strides[0],
            stride_head=self.strides[1],
            stride_slot=self.strides[2],
            block_size=self.block_size,
            dim=self.dim,
            dtype=_native.dtype_code(self.dtype),
            num_reqs=idx_mapping.shape[0],
            layers=self.layer_ptrs.shape[0],
            heads=self.num_heads,
        )
        _native.launch("eagle4_compact_kv", args, self.device)


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
    """Rewrite the round's ``input_ids`` / ``positions`` in place for the draft's prefill and fill ``src_rows``
    (preset to the identity): row ``i`` of the draft's input takes the hidden state of target row ``src_rows[i]``.
    Only the rows of a verified tree change (vllm/round_commit.py:182-215)."""
    for name, t in (("input_ids", input_ids), ("positions", positions), ("src_rows", src_rows)):
        if t.dtype not in (torch.int32, torch.int64) or t.stride(0) != 1:
            raise _native.NotCovered(f"{name} must be a contiguous int32 / int64 vector")
    if sampled.stride(-1) != 1:
        raise _native.NotCovered("sampled rows must be contiguous")
    rows = 1 << max(int(width) - 1, 0).bit_length()  # the power of two >= width, as the reference's arange
    if rows > 64:
        raise _native.NotCovered("tree widths above 64 rows")
    args = _native.ChainizeArgs(
        idx_mapping=_native.itab(idx_mapping),
        query_start_loc=_native.itab(query_start_loc),
        cu_num_logits=_native.itab(cu_num_logits),
        seq_lens=_native.itab(seq_lens),
        path=_native.itab(path),
        path_len=_native.itab(path_len),
        sampled=_native.itab(sampled),
        input_ids=input_ids.data_ptr(),
        positions=positions.data_ptr(),
        src_rows=src_rows.data_ptr(),
        input_ids_dtype=_native.dtype_code(input_ids.dtype),
        positions_dtype=_native.dtype_code(positions.dtype),
        src_rows_dtype=_native.dtype_code(src_rows.dtype),
        rows=rows,
        num_reqs=idx_mapping.shape[0],
    )
    _native.launch("eagle4_chainize", args, input_ids.device)
