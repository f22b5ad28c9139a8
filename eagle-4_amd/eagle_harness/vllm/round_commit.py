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
        # The backend's cache is (blocks, heads, slots in a block, 2 * head_dim), a token's K and V adjacent; the
        # kernel walks (block, slot, head), so validate on that order. The checks and messages are the reference's
        # (vllm/round_commit.py:93-116), which callers may rely on.
        views = [cache.transpose(1, 2) for cache in kv_caches]
        ref = views[0]
        for cache, v in zip(kv_caches, views):
            if v.stride() != ref.stride() or cache.dtype != kv_caches[0].dtype:
                raise ValueError("the target's full-attention layers must share one KV cache layout")
        if ref.stride(3) != 1:
            raise ValueError("KV cache rows must be contiguous")
        for table in block_tables:
            if table.dtype != torch.int32:
                raise ValueError("block tables must be int32")
        stride_block, stride_slot, stride_head = ref.stride(0), ref.stride(1), ref.stride(2)
        self.strides = (stride_block, stride_head, stride_slot)
        self.block_size, self.num_heads, self.dim = ref.shape[1], ref.shape[2], ref.shape[3]
        self.dtype = kv_caches[0].dtype
        self.device = device

        def on_device(values, dtype):
            return torch.tensor(list(values), dtype=dtype, device=device)

        self.layer_ptrs = on_device((c.data_ptr() for c in kv_caches), torch.uint64)
        self.table_ptrs = on_device((t.data_ptr() for t in block_tables), torch.uint64)
        self.table_strides = on_device((t.stride(0) for t in block_tables), torch.int64)
        self.table_block_sizes = on_device(table_block_sizes, torch.int32)
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
