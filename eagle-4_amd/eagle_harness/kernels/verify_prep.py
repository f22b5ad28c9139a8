"""One launch that writes a tree verify's tail-mask words, batch size 1 (kernels/verify_prep.py).

The tail mask is the part of a tree verify's mask that is not "everything before the tree is visible": one 64-bit
word per query row, bit ``j`` set when the row sees tree key ``j``, read from the verify input's flattened
``[width, kv_len]`` bool mask. The committed length is read on the device, so the launch can sit inside a captured
graph.
"""

from __future__ import annotations

import torch

from eagle_harness.kernels import _native

MAX_TAIL_WIDTH = 64  # one uint64 per row


def tree_tail_words(mask: torch.Tensor, committed_len: torch.Tensor, tail_bits: torch.Tensor, width: int) -> None:
    """Write ``tail_bits[:width]`` (int64) from ``mask`` (flattened ``[width, kv_len]``, bool or uint8) after
    ``committed_len`` (a one-element device tensor) KV slots (kernels/verify_prep.py:36-45)."""
    if not 0 < width <= MAX_TAIL_WIDTH:
        raise ValueError(f"verify width {width} outside 1..{MAX_TAIL_WIDTH}")
    args = _native.TailWordsArgs(
        mask=mask.view(torch.uint8).data_ptr(),
        committed_len=_native.itab(committed_len),
        tail_bits=tail_bits.data_ptr(),
        width=width,
    )
    _native.launch("eagle4_tree_tail_words", args, tail_bits.device)
