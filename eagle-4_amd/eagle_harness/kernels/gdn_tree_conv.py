"""GDN tree verify: the width-4 causal conv1d of every tree node through the ancestor table
(kernels/gdn_tree_conv.py).

A node's conv taps are the inputs of the node and of its parent, grandparent and great-grandparent; above the root
they come from the request's history columns. The table of those three ancestors per node is built once per
forward (:func:`~eagle_harness.kernels.gdn_tree.gdn_tree_ancestors`). Every product
is rounded to the 16-bit input dtype before the fp32 accumulation, then SiLU, as the reference's kernels compute it;
windows and the state roll are copies. One gfx950 kernel serves both engines' layouts (``csrc/gdn_tree_conv.hip``):
a thread owns 8 adjacent channels of a request and streams its nodes with 16-byte loads and stores.
"""

from __future__ import annotations

from typing import Optional, Union

import torch

from eagle_harness.kernels import _native
from eagle_harness.kernels.gdn_tree import PAD_SLOT_ID

# The reference picks between a gather and a serial kernel with these thresholds (kernels/gdn_tree_conv.py:397-399);
# the gfx950 kernel has one form for both, and the names stay for callers that read them.
CONV_SERIAL_MIN_BATCH_DIM = 81920
CONV_SERIAL_MAX_WIDTH = 16


def gdn_tree_conv1d_update(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    activation: Union[bool, str, None],
    conv_state_indices: torch.Tensor,
    intermediate_conv_window: Optional[torch.Tensor],
    intermediate_state_indices: Optional[torch.Tensor],
    tree_ancestors: torch.Tensor,
    pad_slot_id: int = PAD_SLOT_ID,
    out: Optional[torch.Tensor] = None,
    *,
    num_accepted_tokens: Optional[torch.Tensor] = None,
    query_start_loc: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``causal_conv1d_update`` of a tree verify (width-4 kernel) whose ancestor table came from
    ``gdn_tree_ancestors`` (kernels/gdn_tree_conv.py:402-497). x: (batch, dim, seqlen) with any strides; weight:
    (dim, 4). out (same shape, any strides) defaults to ``torch.empty_like(x)``.

    Request n's history is the 3 columns of ``conv_state[conv_state_indices[n]]`` from column 0, or from column
    ``num_accepted_tokens[n] - 1``; a row whose index is <= ``pad_slot_id`` is padding. With ``query_start_loc`` x is
    (1, dim, tokens) and request n's nodes are tokens ``query_start_loc[n]:query_start_loc[n + 1]``. Each node's
    window goes to ``intermediate_conv_window[intermediate_state_indices[n], node]`` if given; the state row keeps
    the newest ``min(conv_state.shape[-1], nodes + 2)`` entries of (history ++ inputs). 16-bit inputs only.
    """
    if isinstance(activation, bool):
        activation = "silu" if activation is True else None
    batch, dim, seqlen = x.shape
    width = tree_ancestors.shape[2]
    if query_start_loc is not None:
        assert batch == 1
        batch, seqlen = query_start_loc.shape[0] - 1, width
    assert x.element_size() == 2 and weight.element_size() == 2 and conv_state.element_size() == 2
    assert weight.shape[1] == 4 and tree_ancestors.shape[0] >= batch and tree_ancestors.shape[1:] == (3, seqlen)
    assert tree_ancestors.is_contiguous() and conv_state.shape[-1] >= 3
    has_windows = intermediate_conv_window is not None
    if out is None:
        out = torch.empty_like(x)
    assert out.shape == x.shape and out.dtype == x.dtype
    if not (x.dtype == weight.dtype == conv_state.dtype and (not has_windows or intermediate_conv_window.dtype == x.dtype)):
        raise _native.NotCovered("the gfx950 tree conv takes x, weight, conv state and windows of one 16-bit dtype")
    if tree_ancestors.dtype != torch.int32:
        raise _native.NotCovered("tree_ancestors must be int32")
    qsl = query_start_loc is not None
    args = _native.ConvArgs(
        x=x.data_ptr(),
        stride_x_seq=0 if qsl else x.stride(0),
        stride_x_dim=x.stride(1),
        stride_x_token=x.stride(2),
        weight=weight.data_ptr(),
        stride_w_dim=weight.stride(0),
        stride_w_width=weight.stride(1),
        bias=_native.ptr(bias),
        conv_state=conv_state.data_ptr(),
        stride_cs_seq=conv_state.stride(0),
        stride_cs_dim=conv_state.stride(1),
        stride_cs_tok=conv_state.stride(2),
        conv_state_indices=_native.itab(conv_state_indices),
        num_accepted=_native.itab(num_accepted_tokens),
        query_start_loc=_native.itab(query_start_loc),
        window=_native.ptr(intermediate_conv_window),
        stride_win_seq=intermediate_conv_window.stride(0) if has_windows else 0,
        stride_win_step=intermediate_conv_window.stride(1) if has_windows else 0,
        stride_win_dim=intermediate_conv_window.stride(2) if has_windows else 0,
        stride_win_win=intermediate_conv_window.stride(3) if has_windows else 0,
        window_indices=_native.itab(intermediate_state_indices if has_windows else None),
        ancestors=tree_ancestors.data_ptr(),
        out=out.data_ptr(),
        stride_o_seq=0 if qsl else out.stride(0),
        stride_o_dim=out.stride(1),
        stride_o_token=out.stride(2),
        batch=batch,
        dim=dim,
        seqlen=seqlen,
        state_len=conv_state.shape[-1],
        pad_slot_id=pad_slot_id,
        silu=1 if activation in ("silu", "swish") else 0,
        dtype=_native.dtype_code(x.dtype),
        bias_dtype=_native.dtype_code(bias.dtype) if bias is not None else _native.F32,
    )
    _native.launch("eagle4_gdn_tree_conv1d_update", args, x.device)
    return out
