"""Width-4 tree causal conv1d, restated on the CPU (oracle; test infrastructure only).

Follows ``gdn_tree_conv1d_update`` and its gather kernel (kernels/gdn_tree_conv.py:96-128, 132-279, 402-497): each
node's window is its three nearest ancestors' inputs, or the request's history columns above the root; every
product is rounded to the 16-bit input dtype before the fp32 accumulation (the reference's bf16 x bf16 product),
then SiLU; windows and the state roll are plain copies.
"""

from __future__ import annotations

from typing import Optional

import torch


def _window_value(code: int, x_anc: torch.Tensor, cols: list[torch.Tensor]) -> torch.Tensor:
    """``_window_value`` (kernels/gdn_tree_conv.py:95-98): node ``code`` or history column 2 / 1 / 0."""
    if code >= 0:
        return x_anc
    if code == -1:
        return cols[2]
    if code == -2:
        return cols[1]
    return cols[0]


def gdn_tree_conv1d_update(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    activation,
    conv_state_indices: torch.Tensor,
    intermediate_conv_window: Optional[torch.Tensor],
    intermediate_state_indices: Optional[torch.Tensor],
    tree_ancestors: torch.Tensor,
    pad_slot_id: int = -1,
    out: Optional[torch.Tensor] = None,
    *,
    num_accepted_tokens: Optional[torch.Tensor] = None,
    query_start_loc: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """The reference's signature (kernels/gdn_tree_conv.py:402-417) on CPU tensors; mutates ``conv_state`` and the
    windows like the kernel and returns ``out``."""
    if isinstance(activation, bool):
        activation = "silu" if activation else None
    silu = activation in ("silu", "swish")
    batch, dim, seqlen = x.shape
    width = tree_ancestors.shape[2]
    if query_start_loc is not None:
        batch, seqlen = query_start_loc.shape[0] - 1, width
    if out is None:
        out = torch.empty_like(x)
    dt = x.dtype
    state_len = conv_state.shape[-1]
    anc = tree_ancestors.reshape(-1)  # the kernel addresses the table as contiguous (batch, 3, seqlen)
    for n in range(batch):  # _conv_request, :43-56
        slot = int(conv_state_indices[n])
        bos, num_tokens, history = 0, seqlen, 0
        if query_start_loc is not None:
            bos = int(query_start_loc[n])
            num_tokens = int(query_start_loc[n + 1]) - bos
        if num_accepted_tokens is not None:
            history = int(num_accepted_tokens[n]) - 1
        if not (slot > pad_slot_id and num_tokens > 0):
            continue
        xs = 0 if query_start_loc is not None else n
        cols = [conv_state[slot, :, history + j].clone() for j in range(3)]  # :70-76
        w = weight
        b32 = bias.float() if bias is not None else torch.zeros(dim)
        xrow = lambda t: x[xs, :, bos + t]  # noqa: E731
        for t in range(num_tokens):
            codes = [int(anc[n * 3 * seqlen + i * seqlen + t]) for i in range(3)]
            vals = [_window_value(c, xrow(c) if c >= 0 else None, cols) for c in codes]
            acc = b32.clone()
            # the upstream products and order (:225-229), each product rounded to the 16-bit dtype
            acc = acc + (xrow(t).float() * w[:, 3].float()).to(dt).float()
            acc = acc + (vals[0].float() * w[:, 2].float()).to(dt).float()
            acc = acc + (vals[1].float() * w[:, 1].float()).to(dt).float()
            acc = acc + (vals[2].float() * w[:, 0].float()).to(dt).float()
            if silu:
                acc = acc / (1 + torch.exp(-acc))
            out[xs, :, bos + t] = acc.to(out.dtype)
            if intermediate_conv_window is not None:  # :241-264: slot 0 grandparent, 1 parent, 2 self
                coord = int(intermediate_state_indices[n])
                wd = intermediate_conv_window.dtype
                intermediate_conv_window[coord, t, :, 0] = vals[1].to(wd)
                intermediate_conv_window[coord, t, :, 1] = vals[0].to(wd)
                intermediate_conv_window[coord, t, :, 2] = xrow(t).to(wd)
        # the roll (:266-278): entry e of (col0, col1, col2, x_0, ..) goes to column e + shift when >= 0
        shift = min(num_tokens + 2, state_len) - num_tokens - 3
        entries = cols + [xrow(t).clone() for t in range(num_tokens)]
        for e, val in enumerate(entries):
            if e + shift >= 0:
                conv_state[slot, :, e + shift] = val.to(conv_state.dtype)
    return out


def dense_conv_reference(x_nodes, history, weight, bias, parents):
    """The reference test's independent dense form (tests/test_gdn_tree_conv.py:38-48): node outputs
    [nodes, dim] fp32 and windows [nodes, dim, 3] (grandparent, parent, self)."""
    from oracle.tables import window_codes

    outs, windows = [], []
    for node, codes in enumerate(window_codes(parents)):
        vals = [x_nodes[c] if c >= 0 else history[:, 3 + c] for c in codes]
        y = bias.float() + (x_nodes[node] * weight[:, 3]).float()
        for v, w in zip(vals, (weight[:, 2], weight[:, 1], weight[:, 0])):
            y = y + (v * w).float()
        outs.append(y * torch.sigmoid(y))
        windows.append(torch.stack([vals[1], vals[0], x_nodes[node]], dim=-1))
    return torch.stack(outs), torch.stack(windows)
