"""Mamba2 tree verify (kernels/mamba2_tree.py): the selective state update of every tree node, each continuing from
its parent, on the gfx950 kernel of ``csrc/mamba2_tree.hip``.

The verify rows of a request are its draft-tree nodes, each after its parent. A node takes the SSM state its parent
left (the root takes the request's own state), applies its token, and stores the new state in the node's own slot:
one slot per verify row, as vLLM lays out a chain verify. When the parent is the row just before, the state is
still in registers; otherwise it is read back from the parent's slot. A chain therefore reproduces vLLM's chain
update exactly.
"""

from __future__ import annotations

from typing import Optional

import torch

from eagle_harness.kernels import _native
from eagle_harness.kernels.gdn_tree import PAD_SLOT_ID


def mamba2_tree_state_update(
    state: torch.Tensor,
    x: torch.Tensor,
    dt: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor],
    dt_bias: Optional[torch.Tensor],
    out: torch.Tensor,
    *,
    state_indices: torch.Tensor,
    parents: torch.Tensor,
    query_start_loc: torch.Tensor,
    num_accepted_tokens: Optional[torch.Tensor] = None,
    dt_softplus: bool = True,
    pad_slot_id: int = PAD_SLOT_ID,
) -> torch.Tensor:
    """Mamba2's selective state update of a tree verify, in place (kernels/mamba2_tree.py:177-240).

    ``state`` (slots, heads, head_dim, dstate) with a contiguous last dim; ``x`` and ``out`` (tokens, heads, head_dim)
    and ``dt`` (tokens, heads), any token and head strides with contiguous head dims; ``B`` / ``C`` (tokens, groups,
    dstate), contiguous last dim; ``A`` (float32, ``-exp(A_log)``), ``D`` and ``dt_bias`` (heads,). Request ``b``'s rows
    are tokens ``query_start_loc[b]:query_start_loc[b + 1]``; row ``t`` continues from row ``parents[b, t]`` (``-1``
    for row 0: the state at ``state_indices[b, num_accepted_tokens[b] - 1]``, or column 0 without accepted counts) and
    stores its state at ``state_indices[b, t]``; a slot equal to ``pad_slot_id`` is neither read (zeros) nor written.
    ``out[t] = C_t . state_t + D * x_t`` with ``state_t = exp(A dt_t) state_parent + dt_t B_t x_t`` and
    ``dt_t = softplus(dt + dt_bias)`` (``dt_softplus``). dstate 64 / 128 / 256 on the gfx950 kernel (``NotCovered``
    otherwise).
    """
    tokens, heads, head_dim = x.shape
    groups, dstate = B.shape[1], B.shape[2]
    batch = query_start_loc.shape[0] - 1
    assert state.shape[1:] == (heads, head_dim, dstate) and state.stride(-1) == 1
    assert dt.shape == (tokens, heads) and out.shape == x.shape and C.shape == B.shape == (tokens, groups, dstate)
    assert x.stride(-1) == 1 and out.stride(-1) == 1 and B.stride(-1) == 1 and C.stride(-1) == 1
    assert A.shape == (heads,) and A.dtype == torch.float32 and heads % groups == 0
    assert state_indices.shape[0] >= batch and parents.shape[0] >= batch
    assert parents.stride(-1) == 1 and state_indices.stride(-1) == 1
    if B.dtype != x.dtype or C.dtype != x.dtype:
        raise _native.NotCovered("B and C must have x's dtype")
    if D is not None and dt_bias is not None and D.dtype != dt_bias.dtype:
        raise _native.NotCovered("D and dt_bias must share a dtype")
    param = D if D is not None else dt_bias
    A_c = A.contiguous()  # the parameter vectors, kept alive until the launch
    D_c = D.contiguous() if D is not None else None
    bias_c = dt_bias.contiguous() if dt_bias is not None else None
    args = _native.Mamba2Args(
        state=state.data_ptr(),
        stride_state_slot=state.stride(0),
        stride_state_head=state.stride(1),
        stride_state_dim=state.stride(2),
        x=x.data_ptr(),
        stride_x_tok=x.stride(0),
        stride_x_head=x.stride(1),
        dt=dt.data_ptr(),
        stride_dt_tok=dt.stride(0),
        stride_dt_head=dt.stride(1),
        B=B.data_ptr(),
        stride_B_tok=B.stride(0),
        stride_B_group=B.stride(1),
        C=C.data_ptr(),
        stride_C_tok=C.stride(0),
        stride_C_group=C.stride(1),
        A=A_c.data_ptr(),
        D=_native.ptr(D_c),
        dt_bias=_native.ptr(bias_c),
        out=out.data_ptr(),
        stride_out_tok=out.stride(0),
        stride_out_head=out.stride(1),
        slots=_native.itab(state_indices),
        parents=_native.itab(parents),
        num_accepted=_native.itab(num_accepted_tokens),
        query_start_loc=_native.itab(query_start_loc),
        batch=batch,
        heads=heads,
        head_dim=head_dim,
        dstate=dstate,
        groups=groups,
        state_dtype=_native.dtype_code(state.dtype),
        in_dtype=_native.dtype_code(x.dtype),
        dt_dtype=_native.dtype_code(dt.dtype),
        param_dtype=_native.dtype_code(param.dtype) if param is not None else 0,
        out_dtype=_native.dtype_code(out.dtype),
        dt_softplus=int(bool(dt_softplus)),
        pad_slot_id=pad_slot_id,
    )
    _native.launch("eagle4_mamba2_tree_state_update", args, x.device)
    return out
