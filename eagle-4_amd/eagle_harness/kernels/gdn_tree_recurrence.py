"""Gated delta rule recurrence over a draft tree: the SSM half of a GDN layer's tree verify
(kernels/gdn_tree_recurrence.py).

The math (per node, continuing from its parent's state; row 0 from the request's initial state)::

    g    = -exp(A_log) * softplus(a + dt_bias)      # log decay, per value head
    beta = sigmoid(b)                               # write strength, rounded to b's dtype
    q, k = q / |q|, k / |k|;  q *= scale             # L2 norms over K (1e-6 inside the square root)
    h    = h * exp(g);  v' = (v - h^T k) * beta;  h = h + k v'^T;  o = h^T q

Every node's output and state (its snapshot) are written; the request's own state is never written back. States and
snapshots are ``[..., HV, V, K]`` per slot, addressed through the reference's two slot-table layouts (sglang: a
``[slots, steps, HV, V, K]`` scratch with one row per request; vLLM: the ``[slots, HV, V, K]`` pool with one slot per
verify row, resuming at ``num_accepted - 1``). A slot ``<= pad_slot_id`` is padding: never written, read as zero.

The gfx950 kernel (``csrc/gdn_tree_recurrence.hip``) walks each (request, value head) in one workgroup with the
state in registers and writes every snapshot as full 128-byte lines; the reference's path replay (``tree_paths``
with an fp32 state) computes the same fold, so both selections run that walk.
"""

from __future__ import annotations

from typing import Optional

import torch

from eagle_harness.kernels import _native
from eagle_harness.kernels.gdn_tree import PAD_SLOT_ID


def gdn_tree_state_args(
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    num_accepted_tokens: Optional[torch.Tensor],
    intermediate_states_buffer: torch.Tensor,
    intermediate_state_indices: torch.Tensor,
    publish: Optional[torch.Tensor],
) -> dict:
    """Checks how a walk launch addresses its states and returns the addressing values keyed by the reference walk's
    argument names (kernels/gdn_tree_recurrence.py:517-559; the keys and the assertion messages are the interface
    the reference's callers read).

    A per-row slot table ([N, S] into a [slots, HV, V, K] pool, vLLM) or a per-request table ([N] into a
    [slots, steps, HV, V, K] scratch, sglang) selects the layout; ``num_accepted_tokens`` comes with, and only with,
    a 2-D initial-state table; ``publish`` needs per-row slots. Entries the chosen layout does not read hold a
    stride of 0, or a tensor that is safe to pass, and the flags say so."""
    per_row = intermediate_state_indices.dim() == 2
    if per_row:
        assert intermediate_states_buffer.dim() == 4, "one slot per row addresses a [slots, HV, V, K] buffer"
    else:
        assert intermediate_states_buffer.dim() == 5, "one slot per request addresses a [slots, steps, HV, V, K] buffer"
    h0_per_column = initial_state_indices.dim() == 2
    assert h0_per_column == (num_accepted_tokens is not None)
    assert publish is None or per_row, "publish copies a table of per-row slots"

    def inner_stride(t: torch.Tensor) -> int:  # column stride of a 2-D table; 0 for a 1-D one
        return t.stride(1) if t.dim() == 2 else 0

    found = {
        "stride_h0_source": initial_state_source.stride(0),
        "stride_h0_indices_seq": initial_state_indices.stride(0),
        "stride_h0_indices_col": inner_stride(initial_state_indices),
        "num_accepted": num_accepted_tokens if h0_per_column else initial_state_indices,
        "stride_snap_indices_seq": intermediate_state_indices.stride(0),
        "stride_snap_indices_row": inner_stride(intermediate_state_indices),
        "stride_snap_slot": intermediate_states_buffer.stride(0),
        "stride_snap_row": 0 if per_row else intermediate_states_buffer.stride(1),
        "publish": publish if publish is not None else intermediate_state_indices,
        "stride_publish": publish.stride(0) if publish is not None else 0,
        "num_slot_cols": intermediate_state_indices.shape[-1],
    }
    found.update(ROW_SLOTS=per_row, HAS_NUM_ACCEPTED=h0_per_column, PUBLISH=publish is not None)
    return found


def _check_state_layout(t: torch.Tensor, lead: int, HV: int, V: int, K: int, name: str) -> None:
    inner = t.shape[lead:]
    if tuple(inner) != (HV, V, K) or t.stride(-1) != 1 or t.stride(-2) != K or t.stride(-3) != V * K:
        raise _native.NotCovered(f"{name}: each slot must be a contiguous [HV, V, K] = [{HV}, {V}, {K}] state")
    align = 16 if t.dtype == torch.float32 else 8
    if t.data_ptr() % align or any(s % 4 for s in t.stride()[:lead]):
        raise _native.NotCovered(f"{name}: slots must start on {align}-byte boundaries")


def gdn_tree_recurrent_update(
    A_log: torch.Tensor,
    dt_bias: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    intermediate_states_buffer: torch.Tensor,
    intermediate_state_indices: torch.Tensor,
    retrieve_parent_token: torch.Tensor,
    num_accepted_tokens: Optional[torch.Tensor] = None,
    pad_slot_id: int = PAD_SLOT_ID,
    out: Optional[torch.Tensor] = None,
    publish: Optional[torch.Tensor] = None,
    tree_paths: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    softplus_beta: float = 1.0,
    softplus_threshold: float = 20.0,
    gluon: bool = False,
) -> torch.Tensor:
    """Runs the gated delta rule over every node of a verify tree and stores each node's state as a snapshot
    (kernels/gdn_tree_recurrence.py:562-706; same arguments, defaults and assertions).

    Args:
        A_log, dt_bias: [HV] gate parameters of the layer.
        q, k: (1, tokens, H, K); v: (1, tokens, HV, V); token-strided, contiguous over (heads, dim).
        a, b: (tokens, HV) gate inputs; ``beta`` is rounded to ``b``'s dtype.
        initial_state_source: the state pool, [slots, HV, V, K].
        initial_state_indices: [N] pool slot of each request's state, or with ``num_accepted_tokens`` [N, C], where
            the state is at column ``num_accepted_tokens[n] - 1``.
        cu_seqlens: [N + 1] row offsets of the requests; rows are in node order, parents first.
        intermediate_states_buffer: [slots, steps, HV, V, K] (sglang scratch) or [slots, HV, V, K] (vLLM; may be
            ``initial_state_source`` itself).
        intermediate_state_indices: [N] scratch row per request (5-D buffer) or [N, S] slot per row (4-D).
        retrieve_parent_token: [N, >= rows] parent row of each row, within the request; entry 0 is ignored.
        num_accepted_tokens: [N], see ``initial_state_indices``.
        pad_slot_id: slots ``<= pad_slot_id`` are padding (sglang -1, vLLM 0).
        out: optional (1, tokens, HV, V) output, token-strided, contiguous over (HV, V).
        publish: optional [N, >= S] int32; receives the [N, S] slot table (per-row slots only).
        tree_paths: optional path table; with an fp32 pool and scratch the reference selects its path replay, which
            computes the same fold as the walk run here.
        scale: q scale, default ``K ** -0.5``.
        softplus_beta, softplus_threshold: the gate's softplus.
        gluon: accepted for signature compatibility (the Gluon twin is NVIDIA-only); ignored.

    Returns:
        ``out`` when given, otherwise a tensor shaped like ``v`` with ``q``'s dtype and device.
    """
    _, _, H, K = k.shape
    V = v.shape[-1]
    HV = v.shape[2]
    N = cu_seqlens.shape[0] - 1
    assert K & (K - 1) == 0 and K > 0, "K must be a power of two"
    if scale is None:
        scale = K**-0.5
    fp32_state = intermediate_states_buffer.dtype == torch.float32 and initial_state_source.dtype == torch.float32
    if out is None:
        out = q.new_empty(v.shape)
    assert out.shape == v.shape and out.stride(3) == 1 and out.stride(2) == V
    if tree_paths is not None and fp32_state:
        assert tree_paths.shape[0] >= N and tree_paths.dtype == torch.int32
        assert initial_state_indices.ndim == 1 and intermediate_state_indices.ndim == 1 and publish is None
        assert pad_slot_id == PAD_SLOT_ID, "the path replay takes sglang's per-request tables"
    state = gdn_tree_state_args(
        initial_state_source,
        initial_state_indices,
        num_accepted_tokens,
        intermediate_states_buffer,
        intermediate_state_indices,
        publish,
    )
    # layouts the kernel addresses: unit inner strides, heads contiguous, 8 / 16-byte vector loads
    for name, t, d in (("q", q, K), ("k", k, K), ("v", v, V)):
        if t.stride(3) != 1 or t.stride(2) != d or t.stride(1) % 4 or t.data_ptr() % (4 * t.element_size()):
            raise _native.NotCovered(f"{name} must be token-strided and contiguous over (heads, dim)")
    if not (q.dtype == k.dtype == v.dtype) or a.dtype != b.dtype or a.stride(-1) != 1 or b.stride(-1) != 1:
        raise _native.NotCovered("q, k, v must share a dtype, as must a and b (unit stride over heads)")
    if publish is not None and publish.dtype != torch.int32:
        raise _native.NotCovered("publish must be int32")
    _check_state_layout(initial_state_source, 1, HV, V, K, "initial_state_source")
    _check_state_layout(intermediate_states_buffer, state["ROW_SLOTS"] and 1 or 2, HV, V, K, "intermediate_states_buffer")
    args = _native.GdnArgs(
        q=q.data_ptr(),
        k=k.data_ptr(),
        v=v.data_ptr(),
        stride_q=q.stride(1),
        stride_k=k.stride(1),
        stride_v=v.stride(1),
        in_dtype=_native.dtype_code(q.dtype),
        gate_dtype=_native.dtype_code(b.dtype),
        a=a.data_ptr(),
        b=b.data_ptr(),
        stride_a=a.stride(-2),
        stride_b=b.stride(-2),
        A_log=A_log.data_ptr(),
        dt_bias=dt_bias.data_ptr(),
        A_log_dtype=_native.dtype_code(A_log.dtype),
        dt_bias_dtype=_native.dtype_code(dt_bias.dtype),
        softplus_beta=softplus_beta,
        softplus_threshold=softplus_threshold,
        scale=scale,
        out_dtype=_native.dtype_code(out.dtype),
        out=out.data_ptr(),
        stride_o=out.stride(1),
        parents=_native.itab(retrieve_parent_token),
        cu_seqlens=_native.itab(cu_seqlens),
        h0_source=initial_state_source.data_ptr(),
        stride_h0_source=state["stride_h0_source"],
        h0_dtype=_native.dtype_code(initial_state_source.dtype),
        snap_dtype=_native.dtype_code(intermediate_states_buffer.dtype),
        h0_indices=_native.itab(initial_state_indices),
        num_accepted=_native.itab(num_accepted_tokens),
        snap=intermediate_states_buffer.data_ptr(),
        stride_snap_slot=state["stride_snap_slot"],
        stride_snap_row=state["stride_snap_row"],
        snap_indices=_native.itab(intermediate_state_indices),
        publish=_native.ptr(publish),
        stride_publish=state["stride_publish"],
        num_slot_cols=state["num_slot_cols"],
        N=N,
        H=H,
        HV=HV,
        K=K,
        V=V,
        row_slots=int(state["ROW_SLOTS"]),
        skip_chain_reload=int(fp32_state),
        pad_slot_id=pad_slot_id,
    )
    _native.launch("eagle4_gdn_tree_recurrent_update", args, q.device)
    return out
