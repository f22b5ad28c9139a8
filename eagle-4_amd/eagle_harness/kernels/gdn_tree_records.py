"""GDN tree verify, records contract (kernels/gdn_tree_records.py): replay records instead of per-node snapshots.

The verify writes, per node and value head, a record ``(delta [V], key [K], decay)`` (``records[row, node, hv, :V]``
the node's v' = (v - h k^) beta, ``[V:V+K]`` its normalised key, ``[V+K]`` exp(g)); the commit folds the accepted
node's root path of records into the pool. The chunk form (no rounding) of trees with at most 16 nodes and bf16
inputs runs in closed form on the matrix cores (``csrc/gdn_tree_chunk.hip``: one wave per (request, value head,
column slice) solves the whole tree). The path replay (``tree_paths`` given; every parent state rounded to the pool
dtype, as the reference's replay does) and wider trees run the depth-first walk (``csrc/gdn_tree_records.hip``: one
wave walks each (request, value head, V tile) instead of replaying every leaf path); the results are the same folds.
"""

from __future__ import annotations

from typing import Optional

import torch

from eagle_harness.kernels import _native


def _records_layout(records: torch.Tensor, HV: int, V: int, K: int) -> None:
    if records.dtype != torch.float32 or records.ndim < 4:
        raise _native.NotCovered("records must be fp32 [..., rows, steps, HV, REC]")
    rec = records.shape[-1]
    if (records.shape[-2] != HV or records.stride(-1) != 1 or records.stride(-2) != rec
            or records.stride(-3) != HV * rec or rec < V + K + 1):
        raise _native.NotCovered("each record row must be a contiguous [steps, HV, REC >= V + K + 1] block")


def _update(A_log, dt_bias, q, k, v, a, b, state, state_indices, query_start_loc, parent, tree_paths, records,
            record_indices, width, path_replay: bool) -> torch.Tensor:
    _, tokens, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    N = query_start_loc.numel() - 1
    out = torch.empty_like(v)
    if N == 0 or tokens == 0:
        return out
    if width > 64:
        raise ValueError(f"tree width {width} > 64")
    for name, t, d in (("q", q, K), ("k", k, K), ("v", v, V)):
        if t.stride(3) != 1 or t.stride(2) != d or t.stride(1) % 4 or t.data_ptr() % (4 * t.element_size()):
            raise _native.NotCovered(f"{name} must be token-strided and contiguous over (heads, dim)")
    if not (q.dtype == k.dtype == v.dtype) or a.dtype != b.dtype or a.stride(-1) != 1 or b.stride(-1) != 1:
        raise _native.NotCovered("q, k, v must share a dtype, as must a and b (unit stride over heads)")
    if state.shape[1:] != (HV, V, K) or state.stride(-1) != 1 or state.stride(-2) != K or state.stride(-3) != V * K:
        raise _native.NotCovered(f"state must be a pool of contiguous [HV, V, K] = [{HV}, {V}, {K}] slots")
    _records_layout(records, HV, V, K)
    if records.shape[-3] < width:
        raise _native.NotCovered(f"records hold {records.shape[-3]} steps, fewer than the width {width}")
    if path_replay:
        if (tree_paths.dtype != torch.int32 or tree_paths.ndim != 3 or tree_paths.stride(-1) != 1
                or tree_paths.shape[0] < N or tree_paths.shape[-1] < 2 + width):
            raise _native.NotCovered("tree_paths must be int32 [batch, paths, 2 + width] with contiguous entries")
    elif parent.shape[0] < N or parent.shape[1] < width:
        raise _native.NotCovered("parent must hold [batch, width] entries")
    args = _native.RecordsArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
        stride_q=q.stride(1), stride_k=k.stride(1), stride_v=v.stride(1),
        in_dtype=_native.dtype_code(q.dtype), gate_dtype=_native.dtype_code(b.dtype),
        a=a.data_ptr(), b=b.data_ptr(), stride_a=a.stride(-2), stride_b=b.stride(-2),
        A_log=A_log.data_ptr(), dt_bias=dt_bias.data_ptr(),
        A_log_dtype=_native.dtype_code(A_log.dtype), dt_bias_dtype=_native.dtype_code(dt_bias.dtype),
        scale=K**-0.5, out_dtype=_native.dtype_code(out.dtype), out=out.data_ptr(), stride_o=out.stride(1),
        state=state.data_ptr(), stride_state=state.stride(0), state_dtype=_native.dtype_code(state.dtype),
        path_replay=int(path_replay), state_indices=_native.itab(state_indices),
        query_start_loc=_native.itab(query_start_loc), parent=_native.itab(parent),
        tree_paths=_native.itab(tree_paths) if path_replay else _native.itab(None),
        records=records.data_ptr(), stride_records_row=records.stride(-4),
        record_indices=_native.itab(record_indices), rec=records.shape[-1], width=width,
        num_paths=tree_paths.shape[1] if path_replay else 0, N=N, H=H, HV=HV, K=K, V=V,
    )
    _native.launch("eagle4_gdn_tree_records_update", args, q.device)
    return out


def gdn_tree_records_update(
    A_log, dt_bias, q, k, v, a, b, *, state, state_indices, query_start_loc, parent, tree_paths, records,
    record_indices, width,
):
    """Verify with compact replay records, preserving the pool's state precision (kernels/gdn_tree_records.py
    :364-444). bf16 / fp16 pools require ``tree_paths`` (each parent state is rounded before its descendants read
    it); fp32 pools may leave it out (the chunk form, no intermediate rounding: commit with ``round_state=False``).
    Returns the outputs, shaped like ``v``. A request with ``record_indices[n] < 0`` writes no records; in the path
    replay it runs as one chain over its rows."""
    if tree_paths is None:
        if state.dtype != torch.float32:
            raise ValueError("tree_paths are required for low-precision recurrent state")
        return gdn_tree_chunk_update(A_log, dt_bias, q, k, v, a, b, state=state, state_indices=state_indices,
                                     query_start_loc=query_start_loc, parent=parent, records=records,
                                     record_indices=record_indices, width=width)
    return _update(A_log, dt_bias, q, k, v, a, b, state, state_indices, query_start_loc, parent, tree_paths, records,
                   record_indices, width, path_replay=True)


def gdn_tree_chunk_update(
    A_log, dt_bias, q, k, v, a, b, *, state, state_indices, query_start_loc, parent, records, record_indices, width,
    use_flydsl: bool = True,
):
    """Outputs and delta / key / decay records without per-node state snapshots, state kept in fp32 throughout
    (kernels/gdn_tree_records.py:496-579; the accepted-path commit must use ``round_state=False``). ``use_flydsl``
    is accepted for signature compatibility and ignored."""
    return _update(A_log, dt_bias, q, k, v, a, b, state, state_indices, query_start_loc, parent, None, records,
                   record_indices, width, path_replay=False)


def gdn_tree_records_commit(
    state: torch.Tensor,
    records: torch.Tensor,
    state_indices: torch.Tensor,
    record_indices: torch.Tensor,
    commit_steps: torch.Tensor,
    parent: torch.Tensor,
    round_state: bool,
) -> None:
    """Commit the accepted node of every request into ``state`` (all layers, one launch) by replaying its root path's
    records (kernels/gdn_tree_records.py:229-272). state: (L, slots, HV, V, K); records: (L, rows, steps, HV, REC);
    parent: (batch, width), node 0 the root; a negative step, slot or row skips the request."""
    L_layers, _, HV, V, K = state.shape
    n = commit_steps.shape[0]
    if n == 0:
        return
    assert records.shape[0] == L_layers and records.shape[3] == HV and state.stride(-1) == 1
    assert state.stride(3) == K and state.stride(2) == V * K, "contiguous (V, K) state per head"
    _records_layout(records, HV, V, K)
    # the root path walks nodes below both the parent table's width and the records' steps (a parent table may be
    # wider than the tree: its extra columns are never reached)
    dmax = min(parent.shape[1], records.shape[2])
    args = _native.RecordsCommitArgs(
        state=state.data_ptr(), stride_state_layer=state.stride(0), stride_state_slot=state.stride(1),
        state_dtype=_native.dtype_code(state.dtype), round_state=int(bool(round_state)), records=records.data_ptr(),
        stride_records_layer=records.stride(0), stride_records_row=records.stride(1),
        state_indices=_native.itab(state_indices), record_indices=_native.itab(record_indices),
        commit_steps=_native.itab(commit_steps), parent=_native.itab(parent), n=n, layers=L_layers, HV=HV, K=K, V=V,
        rec=records.shape[-1], dmax=dmax, reserved=0,
    )
    _native.launch("eagle4_gdn_tree_records_commit", args, state.device)
