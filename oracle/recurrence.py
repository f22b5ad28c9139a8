"""Gated delta rule over a draft tree (snapshot contract), restated on the CPU (oracle; test infrastructure only).

Follows ``gdn_tree_recurrent_update`` and its walk (kernels/gdn_tree_recurrence.py:116-185, 204-359, 517-706): for
every request the nodes are visited in order; a node starts from its parent's snapshot read back from the snapshot
buffer (row 0 from the initial state, a chain child of an fp32 state from the previous node's registers), applies

    g = -exp(A_log) * softplus(a + dt_bias)         (linear above the threshold)
    beta = sigmoid(b), rounded through b's dtype
    q, k = q / sqrt(|q|^2 + 1e-6) * scale, k / sqrt(|k|^2 + 1e-6)
    h = h * exp(g);  v' = (v - h k) * beta;  h = h + v' k^T;  o = h q

and writes its output and its snapshot. States are [HV, V, K] per slot (K contiguous). All math is fp32, vectorised
over value heads; the walk's serial order over nodes (and every read of the snapshot buffer) is kept, so aliasing
and padding behave like the kernel.
"""

from __future__ import annotations

from typing import Optional

import torch

L2_NORM_EPS = 1e-6


def log_decay(a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor, beta: float = 1.0, threshold: float = 20.0):
    """``_log_decay`` (kernels/gdn_tree_recurrence.py:115-129), fp32."""
    x = a.float() + dt_bias.float()
    bx = beta * x
    sp = torch.where(bx <= threshold, (1.0 / beta) * torch.log(1.0 + torch.exp(bx)), x)
    return -torch.exp(A_log.float()) * sp


def write_strength(b: torch.Tensor) -> torch.Tensor:
    """``_write_strength`` (kernels/gdn_tree_recurrence.py:132-140): sigmoid, rounded through b's dtype."""
    beta = 1.0 / (1.0 + torch.exp(-b.float()))
    return beta.to(b.dtype).float()


def normalized_query_key(q: torch.Tensor, k: torch.Tensor, scale: float):
    """``_normalized_query_key`` (kernels/gdn_tree_recurrence.py:143-151) over the last dim, fp32."""
    q = q.float()
    k = k.float()
    q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + L2_NORM_EPS)
    k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + L2_NORM_EPS)
    return q * scale, k


def delta_rule_step(h, q, k, v, g, beta):
    """``_delta_rule_step`` (kernels/gdn_tree_recurrence.py:167-185) on [HV, V, K] states; q, k [HV, K]; v [HV, V];
    g, beta [HV]. Returns (h, o [HV, V])."""
    h = h * torch.exp(g)[:, None, None]
    v = v - (h * k[:, None, :]).sum(-1)
    v = v * beta[:, None]
    h = h + v[:, :, None] * k[:, None, :]
    o = (h * q[:, None, :]).sum(-1)
    return h, o


def gdn_tree_recurrent_update(
    A_log,
    dt_bias,
    q,
    k,
    v,
    a,
    b,
    *,
    initial_state_source: torch.Tensor,
    initial_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    intermediate_states_buffer: torch.Tensor,
    intermediate_state_indices: torch.Tensor,
    retrieve_parent_token: torch.Tensor,
    num_accepted_tokens: Optional[torch.Tensor] = None,
    pad_slot_id: int = -1,
    out: Optional[torch.Tensor] = None,
    publish: Optional[torch.Tensor] = None,
    tree_paths=None,
    scale: Optional[float] = None,
    softplus_beta: float = 1.0,
    softplus_threshold: float = 20.0,
    gluon: bool = False,
) -> torch.Tensor:
    """The reference signature (kernels/gdn_tree_recurrence.py:562-586) on CPU tensors, walk semantics
    (:204-359). ``tree_paths`` selects the reference's path replay, which computes the same fold over each root
    path (:370-495); the walk below is that fold too."""
    _, _, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    N = cu_seqlens.shape[0] - 1
    if scale is None:
        scale = K**-0.5
    if out is None:
        out = q.new_empty(v.shape)
    row_slots = intermediate_state_indices.ndim == 2
    fp32_state = intermediate_states_buffer.dtype == torch.float32 and initial_state_source.dtype == torch.float32
    skip_chain_reload = fp32_state
    group = HV // H
    A32, dt32 = A_log.float(), dt_bias.float()
    for n in range(N):  # one request at a time; the kernel runs (V tile, request, head) programs in parallel
        if publish is not None and row_slots:  # _publish_slot_table, :188-200
            S = intermediate_state_indices.shape[1]
            publish[n, :S] = intermediate_state_indices[n, :S]
        bos, eos = int(cu_seqlens[n]), int(cu_seqlens[n + 1])
        T = eos - bos
        if num_accepted_tokens is not None:
            idx = int(initial_state_indices[n, int(num_accepted_tokens[n]) - 1])
        else:
            idx = int(initial_state_indices[n] if initial_state_indices.ndim == 1 else initial_state_indices[n, 0])
        h = torch.zeros(HV, V, K)
        if idx > pad_slot_id:  # :286-296
            h = initial_state_source[idx].float().clone()
        cache_idx = int(intermediate_state_indices[n, 0] if row_slots else intermediate_state_indices[n])
        for step in range(T):  # :306-359
            parent = int(retrieve_parent_token[n, step])
            slot, parent_slot = cache_idx, cache_idx
            if row_slots:
                slot = int(intermediate_state_indices[n, step])
                parent_slot = int(intermediate_state_indices[n, parent]) if step != 0 else pad_slot_id
            reload = step != 0 and parent_slot > pad_slot_id
            if skip_chain_reload:
                reload = reload and parent != step - 1
            if reload:
                src = intermediate_states_buffer[parent_slot] if row_slots else intermediate_states_buffer[parent_slot, parent]
                h = src.float().clone()
            t = bos + step
            g = log_decay(a[t], A32, dt32, softplus_beta, softplus_threshold)
            beta = write_strength(b[t])
            qn, kn = normalized_query_key(q[0, t], k[0, t], scale)  # [H, K]
            qn = qn.repeat_interleave(group, 0)
            kn = kn.repeat_interleave(group, 0)
            h, o = delta_rule_step(h, qn, kn, v[0, t].float(), g, beta)
            out[0, t] = o.to(out.dtype)
            if slot > pad_slot_id:
                if row_slots:
                    intermediate_states_buffer[slot] = h.to(intermediate_states_buffer.dtype)
                else:
                    intermediate_states_buffer[slot, step] = h.to(intermediate_states_buffer.dtype)
    return out


def dense_tree_reference(q, k, v, a, b, A_log, dt_bias, init, parents, heads, value_heads):
    """An independent per-row formulation (the reference test's dense form, tests/test_gdn_tree_kernels.py:151-176):
    each row continues from its parent's state; returns (outputs [rows, HV, V], states [rows][HV, V, K]).
    Unlike the walk it keeps beta unrounded (fp32 gate inputs)."""
    outs, states = [], []
    for row, parent in enumerate(parents):
        state = (init if parent < 0 else states[parent]).clone()
        qn, kn = q[row], k[row]
        qn = qn / torch.sqrt((qn * qn).sum(-1, keepdim=True) + 1e-6)
        kn = kn / torch.sqrt((kn * kn).sum(-1, keepdim=True) + 1e-6)
        qn = qn * q.shape[-1] ** -0.5
        g = -torch.exp(A_log) * torch.nn.functional.softplus(a[row] + dt_bias)
        beta = torch.sigmoid(b[row])
        out = torch.zeros_like(v[row])
        for hv in range(value_heads):
            h = hv // (value_heads // heads)
            s = state[hv] * torch.exp(g[hv])
            delta = (v[row, hv] - s @ kn[h]) * beta[hv]
            s = s + delta[:, None] * kn[h][None, :]
            state[hv] = s
            out[hv] = s @ qn[h]
        outs.append(out)
        states.append(state)
    return torch.stack(outs), states
