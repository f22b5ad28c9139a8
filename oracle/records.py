"""Replay records, accepted-path commit and the parallel chunk form, restated on the CPU (oracle; test
infrastructure only).

Follows kernels/gdn_tree_records.py. Per node a record ``(delta [V], key [K], decay)`` is kept instead of a state
snapshot (REC = V + K + 4 floats; the 3 floats after the decay are never written). ``gdn_tree_records_update``
replays every leaf's root path from the pool state, rounding each parent state to the pool dtype before its children
read it (:44-101, ``ROUND_STATE``); ``gdn_tree_chunk_update`` is the fp32 closed form over the ancestor closure
(:276-361); ``gdn_tree_records_commit`` folds the accepted node's root path back into the pool (:160-226).
"""

from __future__ import annotations

import torch

from oracle.recurrence import log_decay, normalized_query_key, write_strength


def gdn_tree_pre(A_log, dt_bias, q, k, a, b, scale, softplus_beta=1.0, softplus_threshold=20.0):
    """``_gdn_tree_pre_kernel`` (kernels/gdn_tree_records.py:104-156): fp32 q_pre, k_pre [tokens, H, K] and gb_pre
    [tokens, HV, 2] = (exp(g), beta)."""
    g = log_decay(a, A_log, dt_bias, softplus_beta, softplus_threshold)  # [tokens, HV]
    beta = write_strength(b)
    qn, kn = normalized_query_key(q[0], k[0], scale)
    return qn, kn, torch.stack([torch.exp(g), beta], -1)


def gdn_tree_records_update(A_log, dt_bias, q, k, v, a, b, *, state, state_indices, query_start_loc, parent,
                            tree_paths, records, record_indices, width):
    """``gdn_tree_records_update`` with ``tree_paths`` (kernels/gdn_tree_records.py:364-444): the rounded path replay.

    Writes ``records[record_indices[n], node]`` for every node and returns the output shaped like ``v``."""
    _, tokens, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    group = HV // H
    out = torch.empty_like(v)
    qp, kp, gb = gdn_tree_pre(A_log, dt_bias, q, k, a, b, K**-0.5)
    N = query_start_loc.numel() - 1
    P = tree_paths.shape[1]
    for n in range(N):
        bos, eos = int(query_start_loc[n]), int(query_start_loc[n + 1])
        rec_idx = int(record_indices[n])
        linear = rec_idx < 0
        for p in range(P):
            if linear:
                L = (eos - bos) if p == 0 else 0
                wfrom = 0
            else:
                L = int(tree_paths[n, p, 0])
                wfrom = int(tree_paths[n, p, 1])
            if L <= 0:
                continue
            idx = int(state_indices[n])
            h = state[idx].float().clone() if idx >= 0 else torch.zeros(HV, V, K)
            for d in range(L):
                t = bos + (d if linear else int(tree_paths[n, p, 2 + d]))
                uq = qp[t].repeat_interleave(group, 0)
                uk = kp[t].repeat_interleave(group, 0)
                eg, beta = gb[t, :, 0], gb[t, :, 1]
                if d > 0 and rec_idx >= 0:  # ROUND_STATE (:86-88)
                    h = h.to(state.dtype).float()
                h = h * eg[:, None, None]
                dv = (v[0, t].float() - (h * uk[:, None, :]).sum(-1)) * beta[:, None]
                h = h + dv[:, :, None] * uk[:, None, :]
                if d >= wfrom:
                    out[0, t] = (h * uq[:, None, :]).sum(-1).to(out.dtype)
                    if rec_idx >= 0:
                        node = t - bos
                        records[rec_idx, node, :, :V] = dv
                        records[rec_idx, node, :, V : V + K] = uk
                        records[rec_idx, node, :, V + K] = eg
    return out


def gdn_tree_chunk_update(A_log, dt_bias, q, k, v, a, b, *, state, state_indices, query_start_loc, parent, records,
                          record_indices, width):
    """``gdn_tree_chunk_update`` / ``_gdn_tree_chunk_kernel`` (kernels/gdn_tree_records.py:276-361, 496-579): per
    (request, value head) in closed form, fp32, no per-node rounding:

        R = strict-ancestor closure of the parent links, G_t = prod of exp(g) along t's root path,
        D = (I + diag(beta) (R o G_t/G_j o K K^T))^-1 diag(beta) (V - diag(G) K S0^T),
        O = diag(G) Q S0^T + ((R + I) o G_t/G_j o Q K^T) D.

    (S0 is the [V, K] pool state, so K S0^T is [nodes, V].)"""
    _, tokens, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    group = HV // H
    out = torch.empty_like(v)
    qp, kp, gb = gdn_tree_pre(A_log, dt_bias, q, k, a, b, K**-0.5)
    N = query_start_loc.numel() - 1
    for n in range(N):
        bos, eos = int(query_start_loc[n]), int(query_start_loc[n + 1])
        T = eos - bos
        if T <= 0:
            continue
        par = [int(parent[n, t]) if t > 0 else -1 for t in range(T)]
        R = torch.zeros(T, T)
        for t in range(T):  # strict ancestors
            p = par[t]
            while p >= 0:
                R[t, p] = 1.0
                p = par[p]
        eye = torch.eye(T)
        M = R + eye
        idx = int(state_indices[n])
        row = int(record_indices[n])
        for hv in range(HV):
            h = hv // group
            Kt = kp[bos:eos, h]
            Qt = qp[bos:eos, h]
            eg = gb[bos:eos, hv, 0]
            beta = gb[bos:eos, hv, 1]
            logG = M @ torch.log(torch.clamp(eg, min=1e-30))
            G = torch.exp(logG)
            ratio = torch.where(M > 0, torch.exp(logG[:, None] - logG[None, :]), torch.zeros(T, T))
            L = beta[:, None] * (R * ratio * (Kt @ Kt.T))
            S0 = state[idx, hv].float() if idx >= 0 else torch.zeros(V, K)
            rhs = beta[:, None] * (v[0, bos:eos, hv].float() - G[:, None] * (Kt @ S0.T))
            D = torch.linalg.solve(eye + L, rhs)
            O = G[:, None] * (Qt @ S0.T) + (ratio * (Qt @ Kt.T)) @ D
            out[0, bos:eos, hv] = O.to(out.dtype)
            if row >= 0:
                records[row, :T, hv, :V] = D
                records[row, :T, hv, V : V + K] = Kt
                records[row, :T, hv, V + K] = eg
    return out


def gdn_tree_records_commit(state, records, state_indices, record_indices, commit_steps, parent, round_state):
    """``gdn_tree_records_commit`` (kernels/gdn_tree_records.py:160-272): for every layer and request with
    non-negative step, slot and record row, fold ``S <- S * decay + delta key^T`` over the accepted node's root path
    (rounded to the pool dtype between nodes with ``round_state``) and store it in the pool."""
    L_layers, _, HV, V, K = state.shape
    dmax = parent.shape[1]
    for layer in range(L_layers):
        for n in range(commit_steps.shape[0]):
            step, slot, row = int(commit_steps[n]), int(state_indices[n]), int(record_indices[n])
            if not (step >= 0 and slot >= 0 and row >= 0):
                continue
            path, node = [], step
            for _ in range(dmax):  # :192-201
                path.append(node)
                node = int(parent[n, node]) if node > 0 else -1
                if node < 0:
                    break
            h = state[layer, slot].float().clone()
            for d, node in enumerate(reversed(path)):
                rec = records[layer, row, node]
                if round_state and d > 0:
                    h = h.to(state.dtype).float()
                h = h * rec[:, V + K][:, None, None]
                h = h + rec[:, :V][:, :, None] * rec[:, V : V + K][:, None, :]
            state[layer, slot] = h.to(state.dtype)
