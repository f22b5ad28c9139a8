"""Mamba2 tree verify restated on the CPU (oracle; test infrastructure only).

Follows kernels/mamba2_tree.py:41-160 (``_tree_ssu_kernel``): request ``b``'s rows are tokens
``query_start_loc[b] .. query_start_loc[b + 1] - 1``; row 0 starts from ``state[slots[b, max(num_accepted[b] - 1,
0)]]`` (:99-104), a row whose parent is the previous row continues from the unrounded state, any other reloads its
parent's stored slot (:121-131); each row computes ``dt = softplus(dt + dt_bias)`` (:133-137, softplus :38-39),
``state = state * exp(A dt) + (B dt) x`` (:138-142), stores it (rounded to the pool dtype) unless its slot is the pad
slot (:143-145), and ``out = C . state + D x`` (:146-149). A pad slot reads as zeros. Computed in float64; the stored
state is rounded through the pool's dtype as the reference's store rounds it.
"""

from __future__ import annotations

import math

import torch


def _softplus(dt: float) -> float:
    return math.log(math.exp(dt) + 1.0) if dt <= 20.0 else dt


def mamba2_tree_state_update(state, x, dt, A, B, C, D, dt_bias, out, *, state_indices, parents, query_start_loc,
                             num_accepted_tokens=None, dt_softplus=True, pad_slot_id=-1):
    """In place on ``state`` and ``out`` (CPU tensors, the shapes of kernels/mamba2_tree.py:177-202)."""
    tokens, heads, head_dim = x.shape
    groups = B.shape[1]
    hpg = heads // groups
    batch = query_start_loc.shape[0] - 1
    for b in range(batch):
        bos, eos = int(query_start_loc[b]), int(query_start_loc[b + 1])
        if eos <= bos:
            continue
        init = max(int(num_accepted_tokens[b]) - 1, 0) if num_accepted_tokens is not None else 0
        for h in range(heads):
            g = h // hpg

            def read(slot):
                if slot == pad_slot_id:
                    return torch.zeros(head_dim, state.shape[-1], dtype=torch.float64)
                return state[slot, h].double()

            s = read(int(state_indices[b, init]))
            for t in range(eos - bos):
                tok = bos + t
                p = int(parents[b, t])
                if t > 0 and p != t - 1:
                    s = read(int(state_indices[b, p]))
                d = float(dt[tok, h]) + (float(dt_bias[h]) if dt_bias is not None else 0.0)
                if dt_softplus:
                    d = _softplus(d)
                xv = x[tok, h].double()
                s = s * math.exp(float(A[h]) * d) + (B[tok, g].double() * d)[None, :] * xv[:, None]
                slot = int(state_indices[b, t])
                if slot != pad_slot_id:
                    state[slot, h] = s.to(state.dtype)
                o = s @ C[tok, g].double()
                if D is not None:
                    o = o + xv * float(D[h])
                out[tok, h] = o.to(out.dtype)
    return out
