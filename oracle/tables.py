"""Tree tables of the verify round, restated on the CPU (oracle; test infrastructure only).

Every function mirrors one reference kernel lane by lane, including the values it produces for malformed input
(parents that point forward, out of range or at padding), so the HIP kernels can be compared bit for bit.
"""

from __future__ import annotations

from typing import Optional

import numpy as np


def _np2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def _to_i64(v: int) -> int:
    """Two's complement int64 of an unsigned 64-bit pattern."""
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= 1 << 63 else v


def stage_tree(
    parents: np.ndarray,
    idx_mapping: np.ndarray,
    query_start_loc: np.ndarray,
    cu_num_logits: np.ndarray,
    positions: np.ndarray,
    stage_parents: np.ndarray,
    stage_anc: np.ndarray,
    stage_mask: np.ndarray,
    context_lens: np.ndarray,
    slot_parents: np.ndarray,
    slot_depths: np.ndarray,
    num_reqs: int,
    width: int,
    tree: bool,
) -> None:
    """``_stage_tree_kernel`` (vllm/verify_layout.py:31-86), in place on numpy arrays.

    parents [slots, W] int32 (row 0: -1); idx_mapping [R]; query_start_loc / cu_num_logits [R + 1]; positions
    [tokens] int64 (chain in, depth out); stage_parents [R, W]; stage_anc [R, 3, W]; stage_mask [R, W] int64;
    context_lens [R]; slot_parents / slot_depths [slots, W].
    """
    W = width
    WP = _np2(W)
    for b in range(num_reqs):
        slot = int(idx_mapping[b])
        start = int(query_start_loc[b])
        w = int(query_start_loc[b + 1]) - start
        context_lens[b] = np.int32(np.int64(positions[start]).astype(np.int32))  # :52
        is_tree = tree and w > 1 and w == int(cu_num_logits[b + 1]) - int(cu_num_logits[b])  # :54
        rows = list(range(WP))
        par = [int(parents[slot, r]) if r < W else -1 for r in rows]  # :57
        if not is_tree:
            par = [r - 1 for r in rows]  # :59
        depth = [0] * WP
        anc1 = [-1] * WP
        anc2 = [-2] * WP
        anc3 = [-3] * WP
        mask = [1] * WP

        def at(arr, p):
            return arr[p] if 0 <= p < WP else 0

        for r in range(1, W):  # :66-74, updates in the kernel's order
            p = par[r]
            depth[r] = at(depth, p) + 1
            anc1[r] = p
            anc2[r] = at(anc1, p)
            anc3[r] = at(anc2, p)
            mask[r] = _to_i64(at(mask, p) | (1 << r))
        for r in range(W):
            stage_parents[b, r] = par[r]
            stage_anc[b, 0, r] = anc1[r]
            stage_anc[b, 1, r] = anc2[r]
            stage_anc[b, 2, r] = anc3[r]
            stage_mask[b, r] = mask[r]
            slot_parents[slot, r] = par[r]
            slot_depths[slot, r] = depth[r]
        if is_tree:  # :85-86
            for r in range(min(w, W)):
                positions[start + r] = int(positions[start + r]) - r + depth[r]


def tree_masks(parents: list[int], width: Optional[int] = None) -> list[int]:
    """Ancestor-or-self bit masks of a parent-first tree, signed int64 (the stage's ``masks`` rows)."""
    masks: list[int] = []
    for r, p in enumerate(parents):
        masks.append(_to_i64((1 << r) | ((masks[p] & ((1 << 64) - 1)) if p >= 0 else 0)))
    if width is not None:
        masks += [0] * (width - len(masks))
    return masks


def window_codes(parents: list[int]) -> list[list[int]]:
    """Per node: parent, grandparent, great-grandparent; -1/-2/-3 are the history columns 2/1/0."""
    anc = [[-1, -2, -3]]
    for node in range(1, len(parents)):
        p = parents[node]
        anc.append([p, anc[p][0], anc[p][1]])
    return anc


def links_from_parents(parents: list[int], width: int) -> tuple[list[int], list[int]]:
    """sglang's first-child / next-sibling links of a parent-first tree (children in row order), -1 padded."""
    next_token = [-1] * width
    next_sibling = [-1] * width
    last_child: dict[int, int] = {}
    for node in range(1, len(parents)):
        p = parents[node]
        if p in last_child:
            next_sibling[last_child[p]] = node
        else:
            next_token[p] = node
        last_child[p] = node
    return next_token, next_sibling


def _gdn_tree_paths(parents_in: list[int], num_tokens: int, seqlen: int, paths: np.ndarray) -> None:
    """``_gdn_tree_paths`` (kernels/gdn_tree.py:44-89) on one request's [seqlen, 2 + seqlen] path rows."""
    NP = len(parents_in)
    idx = list(range(NP))
    parents = [parents_in[i] if (i > 0 and 0 <= parents_in[i] < i) else max(i - 1, 0) for i in idx]  # :57-61
    packed = [0] * NP
    for t in range(1, seqlen):  # :64-72
        p = parents[t]
        pp = packed[p] if 0 <= p < NP else 0
        depth = (pp & 255) + 1
        chain_depth = depth if pp >= 65536 else (pp >> 8) & 255
        if t < num_tokens:
            packed[t] = depth + (chain_depth << 8)
            if 0 <= p < NP:
                packed[p] |= 65536
    depths = [v & 255 for v in packed]
    is_leaf = [i < num_tokens and packed[i] < 65536 for i in idx]
    num_leaves = sum(is_leaf)
    rank = 0
    leaf_rows = {}
    for i in idx:
        if is_leaf[i]:
            leaf_rows[i] = rank
            paths[rank, 0] = depths[i] + 1  # :78
            paths[rank, 1] = (packed[i] >> 8) & 255  # :79
            rank += 1
    for i in range(num_leaves, seqlen):  # :80-84: only the length column of unused rows
        paths[i, 0] = 0
    for i, row in leaf_rows.items():  # :86-89, leaf first
        node = i
        for step in range(depths[i] + 1):
            paths[row, 2 + depths[i] - step] = node
            node = parents[node] if 0 <= node < NP else 0


def gdn_tree_ancestors(
    next_token: np.ndarray,
    next_sibling: np.ndarray,
    parent_token: np.ndarray,
    conv_state_indices: np.ndarray,
    width: int,
    ancestors: np.ndarray,
    query_start_loc: Optional[np.ndarray] = None,
    paths: Optional[np.ndarray] = None,
    pad_slot_id: int = -1,
) -> None:
    """``gdn_tree_ancestors`` / ``_gdn_tree_ancestors_kernel`` (kernels/gdn_tree.py:93-237), in place.

    Writes ``parent_token[:, :width]``, ``ancestors`` [batch, 3, width] and, with ``paths`` [batch, width, 2 + width],
    the path table.
    """
    batch = ancestors.shape[0]
    NP = _np2(width)
    for s in range(batch):
        coord = int(conv_state_indices[s])
        num_tokens = 0
        if paths is not None:
            num_tokens = min(max(int(query_start_loc[s + 1]) - int(query_start_loc[s]), 0), width)  # :123-126
        if coord == pad_slot_id:  # :127-138
            if paths is not None:
                par = [int(parent_token[s, i]) if i < width else 0 for i in range(NP)]
                _gdn_tree_paths(par, num_tokens, width, paths[s])
            continue
        nxt = [int(next_token[s, i]) if i < width else -1 for i in range(NP)]
        sib = [int(next_sibling[s, i]) if i < width else -1 for i in range(NP)]
        par = [0] * NP
        a1 = [-1] * NP
        a2 = [-2] * NP
        a3 = [-3] * NP
        for t in range(width):  # :155-172
            n = nxt[t]
            if n != -1 and 0 <= n < NP:
                par[n] = t
            sb = sib[t]
            p = par[t]
            if sb != -1 and 0 <= sb < NP:
                par[sb] = p
            g = par[p] if 0 <= p < NP else 0
            g = g if p > 0 else p - 1
            gg = par[g] if 0 <= g < NP else 0
            gg = gg if g > 0 else g - 1
            if t > 0:
                a1[t], a2[t], a3[t] = p, g, gg
        for i in range(width):
            parent_token[s, i] = par[i]
            ancestors[s, 0, i] = a1[i]
            ancestors[s, 1, i] = a2[i]
            ancestors[s, 2, i] = a3[i]
        if paths is not None:
            _gdn_tree_paths(par, num_tokens, width, paths[s])


def tree_tail_words(mask_flat: np.ndarray, committed_len: int, width: int) -> list[int]:
    """``_tail_words_kernel`` (kernels/verify_prep.py:23-33): one signed int64 word per row of a ``[width, kv_len]``
    bool mask, bit ``j`` = the row sees tree key ``j`` (column ``kv_len - width + j``)."""
    if not 0 < width <= 64:
        raise ValueError(f"verify width {width} outside 1..64")
    kv_len = committed_len + width
    words = []
    for r in range(width):
        w = 0
        for j in range(width):
            if mask_flat[r * kv_len + (kv_len - width) + j]:
                w |= 1 << j
        words.append(_to_i64(w))
    return words
