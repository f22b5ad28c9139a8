"""The depth-first walk plan of ``csrc/walk_plan.h`` (``build_plan``), emulated lane by lane on the CPU, against a
serial pre-order walk of the same tree.

``build_plan`` runs in one 64-lane wave, lane u holding row u: child masks and first children by LDS atomics, depths
and the successor's ancestor by pointer jumping over lane shuffles, Sethi-Ullman needs one tree level at a time
through per-row byte histograms. The emulation below performs the same steps on 64-entry arrays (a shuffle reads
another lane's value, an LDS atomic updates a shared entry, a ballot asks whether any lane holds a condition) in the
kernel's order. The serial side is the plan's definition: the pre-order walk with each node's children taken in
increasing (need, index) order, or index order, and for every row the row walked after it, whether that row is its
first child, whether it is the last child of its parent (the parked state is popped) and whether the row has
several children (its state is parked).
"""

from __future__ import annotations

import numpy as np
import pytest

NO_NEXT, FIRST, LAST, MULTI = 127, 1 << 7, 1 << 8, 1 << 9
LANES = 64


def _need_of(hist: int) -> int:
    """walk_plan.h need_of: the stack entries below a row from the byte histogram of its children's needs."""
    if hist == 0:
        return 0
    m1 = (hist.bit_length() - 1) >> 3
    if (hist >> (8 * m1)) & 0xFF >= 2:
        return m1 + 1
    rest = hist & ~(0xFF << (8 * m1))
    if rest == 0:
        return m1
    m2 = (rest.bit_length() - 1) >> 3
    return m1 if m1 > m2 + 1 else m2 + 1


def emulate_build_plan(parents: list[int], by_need: bool) -> list[int]:
    """The packed plan of every row, computed with build_plan's lane-parallel steps."""
    T = len(parents)
    lane = np.arange(LANES)
    par = np.array(list(parents) + [0] * (LANES - T))
    par[0] = 0
    child = (lane > 0) & (lane < T)
    kids = [0] * LANES
    hist = [0] * LANES
    first_key = [0x7FFFFFFF] * LANES
    for u in np.flatnonzero(child):  # atomicOr(kids[par], 1 << lane)
        kids[par[u]] |= 1 << int(u)
    need = np.zeros(LANES, dtype=np.int64)
    if by_need:
        dep = np.where(child, 1, 0)
        up = np.where(child, par, lane)
        for _ in range(6):  # pointer jumping to the root
            if not np.any((lane < T) & (up != 0)):
                break
            d2, u2 = dep[up], up[up]
            dep = dep + d2
            up = u2
        deepest = 0  # bit by bit from ballots
        for b in range(5, -1, -1):
            if np.any((lane < T) & (dep >= (deepest | (1 << b)))):
                deepest |= 1 << b
        for level in range(deepest, 0, -1):  # the deepest level first
            mine = child & (dep == level)
            if not mine.any():
                continue
            rows = np.flatnonzero(mine)
            for u in rows:
                need[u] = _need_of(hist[u])
            for u in rows:  # atomicAdd(hist[par], 1 << 8 * need)
                hist[par[u]] += 1 << (8 * int(need[u]))
    if by_need:
        key = need * 64 + lane
        for u in np.flatnonzero(child):  # atomicMin(first[par], key)
            first_key[par[u]] = min(first_key[par[u]], int(key[u]))
        first = np.array([-1 if fk == 0x7FFFFFFF else fk & 63 for fk in first_key])
        after = np.full(LANES, -1)
        for u in np.flatnonzero(child):
            best = 0x7FFFFFFF
            sib = kids[par[u]] & ~(1 << int(u))
            while sib:
                s = (sib & -sib).bit_length() - 1
                sib &= sib - 1
                if key[u] < key[s] < best:
                    best = int(key[s])
            after[u] = -1 if best == 0x7FFFFFFF else best & 63
    else:  # index order from the masks' lowest bits: the first child, the next sibling above the row (64-bit masks)
        first = np.array([(k & -k).bit_length() - 1 if k else -1 for k in kids])
        after = np.full(LANES, -1)
        for u in np.flatnonzero(child):
            above = kids[par[u]] & ~(((2 << int(u)) - 1) & (2**64 - 1)) & (2**64 - 1)
            after[u] = (above & -above).bit_length() - 1 if above else -1
    marked = (lane == 0) | (lane >= T) | (after >= 0)
    J = np.where(marked, lane, par)
    for _ in range(6):
        JJ = J[J]
        if np.all(JJ == J):
            break
        J = JJ
    after_J = after[J]
    nxt = np.where(first >= 0, first, np.where(J == 0, -1, after_J))
    after_next = after[nxt & 63]
    last = (first < 0) & (nxt >= 0) & (after_next < 0)
    multi = np.array([bin(k).count("1") >= 2 for k in kids])
    plan = np.where(nxt < 0, NO_NEXT, nxt) | np.where(first >= 0, FIRST, 0) | np.where(last, LAST, 0) | np.where(
        multi, MULTI, 0)
    return [int(p) for p in plan[:T]]


def serial_plan(parents: list[int], by_need: bool) -> list[int]:
    """The plan's definition: a serial pre-order walk."""
    T = len(parents)
    kids = [[] for _ in range(T)]
    for u in range(1, T):
        kids[parents[u]].append(u)
    need = [0] * T
    for u in reversed(range(T)):  # parents first, so a reverse scan sees children before parents
        ns = sorted((need[c] for c in kids[u]), reverse=True)
        if len(ns) == 1:
            need[u] = ns[0]
        elif ns:
            need[u] = ns[0] + 1 if ns[0] == ns[1] else ns[0]
    order_of = {u: sorted(kids[u], key=lambda c: (need[c], c) if by_need else c) for u in range(T)}
    walk, stack = [], [0]
    while stack:
        u = stack.pop()
        walk.append(u)
        stack.extend(reversed(order_of[u]))
    plan = [0] * T
    for i, u in enumerate(walk):
        nxt = walk[i + 1] if i + 1 < len(walk) else -1
        bits = NO_NEXT if nxt < 0 else nxt
        if order_of[u]:
            bits |= FIRST  # the next row is u's first child
        elif nxt >= 0 and order_of[parents[nxt]][-1] == nxt:
            bits |= LAST
        if len(kids[u]) >= 2:
            bits |= MULTI
        plan[u] = bits
    return plan


def _trees(rng: np.random.Generator):
    for T in range(1, LANES + 1):
        yield [-1] + list(range(T - 1))  # chain
        yield [-1] + [0] * (T - 1)  # star
        yield [-1] + [(u - 1) // 2 for u in range(1, T)]  # complete binary tree
        yield [-1] + [u - 1 if u % 2 else max(u - 2, 0) for u in range(1, T)]  # comb
        for _ in range(40):
            yield [-1] + [int(rng.integers(0, u)) for u in range(1, T)]  # any parent before the row
        for _ in range(20):  # topk <= 4, depth <= 12, as the verify trees are drafted
            par, depth, nkids = [-1], [0], [0]
            for u in range(1, T):
                ok = [j for j in range(u) if nkids[j] < 4 and depth[j] < 12] or [u - 1]
                p = int(ok[int(rng.integers(0, len(ok)))])
                par.append(p)
                depth.append(depth[p] + 1)
                nkids[p] += 1
                nkids.append(0)
            yield par


@pytest.mark.parametrize("by_need", [True, False])
def test_parallel_plan_equals_the_serial_walk(by_need):
    rng = np.random.default_rng(7)
    count = 0
    for parents in _trees(rng):
        assert emulate_build_plan(parents, by_need) == serial_plan(parents, by_need), parents
        count += 1
    assert count == 64 * 64


def test_known_plan():
    """Rows [-1, 0, 0, 1, 1, 2, 3]: in need order the walk is 0 2 5 1 3 6 4 (row 2's subtree needs no parked state,
    row 1's needs one: its two children need none each), in index order 0 1 3 6 4 2 5."""
    parents = [-1, 0, 0, 1, 1, 2, 3]
    plan = serial_plan(parents, True)
    walk, u = [0], 0
    while plan[u] & NO_NEXT != NO_NEXT:
        u = plan[u] & NO_NEXT
        walk.append(u)
    assert walk == [0, 2, 5, 1, 3, 6, 4]
    plan = serial_plan(parents, False)
    walk, u = [0], 0
    while plan[u] & NO_NEXT != NO_NEXT:
        u = plan[u] & NO_NEXT
        walk.append(u)
    assert walk == [0, 1, 3, 6, 4, 2, 5]
    assert plan[0] & MULTI and plan[1] & MULTI and not plan[2] & MULTI
    assert plan[6] & LAST  # after row 6, row 4 is row 1's last child: row 1's parked state is popped
