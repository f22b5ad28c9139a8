"""Pins of the oracle's tree tables (CPU): the reference tests' known answers and closed forms, plus independent
brute-force formulations (ancestor bits by walking up, links round trips, chain cover of the path table)."""

import numpy as np
import pytest

from oracle import tables as ot
from workloads import root_path, seeded_tree

PARENTS = [-1, 0, 0, 1, 1, 2, 3]


def _stage(parents_rows, widths, tree=True, W=None, positions=None, idx=None):
    W = W or max(len(p) for p in parents_rows)
    R = len(parents_rows)
    slots = R + 2
    par = np.full((slots, W), -1, np.int32)
    idx = np.arange(R, dtype=np.int32) + 1 if idx is None else idx
    for b, p in enumerate(parents_rows):
        par[idx[b], : len(p)] = p
    qsl = np.concatenate([[0], np.cumsum(widths)]).astype(np.int32)
    pos = (np.concatenate([100 + 10 * b + np.arange(w) for b, w in enumerate(widths)]) if positions is None
           else positions).astype(np.int64)
    out = dict(sp=np.zeros((R, W), np.int32), sa=np.zeros((R, 3, W), np.int32), sm=np.zeros((R, W), np.int64),
               cl=np.zeros(R, np.int32), slp=np.zeros((slots, W), np.int32), sld=np.zeros((slots, W), np.int32))
    ot.stage_tree(par, idx, qsl, qsl, pos, out["sp"], out["sa"], out["sm"], out["cl"], out["slp"], out["sld"], R, W,
                  tree)
    return out, pos, idx


def test_stage_known_answer():
    """PARENTS = [-1, 0, 0, 1, 1, 2, 3]: masks [1, 3, 5, 11, 19, 37, 75], depths [0, 1, 1, 2, 2, 2, 3]."""
    out, pos, idx = _stage([PARENTS], [7])
    assert out["sm"][0].tolist() == [1, 3, 5, 11, 19, 37, 75]
    assert out["sld"][idx[0]].tolist() == [0, 1, 1, 2, 2, 2, 3]
    assert (pos - 100).tolist() == [0, 1, 1, 2, 2, 2, 3]  # tree positions: context + depth
    assert out["cl"][0] == 100
    assert out["sa"][0].T.tolist() == [[-1, -2, -3], [0, -1, -2], [0, -1, -2], [1, 0, -1], [1, 0, -1], [2, 0, -1],
                                       [3, 1, 0]]


def _random_parents(width, seed):
    rng = np.random.default_rng(seed)
    return [-1] + [int(rng.integers(0, r)) for r in range(1, width)]


@pytest.mark.parametrize("parents", [PARENTS, _random_parents(16, 1), _random_parents(64, 3), [-1, 0, 1, 2, 3]])
def test_stage_matches_reference_closed_form(parents):
    """The reference test's recurrence (tests/test_gpu_kernels.py:47-64): depth = depth[p] + 1, window = [p,
    window[p][0], window[p][1]], mask = 1 << row | mask[p], signed int64."""
    width = len(parents)
    out, pos, idx = _stage([parents, parents], [width, width])
    depth, window, mask = [0], [[-1, -2, -3]], [1]
    for row in range(1, width):
        p = parents[row]
        depth.append(depth[p] + 1)
        window.append([p, window[p][0], window[p][1]])
        mask.append(1 << row | mask[p])
    mask = [m - (1 << 64) if m >= 1 << 63 else m for m in mask]
    for b in range(2):
        assert out["sa"][b].T.tolist() == window
        assert out["sm"][b].tolist() == mask
        assert out["sp"][b].tolist() == parents
        assert out["slp"][idx[b]].tolist() == parents
        assert out["sld"][idx[b]].tolist() == depth
        assert (pos[b * width : (b + 1) * width] - 100 - 10 * b).tolist() == depth


@pytest.mark.parametrize("seed", range(6))
def test_stage_masks_are_ancestor_sets(seed):
    """Independent form: bit j of row r's mask is set iff j lies on r's root path (walked up through parents)."""
    parents = seeded_tree(np.random.default_rng(seed), 16)
    out, _, _ = _stage([parents], [16])
    for r in range(16):
        path = set(root_path(parents, r))
        m = int(out["sm"][0, r]) & ((1 << 64) - 1)
        assert {j for j in range(16) if m >> j & 1} == path


def test_stage_chains_and_non_trees():
    """tree=False stages chains (parents r - 1) and leaves positions; a request whose width differs from its logits
    count (a prefill chunk) is staged as a chain too (vllm/verify_layout.py:53-59)."""
    out, pos, idx = _stage([PARENTS], [7], tree=False)
    assert out["sp"][0].tolist() == list(range(-1, 6))
    assert (pos - 100).tolist() == list(range(7))
    assert out["sm"][0].tolist() == [(1 << (r + 1)) - 1 for r in range(7)]


def test_stage_width_over_64_is_rejected_by_the_host():
    from eagle_harness.vllm.verify_layout import VerifyStage

    with pytest.raises(ValueError, match="at most 64 rows"):
        VerifyStage(2, 10, 65, "cpu")


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("width", [1, 2, 7, 16, 33])
def test_ancestors_round_trip_links(seed, width):
    """The parent derivation from first-child / next-sibling links returns the tree's parents (a first child's parent
    is the node; a sibling inherits its predecessor's), and the window codes are the closed form's."""
    parents = seeded_tree(np.random.default_rng(seed), width)
    nxt, sib = ot.links_from_parents(parents, width)
    par = np.zeros((1, width), np.int64)
    anc = np.zeros((1, 3, width), np.int32)
    paths = np.zeros((1, width, 2 + width), np.int32)
    ot.gdn_tree_ancestors(np.array([nxt]), np.array([sib]), par, np.array([5]), width, anc, np.array([0, width]),
                          paths)
    assert par[0, 1:].tolist() == parents[1:]
    assert anc[0].T.tolist() == ot.window_codes(parents)
    _check_paths(parents, paths[0], width)


def _check_paths(parents, paths, width):
    """Path-table invariants (kernels/gdn_tree.py:52-56): one row per leaf in node order, [len, write_from, root
    path]; the rows' chains (depths >= write_from) cover every node exactly once; rows past the leaf count have
    length 0."""
    children = {p for p in parents[1:]}
    leaves = [n for n in range(len(parents)) if n not in children]
    covered = []
    for r, leaf in enumerate(leaves):
        path = root_path(parents, leaf)
        assert paths[r, 0] == len(path)
        assert paths[r, 2 : 2 + len(path)].tolist() == path
        wf = paths[r, 1]
        # the chain starts where the path stops being a run of first children
        first_child = {n: min(c for c in range(1, len(parents)) if parents[c] == n) for n in children}
        start = len(path) - 1
        while start > 0 and first_child[path[start - 1]] == path[start]:
            start -= 1
        assert wf == start
        covered += path[wf:]
    assert sorted(covered) == list(range(len(parents)))
    assert all(paths[r, 0] == 0 for r in range(len(leaves), width))


def test_ancestors_pad_rows_keep_parents_and_follow_them():
    """A padded request keeps its parent links and ancestor rows; its paths follow its current parents."""
    parents = [-1, 0, 0, 1, 2]
    par = np.array([[9, 0, 0, 1, 2]], np.int64)
    anc = np.full((1, 3, 5), 77, np.int32)
    paths = np.zeros((1, 5, 7), np.int32)
    ot.gdn_tree_ancestors(np.full((1, 5), -1), np.full((1, 5), -1), par, np.array([-1]), 5, anc, np.array([0, 5]),
                          paths)
    assert par.tolist() == [[9, 0, 0, 1, 2]] and (anc == 77).all()
    _check_paths(parents, paths[0], 5)


@pytest.mark.parametrize("num_tokens", [1, 2, 5, 11, 15])
def test_paths_of_a_partial_request(num_tokens):
    """A request verifying fewer rows than the tree width (num_tokens < width): the path table is the one of the
    tree's first num_tokens rows (a prefix of a parent-first tree is a tree), checked against that truncated tree's
    own leaves, root paths and first-child runs; the remaining rows have length 0."""
    rng = np.random.default_rng(num_tokens)
    width = 16
    for _ in range(5):
        parents = [-1] + [int(rng.integers(0, i)) for i in range(1, width)]
        paths = np.full((width, 2 + width), 99, np.int32)
        ot._gdn_tree_paths(parents, num_tokens, width, paths)
        _check_paths(parents[:num_tokens], paths, width)
        # and through the public entry with a query_start_loc that gives the request num_tokens rows
        first, sibling = [-1] * width, [-1] * width
        last = {}
        for node in range(1, width):
            p = parents[node]
            if p in last:
                sibling[last[p]] = node
            else:
                first[p] = node
            last[p] = node
        par = np.zeros((1, width), np.int64)
        anc = np.zeros((1, 3, width), np.int32)
        table = np.full((1, width, 2 + width), 99, np.int32)
        ot.gdn_tree_ancestors(np.array([first]), np.array([sibling]), par, np.array([0]), width, anc,
                              np.array([0, num_tokens]), table)
        _check_paths(parents[:num_tokens], table[0], width)


def test_paths_sanitise_forward_parents():
    """Parents that are not ancestor-first are replaced by node - 1 so the table stays in bounds (:57-61)."""
    paths = np.zeros((4, 6), np.int32)
    ot._gdn_tree_paths([0, 3, 0, 1], 4, 4, paths)  # node 1's parent 3 is forward: becomes 0
    _check_paths([-1, 0, 0, 1], paths, 4)


def test_tail_words_closed_form():
    rng = np.random.default_rng(0)
    width, committed = 5, 30
    mask = rng.integers(0, 2, width * (committed + width)).astype(bool)
    words = ot.tree_tail_words(mask, committed, width)
    rows = mask.reshape(width, committed + width)[:, committed:]
    assert words == [sum(int(b) << j for j, b in enumerate(row)) for row in rows]
    with pytest.raises(ValueError):
        ot.tree_tail_words(mask, committed, 65)
