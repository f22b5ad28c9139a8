"""Pins of the CPU oracle's accept walks, row compaction and vLLM state commit (oracle/accept.py, oracle/commit.py):
the reference test's planted-path known answers (tests/test_tree_rejection_sampler.py:26-28, 56-71), the bs1 tail
walk agreeing with the tree walk on the same tree, compaction's closed form (kernels/accept_tail.py:190-224), and the
commit's defining property — the next round resumes exactly where the accepted path run as a chain ends
(tests/test_gdn_tree_kernels.py:391-547 checks the same against vLLM's chain kernels)."""

import numpy as np
import torch

from oracle import accept as oac
from oracle import commit as ocm
from oracle import conv as oc
from oracle import recurrence as orr
from oracle.tables import links_from_parents
from workloads import seeded_tree, window_codes

# (parents, accepted path, state slot): the reference test's two requests
TREES = [([-1, 0, 0, 1, 1, 2, 3, 5], [0, 2, 5, 7], 3), ([-1, 0, 0, 1, 1], [0, 1, 4], 1)]


def _planted(parents, path, vocab, gen):
    """Target logits and drafted tokens such that the greedy walk accepts ``path`` and nothing off it."""
    n = len(parents)
    logits = torch.randn(n, vocab, generator=gen)
    drafted = torch.randint(0, vocab, (n,), generator=gen)
    top = logits.argmax(-1)
    for row in range(1, n):
        if drafted[row] == top[parents[row]]:
            drafted[row] = (top[parents[row]] + 1) % vocab
    for parent, child in zip(path, path[1:]):
        drafted[child] = top[parent]
    return logits, drafted


def test_argmax_takes_the_first_index_on_ties():
    logits = torch.zeros(2, 10)
    logits[0, [3, 7]] = 5.0
    logits[1, [9, 0]] = -1.0
    logits[1, 1:9] = -2.0
    assert oac.argmax_rows(logits).tolist() == [3, 0]


def test_accept_tree_planted_paths_known_answer():
    W, vocab, slots = 8, 64, 4
    gen = torch.Generator().manual_seed(7)
    logits, drafted, parents_tab = [], [], torch.full((slots, W), -1, dtype=torch.int32)
    for parents, path, slot in TREES:
        lg, dr = _planted(parents, path, vocab, gen)
        logits.append(lg)
        drafted.append(dr)
        parents_tab[slot, : len(parents)] = torch.tensor(parents)
    sizes = [len(p) for p, _, _ in TREES]
    cu = torch.tensor([0, sizes[0], sizes[0] + sizes[1]], dtype=torch.int32)
    target = oac.argmax_rows(torch.cat(logits))
    path_tab = torch.full((slots, W), -5, dtype=torch.int32)
    path_len = torch.zeros(slots, dtype=torch.int32)
    sampled, num = oac.accept_tree(target, torch.cat(drafted), cu, torch.tensor([3, 1], dtype=torch.int32), parents_tab,
                                   path_tab, path_len, W)
    assert path_tab[3, :4].tolist() == [0, 2, 5, 7] and path_tab[1, :3].tolist() == [0, 1, 4]
    assert path_len[3] == 4 and path_len[1] == 3 and num.tolist() == [4, 3]
    assert sampled[0, :4].tolist() == target[[0, 2, 5, 7]].tolist()
    assert sampled[1, :3].tolist() == target[sizes[0] + torch.tensor([0, 1, 4])].tolist()


def test_accept_tail_walks_the_same_path_as_the_tree_walk():
    """bs1 links (first child / next sibling in row order): the first matching sibling is the lowest-index matching
    child, so both walks accept the same nodes; predictions move the path to the front."""
    rng = np.random.default_rng(11)
    for trial in range(20):
        W, depth, vocab = 16, 8, 50
        parents = seeded_tree(rng, W)
        leaf = int(rng.integers(W))
        path, node = [], leaf
        while node >= 0:
            path.append(node)
            node = parents[node]
        path = path[::-1][:depth]
        gen = torch.Generator().manual_seed(trial)
        logits, drafted = _planted(parents, path, vocab, gen)
        target = oac.argmax_rows(logits)
        nxt, sib = links_from_parents(parents, W)
        seq_len = 30
        req_to_token = torch.arange(200, dtype=torch.int64).view(2, 100) + 1000
        out_loc = torch.arange(W, dtype=torch.int64) + 500
        # tree position i is flattened row perm[i] (retrieve_index): candidates go by position, targets by row
        perm = torch.randperm(W, generator=gen)
        target_rows = torch.empty_like(target)
        target_rows[perm] = target
        got = oac.accept_tail(target_rows.to(torch.int32), drafted.to(torch.int32), perm.to(torch.int32),
                              torch.tensor(nxt, dtype=torch.int32), torch.tensor(sib, dtype=torch.int32),
                              torch.tensor([seq_len], dtype=torch.int32), out_loc, req_to_token,
                              torch.tensor([1]), depth)
        n = len(path)
        assert got["accept_index"][0, :n].tolist() == perm[path].tolist()
        assert got["accept_index"][0, n:].tolist() == [-1] * (depth - n)
        assert int(got["accept_lens"][0]) == n and int(got["new_seq_lens"][0]) == seq_len + n
        assert int(got["bonus_tokens"][0]) == int(target[path[-1]])
        assert got["predict"][:n].tolist() == target[path].tolist()
        assert got["accepted_slots"][:n].tolist() == (out_loc[perm[path]]).tolist()
        assert got["committed_slots"][:n].tolist() == req_to_token[1, seq_len : seq_len + n].tolist()
        # and the tree walk agrees
        ptab = torch.tensor([parents], dtype=torch.int32)
        pt, pl = torch.zeros(1, W, dtype=torch.int32), torch.zeros(1, dtype=torch.int32)
        oac.accept_tree(target, drafted, torch.tensor([0, W], dtype=torch.int32), torch.tensor([0], dtype=torch.int32),
                        ptab, pt, pl, W)
        walked = pt[0, : int(pl[0])].tolist()
        assert walked[:depth] == path


def test_compact_rows_known_answer():
    rows = torch.arange(8 * 3).view(8, 3)
    out = oac.compact_rows(rows, torch.tensor([[0, 3, 5, -1]], dtype=torch.int32))
    assert out[:4].tolist() == [rows[0].tolist(), rows[3].tolist(), rows[5].tolist(), rows[0].tolist()]
    assert torch.equal(out[4:], rows[4:])


def test_accepted_rows_first_known_answer():
    """vllm/tree_accept.py:118-126: a request's first path_len rows point at its accepted rows, the rest at
    themselves (the reference test's two requests, rows of slot 3 then slot 1)."""
    mapping = torch.tensor([3] * 8 + [1] * 5, dtype=torch.int32)
    local = torch.tensor(list(range(8)) + list(range(5)), dtype=torch.int32)
    path = torch.zeros(4, 8, dtype=torch.int32)
    path[3, :4] = torch.tensor([0, 2, 5, 7])
    path[1, :3] = torch.tensor([0, 1, 4])
    path_len = torch.tensor([0, 3, 0, 4], dtype=torch.int32)
    got = oac.accepted_rows_first(mapping, local, path, path_len)
    assert got.tolist() == [0, 2, 5, 7, 4, 5, 6, 7, 8, 9, 12, 11, 12]


def test_commit_resumes_where_the_accepted_chain_ends():
    """A tree round (conv + walk, vLLM per-row slots) then the commit leaves the request's window and recurrent state
    exactly where running the accepted path as a chain leaves them."""
    parents = [-1, 0, 0, 1, 2, 4, 4]
    path = [0, 2, 4, 5]
    T, n = len(parents), len(path)
    H, HV, K, V, dim = 1, 2, 8, 8, 12
    gen = torch.Generator().manual_seed(21)
    hist = torch.randn(dim, 3, generator=gen)
    x = torch.randn(T, dim, generator=gen)
    weight = torch.randn(dim, 4, generator=gen)
    q, k = torch.randn(1, T, H, K, generator=gen), torch.randn(1, T, H, K, generator=gen)
    v = torch.randn(1, T, HV, V, generator=gen)
    a, b = torch.randn(T, HV, generator=gen), torch.randn(T, HV, generator=gen)
    A_log, dt_bias = torch.randn(HV, generator=gen), torch.randn(HV, generator=gen)
    init = torch.randn(HV, V, K, generator=gen) * 0.1

    def run(par, xs, qs, ks, vs, as_, bs_, num_slots):
        W = len(par)
        conv = torch.zeros(num_slots, dim, 3 + W)
        conv[1, :, :3] = hist
        pool = torch.zeros(num_slots, HV, V, K)
        pool[1] = init
        sl = (1 + torch.arange(W + 1, dtype=torch.int32))[None]
        qsl = torch.tensor([0, W], dtype=torch.int32)
        acc = torch.tensor([1], dtype=torch.int32)
        anc = torch.tensor([list(zip(*window_codes(par)))], dtype=torch.int32)
        oc.gdn_tree_conv1d_update(xs.t()[None], conv, weight, None, "silu", sl[:, 0].contiguous(), None, None, anc,
                                  pad_slot_id=0, out=torch.empty_like(xs).t()[None], num_accepted_tokens=acc,
                                  query_start_loc=qsl)
        orr.gdn_tree_recurrent_update(A_log, dt_bias, qs, ks, vs, as_, bs_, initial_state_source=pool,
                                      initial_state_indices=sl, cu_seqlens=qsl, intermediate_states_buffer=pool,
                                      intermediate_state_indices=sl, retrieve_parent_token=torch.tensor([par]),
                                      num_accepted_tokens=acc, pad_slot_id=0)
        return conv, pool, sl

    conv, pool, sl = run(parents, x, q, k, v, a, b, T + 2)
    ptab = torch.full((1, T), -1, dtype=torch.int32)
    ptab[0, :n] = torch.tensor(path)
    ocm.linear_state_commit([conv], [pool], [sl], torch.tensor([0], dtype=torch.int32), ptab,
                            torch.tensor([n], dtype=torch.int32))
    chain = [-1] + list(range(n - 1))
    idx = torch.tensor(path)
    cconv, cpool, csl = run(chain, x[idx], q[:, idx], k[:, idx], v[:, idx], a[idx], b[idx], n + 2)
    # the next round reads window columns n - 1 .. n + 1 and the state of row n - 1
    assert torch.equal(conv[1, :, n - 1 : n + 2], cconv[1, :, n - 1 : n + 2])
    assert torch.equal(conv[1, :, n - 1 : n + 2], torch.cat([hist, x[idx].t()], 1)[:, -3:])
    torch.testing.assert_close(pool[int(sl[0, n - 1])], cpool[int(csl[0, n - 1])], atol=0, rtol=1e-6)
