"""Pins of the CPU oracle of vLLM's round commit (oracle/round_commit.py): the reference tests' known answers for the
KV compaction (tests/test_gpu_kernels.py:67-111: both cache layouts, table blocks of 1 and 4 cache blocks) and for
chainize (tests/test_tree_round_kernels.py:92-123), and the property the GPU kernel relies on — the ordered moves
equal one gather from the cache as it was (a row is never read after an earlier move wrote it)."""

import numpy as np
import pytest
import torch

from oracle import round_commit as orc
from workloads import committed_path, seeded_tree

W = 8


@pytest.mark.parametrize("slot_major", [False, True])
@pytest.mark.parametrize("blocks_per_table_block", [1, 4])
def test_kv_compaction_known_answer(slot_major, blocks_per_table_block):
    block_size, heads, d, num_layers = 16, 4, 8, 2
    table_block_size = block_size * blocks_per_table_block
    num_cache_blocks = 12 * blocks_per_table_block
    gen = torch.Generator().manual_seed(0)
    shape = (num_cache_blocks, block_size, heads, 2 * d) if slot_major else (num_cache_blocks, heads, block_size, 2 * d)
    raw = [torch.randn(shape, generator=gen).to(torch.bfloat16) for _ in range(num_layers)]
    caches = [r.transpose(1, 2) if slot_major else r for r in raw]
    before = [c.clone() for c in caches]
    table = torch.tensor([[3, 1, 7, 2, 5, 9]], dtype=torch.int32)
    path = torch.zeros(2, 7, dtype=torch.int32)
    path_len = torch.ones(2, dtype=torch.int32)
    path[1, :4] = torch.tensor([0, 2, 5, 6], dtype=torch.int32)
    path_len[1] = 4
    context, width = 20 * blocks_per_table_block + 9, 7
    qsl = torch.tensor([0, width], dtype=torch.int32)
    orc.compact_kv(caches, [table] * num_layers, [table_block_size] * num_layers, torch.ones(1, dtype=torch.int32),
                   qsl, qsl, torch.tensor([context + width], dtype=torch.int32), path, path_len)

    def where(token):
        block = int(table[0, token // table_block_size]) * blocks_per_table_block
        return block + token % table_block_size // block_size, token % block_size

    for layer in range(num_layers):
        for j, row in enumerate([0, 2, 5, 6]):
            (sb, ss), (db, ds) = where(context + row), where(context + j)
            assert torch.equal(caches[layer][db, :, ds], before[layer][sb, :, ss])
        untouched = torch.ones(num_cache_blocks, block_size, dtype=torch.bool)
        for j in range(1, 4):
            untouched[where(context + j)] = False
        assert torch.equal(caches[layer].transpose(1, 2)[untouched], before[layer].transpose(1, 2)[untouched])


def test_chainize_known_answer():
    path = torch.zeros(4, W, dtype=torch.int32)
    path_len = torch.ones(4, dtype=torch.int32)
    path[2, :4] = torch.tensor([0, 2, 5, 7], dtype=torch.int32)
    path_len[2] = 4
    context = 30
    qsl = torch.tensor([0, W, W + 1], dtype=torch.int32)
    cu = torch.tensor([0, W, W + 1], dtype=torch.int32)  # the second request is a plain decode
    seq_lens = torch.tensor([context + W, 50], dtype=torch.int32)
    input_ids = torch.arange(100, 100 + W + 1, dtype=torch.int64)
    positions = torch.tensor([context + d for d in (0, 1, 1, 2, 2, 2, 3, 3)] + [49], dtype=torch.int64)
    sampled = torch.tensor([[11, 12, 13, 14] + [0] * 4, [9] + [0] * 7], dtype=torch.int64)
    src = torch.arange(W + 1, dtype=torch.int64)
    orc.chainize(input_ids, positions, src, idx_mapping=torch.tensor([2, 0]), query_start_loc=qsl, cu_num_logits=cu,
                 seq_lens=seq_lens, path=path, path_len=path_len, sampled=sampled, width=W)
    assert src[:W].tolist() == [0, 2, 5, 7, 4, 5, 6, 7] and src[W] == W
    assert positions[:W].tolist() == [context + r for r in range(W)] and positions[W] == 49
    assert input_ids[:4].tolist() == [100, 11, 12, 13]
    assert input_ids[4:W].tolist() == [104, 105, 106, 107]


def test_ordered_moves_equal_one_gather():
    """For any parent-first tree and accepted path, moving rows one at a time in path order lands what a single
    gather from the untouched cache gives: row context + j <- row context + path[j]."""
    rng = np.random.default_rng(3)
    for trial in range(20):
        width = int(rng.integers(2, 17))
        parents = seeded_tree(rng, width)
        path_rows = committed_path(parents, int(rng.integers(1, 13)))
        block_size, heads, d = 4, 2, 3
        cache = torch.randn(16, heads, block_size, 2 * d, generator=torch.Generator().manual_seed(trial))
        table = torch.tensor([list(rng.permutation(16))], dtype=torch.int32)
        context = int(rng.integers(0, 16 * block_size - width))
        path = torch.zeros(1, width, dtype=torch.int32)
        path[0, : len(path_rows)] = torch.tensor(path_rows, dtype=torch.int32)
        path_len = torch.tensor([len(path_rows)], dtype=torch.int32)
        qsl = torch.tensor([0, width], dtype=torch.int32)
        before = cache.clone()
        orc.compact_kv([cache], [table], [block_size], torch.zeros(1, dtype=torch.int32), qsl, qsl,
                       torch.tensor([context + width], dtype=torch.int32), path, path_len)

        def where(pos):
            token = int(table[0, pos // block_size]) * block_size + pos % block_size
            return token // block_size, token % block_size

        want = before.clone()
        for j, row in enumerate(path_rows):
            (sb, ss), (db, ds) = where(context + row), where(context + j)
            want[db, :, ds] = before[sb, :, ss]
        assert torch.equal(cache, want)


def test_requests_that_are_not_trees_are_left_alone():
    """One row, or fewer logits than rows (:26-29): nothing moves, nothing is rewritten."""
    cache = torch.randn(4, 1, 4, 4, generator=torch.Generator().manual_seed(1))
    before = cache.clone()
    table = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 3]], dtype=torch.int32)
    path = torch.tensor([[0, 2, 3, 0], [0, 1, 0, 0]], dtype=torch.int32)
    path_len = torch.tensor([3, 2], dtype=torch.int32)
    qsl = torch.tensor([0, 4, 5], dtype=torch.int32)
    cu = torch.tensor([0, 3, 4], dtype=torch.int32)  # request 0: 4 rows, 3 logits; request 1: one row
    seq = torch.tensor([10, 8], dtype=torch.int32)
    orc.compact_kv([cache], [table], [4], torch.tensor([0, 1]), qsl, cu, seq, path, path_len)
    assert torch.equal(cache, before)
    ids, pos, src = torch.arange(5), torch.arange(5), torch.arange(5)
    orc.chainize(ids, pos, src, idx_mapping=torch.tensor([0, 1]), query_start_loc=qsl, cu_num_logits=cu, seq_lens=seq,
                 path=path, path_len=path_len, sampled=torch.zeros(2, 4, dtype=torch.int64), width=4)
    assert ids.tolist() == pos.tolist() == src.tolist() == list(range(5))
