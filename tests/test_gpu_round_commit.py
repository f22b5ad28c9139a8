"""vLLM's round commit on the GPU against the oracle (vllm/round_commit.py): the KV compaction of accepted rows in the
reference test's scenario (tests/test_gpu_kernels.py:67-111: both cache layouts, table blocks of 1 and 4 cache blocks)
and on seeded batches (trees, decodes and prefills mixed, several layers, head dims on and off the 16-byte path, bf16
and fp16), and chainize in the reference test's scenario (tests/test_tree_round_kernels.py:92-123) and on seeded
batches with int32 and int64 rows. Integer and byte work: bit-exact."""

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import round_commit as orc
from workloads import committed_path, seeded_tree

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("slot_major", [False, True])
@pytest.mark.parametrize("blocks_per_table_block", [1, 4])
def test_kv_compaction_reference_scenario(dev, slot_major, blocks_per_table_block):
    from eagle_harness.vllm.round_commit import KvCompactor
    from eagle_harness.vllm.verify_layout import TreeStore

    announce(f"kv compaction reference scenario slot_major={slot_major} table blocks={blocks_per_table_block}")
    block_size, heads, d, num_layers = 16, 4, 8, 2
    table_block_size = block_size * blocks_per_table_block
    num_cache_blocks = 12 * blocks_per_table_block
    gen = torch.Generator().manual_seed(0)
    shape = (num_cache_blocks, block_size, heads, 2 * d) if slot_major else (num_cache_blocks, heads, block_size, 2 * d)
    raw = [torch.randn(shape, generator=gen).to(torch.bfloat16).to(dev) for _ in range(num_layers)]
    caches = [r.transpose(1, 2) if slot_major else r for r in raw]
    before = [c.clone() for c in caches]
    table = torch.tensor([[3, 1, 7, 2, 5, 9]], dtype=torch.int32, device=dev)
    store = TreeStore(2, 7, dev)
    store.path[1, :4] = torch.tensor([0, 2, 5, 6], dtype=torch.int32, device=dev)
    store.path_len[1] = 4
    context, width = 20 * blocks_per_table_block + 9, 7
    qsl = torch.tensor([0, width], dtype=torch.int32, device=dev)
    seq = torch.tensor([context + width], dtype=torch.int32, device=dev)
    ones = torch.ones(1, dtype=torch.int32, device=dev)
    KvCompactor(caches, [table] * num_layers, [table_block_size] * num_layers, dev).compact(
        ones, qsl, qsl, seq, store.path, store.path_len)
    torch.cuda.synchronize()
    want = [c.cpu() for c in before]
    orc.compact_kv(want, [table.cpu()] * num_layers, [table_block_size] * num_layers, ones.cpu(), qsl.cpu(), qsl.cpu(),
                   seq.cpu(), store.path.cpu(), store.path_len.cpu())

    def where(token):
        block = int(table[0, token // table_block_size]) * blocks_per_table_block
        return block + token % table_block_size // block_size, token % block_size

    for layer in range(num_layers):
        got = caches[layer].cpu()
        assert torch.equal(got, want[layer])
        for j, row in enumerate([0, 2, 5, 6]):
            (sb, ss), (db, ds) = where(context + row), where(context + j)
            assert torch.equal(got[db, :, ds], before[layer][sb, :, ss].cpu())


@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (64, torch.float16), (5, torch.bfloat16)])
def test_kv_compaction_seeded_batches(dev, d, dtype):
    """A batch of trees, decodes and prefills over shuffled, shared-nothing blocks, 3 layers, several heads; the
    head dim of 5 takes the element-wise path."""
    from eagle_harness.vllm.round_commit import KvCompactor

    announce(f"kv compaction seeded d={d} {dtype}")
    rng = np.random.default_rng(d)
    B, heads, block_size, layers, width = 12, 3, 16, 3, 16
    max_blocks = 12
    num_blocks = B * max_blocks + 5
    perm = rng.permutation(num_blocks)
    table = torch.tensor(perm[: B * max_blocks].reshape(B, max_blocks), dtype=torch.int32)
    qsl, cu, seq = [0], [0], []
    paths, plen = torch.zeros(B + 2, width, dtype=torch.int32), torch.ones(B + 2, dtype=torch.int32)
    for b in range(B):
        kind = b % 4
        w = width if kind < 2 else (1 if kind == 2 else 5)  # trees, a decode, a prefill (5 rows, 1 logit)
        qsl.append(qsl[-1] + w)
        cu.append(cu[-1] + (w if kind < 2 else 1))
        seq.append(int(rng.integers(w + 1, max_blocks * block_size - 1)))
        parents = seeded_tree(rng, width)
        p = committed_path(parents, int(rng.integers(1, 13)))
        paths[B - b, : len(p)] = torch.tensor(p, dtype=torch.int32)
        plen[B - b] = len(p)
    idx = torch.tensor([B - b for b in range(B)], dtype=torch.int32)  # state slots in reverse
    gen = torch.Generator().manual_seed(d)
    caches = [torch.randn(num_blocks, heads, block_size, 2 * d, generator=gen).to(dtype) for _ in range(layers)]
    want = [c.clone() for c in caches]
    qsl_t, cu_t, seq_t = (torch.tensor(x, dtype=torch.int32) for x in (qsl, cu, seq))
    orc.compact_kv(want, [table] * layers, [block_size] * layers, idx, qsl_t, cu_t, seq_t, paths, plen)
    gc = [c.to(dev) for c in caches]
    KvCompactor(gc, [table.to(dev)] * layers, [block_size] * layers, dev).compact(
        idx.to(dev), qsl_t.to(dev), cu_t.to(dev), seq_t.to(dev), paths.to(dev), plen.to(dev))
    torch.cuda.synchronize()
    for layer in range(layers):
        assert torch.equal(gc[layer].cpu(), want[layer])
    assert any(not torch.equal(w, c) for w, c in zip(want, caches))  # something moved


def test_chainize_reference_scenario(dev):
    from eagle_harness.vllm.round_commit import chainize
    from eagle_harness.vllm.verify_layout import TreeStore

    announce("chainize reference scenario")
    W = 8
    store = TreeStore(4, W, dev)
    store.path[2, :4] = torch.tensor([0, 2, 5, 7], dtype=torch.int32, device=dev)
    store.path_len[2] = 4
    context = 30
    qsl = torch.tensor([0, W, W + 1], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, W, W + 1], dtype=torch.int32, device=dev)
    seq_lens = torch.tensor([context + W, 50], dtype=torch.int32, device=dev)
    input_ids = torch.arange(100, 100 + W + 1, dtype=torch.int64, device=dev)
    positions = torch.tensor([context + d for d in (0, 1, 1, 2, 2, 2, 3, 3)] + [49], dtype=torch.int64, device=dev)
    sampled = torch.tensor([[11, 12, 13, 14] + [0] * 4, [9] + [0] * 7], dtype=torch.int64, device=dev)
    src = torch.arange(W + 1, dtype=torch.int64, device=dev)
    chainize(input_ids, positions, src, idx_mapping=torch.tensor([2, 0], dtype=torch.int64, device=dev),
             query_start_loc=qsl, cu_num_logits=cu, seq_lens=seq_lens, path=store.path, path_len=store.path_len,
             sampled=sampled, width=W)
    torch.cuda.synchronize()
    assert src[:W].tolist() == [0, 2, 5, 7, 4, 5, 6, 7] and src[W] == W
    assert positions[:W].tolist() == [context + r for r in range(W)] and positions[W] == 49
    assert input_ids[:4].tolist() == [100, 11, 12, 13]
    assert input_ids[4:W].tolist() == [104, 105, 106, 107]


@pytest.mark.parametrize("ids_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("width", [3, 16, 64])
def test_chainize_seeded_batches(dev, ids_dtype, width):
    """Trees of every accept length, decodes and prefills mixed, state slots permuted; int32 or int64 rows."""
    from eagle_harness.vllm.round_commit import chainize

    announce(f"chainize seeded width={width} {ids_dtype}")
    rng = np.random.default_rng(width)
    B = 10
    qsl, cu, seq = [0], [0], []
    paths, plen = torch.zeros(B, width, dtype=torch.int32), torch.ones(B, dtype=torch.int32)
    slots = rng.permutation(B)
    for b in range(B):
        kind = b % 3
        w = width if kind == 0 or b == 1 else (1 if kind == 1 else min(4, width))
        qsl.append(qsl[-1] + w)
        cu.append(cu[-1] + (w if kind == 0 or b == 1 else 1))
        seq.append(int(rng.integers(w, 5000)))
        parents = seeded_tree(rng, width)
        p = committed_path(parents, int(rng.integers(1, 13)))
        paths[slots[b], : len(p)] = torch.tensor(p, dtype=torch.int32)
        plen[slots[b]] = len(p)
    T = qsl[-1]
    ids = torch.tensor(rng.integers(0, 150000, T), dtype=ids_dtype)
    pos = torch.arange(T, dtype=torch.int64) * 7
    src = torch.arange(T, dtype=torch.int64)
    sampled = torch.tensor(rng.integers(0, 150000, (B, width)), dtype=torch.int64)
    kw = dict(idx_mapping=torch.tensor(slots, dtype=torch.int64), query_start_loc=torch.tensor(qsl, dtype=torch.int32),
              cu_num_logits=torch.tensor(cu, dtype=torch.int32), seq_lens=torch.tensor(seq, dtype=torch.int32),
              path=paths, path_len=plen, sampled=sampled)
    w_ids, w_pos, w_src = ids.clone(), pos.clone(), src.clone()
    orc.chainize(w_ids, w_pos, w_src, width=width, **kw)
    g_ids, g_pos, g_src = ids.to(dev), pos.to(dev), src.to(dev)
    chainize(g_ids, g_pos, g_src, width=width, **{k: v.to(dev) for k, v in kw.items()})
    torch.cuda.synchronize()
    assert torch.equal(g_ids.cpu(), w_ids) and torch.equal(g_pos.cpu(), w_pos) and torch.equal(g_src.cpu(), w_src)
    if width >= 16:
        assert not torch.equal(w_src, src)  # some tree moved (3-node trees accept a chain prefix: nothing moves)
