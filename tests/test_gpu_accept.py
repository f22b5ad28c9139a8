"""Greedy acceptance on the GPU against the oracle, bit for bit: first-index argmax over the vocab, the tree walk
(vllm/tree_accept.py:45-115) with the reference test's planted paths, the bs1 accept tail (kernels/accept_tail.py:
56-187), row compaction and the vLLM state commit (vllm/gdn_tree_verify.py:186-322)."""

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import accept as oacc
from oracle import commit as ocm
from oracle.tables import links_from_parents
from workloads import seeded_tree

pytestmark = pytest.mark.gpu

W, VOCAB, SLOTS = 8, 64, 4
# Two requests (state slots 3 and 1): accepted rows [0, 2, 5, 7] and [0, 1, 4] (tests/test_tree_rejection_sampler.py:28)
TREES = [([-1, 0, 0, 1, 1, 2, 3, 5], [0, 2, 5, 7], 3), ([-1, 0, 0, 1, 1], [0, 1, 4], 1)]


def _planted():
    gen = torch.Generator().manual_seed(7)
    sizes = [len(p) for p, _, _ in TREES]
    logits = torch.randn(sum(sizes), VOCAB, generator=gen)
    drafted = torch.randint(0, VOCAB, (sum(sizes),), generator=gen)
    start = 0
    for (parents, path, _), size in zip(TREES, sizes):
        argmax = logits[start : start + size].argmax(-1)
        for row in range(1, size):
            if drafted[start + row] == argmax[parents[row]]:
                drafted[start + row] = (argmax[parents[row]] + 1) % VOCAB
        for parent, child in zip(path, path[1:]):
            drafted[start + child] = argmax[parent]
        start += size
    return logits, drafted, sizes


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_argmax_first_index_on_ties(dev, dtype):
    from eagle_harness.vllm.tree_accept import greedy_targets

    announce(f"argmax {dtype}")
    gen = torch.Generator().manual_seed(3)
    for rows, vocab in ((5, 64), (3, 151936), (2, 1001)):
        logits = torch.randn(rows, vocab, generator=gen).to(dtype)
        logits[0, 17] = logits[0, 900 % vocab] = 50.0  # a tie: the first index wins
        got = greedy_targets(logits.to(dev)).cpu()
        assert got.tolist() == oacc.argmax_rows(logits).tolist() == logits.float().argmax(-1).tolist()


def test_accept_tree_planted_paths(dev):
    from eagle_harness.vllm.tree_accept import accept_tree, greedy_targets
    from eagle_harness.vllm.verify_layout import TreeStore

    announce("accept tree planted")
    logits, drafted, sizes = _planted()
    parents = torch.full((SLOTS, W), -1, dtype=torch.int32)
    for p, _, slot in TREES:
        parents[slot, : len(p)] = torch.tensor(p, dtype=torch.int32)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int32)
    idx = torch.tensor([slot for _, _, slot in TREES], dtype=torch.int32)
    store = TreeStore(SLOTS, W, dev)
    target = greedy_targets(logits.to(dev))
    sampled, num = accept_tree(target, drafted.to(dev), cu.to(dev), idx.to(dev), parents.to(dev), store)
    torch.cuda.synchronize()
    path_o = torch.zeros(SLOTS, W, dtype=torch.int32)
    plen_o = torch.ones(SLOTS, dtype=torch.int32)
    s_o, n_o = oacc.accept_tree(logits.argmax(-1), drafted, cu, idx, parents, path_o, plen_o, W)
    for b, (_, path, slot) in enumerate(TREES):
        assert int(num[b]) == len(path) == int(n_o[b])
        assert store.path[slot, : len(path)].cpu().tolist() == path == path_o[slot, : len(path)].tolist()
        assert int(store.path_len[slot]) == len(path)
        assert sampled[b, : len(path)].cpu().tolist() == s_o[b, : len(path)].tolist()
        assert sampled[b, : len(path)].cpu().tolist() == [int(logits[cu[b] + r].argmax()) for r in path]


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_accept_tail_matches_oracle(dev, seed):
    from eagle_harness.kernels.accept_tail import accept_tail, compact_rows

    announce(f"accept tail seed={seed}")
    rng = np.random.default_rng(seed)
    width, depth = 16, 12
    parents = seeded_tree(rng, width)
    nxt, sib = links_from_parents(parents, width)
    target = torch.from_numpy(rng.integers(0, 20, width)).long()
    cand = torch.from_numpy(rng.integers(0, 20, width)).long()
    node = 0  # plant a few matches down the first-child chain
    for _ in range(3):
        child = nxt[node]
        if child < 0:
            break
        cand[child] = target[node]
        node = child
    args = (target, cand, torch.arange(width).long()[None], torch.tensor([nxt]).long(), torch.tensor([sib]).long(),
            torch.tensor([40]).long(), torch.from_numpy(rng.integers(0, 1000, width)).long(),
            torch.from_numpy(rng.integers(0, 5000, (2, 80))).int(), torch.tensor([1]).long())
    want = oacc.accept_tail(*args, depth)
    got = accept_tail(*[a.to(dev) for a in args], depth)
    torch.cuda.synchronize()
    for name in want:
        assert getattr(got, {"bonus_tokens": "bonus_tokens"}.get(name, name)).cpu().tolist() == want[name].tolist(), name
    rows = torch.randn(width, 300, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    got_rows = compact_rows(rows.to(dev), got.accept_index).cpu()
    assert torch.equal(got_rows, oacc.compact_rows(rows, want["accept_index"]))


@pytest.mark.parametrize("ssm_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout,conv_dtype,dim", [("rows", torch.bfloat16, 40), ("rows", torch.bfloat16, 600),
                                                   ("rows", torch.float32, 300), ("columns", torch.bfloat16, 600)])
def test_linear_state_commit_matches_oracle(dev, ssm_dtype, layout, conv_dtype, dim):
    """Window caches with contiguous rows (moved as whole 16-byte pieces; rows of 10 elements, so pieces straddle
    channels; blocks of 256 / 128 channels and a partial last block) and column-major ones (moved element-wise)."""
    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit

    announce(f"state commit {ssm_dtype} {layout} {conv_dtype} dim {dim}")
    gen = torch.Generator().manual_seed(4)
    layers, reqs, width, hv, d = 2, 3, 8, 2, 16
    slots_n = 1 + reqs * width
    if layout == "rows":
        convs = [torch.randn(slots_n, dim, 2 + width, generator=gen).to(conv_dtype) for _ in range(layers)]
    else:
        convs = [torch.randn(slots_n, 2 + width, dim, generator=gen).to(conv_dtype).transpose(1, 2)
                 for _ in range(layers)]
    ssms = [torch.randn(slots_n, hv, d, d, generator=gen).to(ssm_dtype) for _ in range(layers)]
    slots = (1 + torch.arange(reqs * width, dtype=torch.int32)).view(reqs, width)
    slots[2] = 0  # a padded request
    idx = torch.tensor([2, 0, 1], dtype=torch.int32)
    path = torch.zeros(reqs, width, dtype=torch.int32)
    plen = torch.ones(reqs, dtype=torch.int32)
    for s, p in ((2, [0, 2, 5, 7]), (0, [0, 1, 2]), (1, [0, 3])):
        path[s, : len(p)] = torch.tensor(p, dtype=torch.int32)
        plen[s] = len(p)
    want_c, want_s = [c.clone() for c in convs], [s.clone() for s in ssms]
    ocm.linear_state_commit(want_c, want_s, [slots] * layers, idx, path, plen)
    gc, gs = [c.to(dev) for c in convs], [s.to(dev) for s in ssms]
    commit = LinearStateCommit(list(zip(gc, gs)), [slots.to(dev)] * layers, dev)
    commit.commit(idx.to(dev), path.to(dev), plen.to(dev))
    torch.cuda.synchronize()
    for layer in range(layers):
        assert torch.equal(gc[layer].cpu(), want_c[layer])
        assert torch.equal(gs[layer].cpu(), want_s[layer])


@pytest.mark.parametrize("dim_first", [True, False])
def test_linear_state_commit_from_layer_objects(dev, dim_first):
    """The speculator builds the commit from vLLM layer objects (``kv_cache`` = [conv state, ssm state]) with the conv
    state in vLLM's own layout: [slots, dim, len] when dim-first, else [slots, len, dim], which the commit views
    dim-first (vllm/gdn_tree_verify.py:261-265). Both layouts land bit for bit on the oracle's moves."""
    from types import SimpleNamespace

    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit

    announce(f"state commit from layer objects, dim_first={dim_first}")
    gen = torch.Generator().manual_seed(11)
    layers, reqs, width, dim = 3, 4, 8, 520
    slots_n = 1 + reqs * width
    raw = [torch.randn((slots_n, dim, 2 + width) if dim_first else (slots_n, 2 + width, dim), generator=gen)
           .to(torch.bfloat16) for _ in range(layers)]
    ssms = [torch.randn(slots_n, 2, 16, 16, generator=gen) for _ in range(layers)]
    slots = (1 + torch.arange(reqs * width, dtype=torch.int32)).view(reqs, width)
    idx = torch.tensor([1, 3, 0, 2], dtype=torch.int32)
    path = torch.zeros(reqs, width, dtype=torch.int32)
    plen = torch.ones(reqs, dtype=torch.int32)
    for s, p in ((0, [0, 2, 5, 7]), (1, [0, 1, 2]), (2, [0, 3, 6]), (3, [0])):
        path[s, : len(p)] = torch.tensor(p, dtype=torch.int32)
        plen[s] = len(p)
    view = (lambda c: c) if dim_first else (lambda c: c.transpose(1, 2))
    want_c, want_s = [view(c).clone() for c in raw], [s.clone() for s in ssms]
    ocm.linear_state_commit(want_c, want_s, [slots] * layers, idx, path, plen)
    objs = [SimpleNamespace(kv_cache=[c.to(dev), s.to(dev)]) for c, s in zip(raw, ssms)]
    commit = LinearStateCommit(objs, [slots.to(dev)] * layers, dev, dim_first=dim_first)
    assert commit.dim == dim
    commit.commit(idx.to(dev), path.to(dev), plen.to(dev))
    torch.cuda.synchronize()
    for layer in range(layers):
        assert torch.equal(view(objs[layer].kv_cache[0]).cpu(), want_c[layer])
        assert torch.equal(objs[layer].kv_cache[1].cpu(), want_s[layer])


def _linked_tree(width, rng):
    """A random tree as first-child / next-sibling links (about half the nodes continue a chain), draft tokens in a
    small vocabulary and a target that follows a child's draft 80 % of the time (the shape of
    tests/test_accept_tail_gpu.py:23-39)."""
    parent = [-1] + [rng.randrange(0, i) if rng.random() < 0.5 else i - 1 for i in range(1, width)]
    kids = [[j for j in range(width) if parent[j] == i] for i in range(width)]
    first = [c[0] if c else -1 for c in kids]
    sibling = [-1] * width
    for c in kids:
        for x, y in zip(c, c[1:]):
            sibling[x] = y
    cand = [rng.randrange(0, 6) for _ in range(width)]
    target = [cand[rng.choice(kids[i])] if kids[i] and rng.random() < 0.8 else rng.randrange(0, 6) for i in range(width)]
    return cand, first, sibling, target


@pytest.mark.parametrize("width,depth", [(16, 12), (9, 8), (4, 4), (2, 2), (31, 12), (32, 32), (8, 1)])
def test_accept_tail_served_shapes(dev, width, depth):
    """The widths and depths the reference serves after its warm-up (tests/test_accept_tail_gpu.py:69-153):
    int64 tables, an out_cache_loc that is a slice of a slot list (8-byte aligned), compaction into the rows of a
    wider hidden buffer; every field against the oracle."""
    import random

    from eagle_harness.kernels.accept_tail import accept_tail, compact_rows, warm_up

    announce(f"accept tail width={width} depth={depth}")
    hidden = torch.zeros(64, 5120, dtype=torch.bfloat16, device=dev)
    warm_up(hidden, torch.bfloat16)
    rng = random.Random(7 + width * 100 + depth)
    cand, first, sibling, target = _linked_tree(width, rng)
    long = dict(dtype=torch.int64)
    slots_all = torch.tensor([rng.randrange(1, 1 << 20) for _ in range(width + 1)], **long)
    args = (torch.tensor(target, **long), torch.tensor(cand, **long), torch.arange(width, **long).reshape(1, width),
            torch.tensor(first, **long).reshape(1, width), torch.tensor(sibling, **long).reshape(1, width),
            torch.tensor([rng.randrange(1, 150)], **long), slots_all[1:],
            torch.tensor([[rng.randrange(1, 1 << 20) for _ in range(200 + width)] for _ in range(3)], dtype=torch.int32),
            torch.tensor([1], **long))
    want = oacc.accept_tail(*args, depth)
    slots_dev = slots_all.to(dev)
    dev_args = [x.to(dev) for x in args]
    dev_args[6] = slots_dev[1:]  # the slice itself, not a copy: its data starts 8 bytes into the allocation
    got = accept_tail(*dev_args, depth)
    rows = torch.randn(width, 5120, generator=torch.Generator().manual_seed(width)).to(torch.bfloat16)
    compact_rows(rows.to(dev), got.accept_index, out=hidden[:width])
    torch.cuda.synchronize()
    for name in want:
        assert getattr(got, name).cpu().tolist() == want[name].tolist(), name
    assert torch.equal(hidden[:width].cpu(), oacc.compact_rows(rows, want["accept_index"]))
    assert not hidden[width:].any().item()


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the capture records nothing: it reads a flag
def test_graph_capture_stages_the_tree_path_whatever_was_staged_last(dev):
    """The layers ask ``VerifyStage.verifying``; it is true while a graph is captured even when the last staged batch
    was a chain (tests/test_gpu_kernels.py:113-125)."""
    from eagle_harness.vllm.verify_layout import VerifyStage

    announce("verify stage graph capture")
    stage = VerifyStage(2, 16, 8, dev)
    stage.active = False
    assert not stage.verifying
    seen = []
    torch.zeros(1, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        seen.append(stage.verifying)
    assert seen == [True]
    stage.active = True
    assert stage.verifying
