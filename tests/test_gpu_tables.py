"""Tree tables on the GPU against the oracle, bit for bit: the verify stage (vllm/verify_layout.py:31-86), the
link -> parent derivation with window codes and path table (kernels/gdn_tree.py:93-237) and the tail-mask words
(kernels/verify_prep.py:23-45)."""

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import tables as ot
from workloads import seeded_tree

pytestmark = pytest.mark.gpu

PARENTS = [-1, 0, 0, 1, 1, 2, 3]


def _random_parents(width, seed):
    gen = torch.Generator().manual_seed(seed)
    return [-1] + [int(torch.randint(0, r, (1,), generator=gen)) for r in range(1, width)]


@pytest.mark.parametrize(
    "parents", [PARENTS, _random_parents(16, 1), _random_parents(16, 2), _random_parents(64, 3), [-1, 0, 1, 2, 3],
                # not parent first (a forward parent, one past the row range, a negative one): the serial update order
                [-1, 3, 0, 1, 9, 2, -5]]
)
@pytest.mark.parametrize("tree", [True, False])
def test_stage_matches_oracle(dev, parents, tree):
    from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage

    announce(f"stage width={len(parents)} tree={tree}")
    width, num_reqs, slots = len(parents), 3, 8
    store = TreeStore(slots, width, dev)
    rows = torch.tensor(parents, dtype=torch.int32)
    store.parents[:] = rows.to(dev)
    stage = VerifyStage(slots, slots * width, width, dev)
    widths = [width, max(1, width - 2), 1]  # a full tree, a prefix of it, a chain of one
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(widths)]), dtype=torch.int32)
    cu = qsl.clone()
    cu[-1] -= 0
    positions = torch.cat([100 + 7 * b + torch.arange(w) for b, w in enumerate(widths)]).to(torch.int64)
    idx = torch.tensor([2, 5, 0], dtype=torch.int32)
    pos_d = positions.to(dev)
    stage.stage(store, idx.to(dev), qsl.to(dev), cu.to(dev), pos_d, num_reqs, int(qsl[-1]), tree=tree)

    o_parents = np.zeros((slots, width), np.int32)
    o_parents[:] = -1
    o_parents[:, :width] = parents
    want = dict(
        stage_parents=np.zeros((slots, width), np.int32), stage_anc=np.zeros((slots, 3, width), np.int32),
        stage_mask=np.ones((slots, width), np.int64), context_lens=np.zeros(slots, np.int32),
        slot_parents=np.zeros((slots, width), np.int32), slot_depths=np.zeros((slots, width), np.int32),
    )
    pos = positions.numpy().copy()
    ot.stage_tree(o_parents, idx.numpy(), qsl.numpy(), cu.numpy(), pos, want["stage_parents"], want["stage_anc"],
                  want["stage_mask"], want["context_lens"], want["slot_parents"], want["slot_depths"], num_reqs, width,
                  tree)
    torch.cuda.synchronize()
    assert stage.parents[:num_reqs].cpu().numpy().tolist() == want["stage_parents"][:num_reqs].tolist()
    assert stage.ancestors[:num_reqs].cpu().numpy().tolist() == want["stage_anc"][:num_reqs].tolist()
    assert stage.masks[:num_reqs].cpu().numpy().tolist() == want["stage_mask"][:num_reqs].tolist()
    assert stage.context_lens[:num_reqs].cpu().numpy().tolist() == want["context_lens"][:num_reqs].tolist()
    for s in idx.tolist():
        assert stage.slot_parents[s].cpu().tolist() == want["slot_parents"][s].tolist()
        assert stage.slot_depths[s].cpu().tolist() == want["slot_depths"][s].tolist()
    assert pos_d.cpu().numpy().tolist() == pos.tolist()
    # the same launch saved the chain positions the stage rewrote
    assert stage.chain_positions[: int(qsl[-1])].cpu().tolist() == positions.tolist()


def _links_case(widths, seed, pad_rows=()):
    rng = np.random.default_rng(seed)
    W = max(widths)
    B = len(widths)
    nxt = np.full((B, W), -1, np.int64)
    sib = np.full((B, W), -1, np.int64)
    parents = []
    for b, w in enumerate(widths):
        p = seeded_tree(rng, w)
        parents.append(p)
        n, s = ot.links_from_parents(p, W)
        nxt[b], sib[b] = n, s
    par = np.full((B, W), 5, np.int64)  # pad rows keep these
    csi = np.arange(B, dtype=np.int32) + 3
    for b in pad_rows:
        csi[b] = -1
    qsl = np.concatenate([[0], np.cumsum(widths)]).astype(np.int32)
    return parents, nxt, sib, par, csi, qsl, W


@pytest.mark.parametrize("widths,pad_rows", [([7], ()), ([16, 16, 11], ()), ([16, 5, 16], (1,)), ([33, 2], ())])
@pytest.mark.parametrize("link_dtype", [torch.int64, torch.int32])
def test_ancestors_and_paths_match_oracle(dev, widths, pad_rows, link_dtype):
    from eagle_harness.kernels.gdn_tree import gdn_tree_ancestors, gdn_tree_paths_buffer

    announce(f"ancestors widths={widths} pad={pad_rows} {link_dtype}")
    parents, nxt, sib, par, csi, qsl, W = _links_case(widths, seed=sum(widths), pad_rows=pad_rows)
    B = len(widths)
    want_par, want_anc = par.copy(), np.zeros((B, 3, W), np.int32)
    want_paths = np.zeros((B, W, 2 + W), np.int32)
    ot.gdn_tree_ancestors(nxt, sib, want_par, csi, W, want_anc, qsl, want_paths)
    g_par = torch.from_numpy(par).to(link_dtype).to(dev)
    g_anc = torch.zeros(B, 3, W, dtype=torch.int32, device=dev)
    g_paths = gdn_tree_paths_buffer(B, W, dev)
    gdn_tree_ancestors(
        torch.from_numpy(nxt).to(link_dtype).to(dev), torch.from_numpy(sib).to(link_dtype).to(dev), g_par,
        torch.from_numpy(csi).to(dev), W, g_anc, query_start_loc=torch.from_numpy(qsl).to(dev), paths=g_paths,
    )
    torch.cuda.synchronize()
    assert g_par.cpu().numpy().tolist() == want_par.tolist()
    live = [b for b in range(B) if b not in pad_rows]
    assert g_anc.cpu().numpy()[live].tolist() == want_anc[live].tolist()
    assert g_paths.cpu().numpy().tolist() == want_paths.tolist()
    # the derived parents are the trees' parents (links round trip)
    for b in live:
        assert g_par[b, 1 : widths[b]].cpu().tolist() == parents[b][1:]


def _signed(word: int) -> int:
    return word - (1 << 64) if word >= 1 << 63 else word


@pytest.mark.parametrize("width,kv_len", [(1, 7), (5, 40), (16, 3000), (64, 5000), (16, 70000)])
def test_tail_words_match_oracle(dev, width, kv_len):
    from eagle_harness.kernels.verify_prep import tree_tail_words

    announce(f"tail words width={width} kv_len={kv_len}")
    gen = torch.Generator().manual_seed(width)
    mask = torch.randint(0, 2, (width * kv_len,), generator=gen, dtype=torch.uint8).bool()
    committed = torch.tensor([kv_len - width], dtype=torch.int64)
    tail = torch.full((width + 1,), 7, dtype=torch.int64, device=dev)
    tree_tail_words(mask.to(dev), committed.to(dev), tail, width)
    want = ot.tree_tail_words(mask.numpy(), kv_len - width, width)
    rows = mask.view(width, kv_len)[:, kv_len - width :].int().tolist()
    closed = [_signed(sum(bit << j for j, bit in enumerate(row))) for row in rows]
    assert tail[:width].cpu().tolist() == want == closed
    assert int(tail[width]) == 7

