"""The verify path at the benchmark workloads' own sizes on the GPU, against the oracle.

- Batch 64 bf16 tree-verify attention (16-node seeded trees, 24 / 4 heads, D 256, page 16, permuted page tables,
  prefixes U[1024, 8192]) on the default streamed schedule: all 64 requests against the dense oracle.
- GDN layers at batch 256 and 512 (16 / 32 heads, K = V = 128, fp32 states, vLLM per-row slots): the tree conv over
  the 8192 qkv channels, the walk on q / k / v views of the conv output, then the accepted-path commit for seeded
  accept lengths U[1, 12]. Sampled requests against the oracle (conv, walk and commit; requests are independent, so
  the oracle runs on a compact copy of their slots); for every request, the committed state equals the walk's
  snapshot of the accepted node and the window columns follow the accepted path, bit for bit.
- The batch-512 quantized round's parts: fp8-e4m3 attention (prefixes U[512, 4096]) on sampled requests against
  the dequantised oracle; the greedy targets over 8192 x 151936 bf16 logits against ``torch.argmax`` on the device
  (first index on ties, bit for bit); the tree walk of all 512 requests against the oracle walk.

Tolerances: 2e-2 abs / 1e-2 rel for 16-bit outputs, 1e-5 abs / 1e-4 rel for fp32 states; bit for bit for indices,
moved bytes and argmax."""

import numpy as np
import pytest
import torch

from conftest import announce, assert_states_close
from oracle import accept as oacc
from oracle import attention as oa
from oracle import commit as ocm
from oracle import conv as oc
from oracle import recurrence as orr
from workloads import ATTN_B64, ATTN_B512_FP8, GdnShape, accept_paths, attention_inputs, gdn_inputs, seeded_tree

pytestmark = pytest.mark.gpu


def _close16(got, want):
    torch.testing.assert_close(got.float(), want.float(), atol=2e-2, rtol=1e-2)


def _attention_subset(inp, reqs):
    """The dense oracle over requests ``reqs`` only (CPU tensors; the caches stay whole, the tables are sliced)."""
    W = inp["max_query_len"]
    rows = torch.cat([torch.arange(r * W, (r + 1) * W) for r in reqs])
    idx = torch.tensor(reqs)
    out = torch.empty(len(reqs) * W, *inp["q"].shape[1:], dtype=inp["q"].dtype)
    kw = dict(k_scale=inp["k_scale"], v_scale=inp["v_scale"]) if "k_scale" in inp else {}
    oa.verify_attention(inp["q"][rows], inp["k_new"][rows], inp["v_new"][rows], inp["key_cache"], inp["value_cache"],
                        inp["block_table"][idx], inp["context_lens"][idx],
                        torch.arange(0, len(reqs) * W + 1, W, dtype=torch.int32), inp["masks"][idx], inp["scale"], out,
                        max_query_len=W, **kw)
    return rows, out


def _verify_attention(g, out, fp8=False):
    from eagle_harness.vllm.verify_attention import verify_attention

    kw = dict(k_scale=g["k_scale"], v_scale=g["v_scale"]) if fp8 else {}
    verify_attention(g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"],
                     g["context_lens"], g["query_start_loc"], g["masks"], g["scale"], out,
                     max_query_len=g["max_query_len"], **kw)
    torch.cuda.synchronize()


def test_attention_b64_every_request(dev):
    """Batch 64 x 16 nodes, 24 / 4 heads, D 256, bf16 pages of 16, prefixes U[1024, 8192]: all 64 requests."""
    announce("config attention b64 d256 l1024-8192, all requests")
    inp = attention_inputs(ATTN_B64, seed=0)
    assert int(inp["context_lens"].max()) > 7000 and int(inp["context_lens"].min()) < 2000
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = torch.full_like(g["q"], 7.0)
    _verify_attention(g, out)
    got = out.cpu()
    for lo in range(0, 64, 16):
        rows, want = _attention_subset(inp, list(range(lo, lo + 16)))
        _close16(got[rows], want)


def test_attention_b512_fp8_sampled_requests(dev):
    """Batch 512 x 16 nodes over fp8-e4m3 pages with per-(page, KV head) scales, prefixes U[512, 4096]: every output
    finite, 24 sampled requests (the longest and shortest among them) against the dequantised oracle."""
    announce("config attention b512 fp8 sampled")
    g = attention_inputs(ATTN_B512_FP8, seed=3, device=dev, fp8=True, gen_device=dev)
    out = torch.full_like(g["q"], 7.0)
    _verify_attention(g, out, fp8=True)
    assert bool(torch.isfinite(out.float()).all())
    lens = g["context_lens"].cpu()
    rng = np.random.default_rng(5)
    reqs = sorted({int(lens.argmax()), int(lens.argmin()), *map(int, rng.choice(512, 22, replace=False))})
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in g.items()}
    rows, want = _attention_subset(cpu, reqs)
    _close16(out.cpu()[rows], want)


def _gdn_subset(g, reqs, W):
    """CPU copy of requests ``reqs`` of a vLLM-layout GDN workload, with their slots renumbered into a compact pool
    (slot 0 stays the null block)."""
    n = len(reqs)
    rows = torch.cat([torch.arange(r * W, (r + 1) * W) for r in reqs])
    idx = torch.tensor(reqs)
    old = g["slots"].cpu()[idx]  # [n, W + 1]
    new = (1 + torch.arange(n * (W + 1), dtype=torch.int32)).view(n, W + 1)
    pool = torch.zeros(1 + n * (W + 1), *g["pool"].shape[1:], dtype=g["pool"].dtype)
    pool[new.flatten().long()] = g["pool"][old.flatten().long().to(g["pool"].device)].cpu()
    conv_state = torch.zeros(1 + n * (W + 1), *g["conv_state"].shape[1:], dtype=g["conv_state"].dtype)
    conv_state[new[:, 0].long()] = g["conv_state"][old[:, 0].long().to(g["conv_state"].device)].cpu()
    return dict(rows=rows, old_slots=old, slots=new, pool=pool, conv_state=conv_state, x=g["x"].cpu()[rows],
                a=g["a"].cpu()[rows], b=g["b"].cpu()[rows], parent_table=g["parent_table"].cpu()[idx],
                ancestors=g["ancestors"].cpu()[idx], num_accepted=g["num_accepted"].cpu()[idx],
                query_start_loc=torch.arange(0, n * W + 1, W, dtype=torch.int32))


@pytest.mark.parametrize("batch", [256, 512])
def test_gdn_layer_conv_walk_commit(dev, batch):
    """One GDN layer at batch ``batch`` x 16 nodes (the cfg2 heads): conv -> walk on views of the conv output ->
    commit of the seeded accepted paths."""
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit

    announce(f"config gdn layer batch={batch} conv+walk+commit")
    shape = GdnShape(batch, 16, 16, 32, 128, 128)
    W, H, HV, K, V = shape.width, shape.h, shape.hv, shape.k, shape.v
    g = gdn_inputs(shape, seed=21 + batch, device=dev, gen_device=dev)
    tokens, dim = batch * W, g["dim"]
    rng = np.random.default_rng(batch)
    reqs = sorted({0, batch - 1, *map(int, rng.choice(batch, 10, replace=False))})
    sub = _gdn_subset(g, reqs, W)  # before anything runs: the initial states and windows

    slots = g["slots"]
    mixed = torch.empty(tokens, dim, dtype=torch.bfloat16, device=dev)
    gdn_tree_conv1d_update(g["x"].t()[None], g["conv_state"], g["conv_weight"], None, "silu", slots[:, 0].contiguous(),
                           None, None, g["ancestors"], pad_slot_id=0, out=mixed.t()[None],
                           num_accepted_tokens=g["num_accepted"], query_start_loc=g["query_start_loc"])
    q, k, v = (mixed[:, lo:hi] for lo, hi in ((0, H * K), (H * K, 2 * H * K), (2 * H * K, dim)))
    out = gdn_tree_recurrent_update(
        g["A_log"], g["dt_bias"], q.view(1, tokens, H, K), k.view(1, tokens, H, K), v.view(1, tokens, HV, V), g["a"],
        g["b"], initial_state_source=g["pool"], initial_state_indices=slots, cu_seqlens=g["query_start_loc"],
        intermediate_states_buffer=g["pool"], intermediate_state_indices=slots,
        retrieve_parent_token=g["parent_table"], num_accepted_tokens=g["num_accepted"], pad_slot_id=0)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())

    # the oracle on the sampled requests: the conv on their x, the walk on the kernel's own conv output
    n = len(reqs)
    s_conv = sub["conv_state"].clone()
    o_conv = torch.zeros(n * W, dim, dtype=torch.bfloat16)
    oc.gdn_tree_conv1d_update(sub["x"].t()[None], s_conv, g["conv_weight"].cpu(), None, "silu", sub["slots"][:, 0],
                              None, None, sub["ancestors"], pad_slot_id=0, out=o_conv.t()[None],
                              num_accepted_tokens=sub["num_accepted"], query_start_loc=sub["query_start_loc"])
    mixed_sub = mixed.cpu()[sub["rows"]]
    _close16(mixed_sub, o_conv)
    old = sub["old_slots"]
    assert torch.equal(g["conv_state"][old[:, 0].long().to(dev)].cpu(), s_conv[sub["slots"][:, 0].long()])
    pool = sub["pool"].clone()
    o_walk = orr.gdn_tree_recurrent_update(
        g["A_log"].cpu(), g["dt_bias"].cpu(), mixed_sub[:, : H * K].reshape(1, n * W, H, K),
        mixed_sub[:, H * K : 2 * H * K].reshape(1, n * W, H, K), mixed_sub[:, 2 * H * K :].reshape(1, n * W, HV, V),
        sub["a"], sub["b"], initial_state_source=pool, initial_state_indices=sub["slots"],
        cu_seqlens=sub["query_start_loc"], intermediate_states_buffer=pool, intermediate_state_indices=sub["slots"],
        retrieve_parent_token=sub["parent_table"], num_accepted_tokens=sub["num_accepted"], pad_slot_id=0)
    _close16(out.cpu()[0, sub["rows"]], o_walk[0])
    snaps = g["pool"][old.flatten().long().to(dev)].cpu()
    assert_states_close(snaps, pool[sub["slots"].flatten().long()])

    # the commit of every request, checked against its own snapshots and windows taken just before it
    path, plen = accept_paths(g["parents"], seed=batch, width=W)
    last = path[torch.arange(batch), (plen - 1).long()]
    slots_cpu = slots.cpu()
    src_state = slots_cpu[torch.arange(batch), last.long()].long()
    dst_state = slots_cpu[torch.arange(batch), (plen - 1).long()].long()
    want_states = g["pool"][src_state.to(dev)].clone()
    windows = g["conv_state"][slots[:, 0].long()].clone()  # [B, dim, 3 + W]
    want_windows = windows.clone()
    for b in range(batch):  # column 2 + path[j] -> 2 + j, ascending j (a source never precedes its destination)
        for j in range(1, int(plen[b])):
            want_windows[b, :, 2 + j] = want_windows[b, :, 2 + int(path[b, j])]
    commit = LinearStateCommit([(g["conv_state"], g["pool"])], [slots], dev)
    commit.commit(torch.arange(batch, dtype=torch.int32, device=dev), path.to(dev), plen.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(g["pool"][dst_state.to(dev)], want_states)
    assert torch.equal(g["conv_state"][slots[:, 0].long()], want_windows)

    # and the oracle's commit on the sampled requests' compact copy: the same window bytes, the same state (within
    # the walk's tolerance: the oracle moves its own snapshot)
    ocm.linear_state_commit([s_conv], [pool], [sub["slots"]], torch.arange(n, dtype=torch.int32), path[reqs],
                            plen[reqs])
    for i, r in enumerate(reqs):
        d_new = int(sub["slots"][i, int(plen[r]) - 1])
        assert_states_close(g["pool"][int(dst_state[r])].cpu(), pool[d_new])
        assert torch.equal(g["conv_state"][int(slots_cpu[r, 0])].cpu(), s_conv[int(sub["slots"][i, 0])])


def test_accept_b512_argmax_and_walk(dev):
    """8192 rows x 151936 bf16 logits: greedy targets equal ``torch.argmax`` on the device; the tree walk of 512
    seeded 16-node trees with planted drafts equals the oracle walk (paths, lengths, sampled tokens)."""
    from eagle_harness.vllm.tree_accept import accept_tree, greedy_targets
    from eagle_harness.vllm.verify_layout import TreeStore

    announce("config accept b512 argmax vocab 151936 + walk")
    B, W, vocab = 512, 16, 151936
    gen = torch.Generator(device=dev).manual_seed(17)
    logits = torch.randn(B * W, vocab, device=dev, generator=gen).bfloat16()
    target = greedy_targets(logits)
    want = torch.argmax(logits, dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(target, want)
    del logits

    rng = np.random.default_rng(19)
    trees = [seeded_tree(rng, W) for _ in range(B)]
    tgt = target.cpu()
    drafted = torch.from_numpy(rng.integers(0, vocab, B * W)).long()
    for b, parents in enumerate(trees):  # plant: a random child of each planted node carries its parent's target
        node = 0
        while True:
            kids = [c for c in range(W) if parents[c] == node]
            if not kids or rng.random() < 0.15:
                break
            node = kids[int(rng.integers(len(kids)))]
            drafted[b * W + node] = tgt[b * W + parents[node]]
    parents_t = torch.tensor(trees, dtype=torch.int32)
    cu = torch.arange(0, B * W + 1, W, dtype=torch.int32)
    idx = torch.arange(B, dtype=torch.int32)
    store = TreeStore(B, W, dev)
    sampled, num = accept_tree(target, drafted.to(dev), cu.to(dev), idx.to(dev), parents_t.to(dev), store)
    torch.cuda.synchronize()
    path_o, plen_o = torch.zeros(B, W, dtype=torch.int32), torch.ones(B, dtype=torch.int32)
    sampled_o, num_o = oacc.accept_tree(tgt, drafted, cu, idx, parents_t, path_o, plen_o, W)
    assert torch.equal(num.cpu(), num_o)
    assert int(num_o.max()) > 3  # the planted paths are accepted past the root
    assert torch.equal(store.path_len.cpu(), plen_o)
    for b in range(B):
        n = int(num_o[b])
        assert torch.equal(store.path[b, :n].cpu(), path_o[b, :n])
        assert torch.equal(sampled[b, :n].cpu(), sampled_o[b, :n])
