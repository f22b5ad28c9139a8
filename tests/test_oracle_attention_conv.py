"""Pins of the CPU oracle's tree-verify attention and tree conv (oracle/attention.py, oracle/conv.py) against library
routines and invariants, so a mistake in the oracle (a wrong page index, a transposed mask, a dropped tap) fails here
before it can hide a kernel's: chains reduce to torch's scaled_dot_product_attention / depthwise conv1d, every tree
row equals its root path run as a chain, fp8 pages follow torch's float8_e4m3fn, and the conv's state roll is the
reference tests' known answer (tests/test_gdn_tree_conv.py:79, :118-121)."""

import torch
import torch.nn.functional as F
from oracle import attention as oa
from oracle import conv as oc
import numpy as np

from workloads import seeded_tree, tree_masks, window_codes


def _paged(keys_ctx, page, blocks_total, gen):
    """Scatters [L, Hkv, D] context rows into a shuffled paged cache; returns (cache, block_table row)."""
    L, hkv, d = keys_ctx.shape
    npages = (L + page - 1) // page
    perm = torch.randperm(blocks_total, generator=gen)[:npages]
    cache = torch.randn(blocks_total, page, hkv, d, generator=gen) * 100  # poison everywhere else
    for p in range(npages):
        rows = keys_ctx[p * page : (p + 1) * page]
        cache[perm[p], : rows.shape[0]] = rows
    return cache, perm.to(torch.int32)


def _case(parents, L, hq=4, hkv=2, d=16, page=16, seed=0):
    gen = torch.Generator().manual_seed(seed)
    W = len(parents)
    kctx, vctx = torch.randn(L, hkv, d, generator=gen), torch.randn(L, hkv, d, generator=gen)
    blocks = (L + page - 1) // page + 5
    kc, table = _paged(kctx, page, blocks, gen)
    gen2 = torch.Generator().manual_seed(seed + 1)
    vc = torch.randn(blocks, page, hkv, d, generator=gen2) * 100
    for p in range((L + page - 1) // page):
        rows = vctx[p * page : (p + 1) * page]
        vc[table[p], : rows.shape[0]] = rows
    q = torch.randn(W, hq, d, generator=gen)
    kn, vn = torch.randn(W, hkv, d, generator=gen), torch.randn(W, hkv, d, generator=gen)
    masks = torch.tensor([tree_masks(parents)], dtype=torch.int64)
    bt = torch.zeros(1, max(1, len(table)) + 2, dtype=torch.int32)
    bt[0, : len(table)] = table
    out = torch.full((W + 3, hq, d), 7.0)
    oa.verify_attention(q, kn, vn, kc, vc, bt, torch.tensor([L], dtype=torch.int32),
                        torch.tensor([0, W], dtype=torch.int32), masks, d**-0.5, out, max_query_len=W)
    return dict(q=q, kn=kn, vn=vn, kctx=kctx, vctx=vctx, out=out, W=W, hq=hq, hkv=hkv, d=d)


def _sdpa(q, keys, values, visible, group):
    """torch's attention over explicit keys: q [W, Hq, D], keys [S, Hkv, D], visible [W, S] bool."""
    k = keys.repeat_interleave(group, 1).permute(1, 0, 2)
    v = values.repeat_interleave(group, 1).permute(1, 0, 2)
    return F.scaled_dot_product_attention(q.permute(1, 0, 2), k, v, attn_mask=visible[None]).permute(1, 0, 2)


def test_chain_without_context_is_causal_sdpa():
    c = _case([-1, 0, 1, 2, 3, 4], L=0)
    want = F.scaled_dot_product_attention(
        c["q"].permute(1, 0, 2), c["kn"].repeat_interleave(2, 1).permute(1, 0, 2),
        c["vn"].repeat_interleave(2, 1).permute(1, 0, 2), is_causal=True).permute(1, 0, 2)
    torch.testing.assert_close(c["out"][: c["W"]], want, atol=1e-5, rtol=1e-5)
    assert torch.all(c["out"][c["W"] :] == 7.0)  # rows past the batch keep the sentinel


def test_chain_with_a_ragged_paged_context_is_masked_sdpa():
    L = 37  # not a multiple of the page: the last page is partly filled
    c = _case([-1, 0, 1, 2, 3], L=L)
    W = c["W"]
    keys, values = torch.cat([c["kctx"], c["kn"]]), torch.cat([c["vctx"], c["vn"]])
    visible = torch.cat([torch.ones(W, L, dtype=torch.bool), torch.ones(W, W).tril().bool()], 1)
    want = _sdpa(c["q"], keys, values, visible, c["hq"] // c["hkv"])
    torch.testing.assert_close(c["out"][:W], want, atol=1e-5, rtol=1e-5)


def test_tree_rows_equal_their_root_path_chain():
    """Row r sees the context and exactly its ancestors-or-self among the draft keys."""
    parents = seeded_tree(np.random.default_rng(3), 12)
    L = 20
    c = _case(parents, L=L, seed=3)
    W = c["W"]
    for r in range(W):
        path, node = [], r
        while node >= 0:
            path.append(node)
            node = parents[node]
        path = sorted(path)
        keys = torch.cat([c["kctx"], c["kn"][path]])
        values = torch.cat([c["vctx"], c["vn"][path]])
        want = _sdpa(c["q"][r : r + 1], keys, values, torch.ones(1, L + len(path), dtype=torch.bool),
                     c["hq"] // c["hkv"])
        torch.testing.assert_close(c["out"][r : r + 1], want, atol=1e-5, rtol=1e-5)


def test_fp8_pages_are_torch_e4m3fn_with_per_page_head_scales():
    gen = torch.Generator().manual_seed(4)
    cache = torch.randn(6, 16, 3, 8, generator=gen) * torch.tensor([0.01, 1.0, 300.0])[None, None, :, None]
    cache[2, :, 1] = 0.0  # an all-zero (page, head): scale 1
    q8, scale = oa.quantize_fp8_pages(cache)
    assert q8.dtype == torch.float8_e4m3fn and scale.shape == (6, 3)
    assert scale[2, 1] == 1.0
    # the amax of every (page, head) lands on the format's largest finite value, 448
    amax8 = q8.float().abs().amax(dim=(1, 3))
    nz = cache.abs().amax(dim=(1, 3)) > 0
    assert torch.all(amax8[nz] == 448.0)
    # round to nearest with 3 mantissa bits: relative error within 2^-4 for normal values
    deq = oa.dequantize_fp8_pages(q8, scale)
    normal = cache.abs() >= 2.0**-6 * scale[:, None, :, None]
    rel = ((deq - cache).abs() / cache.abs().clamp_min(1e-30))[normal]
    assert rel.max() <= 2.0**-4 + 1e-6


def test_fp8_attention_equals_attention_on_the_dequantized_cache():
    """k_scale / v_scale index (block, KV head): scales that differ per page and head must be applied per row."""
    gen = torch.Generator().manual_seed(5)
    W, hq, hkv, d, page, blocks = 5, 4, 2, 16, 16, 8
    parents = [-1, 0, 0, 1, 2]
    kc = torch.randn(blocks, page, hkv, d, generator=gen) * torch.linspace(0.1, 10, blocks)[:, None, None, None]
    vc = torch.randn(blocks, page, hkv, d, generator=gen) * torch.tensor([0.5, 20.0])[None, None, :, None]
    k8, ks = oa.quantize_fp8_pages(kc)
    v8, vs = oa.quantize_fp8_pages(vc)
    q = torch.randn(W, hq, d, generator=gen)
    kn, vn = torch.randn(W, hkv, d, generator=gen), torch.randn(W, hkv, d, generator=gen)
    bt = torch.tensor([[5, 2, 7, 0]], dtype=torch.int32)
    args = (torch.tensor([50], dtype=torch.int32), torch.tensor([0, W], dtype=torch.int32),
            torch.tensor([tree_masks(parents)], dtype=torch.int64), d**-0.5)
    got = torch.zeros(W, hq, d)
    oa.verify_attention(q, kn, vn, k8, v8, bt, *args, got, max_query_len=W, k_scale=ks, v_scale=vs)
    want = torch.zeros(W, hq, d)
    oa.verify_attention(q, kn, vn, oa.dequantize_fp8_pages(k8, ks), oa.dequantize_fp8_pages(v8, vs), bt, *args, want,
                        max_query_len=W)
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)


# ---- tree conv --------------------------------------------------------------------------------------------------------

def _conv_case(parents, dim=6, seed=0, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    W = len(parents)
    x = torch.randn(W, dim, generator=gen).to(dtype)
    w = torch.randn(dim, 4, generator=gen).to(dtype)
    bias = torch.randn(dim, generator=gen).to(dtype)
    hist = torch.randn(dim, 3, generator=gen).to(dtype)
    anc = torch.tensor([list(zip(*window_codes(parents)))], dtype=torch.int32)  # [1, 3, W]
    state = torch.zeros(2, dim, 3, dtype=dtype)
    state[1] = hist
    out = oc.gdn_tree_conv1d_update(x.t()[None].contiguous(), state, w, bias, "silu",
                                    torch.tensor([1], dtype=torch.int32), None, None, anc)
    return x, w, bias, hist, state, out[0].t()


def _chain_conv(x_chain, hist, w, bias):
    """Depthwise causal conv1d (torch) over [history, x_chain] with SiLU: [len, dim]."""
    seq = torch.cat([hist, x_chain.t()], 1)[None]  # [1, dim, 3 + len]
    y = F.conv1d(seq, w[:, None, :], bias, groups=w.shape[0])[0]  # [dim, len]
    return F.silu(y).t()


def test_conv_chain_is_torch_depthwise_conv1d():
    x, w, bias, hist, _, out = _conv_case([-1, 0, 1, 2, 3, 4, 5])
    torch.testing.assert_close(out, _chain_conv(x, hist, w, bias), atol=1e-5, rtol=1e-5)


def test_conv_tree_rows_equal_their_root_path_chain():
    parents = seeded_tree(np.random.default_rng(8), 14)
    x, w, bias, hist, _, out = _conv_case(parents, seed=8)
    for r in range(len(parents)):
        path, node = [], r
        while node >= 0:
            path.append(node)
            node = parents[node]
        path = sorted(path)
        torch.testing.assert_close(out[r], _chain_conv(x[path], hist, w, bias)[-1], atol=1e-5, rtol=1e-5)


def test_conv_matches_the_reference_tests_dense_form():
    parents = seeded_tree(np.random.default_rng(9), 10)
    x, w, bias, hist, _, out = _conv_case(parents, seed=9)
    want, _ = oc.dense_conv_reference(x, hist, w, bias, parents)
    torch.testing.assert_close(out, want.float(), atol=1e-5, rtol=1e-5)


def test_conv_roll_known_answers():
    """sglang layout (3 history columns): the state becomes the last 3 of [history, x] (tests/test_gdn_tree_conv.py:79);
    vLLM layout: [history[1:], x] from the resume column on, later columns untouched (:118-121)."""
    parents = [-1, 0, 0, 1]
    x, _, _, hist, state, _ = _conv_case(parents, seed=2)
    assert torch.equal(state[1], torch.cat([hist, x.t()], 1)[:, -3:])
    assert torch.equal(state[0], torch.zeros_like(state[0]))  # other slots untouched
    # vLLM: state_len 3 + W, resume column a - 1 with a = 2 accepted
    gen = torch.Generator().manual_seed(3)
    dim, W = 5, len(parents)
    xv = torch.randn(W, dim, generator=gen)
    st0 = torch.randn(3, dim, 3 + W + 2, generator=gen)
    st = st0.clone()
    anc = torch.tensor([list(zip(*window_codes(parents)))], dtype=torch.int32)
    oc.gdn_tree_conv1d_update(xv.t()[None], st, torch.randn(dim, 4, generator=gen), None, "silu",
                              torch.tensor([2], dtype=torch.int32), None, None, anc, pad_slot_id=0,
                              num_accepted_tokens=torch.tensor([2], dtype=torch.int32),
                              query_start_loc=torch.tensor([0, W], dtype=torch.int32))
    history = st0[2, :, 1:4]
    rolled = torch.cat([history[:, 1:], xv.t()], 1)
    assert torch.equal(st[2, :, : rolled.shape[1]], rolled)
    assert torch.equal(st[2, :, rolled.shape[1] :], st0[2, :, rolled.shape[1] :])
    assert torch.equal(st[:2], st0[:2])
