"""The GDN tree recurrence (snapshot contract) on the GPU against the oracle walk
(kernels/gdn_tree_recurrence.py:204-359, 562-706): outputs within the output dtype's tolerance, fp32 states within
1e-4 relative, both engines' slot tables, 16-bit snapshot buffers, publish and padding."""

import pytest
import torch

from conftest import announce, assert_states_close
from oracle import recurrence as orr
from workloads import GDN_B1, GdnShape, gdn_inputs, seeded_tree

pytestmark = pytest.mark.gpu

TREE = [-1, 0, 0, 1, 1, 2, 3]
CHAIN = [-1, 0, 1, 2, 3]


def _random_tree(width, seed):
    gen = torch.Generator().manual_seed(seed)
    return [-1] + [int(torch.randint(0, r, (1,), generator=gen)) for r in range(1, width)]


def _requests(parent_lists, width):
    parents = torch.zeros(len(parent_lists), width, dtype=torch.int32)
    qsl = [0]
    for b, plist in enumerate(parent_lists):
        parents[b, : len(plist)] = torch.tensor(plist)
        qsl.append(qsl[-1] + len(plist))
    return parents, torch.tensor(qsl, dtype=torch.int32)


def _to(d, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _state_close(got, want):
    assert_states_close(got.float(), want.float())


def _vllm_case(dev, parent_lists, dims, state_dtype=torch.float32, edit_slots=None, seed=1):
    """One slot per row (the vLLM layout); runs the GPU walk and the oracle walk on the same inputs and compares."""
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

    gen = torch.Generator().manual_seed(seed)
    width = max(map(len, parent_lists))
    (heads, value_heads, dk, dv) = dims
    parents, qsl = _requests(parent_lists, width)
    tokens = int(qsl[-1])
    q, k = torch.randn(1, tokens, heads, dk, generator=gen), torch.randn(1, tokens, heads, dk, generator=gen)
    v = torch.randn(1, tokens, value_heads, dv, generator=gen)
    a, b = torch.randn(tokens, value_heads, generator=gen), torch.randn(tokens, value_heads, generator=gen)
    A_log, dt_bias = torch.randn(value_heads, generator=gen), torch.randn(value_heads, generator=gen)
    slots = torch.arange(1, 1 + len(parent_lists) * (width + 1), dtype=torch.int32).view(len(parent_lists), width + 1)
    if edit_slots is not None:
        edit_slots(slots)
    num_slots = int(slots.max()) + 2
    state = (torch.randn(num_slots, value_heads, dv, dk, generator=gen) * 0.1).to(state_dtype)
    accepted = torch.tensor([1 + (i % 2) for i in range(len(parent_lists))], dtype=torch.int32)
    kw = dict(num_accepted_tokens=accepted, pad_slot_id=0)
    s_want = state.clone()
    o_want = orr.gdn_tree_recurrent_update(A_log, dt_bias, q, k, v, a, b, initial_state_source=s_want,
                                           initial_state_indices=slots, cu_seqlens=qsl,
                                           intermediate_states_buffer=s_want, intermediate_state_indices=slots,
                                           retrieve_parent_token=parents, **kw)
    g = _to(dict(q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt_bias=dt_bias, state=state, slots=slots, parents=parents,
                 qsl=qsl, accepted=accepted), dev)
    o_got = gdn_tree_recurrent_update(g["A_log"], g["dt_bias"], g["q"], g["k"], g["v"], g["a"], g["b"],
                                      initial_state_source=g["state"], initial_state_indices=g["slots"],
                                      cu_seqlens=g["qsl"], intermediate_states_buffer=g["state"],
                                      intermediate_state_indices=g["slots"], retrieve_parent_token=g["parents"],
                                      num_accepted_tokens=g["accepted"], pad_slot_id=0)
    torch.cuda.synchronize()
    if state_dtype == torch.float32:
        torch.testing.assert_close(o_got.cpu(), o_want, atol=1e-4, rtol=1e-4)
        _state_close(g["state"].cpu(), s_want)
    else:  # 16-bit snapshots: within one rounding of the oracle's (the fp32 math differs in summation order)
        torch.testing.assert_close(o_got.cpu().float(), o_want.float(), atol=2e-2, rtol=1e-2)
        torch.testing.assert_close(g["state"].cpu().float(), s_want.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("parent_lists", [[TREE, CHAIN], [TREE, TREE[:5]], [_random_tree(16, 2), _random_tree(16, 3)]])
@pytest.mark.parametrize("dims", [(2, 4, 8, 8), (2, 6, 128, 128), (1, 2, 64, 32), (4, 8, 256, 128)])
def test_vllm_row_slots_fp32_match_oracle(dev, parent_lists, dims):
    """The reference test's layout (tests/test_gdn_tree_kernels.py:179-219): fp32 inputs, one slot per row."""
    announce(f"recurrence vllm fp32 dims={dims} widths={[len(p) for p in parent_lists]}")
    _vllm_case(dev, parent_lists, dims)


# Nodes 0..5 each have two children, the lower-index one leading deeper, so six states are parked at once (more
# than the walk's LDS stack holds: the deepest ones are reloaded from their snapshots).
NESTED = [-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 0, 1, 2, 3, 4, 5]


# A complete binary tree: walked neediest-child-last (fp32 snapshots) it needs three parked states, one more than the
# two that the large grids' walk holds, so the deepest branch points reload their snapshots there.
BINARY = [-1] + [(i - 1) // 2 for i in range(1, 16)]


# Value heads: 4 is a small grid (16 lanes per row, children in index order, four parked states), 64 a large one
# (8 lanes per row, children in need order, two parked states).
@pytest.mark.parametrize("value_heads", [4, 64])
@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_nested_branches_beyond_the_parked_states(dev, state_dtype, value_heads):
    announce(f"recurrence nested branches {state_dtype} HV {value_heads}")
    _vllm_case(dev, [NESTED, BINARY, _random_tree(16, 4), [-1] + [0] * 15], (2, value_heads, 128, 128),
               state_dtype=state_dtype)


COMB = [-1] + [2 * ((i - 1) // 2) for i in range(1, 64)]  # even rows a 32-row spine, every spine row with a leaf too


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_depth_first_plans_up_to_64_rows(dev, state_dtype):
    """The widest depth-first requests: 64 rows (random, a 64-row chain, a deep comb) and 33 rows, whose plans need
    every round of the plan's pointer jumping (the chain: 63 levels) and nested parked states (the comb)."""
    announce(f"recurrence 64-row plans {state_dtype}")
    _vllm_case(dev, [_random_tree(64, 9), list(range(-1, 63)), COMB, _random_tree(33, 10)], (1, 2, 64, 32),
               state_dtype=state_dtype)


def _pad_row(slots):
    slots[0, 3] = 0  # row 3's snapshot is not written; its children continue from the previous row's state


def _shared_slot(slots):
    slots[1, 5] = slots[1, 2]  # rows 2 and 5 share a slot: row 2's later children read row 5's snapshot


@pytest.mark.parametrize("case", ["pad_row", "shared_slot", "long_request"])
def test_reference_index_order_for_other_slot_tables(dev, case):
    """Slot tables whose reloads do not return the parent's own state keep the reference's index-order walk
    (kernels/gdn_tree_recurrence.py:312-329), as does a request of more than 64 rows."""
    announce(f"recurrence index-order walk {case}")
    if case == "long_request":
        _vllm_case(dev, [_random_tree(80, 6), TREE], (1, 2, 64, 32))
    else:
        _vllm_case(dev, [_random_tree(16, 7), _random_tree(16, 8)], (2, 4, 128, 128),
                   edit_slots=_pad_row if case == "pad_row" else _shared_slot)


@pytest.mark.parametrize("batch", [1, 4])
def test_gdn_b1_heads_sglang_scratch_match_oracle(dev, batch):
    """The 16 / 32-head layer with bf16 inputs, an fp32 pool and sglang's per-request snapshot scratch."""
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

    announce(f"recurrence sglang bf16 batch={batch}")
    shape = GdnShape(batch, 16, 16, 32, 128, 128)
    inp = gdn_inputs(shape, seed=5, layout="sglang")
    want_scr = inp["scratch"].clone()
    o_want = orr.gdn_tree_recurrent_update(
        inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
        initial_state_source=inp["pool"], initial_state_indices=inp["state_indices"],
        cu_seqlens=inp["query_start_loc"], intermediate_states_buffer=want_scr,
        intermediate_state_indices=inp["scratch_indices"], retrieve_parent_token=inp["parent_table"])
    g = _to(inp, dev)
    o_got = gdn_tree_recurrent_update(
        g["A_log"], g["dt_bias"], g["q"], g["k"], g["v"], g["a"], g["b"],
        initial_state_source=g["pool"], initial_state_indices=g["state_indices"],
        cu_seqlens=g["query_start_loc"], intermediate_states_buffer=g["scratch"],
        intermediate_state_indices=g["scratch_indices"], retrieve_parent_token=g["parent_table"])
    torch.cuda.synchronize()
    torch.testing.assert_close(o_got.cpu().float(), o_want.float(), atol=2e-2, rtol=1e-2)
    _state_close(g["scratch"].cpu(), want_scr)
    assert torch.equal(g["pool"].cpu(), inp["pool"])  # the request's own state is never written


@pytest.mark.parametrize("state_dtype", [torch.bfloat16, torch.float16])
def test_16bit_pool_reloads_rounded_parents(dev, state_dtype):
    """A 16-bit pool / snapshot buffer: every non-root node reloads its parent's rounded snapshot (no register
    chain), as the walk does without SKIP_CHAIN_RELOAD (kernels/gdn_tree_recurrence.py:633-635, 318-329)."""
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

    announce(f"recurrence vllm 16-bit pool {state_dtype}")
    shape = GdnShape(3, 16, 4, 12, 128, 128)
    inp = gdn_inputs(shape, seed=9, layout="vllm", state_dtype=state_dtype)
    want_pool = inp["pool"].clone()
    o_want = orr.gdn_tree_recurrent_update(
        inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
        initial_state_source=want_pool, initial_state_indices=inp["slots"], cu_seqlens=inp["query_start_loc"],
        intermediate_states_buffer=want_pool, intermediate_state_indices=inp["slots"],
        retrieve_parent_token=inp["parent_table"], num_accepted_tokens=inp["num_accepted"], pad_slot_id=0)
    g = _to(inp, dev)
    o_got = gdn_tree_recurrent_update(
        g["A_log"], g["dt_bias"], g["q"], g["k"], g["v"], g["a"], g["b"],
        initial_state_source=g["pool"], initial_state_indices=g["slots"], cu_seqlens=g["query_start_loc"],
        intermediate_states_buffer=g["pool"], intermediate_state_indices=g["slots"],
        retrieve_parent_token=g["parent_table"], num_accepted_tokens=g["num_accepted"], pad_slot_id=0)
    torch.cuda.synchronize()
    torch.testing.assert_close(o_got.cpu().float(), o_want.float(), atol=2e-2, rtol=1e-2)
    # 16-bit snapshots: within one rounding of the oracle's (the fp32 math differs only in summation order)
    torch.testing.assert_close(g["pool"].cpu().float(), want_pool.float(), atol=1e-2, rtol=1e-2)


def test_publish_and_padded_request(dev):
    """publish receives every request's slots, a padded request's too, and leaves later columns alone
    (tests/test_gdn_tree_kernels.py:658-697); outputs do not change with publish."""
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

    announce("recurrence publish")
    gen = torch.Generator().manual_seed(5)
    heads, value_heads, d, width = 1, 2, 128, 4
    parents = torch.tensor([[-1, 0, 0, 1], [-1, 0, 1, 2], [0, 0, 0, 0]], dtype=torch.int32, device=dev)
    qsl = torch.tensor([0, 4, 8, 8], dtype=torch.int32, device=dev)
    tokens = 8
    q, k = (torch.randn(1, tokens, heads, d, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2))
    v = torch.randn(1, tokens, value_heads, d, generator=gen).to(torch.bfloat16).to(dev)
    a, b = (torch.randn(tokens, value_heads, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2))
    A_log, dt_bias = torch.zeros(value_heads, device=dev), torch.zeros(value_heads, device=dev, dtype=torch.bfloat16)
    slots = torch.arange(1, 1 + 3 * (width + 1), dtype=torch.int32, device=dev).view(3, width + 1)
    slots[2] = 0
    accepted = torch.tensor([1, 2, 1], dtype=torch.int32, device=dev)
    state0 = torch.randn(slots.numel() + 1, value_heads, d, d, generator=gen).to(dev) * 0.05
    results = []
    for publish in (None, torch.full((3, width + 3), -7, dtype=torch.int32, device=dev)):
        state = state0.clone()
        out = gdn_tree_recurrent_update(A_log, dt_bias, q, k, v, a, b, initial_state_source=state,
                                        initial_state_indices=slots, num_accepted_tokens=accepted, cu_seqlens=qsl,
                                        intermediate_states_buffer=state, intermediate_state_indices=slots,
                                        retrieve_parent_token=parents, pad_slot_id=0, publish=publish)
        results.append((out, state, publish))
    torch.cuda.synchronize()
    (out0, st0, _), (out1, st1, published) = results
    assert torch.equal(published[:, : width + 1], slots)
    assert torch.all(published[:, width + 1 :] == -7)
    assert torch.equal(out1, out0) and torch.equal(st1, st0)


def test_full_batch_sampled_requests_match_oracle(dev):
    """The batch-64 layer of the bench: every request runs on the GPU; 3 sampled requests are recomputed by the
    oracle (requests are independent), and every output is finite."""
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

    announce("recurrence batch 64 sampled")
    shape = GdnShape(64, 16, 16, 32, 128, 128)
    inp = gdn_inputs(shape, seed=3, layout="vllm")
    g = _to(inp, dev)
    o_got = gdn_tree_recurrent_update(
        g["A_log"], g["dt_bias"], g["q"], g["k"], g["v"], g["a"], g["b"],
        initial_state_source=g["pool"], initial_state_indices=g["slots"], cu_seqlens=g["query_start_loc"],
        intermediate_states_buffer=g["pool"], intermediate_state_indices=g["slots"],
        retrieve_parent_token=g["parent_table"], num_accepted_tokens=g["num_accepted"], pad_slot_id=0)
    torch.cuda.synchronize()
    assert torch.isfinite(o_got.float()).all()
    W = shape.width
    for r in (0, 31, 63):
        sl = slice(r * W, (r + 1) * W)
        sub_slots = inp["slots"][r : r + 1]
        pool = inp["pool"].clone()
        want = orr.gdn_tree_recurrent_update(
            inp["A_log"], inp["dt_bias"], inp["q"][:, sl], inp["k"][:, sl], inp["v"][:, sl], inp["a"][sl], inp["b"][sl],
            initial_state_source=pool, initial_state_indices=sub_slots, cu_seqlens=torch.tensor([0, W], dtype=torch.int32),
            intermediate_states_buffer=pool, intermediate_state_indices=sub_slots,
            retrieve_parent_token=inp["parent_table"][r : r + 1], num_accepted_tokens=inp["num_accepted"][r : r + 1],
            pad_slot_id=0)
        torch.testing.assert_close(o_got[:, sl].cpu().float(), want.float(), atol=2e-2, rtol=1e-2)
        idx = sub_slots[0].long()
        _state_close(g["pool"][idx.to(dev)].cpu(), pool[idx])


def test_packed_projection_views_equal_contiguous_inputs(dev):
    """The callers' layout (tests/test_gdn_tree_kernels.py:222-309; vllm/gdn_tree_verify.py:84-100): q / k / v as
    token-strided views of one packed projection [tokens, 2 H K + HV V (+ z)] and b / a as the halves of [tokens, 2 HV]
    give the same outputs and snapshots, bit for bit, as contiguous copies of the same values."""
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

    announce("recurrence packed projection views")
    gen = torch.Generator().manual_seed(23)
    plists = [_random_tree(8, 4), TREE]
    width = max(map(len, plists))
    heads, value_heads, dk, dv = 2, 4, 128, 128
    key_dim, value_dim = heads * dk, value_heads * dv
    dim = 2 * key_dim + value_dim
    parents, qsl = _requests(plists, width)
    tokens = int(qsl[-1])
    qkvz = torch.randn(tokens, dim + value_dim, generator=gen).bfloat16().to(dev)  # [q, k, v, z]
    ba = torch.randn(tokens, 2 * value_heads, generator=gen).bfloat16().to(dev)
    b, a = ba.chunk(2, dim=-1)
    A_log, dt_bias = torch.randn(value_heads, generator=gen).to(dev), torch.randn(value_heads, generator=gen).to(dev)
    slots = torch.arange(1, 1 + len(plists) * (width + 1), dtype=torch.int32).view(len(plists), width + 1).to(dev)
    state0 = (torch.randn(slots.numel() + 2, value_heads, dv, dk, generator=gen) * 0.1).to(dev)
    accepted = torch.tensor([1, 2], dtype=torch.int32, device=dev)
    parents, qsl = parents.to(dev), qsl.to(dev)
    q, k, v = qkvz[:, :key_dim], qkvz[:, key_dim : 2 * key_dim], qkvz[:, 2 * key_dim : dim]

    def run(q, k, v, a, b):
        state = state0.clone()
        out = gdn_tree_recurrent_update(A_log, dt_bias, q.view(1, tokens, heads, dk), k.view(1, tokens, heads, dk),
                                        v.view(1, tokens, value_heads, dv), a, b, initial_state_source=state,
                                        initial_state_indices=slots, cu_seqlens=qsl, intermediate_states_buffer=state,
                                        intermediate_state_indices=slots, retrieve_parent_token=parents,
                                        num_accepted_tokens=accepted, pad_slot_id=0)
        torch.cuda.synchronize()
        return out, state

    o_views, s_views = run(q, k, v, a, b)
    o_flat, s_flat = run(q.contiguous(), k.contiguous(), v.contiguous(), a.contiguous(), b.contiguous())
    assert torch.equal(o_views, o_flat) and torch.equal(s_views, s_flat)
