"""Pins of the oracle's GDN tree walk and records contract (CPU).

The walk is checked against forms that share no code with it: the delta rule as a matrix product in float64
(S' = e^g S (I - beta k k^T) + beta v k^T), every row equal to its root path run as a chain, the reference's
parallel chunk closed form (ancestor closure and a triangular solve), single-step closed forms, and the two
engines' slot layouts giving the same snapshots. The records replay and commit are pinned against the walk's
snapshots and the reference tests' known answers (sub-ulp decay)."""

import numpy as np
import pytest
import torch

from oracle import recurrence as orr
from oracle import records as orec
from workloads import GdnShape, gdn_inputs, root_path, seeded_tree


def _chain_matrix_form(q, k, v, a, b, A_log, dt_bias, S0, heads):
    """float64 matrix form of the delta rule over a chain; returns (outputs [T, HV, V], states [T][HV, V, K])."""
    T, HV = v.shape[0], v.shape[1]
    K = k.shape[-1]
    S = S0.double().clone()
    g = -torch.exp(A_log.double()) * torch.nn.functional.softplus(a.double() + dt_bias.double())
    beta = torch.sigmoid(b.double()).to(b.dtype).double() if b.dtype != torch.float64 else torch.sigmoid(b)
    outs, states = [], []
    I = torch.eye(K, dtype=torch.float64)  # noqa: E741
    for t in range(T):
        qn = q[t].double() / torch.sqrt((q[t].double() ** 2).sum(-1, keepdim=True) + 1e-6) * K**-0.5
        kn = k[t].double() / torch.sqrt((k[t].double() ** 2).sum(-1, keepdim=True) + 1e-6)
        o = torch.zeros(HV, v.shape[-1], dtype=torch.float64)
        for hv in range(HV):
            h = hv // (HV // heads)
            kk = kn[h][:, None] @ kn[h][None, :]
            S[hv] = torch.exp(g[t, hv]) * S[hv] @ (I - beta[t, hv] * kk) + beta[t, hv] * v[t, hv].double()[:, None] @ kn[h][None, :]
            o[hv] = S[hv] @ qn[h]
        outs.append(o)
        states.append(S.clone())
    return torch.stack(outs), states


def _walk(inp, parents_tab, qsl, state_dtype=torch.float32):
    pool = inp["pool"].clone()
    out = orr.gdn_tree_recurrent_update(
        inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
        initial_state_source=pool, initial_state_indices=inp["slots"], cu_seqlens=qsl,
        intermediate_states_buffer=pool, intermediate_state_indices=inp["slots"], retrieve_parent_token=parents_tab,
        num_accepted_tokens=inp["num_accepted"], pad_slot_id=0)
    return out, pool


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16])
def test_every_row_equals_its_root_path_as_a_matrix_chain(in_dtype):
    shape = GdnShape(2, 16, 2, 4, 32, 16)
    inp = gdn_inputs(shape, seed=3, layout="vllm", in_dtype=in_dtype)
    out, pool = _walk(inp, inp["parent_table"], inp["query_start_loc"])
    for r, parents in enumerate(inp["parents"]):
        S0 = inp["pool"][int(inp["slots"][r, 0])]
        for row in range(16):
            path = [16 * r + n for n in root_path(parents, row)]
            o, states = _chain_matrix_form(inp["q"][0, path], inp["k"][0, path], inp["v"][0, path], inp["a"][path],
                                           inp["b"][path], inp["A_log"], inp["dt_bias"], S0, shape.h)
            tol = dict(atol=1e-4, rtol=1e-4) if in_dtype == torch.float32 else dict(atol=2e-2, rtol=1e-2)
            torch.testing.assert_close(out[0, 16 * r + row].double(), o[-1].to(out.dtype).double(), **tol)
            torch.testing.assert_close(pool[int(inp["slots"][r, row])].double(), states[-1], atol=1e-5, rtol=1e-4)


def test_walk_matches_the_reference_tests_dense_form():
    """tests/test_gdn_tree_kernels.py:151-176: per-row dense update from the parent's state (fp32 b, no rounding)."""
    shape = GdnShape(1, 16, 2, 6, 16, 8)
    inp = gdn_inputs(shape, seed=4, layout="vllm", in_dtype=torch.float32)
    out, pool = _walk(inp, inp["parent_table"], inp["query_start_loc"])
    init = inp["pool"][int(inp["slots"][0, 0])]
    o, states = orr.dense_tree_reference(inp["q"][0], inp["k"][0], inp["v"][0], inp["a"], inp["b"], inp["A_log"],
                                         inp["dt_bias"], init, inp["parents"][0], shape.h, shape.hv)
    torch.testing.assert_close(out[0], o, atol=1e-5, rtol=1e-5)
    for row in range(16):
        torch.testing.assert_close(pool[int(inp["slots"][0, row])], states[row], atol=1e-6, rtol=1e-5)


def test_walk_matches_the_chunk_closed_form():
    """The reference's parallel form (kernels/gdn_tree_records.py:302-306): ancestor closure, cumulative decays and
    a triangular solve give every node's output; its records replayed by the commit give the walk's snapshots."""
    shape = GdnShape(3, 16, 2, 4, 32, 32)
    inp = gdn_inputs(shape, seed=6, layout="sglang", in_dtype=torch.float32)
    scratch = inp["scratch"].clone()
    walk = orr.gdn_tree_recurrent_update(
        inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
        initial_state_source=inp["pool"], initial_state_indices=inp["state_indices"],
        cu_seqlens=inp["query_start_loc"], intermediate_states_buffer=scratch,
        intermediate_state_indices=inp["scratch_indices"], retrieve_parent_token=inp["parent_table"])
    rec = torch.full((3, 16, 4, 32 + 32 + 4), -999.0)
    chunk = orec.gdn_tree_chunk_update(
        inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"], state=inp["pool"],
        state_indices=inp["state_indices"], query_start_loc=inp["query_start_loc"], parent=inp["parent_table"],
        records=rec, record_indices=inp["scratch_indices"], width=16)
    torch.testing.assert_close(chunk, walk, atol=1e-4, rtol=1e-4)
    for node in (0, 5, 15):
        committed = inp["pool"].clone()[None]
        orec.gdn_tree_records_commit(committed, rec[None], inp["state_indices"], inp["scratch_indices"],
                                     torch.full((3,), node, dtype=torch.int32), inp["parent_table"], False)
        for r in range(3):
            torch.testing.assert_close(committed[0, int(inp["state_indices"][r])], scratch[r, node], atol=1e-5,
                                       rtol=1e-4)


def test_chunk_form_is_independent_of_node_order():
    """The chunk form takes the nodes in any order (kernels/gdn_tree_records.py:276-361 builds the ancestor closure
    from the parent links): relabelling a tree's non-root nodes, with their rows moved along, moves the outputs and
    records the same way."""
    shape = GdnShape(2, 12, 2, 4, 32, 16)
    inp = gdn_inputs(shape, seed=9, layout="sglang", in_dtype=torch.float32)
    rng = np.random.default_rng(10)
    W = shape.width
    # new label of old node j, per request (the root keeps 0)
    labels = [[0] + [int(x) for x in rng.permutation(np.arange(1, W))] for _ in range(shape.batch)]
    rows = torch.arange(shape.batch * W)
    parent = inp["parent_table"].clone()
    for n, lab in enumerate(labels):
        for j in range(W):
            rows[n * W + lab[j]] = n * W + j  # new row lab[j] holds old row j
            if j > 0:
                parent[n, lab[j]] = lab[int(inp["parent_table"][n, j])]
    moved = {key: inp[key][:, rows] if key in ("q", "k", "v") else inp[key][rows] for key in ("q", "k", "v", "a", "b")}

    def run(q, k, v, a, b, par):
        rec = torch.full((shape.batch, W, shape.hv, shape.v + shape.k + 4), -999.0)
        out = orec.gdn_tree_chunk_update(inp["A_log"], inp["dt_bias"], q, k, v, a, b, state=inp["pool"],
                                         state_indices=inp["state_indices"], query_start_loc=inp["query_start_loc"],
                                         parent=par, records=rec, record_indices=inp["scratch_indices"], width=W)
        return out, rec

    out, rec = run(inp["q"], inp["k"], inp["v"], inp["a"], inp["b"], inp["parent_table"])
    out2, rec2 = run(moved["q"], moved["k"], moved["v"], moved["a"], moved["b"], parent)
    assert any(int(parent[n, t]) > t for n in range(shape.batch) for t in range(1, W))  # not parent-first
    torch.testing.assert_close(out2[0], out[0, rows], atol=1e-5, rtol=1e-5)
    node_rows = torch.tensor([[lab.index(t) for t in range(W)] for lab in labels])  # old node at each new label
    for n in range(shape.batch):
        torch.testing.assert_close(rec2[n], rec[n, node_rows[n]], atol=1e-5, rtol=1e-5)


def test_single_step_closed_form():
    """From S0 = 0, one node: S = beta v k^T, o = beta v (k . q) scale (normalised q, k)."""
    shape = GdnShape(1, 1, 1, 2, 8, 4)
    inp = gdn_inputs(shape, seed=1, layout="vllm", in_dtype=torch.float32)
    inp["pool"].zero_()
    out, pool = _walk(inp, inp["parent_table"], inp["query_start_loc"])
    q, k, v, b = inp["q"][0, 0, 0], inp["k"][0, 0, 0], inp["v"][0, 0], inp["b"][0]
    qn, kn = q / q.norm(), k / k.norm()
    beta = torch.sigmoid(b)
    S = beta[:, None, None] * v[:, :, None] * kn[None, None, :]
    torch.testing.assert_close(pool[int(inp["slots"][0, 0])], S, atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(out[0, 0], beta[:, None] * v * (kn @ qn) * 8**-0.5, atol=1e-6, rtol=1e-5)


def test_zero_write_strength_only_decays_the_parent():
    """b -> -inf gives beta = 0: a node's state is its parent's times exp(g), whatever v and k."""
    shape = GdnShape(1, 6, 1, 2, 16, 8)
    inp = gdn_inputs(shape, seed=2, layout="vllm", in_dtype=torch.float32)
    inp["b"].fill_(-1e4)
    _, pool = _walk(inp, inp["parent_table"], inp["query_start_loc"])
    parents = inp["parents"][0]
    g = -torch.nn.functional.softplus(inp["a"])  # A_log = dt_bias = 0
    for row in range(1, 6):
        parent_state = pool[int(inp["slots"][0, parents[row]])]
        torch.testing.assert_close(pool[int(inp["slots"][0, row])], parent_state * torch.exp(g[row])[:, None, None],
                                   atol=1e-7, rtol=1e-6)


def test_beta_rounds_through_b_dtype_and_softplus_goes_linear():
    """beta = sigmoid(b) rounded to b's dtype (kernels/gdn_tree_recurrence.py:132-140); softplus is linear above the
    threshold 20 (:115-129)."""
    b = torch.tensor([0.3, -1.7, 2.2], dtype=torch.bfloat16)
    assert torch.equal(orr.write_strength(b), torch.sigmoid(b.float()).to(torch.bfloat16).float())
    a = torch.tensor([25.0, 19.0, -3.0])
    g = orr.log_decay(a, torch.zeros(3), torch.zeros(3))
    assert g[0] == -25.0
    torch.testing.assert_close(g[1:], -torch.nn.functional.softplus(a[1:]))


def test_engine_layouts_agree():
    """sglang's per-request scratch and vLLM's per-row pool slots hold the same snapshots for the same tree."""
    shape = GdnShape(2, 10, 2, 4, 16, 16)
    v = gdn_inputs(shape, seed=8, layout="vllm", in_dtype=torch.float32)
    s = gdn_inputs(shape, seed=8, layout="sglang", in_dtype=torch.float32)
    for r in range(2):  # the same initial states
        s["pool"][int(s["state_indices"][r])] = v["pool"][int(v["slots"][r, 0])]
    out_v, pool_v = _walk(v, v["parent_table"], v["query_start_loc"])
    scratch = s["scratch"].clone()
    out_s = orr.gdn_tree_recurrent_update(
        s["A_log"], s["dt_bias"], v["q"], v["k"], v["v"], v["a"], v["b"], initial_state_source=s["pool"],
        initial_state_indices=s["state_indices"], cu_seqlens=s["query_start_loc"], intermediate_states_buffer=scratch,
        intermediate_state_indices=s["scratch_indices"], retrieve_parent_token=v["parent_table"])
    assert torch.equal(out_v, out_s)
    for r in range(2):
        for row in range(10):
            assert torch.equal(pool_v[int(v["slots"][r, row])], scratch[r, row])


def test_rounded_records_replay_and_sub_ulp_decay():
    """The bf16-pool records path (kernels/gdn_tree_records.py:44-101): with a per-node decay below half a bf16 ulp
    every parent rounds back to one, so outputs stay constant and the commit leaves the pool unchanged
    (tests/test_gdn_rounded_records_gpu.py:119-162)."""
    width, dim = 32, 16
    state = torch.ones(1, 1, dim, dim, dtype=torch.bfloat16)
    q = torch.zeros(1, width, 1, dim, dtype=torch.bfloat16)
    q[..., 0] = 1
    k, v = torch.zeros_like(q), torch.zeros_like(q)
    a = torch.full((width, 1), -7.0, dtype=torch.bfloat16)
    b = torch.zeros_like(a)
    A = torch.zeros(1)
    slot = torch.zeros(1, dtype=torch.int32)
    qsl = torch.tensor([0, width], dtype=torch.int32)
    parent = (torch.arange(width, dtype=torch.int32) - 1).view(1, width)
    paths = torch.cat((torch.tensor([width, 0], dtype=torch.int32), torch.arange(width, dtype=torch.int32))).view(1, 1, -1)
    records = torch.empty(1, width, 1, dim * 2 + 4)
    out = orec.gdn_tree_records_update(A, A, q, k, v, a, b, state=state, state_indices=slot, query_start_loc=qsl,
                                       parent=parent, tree_paths=paths, records=records, record_indices=slot,
                                       width=width)
    assert torch.equal(out, out[:, :1].expand_as(out))
    committed = state.clone().unsqueeze(0)
    orec.gdn_tree_records_commit(committed, records.unsqueeze(0), slot, slot, torch.full_like(slot, width - 1), parent,
                                 True)
    assert torch.equal(committed[0], state)
    before = committed.clone()
    orec.gdn_tree_records_commit(committed, records.unsqueeze(0), slot, slot, -torch.ones_like(slot), parent, True)
    assert torch.equal(committed, before)  # a negative step commits nothing
