"""The GDN records contract on the GPU against the oracle (kernels/gdn_tree_records.py): the path replay with its
parent rounding for 16-bit and fp32 pools, a request without records run as one chain, the fp32 chunk form, the
accepted-path commit over layers (rounded and not), and the commit of the chunk form landing on the snapshot walk's
accepted state. Outputs within the output dtype's tolerance, fp32 records and states within 1e-4 relative."""

import numpy as np
import pytest
import torch

from conftest import announce, assert_states_close
from oracle import records as orec
from oracle import recurrence as orr
from oracle.tables import _gdn_tree_paths
from workloads import seeded_tree

pytestmark = pytest.mark.gpu

SENTINEL = -999.0


def _inputs(parent_lists, heads, value_heads, dk, dv, pool_dtype, in_dtype=torch.bfloat16, seed=0, width=None):
    gen = torch.Generator().manual_seed(seed)
    N = len(parent_lists)
    width = width or max(map(len, parent_lists))
    qsl = [0]
    for p in parent_lists:
        qsl.append(qsl[-1] + len(p))
    tokens = qsl[-1]
    parent = torch.zeros(N, width, dtype=torch.int32)
    paths = np.zeros((N, width, 2 + width), dtype=np.int32)
    for n, p in enumerate(parent_lists):
        parent[n, : len(p)] = torch.tensor(p)
        parent[n, 0] = -1
        _gdn_tree_paths(list(p) + [0] * (width - len(p)), len(p), width, paths[n])
    inp = dict(
        q=torch.randn(1, tokens, heads, dk, generator=gen).to(in_dtype),
        k=torch.randn(1, tokens, heads, dk, generator=gen).to(in_dtype),
        v=torch.randn(1, tokens, value_heads, dv, generator=gen).to(in_dtype),
        a=torch.randn(tokens, value_heads, generator=gen).to(in_dtype),
        b=torch.randn(tokens, value_heads, generator=gen).to(in_dtype),
        A_log=torch.randn(value_heads, generator=gen) * 0.5,
        dt_bias=torch.randn(value_heads, generator=gen) * 0.5,
        state=(torch.randn(N + 3, value_heads, dv, dk, generator=gen) * 0.1).to(pool_dtype),
        state_indices=torch.tensor([n + 2 for n in range(N)], dtype=torch.int32),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32),
        parent=parent,
        tree_paths=torch.from_numpy(paths),
        records=torch.full((N + 1, width, value_heads, dv + dk + 4), SENTINEL),
        record_indices=torch.tensor([N - n for n in range(N)], dtype=torch.int32),  # rows in reverse
    )
    return inp, width


def _to(d, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _call(fn, inp, width, **kw):
    return fn(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"], state=inp["state"],
              state_indices=inp["state_indices"], query_start_loc=inp["query_start_loc"], parent=inp["parent"],
              records=inp["records"], record_indices=inp["record_indices"], width=width, **kw)


def _compare(got_out, want_out, got_rec, want_rec, fp32_exact, K, V):
    tol = dict(atol=1e-4, rtol=1e-4) if fp32_exact else dict(atol=2e-2, rtol=1e-2)
    # a 16-bit output may round to the neighbouring value where the fp32 results differ in the last bits
    otol = tol if got_out.dtype == torch.float32 else dict(atol=max(tol["atol"], 1e-2), rtol=max(tol["rtol"], 1e-2))
    torch.testing.assert_close(got_out.cpu().float(), want_out.float(), **otol)
    got_rec = got_rec.cpu()
    written = want_rec[..., 0] != SENTINEL
    assert torch.equal(got_rec[..., 0] != SENTINEL, written)  # the same nodes written, sentinels elsewhere
    torch.testing.assert_close(got_rec[..., :V][written], want_rec[..., :V][written], **tol)  # delta
    torch.testing.assert_close(got_rec[..., V : V + K + 1][written], want_rec[..., V : V + K + 1][written],
                               atol=1e-5, rtol=1e-5)  # key and decay
    assert torch.all(got_rec[..., V + K + 1 :] == SENTINEL)  # the record's spare floats are never written


@pytest.mark.parametrize("pool_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_path_replay_matches_oracle(dev, pool_dtype):
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update

    announce(f"records path replay pool={pool_dtype}")
    rng = np.random.default_rng(2)
    trees = [seeded_tree(rng, 16), [-1, 0, 1, 2, 3, 4], [-1, 0, 0, 1, 1, 2, 3, 5], seeded_tree(rng, 12)]
    inp, width = _inputs(trees, 4, 8, 128, 128, pool_dtype, seed=3)
    want_rec = inp["records"].clone()
    want = orec.gdn_tree_records_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"],
                                        inp["b"], state=inp["state"], state_indices=inp["state_indices"],
                                        query_start_loc=inp["query_start_loc"], parent=inp["parent"],
                                        tree_paths=inp["tree_paths"], records=want_rec,
                                        record_indices=inp["record_indices"], width=width)
    g = _to(inp, dev)
    got = _call(gdn_tree_records_update, g, width, tree_paths=g["tree_paths"])
    torch.cuda.synchronize()
    _compare(got, want, g["records"], want_rec, pool_dtype == torch.float32, 128, 128)
    assert torch.equal(g["state"].cpu(), inp["state"])  # the verify never writes the pool


def test_request_without_records_runs_as_one_chain(dev):
    """record_indices < 0: no records, and the replay runs the request's rows as one chain without rounding
    (kernels/gdn_tree_records.py:51-53), whatever its tree."""
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update

    announce("records chain rows")
    rng = np.random.default_rng(5)
    trees = [seeded_tree(rng, 16), seeded_tree(rng, 10)]
    inp, width = _inputs(trees, 2, 4, 64, 32, torch.bfloat16, seed=6)
    inp["record_indices"] = torch.tensor([-1, 1], dtype=torch.int32)
    want_rec = inp["records"].clone()
    want = orec.gdn_tree_records_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"],
                                        inp["b"], state=inp["state"], state_indices=inp["state_indices"],
                                        query_start_loc=inp["query_start_loc"], parent=inp["parent"],
                                        tree_paths=inp["tree_paths"], records=want_rec,
                                        record_indices=inp["record_indices"], width=width)
    g = _to(inp, dev)
    got = _call(gdn_tree_records_update, g, width, tree_paths=g["tree_paths"])
    torch.cuda.synchronize()
    _compare(got, want, g["records"], want_rec, False, 64, 32)


def _nested_branches(levels):
    """A chain c_0 .. c_levels whose every node but the last also has a side child s_i with one leaf, the last two
    leaves: `levels` nested nodes whose two children both have children, parent first."""
    par = [-1]
    chain = [0]
    for _ in range(levels):
        chain.append(len(par))
        par.append(chain[-2])
    side = []
    for i in range(levels):
        side.append(len(par))
        par.append(chain[i])
    for s in side:
        par.append(s)
    par += [chain[-1], chain[-1]]
    return par


def _replay_case(dev, trees, dims, in_dtype, pool_dtype, seed):
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update

    inp, width = _inputs(trees, *dims, pool_dtype, in_dtype=in_dtype, seed=seed)
    want_rec = inp["records"].clone()
    want = orec.gdn_tree_records_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"],
                                        inp["b"], state=inp["state"], state_indices=inp["state_indices"],
                                        query_start_loc=inp["query_start_loc"], parent=inp["parent"],
                                        tree_paths=inp["tree_paths"], records=want_rec,
                                        record_indices=inp["record_indices"], width=width)
    g = _to(inp, dev)
    got = _call(gdn_tree_records_update, g, width, tree_paths=g["tree_paths"])
    torch.cuda.synchronize()
    _compare(got, want, g["records"], want_rec, False, dims[2], dims[3])
    assert torch.equal(g["state"].cpu(), inp["state"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dims", [(4, 8, 128, 128), (2, 4, 64, 32), (1, 2, 256, 128), (2, 2, 32, 64)])
def test_path_replay_same_dtype_head_dims(dev, dtype, dims):
    """16-bit inputs and pool of one dtype take the matrix-core replay: trees of 1-16 nodes (a chain, a star, seeded
    ones), every head dim it covers."""
    announce(f"records path replay {dtype} dims={dims}")
    rng = np.random.default_rng(60)
    trees = [seeded_tree(rng, 16), [-1], [-1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0], [-1, 0, 1, 2, 3, 4, 5], seeded_tree(rng, 9)]
    _replay_case(dev, trees, dims, dtype, dtype, 61)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_path_replay_wide_trees(dev, dtype):
    """Trees of 17-64 nodes: stars wider than one MFMA pass of eight children, deep seeded trees."""
    announce(f"records path replay wide trees {dtype}")
    rng = np.random.default_rng(62)
    trees = [seeded_tree(rng, 64), [-1] + [0] * 30, seeded_tree(rng, 40), [-1, 0, 1] + [2] * 17]
    _replay_case(dev, trees, (2, 4, 128, 128), dtype, dtype, 63)


@pytest.mark.parametrize("levels,dims", [(4, (2, 4, 128, 128)), (6, (2, 4, 64, 64)), (3, (1, 2, 256, 128))])
def test_path_replay_nested_branches_outgrow_the_parked_states(dev, levels, dims):
    """More nested nodes with two branching children than the replay parks: the oldest parked states are dropped and
    recomputed from the pool state along their root paths."""
    announce(f"records path replay nested branches levels={levels} dims={dims}")
    rng = np.random.default_rng(64)
    _replay_case(dev, [_nested_branches(levels), seeded_tree(rng, 12)], dims, torch.bfloat16, torch.bfloat16, 65)


@pytest.mark.parametrize("dims", [(4, 8, 128, 128), (2, 2, 64, 32), (1, 2, 256, 128)])
def test_chunk_form_matches_oracle_closed_form(dev, dims):
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update

    announce(f"records chunk form dims={dims}")
    rng = np.random.default_rng(7)
    trees = [seeded_tree(rng, 16), [-1, 0, 1, 1, 0], seeded_tree(rng, 9)]
    inp, width = _inputs(trees, *dims, torch.float32, seed=8)
    want_rec = inp["records"].clone()
    want = orec.gdn_tree_chunk_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
                                      state=inp["state"], state_indices=inp["state_indices"],
                                      query_start_loc=inp["query_start_loc"], parent=inp["parent"], records=want_rec,
                                      record_indices=inp["record_indices"], width=width)
    g = _to(inp, dev)
    got = _call(gdn_tree_records_update, g, width, tree_paths=None)  # fp32 pool without paths: the chunk form
    torch.cuda.synchronize()
    _compare(got, want, g["records"], want_rec, True, dims[2], dims[3])


def _relabelled_tree(rng, n):
    """A seeded tree with its non-root nodes relabelled at random: rows are no longer parent-first."""
    base = seeded_tree(rng, n)
    label = [0] + [int(x) for x in rng.permutation(np.arange(1, n))]
    par = [-1] * n
    for old in range(1, n):
        par[label[old]] = label[base[old]]
    return par


def _chunk_case(dev, trees, dims, pool_dtype, seed, edit=None):
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_chunk_update

    inp, width = _inputs(trees, *dims, pool_dtype, seed=seed)
    if edit is not None:
        edit(inp)
    want_rec = inp["records"].clone()
    want = orec.gdn_tree_chunk_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
                                      state=inp["state"], state_indices=inp["state_indices"],
                                      query_start_loc=inp["query_start_loc"], parent=inp["parent"], records=want_rec,
                                      record_indices=inp["record_indices"], width=width)
    g = _to(inp, dev)
    got = _call(gdn_tree_chunk_update, g, width)
    torch.cuda.synchronize()
    _compare(got, want, g["records"], want_rec, True, dims[2], dims[3])
    assert torch.equal(g["state"].cpu(), inp["state"])  # the verify never writes the pool


@pytest.mark.parametrize("pool_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_chunk_form_any_pool_and_edge_requests(dev, pool_dtype):
    """The chunk form with 16-bit pools too (state read as is, never rounded), 3 value heads per key head, and the
    edge requests: rows not parent-first, a single node, an empty request, a request without a pool slot (zero
    state) and one without records."""
    announce(f"records chunk form pool={pool_dtype} edges")
    rng = np.random.default_rng(21)
    trees = [seeded_tree(rng, 16), _relabelled_tree(rng, 16), [-1], [], seeded_tree(rng, 11), _relabelled_tree(rng, 7),
             list(range(-1, 15))]

    def edit(inp):
        inp["state_indices"][4] = -1  # no pool slot: the tree starts from zeros
        inp["record_indices"][5] = -1  # outputs only

    _chunk_case(dev, trees, (2, 6, 128, 128), pool_dtype, 22, edit)


@pytest.mark.parametrize("dims", [(1, 1, 32, 16), (2, 4, 64, 64), (1, 3, 256, 32)])
def test_chunk_form_head_dims(dev, dims):
    """Key dims 32 / 64 / 256 and value dims 16 / 32 / 64 (one, two and four 16-column tiles per wave)."""
    announce(f"records chunk form dims={dims}")
    rng = np.random.default_rng(31)
    trees = [seeded_tree(rng, 16), _relabelled_tree(rng, 13), seeded_tree(rng, 5)]
    _chunk_case(dev, trees, dims, torch.bfloat16, 32)


@pytest.mark.parametrize("pool_dtype", [torch.bfloat16, torch.float32])
def test_chunk_form_batch_tilings(dev, pool_dtype):
    """A batch large enough for the wider column slices: 64 requests x 16 value heads take four 16-column tiles per
    wave with a bf16 pool, two with an fp32 pool."""
    announce(f"records chunk form batch 64 pool={pool_dtype}")
    rng = np.random.default_rng(51)
    trees = [seeded_tree(rng, int(rng.integers(1, 17))) for _ in range(64)]
    _chunk_case(dev, trees, (4, 16, 128, 128), pool_dtype, 52)


def test_chunk_form_wide_trees_walk(dev):
    """Trees wider than 16 nodes take the depth-first walk; the same closed form."""
    announce("records chunk form width 24")
    rng = np.random.default_rng(41)
    trees = [seeded_tree(rng, 24), seeded_tree(rng, 20), [-1, 0, 0, 1]]
    _chunk_case(dev, trees, (2, 4, 128, 128), torch.float32, 42)


def test_deep_branching_replays_unparked_parents(dev):
    """More nested branches than the walk parks: the deepest parents are recomputed from the pool state."""
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update

    announce("records deep branching")
    nested = [-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 0, 1, 2, 3, 4, 5]
    for pool_dtype in (torch.bfloat16, torch.float32):
        inp, width = _inputs([nested, nested[:9]], 2, 4, 128, 128, pool_dtype, seed=9)
        want_rec = inp["records"].clone()
        want = orec.gdn_tree_records_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"],
                                            inp["b"], state=inp["state"], state_indices=inp["state_indices"],
                                            query_start_loc=inp["query_start_loc"], parent=inp["parent"],
                                            tree_paths=inp["tree_paths"], records=want_rec,
                                            record_indices=inp["record_indices"], width=width)
        g = _to(inp, dev)
        got = _call(gdn_tree_records_update, g, width, tree_paths=g["tree_paths"])
        torch.cuda.synchronize()
        _compare(got, want, g["records"], want_rec, pool_dtype == torch.float32, 128, 128)


@pytest.mark.parametrize("pool_dtype,round_state", [(torch.bfloat16, True), (torch.float32, False),
                                                    (torch.float16, True)])
def test_commit_matches_oracle_over_layers(dev, pool_dtype, round_state):
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_commit

    announce(f"records commit pool={pool_dtype} round={round_state}")
    gen = torch.Generator().manual_seed(11)
    layers, N, width, HV, K, V = 2, 4, 8, 4, 128, 128
    parent = torch.tensor([[-1, 0, 0, 1, 1, 2, 3, 5]] * N, dtype=torch.int32)
    state = (torch.randn(layers, N + 2, HV, V, K, generator=gen) * 0.1).to(pool_dtype)
    records = torch.randn(layers, N + 1, width, HV, V + K + 4, generator=gen) * 0.1
    records[..., V + K] = torch.rand(layers, N + 1, width, HV, generator=gen) * 0.5 + 0.5  # decays in (0.5, 1)
    state_indices = torch.tensor([1, 2, -1, 4], dtype=torch.int32)  # request 2: no slot
    record_indices = torch.tensor([3, 0, 1, 2], dtype=torch.int32)
    commit_steps = torch.tensor([7, 0, 5, -1], dtype=torch.int32)  # request 3: nothing accepted
    want = state.clone()
    orec.gdn_tree_records_commit(want, records, state_indices, record_indices, commit_steps, parent, round_state)
    got = state.to(dev)
    gdn_tree_records_commit(got, records.to(dev), state_indices.to(dev), record_indices.to(dev),
                            commit_steps.to(dev), parent.to(dev), round_state)
    torch.cuda.synchronize()
    if pool_dtype == torch.float32:
        assert_states_close(got.cpu(), want)
    else:
        torch.testing.assert_close(got.cpu().float(), want.float(), atol=1e-2, rtol=1e-2)
    untouched = [0, 3, 4, 5]  # slots no committed request names
    assert torch.equal(got.cpu()[:, untouched], state[:, untouched])


def test_chunk_then_commit_lands_on_the_walks_accepted_state(dev):
    """fp32: the chunk form's records folded along an accepted path give the snapshot walk's state of that node."""
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_commit, gdn_tree_records_update

    announce("records chunk + commit vs walk")
    tree = [-1, 0, 0, 1, 2, 4, 4, 3]
    accepted = 6
    inp, width = _inputs([tree], 2, 4, 128, 128, torch.float32, seed=12)
    g = _to(inp, dev)
    _call(gdn_tree_records_update, g, width, tree_paths=None)
    pool = g["state"].clone()[None]  # one layer
    gdn_tree_records_commit(pool, g["records"][None], g["state_indices"], g["record_indices"],
                            torch.tensor([accepted], dtype=torch.int32, device=dev), g["parent"], False)
    torch.cuda.synchronize()
    # the oracle walk with one snapshot slot per row
    T = len(tree)
    snaps = torch.zeros(2 + T, 4, 128, 128)
    snaps[1] = inp["state"][int(inp["state_indices"][0])]
    slots = torch.arange(1, T + 2, dtype=torch.int32)[None]
    orr.gdn_tree_recurrent_update(inp["A_log"], inp["dt_bias"], inp["q"], inp["k"], inp["v"], inp["a"], inp["b"],
                                  initial_state_source=snaps, initial_state_indices=slots,
                                  cu_seqlens=inp["query_start_loc"], intermediate_states_buffer=snaps,
                                  intermediate_state_indices=slots, retrieve_parent_token=inp["parent"],
                                  num_accepted_tokens=torch.tensor([1], dtype=torch.int32), pad_slot_id=0)
    want = snaps[int(slots[0, accepted])]
    assert_states_close(pool[0, int(inp["state_indices"][0])].cpu(), want)


def _per_node_rounded(q, k, v, a, b, A, bias, state, slots, parent, width, batch, hv, h, rounded):
    """Every node's state from its parent's, the parent rounded to the pool dtype first when ``rounded`` (the
    reference test's independent form, tests/test_gdn_rounded_records_gpu.py:46-65): (outputs like v, per-request
    node states)."""
    K = k.shape[-1]
    expected = torch.empty_like(v)
    snapshots = []
    for request in range(batch):
        states = []
        for node in range(width):
            token = request * width + node
            prior = state[int(slots[request])].float() if node == 0 else states[int(parent[request, node])]
            if rounded and node > 0:
                prior = prior.to(state.dtype).float()
            key = k[0, token].float()
            key = key / (key.square().sum(-1, keepdim=True) + 1e-6).sqrt()
            query = q[0, token].float()
            query = query / (query.square().sum(-1, keepdim=True) + 1e-6).sqrt() / K**0.5
            key, query = key.repeat_interleave(hv // h, 0), query.repeat_interleave(hv // h, 0)
            decay = (-A.exp() * torch.nn.functional.softplus(a[token].float() + bias)).exp()
            beta = b[token].float().sigmoid().to(b.dtype).float()
            decayed = prior * decay[:, None, None]
            delta = (v[0, token].float() - (decayed * key[:, None, :]).sum(-1)) * beta[:, None]
            current = decayed + delta[:, :, None] * key[:, None, :]
            states.append(current)
            expected[0, token] = (current * query[:, None, :]).sum(-1).to(v.dtype)
        snapshots.append(states)
    return expected, snapshots


@pytest.mark.parametrize("width,batch", [(1, 1), (8, 2), (16, 1), (32, 2)])
@pytest.mark.parametrize("state_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rounded", [True, False], ids=["path_replay", "chunk"])
def test_reference_rounded_records_scenario(dev, width, batch, state_dtype, rounded):
    """The reference's own GPU scenario (tests/test_gdn_rounded_records_gpu.py:10-113): one path row per node (each
    writing only its node), slots and record rows in reverse, a parent table wider than the tree, spare record steps
    and rows left alone; outputs against the per-node form (rounded parents for the path replay, none for the chunk)
    and the oracle; the commit of the last node against its state; a negative step and an int64 parent table."""
    from eagle_harness.kernels.gdn_tree_records import (gdn_tree_chunk_update, gdn_tree_records_commit,
                                                        gdn_tree_records_update)

    announce(f"records reference scenario width={width} batch={batch} {state_dtype} rounded={rounded}")
    gen = torch.Generator().manual_seed(41 + width)
    h, hv, K, V = 4, 12, 128, 128

    def rand(*shape, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=gen) * 0.2).to(dtype)

    q, k = rand(1, batch * width, h, K), rand(1, batch * width, h, K)
    v = rand(1, batch * width, hv, V)
    a, b = rand(batch * width, hv), rand(batch * width, hv)
    A, bias = rand(hv, dtype=torch.float32), rand(hv, dtype=torch.float32)
    state = rand(batch + 2, hv, V, K, dtype=state_dtype)
    slots = torch.arange(1, batch + 1, dtype=torch.int32).flip(0)
    rows = torch.arange(batch, dtype=torch.int32).flip(0)
    qsl = torch.arange(batch + 1, dtype=torch.int32) * width
    parent = torch.zeros(batch, width + 7, dtype=torch.int32)
    for node in range(1, width):
        parent[:, node] = torch.randint(node, (batch,), generator=gen, dtype=torch.int32)
    paths = torch.zeros(batch, width, width + 2, dtype=torch.int32)
    for request in range(batch):
        for node in range(width):
            chain = [node]
            while chain[-1] > 0:
                chain.append(int(parent[request, chain[-1]]))
            chain.reverse()
            paths[request, node, 0], paths[request, node, 1] = len(chain), len(chain) - 1
            paths[request, node, 2 : 2 + len(chain)] = torch.tensor(chain, dtype=torch.int32)
    rec = torch.full((batch + 1, width + 3, hv, V + K + 4), SENTINEL)
    expected, snapshots = _per_node_rounded(q, k, v, a, b, A, bias, state, slots, parent, width, batch, hv, h, rounded)
    want_rec = rec.clone()
    if rounded:
        want = orec.gdn_tree_records_update(A, bias, q, k, v, a, b, state=state, state_indices=slots,
                                            query_start_loc=qsl, parent=parent, tree_paths=paths, records=want_rec,
                                            record_indices=rows, width=width)
    else:
        want = orec.gdn_tree_chunk_update(A, bias, q, k, v, a, b, state=state, state_indices=slots,
                                          query_start_loc=qsl, parent=parent, records=want_rec, record_indices=rows,
                                          width=width)
    # the oracle against the per-node form first (outputs are 16-bit: a rounding step apart at most)
    torch.testing.assert_close(want.float(), expected.float(), atol=2e-3, rtol=2e-2)
    g = _to(dict(q=q, k=k, v=v, a=a, b=b, A=A, bias=bias, state=state, slots=slots, rows=rows, qsl=qsl,
                 parent=parent, paths=paths, rec=rec), dev)
    kw = dict(state=g["state"], state_indices=g["slots"], query_start_loc=g["qsl"], parent=g["parent"],
              records=g["rec"], record_indices=g["rows"], width=width)
    if rounded:
        out = gdn_tree_records_update(g["A"], g["bias"], g["q"], g["k"], g["v"], g["a"], g["b"], tree_paths=g["paths"],
                                      **kw)
    else:
        out = gdn_tree_chunk_update(g["A"], g["bias"], g["q"], g["k"], g["v"], g["a"], g["b"], **kw)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), expected.float(), atol=2e-3, rtol=2e-2)
    _compare(out, want, g["rec"], want_rec, False, K, V)
    assert bool((g["rec"][-1] == SENTINEL).all().item())  # the unused record row
    accepted = torch.full((batch,), width - 1, dtype=torch.int32, device=dev)
    committed = g["state"].clone().unsqueeze(0)
    gdn_tree_records_commit(committed, g["rec"].unsqueeze(0), g["slots"], g["rows"], accepted, g["parent"], rounded)
    torch.cuda.synchronize()
    for request in range(batch):
        torch.testing.assert_close(committed[0, int(slots[request])].cpu().float(),
                                   snapshots[request][-1].to(state_dtype).float(), atol=2e-3, rtol=2e-2)
    assert torch.equal(committed[0, 0].cpu(), state[0]) and torch.equal(committed[0, -1].cpu(), state[-1])
    before = committed.clone()
    gdn_tree_records_commit(committed, g["rec"].unsqueeze(0), g["slots"], g["rows"], -torch.ones_like(accepted),
                            g["parent"], rounded)
    torch.cuda.synchronize()
    assert torch.equal(committed, before)  # a negative step touches nothing
    from_int64 = g["state"].clone().unsqueeze(0)
    gdn_tree_records_commit(from_int64, g["rec"].unsqueeze(0), g["slots"], g["rows"], accepted,
                            g["parent"].to(torch.int64), rounded)
    torch.cuda.synchronize()
    assert torch.equal(from_int64, committed)


def test_parent_rounding_does_not_accumulate_sub_ulp_decay_on_the_device(dev):
    """The reference's known answer (tests/test_gdn_rounded_records_gpu.py:116-162): a 32-node chain from an all-ones
    bf16 state whose per-node decay is below half a bf16 ulp — every rounded parent is the pool state again, so every
    output is the first one and the rounded commit leaves the pool bit for bit."""
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_commit, gdn_tree_records_update

    announce("records sub-ulp decay chain")
    width, dim = 32, 128
    state = torch.ones(1, 1, dim, dim, device=dev, dtype=torch.bfloat16)
    q = torch.zeros(1, width, 1, dim, device=dev, dtype=torch.bfloat16)
    q[..., 0] = 1
    k, v = torch.zeros_like(q), torch.zeros_like(q)
    a = torch.full((width, 1), -7.0, device=dev, dtype=torch.bfloat16)
    b = torch.zeros_like(a)
    A = torch.zeros(1, device=dev)
    slot = torch.zeros(1, device=dev, dtype=torch.int32)
    qsl = torch.tensor([0, width], device=dev, dtype=torch.int32)
    parent = (torch.arange(width, device=dev, dtype=torch.int32) - 1).view(1, width)
    paths = torch.cat((torch.tensor([width, 0], device=dev, dtype=torch.int32),
                       torch.arange(width, device=dev, dtype=torch.int32))).view(1, 1, width + 2)
    records = torch.empty(1, width, 1, dim * 2 + 4, device=dev)
    out = gdn_tree_records_update(A, A, q, k, v, a, b, state=state, state_indices=slot, query_start_loc=qsl,
                                  parent=parent, tree_paths=paths, records=records, record_indices=slot, width=width)
    torch.cuda.synchronize()
    assert torch.equal(out, out[:, :1].expand_as(out))
    committed = state.clone().unsqueeze(0)
    gdn_tree_records_commit(committed, records.unsqueeze(0), slot, slot, torch.full_like(slot, width - 1), parent,
                            True)
    torch.cuda.synchronize()
    assert torch.equal(committed[0], state)


def test_commit_layer_offsets_past_2_31_elements(dev):
    """The reference's known answer for 64-bit layer offsets (tests/test_gdn_tree_records_gpu.py:94-122): a pool
    whose later layers start past 2^31 elements, behind a guard region one layer long; the commit lands only in its
    slot of every layer."""
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_commit

    announce("records commit past 2^31 elements")
    heads, dim, slots = 8, 128, 8193
    layer = slots * heads * dim * dim
    assert layer < 2**31 <= 2 * layer
    pool = torch.zeros(4 * layer, dtype=torch.bfloat16, device=dev)
    guard, state = pool[:layer], pool[layer:].view(3, slots, heads, dim, dim)
    slot = slots - 1
    gen = torch.Generator(device=dev).manual_seed(5)
    before = torch.randn(3, heads, dim, dim, generator=gen, device=dev).to(torch.bfloat16)
    state[:, slot] = before
    records = torch.randn(3, 1, 1, heads, 2 * dim + 4, generator=gen, device=dev)
    records[..., 2 * dim] = torch.rand(3, 1, 1, heads, generator=gen, device=dev)
    one = torch.ones(1, dtype=torch.int32, device=dev)
    root = torch.zeros(1, 1, dtype=torch.int32, device=dev)
    gdn_tree_records_commit(state, records, one * slot, one * 0, one * 0, root, False)
    torch.cuda.synchronize()
    delta, key, decay = records[:, 0, 0, :, :dim], records[:, 0, 0, :, dim : 2 * dim], records[:, 0, 0, :, 2 * dim]
    want = before.float() * decay[..., None, None] + delta[..., :, None] * key[..., None, :]
    torch.testing.assert_close(state[:, slot].float(), want.to(torch.bfloat16).float(), atol=0.01, rtol=0.01)
    assert not guard.any().item(), "a layer's commit landed outside the pool"
    assert not state[:, :slot].any().item(), "a commit landed in another slot"
    del pool
