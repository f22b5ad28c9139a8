"""Pins of the CPU oracle of the Mamba2 tree state update (oracle/mamba2.py): closed forms along each node's root
path (x = 0: the start state decayed by exp(A * sum of dt); A = 0: the start state plus the sum of dt B x^T, read
by C, plus D x), every tree node = the chain of its root path, pad slots (never written, read as zeros), the start
row num_accepted - 1, and with a 16-bit pool a branch child reads its parent's rounded slot while a chain child
continues from the unrounded state (kernels/mamba2_tree.py:99-149)."""

import math

import torch

from oracle import mamba2 as om

TREE = [-1, 0, 0, 1, 2, 2, 4, 1]


def _case(parents_list, heads=2, head_dim=3, dstate=4, groups=1, seed=0, pool_dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    W = len(parents_list)
    x = torch.randn(W, heads, head_dim, generator=gen, dtype=torch.float64)
    dt = torch.randn(W, heads, generator=gen, dtype=torch.float64)
    A = -torch.rand(heads, generator=gen, dtype=torch.float64)
    B = torch.randn(W, groups, dstate, generator=gen, dtype=torch.float64)
    C = torch.randn(W, groups, dstate, generator=gen, dtype=torch.float64)
    D = torch.randn(heads, generator=gen, dtype=torch.float64)
    bias = torch.randn(heads, generator=gen, dtype=torch.float64)
    state = torch.randn(W + 2, heads, head_dim, dstate, generator=gen, dtype=torch.float64).to(pool_dtype)
    slots = torch.arange(1, W + 1, dtype=torch.int32).view(1, W)
    parents = torch.tensor([parents_list], dtype=torch.int32)
    qsl = torch.tensor([0, W], dtype=torch.int32)
    return dict(state=state, x=x, dt=dt, A=A, B=B, C=C, D=D, dt_bias=bias, slots=slots, parents=parents, qsl=qsl)


def _run(c, **kw):
    state = c["state"].clone()
    out = torch.zeros_like(c["x"])
    om.mamba2_tree_state_update(state, c["x"], c["dt"], c["A"], c["B"], c["C"], c.get("Dv", c["D"]), c["dt_bias"], out,
                                state_indices=c["slots"], parents=c["parents"], query_start_loc=c["qsl"], **kw)
    return out, state


def _path(parents_list, t):
    p = [t]
    while parents_list[p[-1]] >= 0:
        p.append(parents_list[p[-1]])
    return p[::-1]


def _sp(v):
    return math.log(math.exp(v) + 1.0) if v <= 20 else v


def test_zero_inputs_decay_the_start_state_along_the_root_path():
    c = _case(TREE, seed=1)
    c["x"].zero_()
    out, _ = _run(c)
    s0 = c["state"][1]  # slots[0, 0]: the start state
    for t in range(len(TREE)):
        for h in range(2):
            total = sum(_sp(float(c["dt"][u, h] + c["dt_bias"][h])) for u in _path(TREE, t))
            want = math.exp(float(c["A"][h]) * total) * (s0[h] @ c["C"][t, 0])
            torch.testing.assert_close(out[t, h], want, rtol=1e-12, atol=1e-12)


def test_no_decay_sums_the_root_path_inputs():
    c = _case(TREE, seed=2)
    c["A"].zero_()
    out, _ = _run(c, dt_softplus=False)
    s0 = c["state"][1]
    for t in range(len(TREE)):
        for h in range(2):
            s = s0[h].clone()
            for u in _path(TREE, t):
                s += float(c["dt"][u, h] + c["dt_bias"][h]) * torch.outer(c["x"][u, h], c["B"][u, 0])
            want = s @ c["C"][t, 0] + float(c["D"][h]) * c["x"][t, h]
            torch.testing.assert_close(out[t, h], want, rtol=1e-12, atol=1e-12)


def test_every_node_is_the_chain_of_its_root_path():
    c = _case(TREE, seed=3)
    out, state = _run(c)
    for t in range(len(TREE)):
        path = _path(TREE, t)
        n = len(path)
        sub = dict(c)
        sub.update(x=c["x"][path], dt=c["dt"][path], B=c["B"][path], C=c["C"][path],
                   slots=torch.tensor([[1] + list(range(20, 19 + n))], dtype=torch.int32) if n > 1 else
                   torch.tensor([[1]], dtype=torch.int32),
                   parents=torch.tensor([[-1] + list(range(n - 1))], dtype=torch.int32),
                   qsl=torch.tensor([0, n], dtype=torch.int32),
                   state=torch.cat([c["state"], torch.zeros(20, *c["state"].shape[1:], dtype=c["state"].dtype)]))
        o_chain, s_chain = _run(sub)
        torch.testing.assert_close(out[t], o_chain[-1], rtol=1e-12, atol=1e-12)
        last = int(sub["slots"][0, n - 1])
        torch.testing.assert_close(state[t + 1], s_chain[last], rtol=1e-12, atol=1e-12)


def test_pad_slots_and_the_start_row():
    c = _case(TREE, seed=4)
    c["slots"][0, 2] = -1  # row 2 is not stored; its children (rows 4, 5) start from zeros
    c["slots"][0, 0] = -1  # row 0's slot is pad: the start state reads as zeros, row 0 is not stored
    before = c["state"].clone()
    out, state = _run(c)
    assert torch.equal(state[1], before[1]) and torch.equal(state[3], before[3])  # slots 1 (row 0), 3 (row 2) kept
    zero = dict(c)
    zero.update(state=torch.zeros_like(c["state"]), parents=torch.tensor([[-1]], dtype=torch.int32),
                slots=torch.tensor([[7]], dtype=torch.int32), qsl=torch.tensor([0, 1], dtype=torch.int32),
                x=c["x"][4:5], dt=c["dt"][4:5], B=c["B"][4:5], C=c["C"][4:5])
    torch.testing.assert_close(out[4], _run(zero)[0][0], rtol=1e-12, atol=1e-12)  # row 4 = a fresh start from zeros
    # num_accepted 2: row 0 starts from slots[0, 1], the same as moving that state into column 0's slot
    c2 = _case(TREE, seed=5)
    out2, _ = _run(c2, num_accepted_tokens=torch.tensor([2], dtype=torch.int32))
    c3 = dict(c2)
    c3["state"] = c2["state"].clone()
    c3["state"][1] = c2["state"][2]  # the state of slot 2 moved to column 0's slot
    torch.testing.assert_close(out2, _run(c3)[0], rtol=0, atol=0)


def test_bf16_pool_branch_children_read_the_rounded_parent():
    c = _case([-1, 0, 0], seed=6, pool_dtype=torch.bfloat16)
    out, state = _run(c)
    # row 2 (a branch) = a one-row request started from row 0's stored slot
    one = dict(c)
    one.update(state=state.clone(), parents=torch.tensor([[-1]], dtype=torch.int32),
               slots=torch.tensor([[1]], dtype=torch.int32), qsl=torch.tensor([0, 1], dtype=torch.int32),
               x=c["x"][2:3], dt=c["dt"][2:3], B=c["B"][2:3], C=c["C"][2:3])
    o_branch = _run(one)[0][0]
    torch.testing.assert_close(out[2], o_branch, rtol=0, atol=0)
    # row 1 (a chain child) continues unrounded: it differs from a start at row 0's rounded slot
    one.update(x=c["x"][1:2], dt=c["dt"][1:2], B=c["B"][1:2], C=c["C"][1:2])
    assert not torch.equal(out[1], _run(one)[0][0])
