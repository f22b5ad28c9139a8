"""The Mamba2 tree state update on the GPU against the oracle (kernels/mamba2_tree.py:41-240): the reference test's
per-rank shapes (tests/test_mamba2_tree_verify_gpu.py:33-38: Nemotron 3 Nano at TP1 / TP4 with fp32 SSM states,
Nemotron 3.5 Super at TP4 with a bf16 state pool), chains and random trees, accepted counts, pad slots, dstate 64 and
256, fp16 inputs. Outputs within 2e-2 abs / 1e-2 rel (16-bit outputs); fp32 states within 1e-5 abs / 1e-4 rel, 16-bit
pool states within 1e-2; 64-row trees with a 16-bit pool within the reference test's 16-bit tolerances."""

import random

import pytest
import torch

from conftest import announce
from oracle import mamba2 as om

pytestmark = pytest.mark.gpu

SHAPES = {  # (heads, head_dim, groups, dstate, state dtype)
    "tp1": (64, 64, 8, 128, torch.float32),
    "tp4": (16, 64, 2, 128, torch.float32),
    "super-tp4": (32, 64, 2, 128, torch.bfloat16),
    "d64": (8, 32, 2, 64, torch.float32),
    "d256": (4, 64, 1, 256, torch.bfloat16),
}


def _tree(kind, width, rng):
    if kind == "chain":
        return [-1] + list(range(width - 1))
    return [-1] + [rng.randrange(t) for t in range(1, width)]


# The reference test's tolerances for 16-bit state pools (tests/test_mamba2_tree_kernels.py:103-109): a state's last
# bit can round either way where the fp32 arithmetic differs in its last bit, and deep trees carry such flips on.
REF_TOL = {torch.float16: (2e-3, 1e-2), torch.bfloat16: (2e-2, 1e-1)}  # (state, output)


def _case(dev, shape, trees, seed, in_dtype=torch.bfloat16, pads=(), accepted=None, ref_tol=False):
    heads, head_dim, groups, dstate, sdt = SHAPES[shape]
    gen = torch.Generator().manual_seed(seed)
    width = max(map(len, trees))
    bs = len(trees)
    qsl = torch.tensor([0] + [sum(map(len, trees[: i + 1])) for i in range(bs)], dtype=torch.int32)
    tokens = int(qsl[-1])
    parents = torch.full((bs, width), -1, dtype=torch.int32)
    for b, tr in enumerate(trees):
        parents[b, : len(tr)] = torch.tensor(tr)
    slots = (2 + torch.arange(bs * width, dtype=torch.int32)).view(bs, width)
    for b, t in pads:
        slots[b, t] = -1
    state = (torch.randn(2 + bs * width, heads, head_dim, dstate, generator=gen) * 0.5).to(sdt)
    x = torch.randn(tokens, heads, head_dim, generator=gen).to(in_dtype)
    dt = torch.randn(tokens, heads, generator=gen).to(in_dtype)
    A = -torch.rand(heads, generator=gen)
    BC = torch.randn(tokens, 2, groups, dstate, generator=gen).to(in_dtype)
    B, C = BC[:, 0], BC[:, 1]  # token-strided views of one buffer
    D, bias = torch.randn(heads, generator=gen), torch.randn(heads, generator=gen)
    acc = None if accepted is None else torch.tensor(accepted, dtype=torch.int32)
    kw = dict(state_indices=slots, parents=parents, query_start_loc=qsl, num_accepted_tokens=acc, pad_slot_id=-1)
    s_want, o_want = state.clone(), torch.zeros(tokens, heads, head_dim, dtype=in_dtype)
    om.mamba2_tree_state_update(s_want, x, dt, A, B, C, D, bias, o_want, **kw)
    from eagle_harness.kernels.mamba2_tree import mamba2_tree_state_update

    g = lambda t: None if t is None else t.to(dev)  # noqa: E731
    s_got, o_got = g(state), torch.zeros(tokens, heads, head_dim, dtype=in_dtype, device=dev)
    BCd = g(BC)
    mamba2_tree_state_update(s_got, g(x), g(dt), g(A), BCd[:, 0], BCd[:, 1], g(D), g(bias), o_got,
                             **{k: g(v) if isinstance(v, torch.Tensor) else v for k, v in kw.items()})
    torch.cuda.synchronize()
    if ref_tol and sdt != torch.float32:
        st_tol, out_tol = REF_TOL[sdt]
        torch.testing.assert_close(o_got.cpu().float(), o_want.float(), atol=out_tol, rtol=out_tol)
        torch.testing.assert_close(s_got.cpu().float(), s_want.float(), atol=st_tol, rtol=st_tol)
        return
    torch.testing.assert_close(o_got.cpu().float(), o_want.float(), atol=2e-2, rtol=1e-2)
    if sdt == torch.float32:
        torch.testing.assert_close(s_got.cpu(), s_want, atol=1e-5, rtol=1e-4)
    else:
        torch.testing.assert_close(s_got.cpu().float(), s_want.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("shape", ["tp1", "tp4", "super-tp4"])
@pytest.mark.parametrize("kind,width,bs", [("chain", 8, 1), ("tree", 16, 1), ("tree", 16, 4), ("tree", 5, 3)])
def test_reference_shapes_match_oracle(dev, shape, kind, width, bs):
    announce(f"mamba2 {shape} {kind} width={width} bs={bs}")
    rng = random.Random(width * 10 + bs)
    _case(dev, shape, [_tree(kind, width, rng) for _ in range(bs)], seed=bs + width)


@pytest.mark.parametrize("shape", ["d64", "d256"])
def test_other_state_sizes_and_fp16(dev, shape):
    announce(f"mamba2 {shape} fp16")
    rng = random.Random(3)
    _case(dev, shape, [_tree("tree", 12, rng), _tree("tree", 7, rng)], seed=7, in_dtype=torch.float16)


# A complete binary tree (16 nodes): walked neediest-child-last it needs three parked states, one more than the stack
# holds; nodes 0..5 with two children each, the lower-index one leading deeper: in index order (16-bit pools) six
# states are parked at once. Both make the walk reload states from their slots.
BINARY = [-1] + [(i - 1) // 2 for i in range(1, 16)]
NESTED = [-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("shape", ["tp4", "super-tp4", "d256"])
def test_trees_beyond_the_parked_states(dev, shape):
    announce(f"mamba2 parked-state overflow {shape}")
    rng = random.Random(11)
    _case(dev, shape, [BINARY, NESTED, _tree("tree", 16, rng), [-1] + [0] * 15], seed=13)


@pytest.mark.parametrize("shape", ["tp4", "super-tp4"])
def test_depth_first_plans_up_to_64_rows(dev, shape):
    """64-row requests (random, a 64-row chain, a comb: even rows a spine, each with a leaf) and a 33-row one: the
    widest depth-first plans (every round of the plan's pointer jumping, up to 63 tree levels). A bf16 pool is held
    to the reference test's bf16 tolerances: over 20-60 levels two outputs of 460800 move by a bf16 step or two."""
    announce(f"mamba2 64-row plans {shape}")
    rng = random.Random(17)
    comb = [-1] + [2 * ((i - 1) // 2) for i in range(1, 64)]
    _case(dev, shape, [_tree("tree", 64, rng), _tree("chain", 64, rng), comb, _tree("tree", 33, rng)], seed=19,
          ref_tol=True)


def test_accepted_counts_pads_and_ragged_requests(dev):
    """Row 0 of each request from slots[b, accepted - 1]; pad slots neither written nor read (zeros); an empty
    request between two others."""
    announce("mamba2 accepted pads ragged")
    rng = random.Random(5)
    trees = [_tree("tree", 16, rng), [], _tree("tree", 9, rng)]
    # qsl of an empty request: the tree list holds an empty list; parents / slots rows are padded
    _case(dev, "tp4", trees, seed=9, pads=((0, 3), (2, 0)), accepted=[3, 1, 2])


def test_mamba2_layer_front_views(dev):
    """TreeVerify.forward_mamba2_spec_rows (vllm/gdn_tree_verify.py:107-148): the tree conv over [x | B | C], then
    the state update on views of the conv output, equals the two kernels run by hand on contiguous copies, bit for
    bit, and the state update matches the oracle on the conv's own x / B / C."""
    from types import SimpleNamespace

    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.mamba2_tree import mamba2_tree_state_update
    from eagle_harness.vllm.gdn_tree_verify import TreeVerify
    from eagle_harness.vllm.verify_layout import set_stage
    from oracle.tables import window_codes

    announce("mamba2 layer front views")
    rng = random.Random(11)
    heads, head_dim, groups, dstate = 16, 64, 2, 128
    trees = [_tree("tree", 16, rng) for _ in range(3)]
    bs, W = len(trees), 16
    tokens, dim = bs * W, heads * head_dim + 2 * groups * dstate
    gen = torch.Generator().manual_seed(12)
    xbc = torch.randn(tokens, dim, generator=gen).bfloat16().to(dev)
    conv_w = (torch.randn(dim, 4, generator=gen) * 0.3).bfloat16().to(dev)
    conv_state = torch.zeros(1 + bs * (W + 1), dim, 3 + W, dtype=torch.bfloat16)
    slots = (1 + torch.arange(bs * (W + 1), dtype=torch.int32)).view(bs, W + 1)
    conv_state[slots[:, 0].long(), :, :3] = torch.randn(bs, dim, 3, generator=gen).bfloat16()
    anc = torch.tensor([list(zip(*window_codes(p))) for p in trees], dtype=torch.int32).to(dev)
    parents = torch.tensor(trees, dtype=torch.int32).to(dev)
    ssm = (torch.randn(1 + bs * (W + 1), heads, head_dim, dstate, generator=gen) * 0.5).to(dev)
    dt = torch.randn(tokens, heads, generator=gen).bfloat16().to(dev)
    A, D, bias = -torch.rand(heads, generator=gen).to(dev), torch.randn(heads).to(dev), torch.randn(heads).to(dev)
    qsl = torch.arange(0, tokens + 1, W, dtype=torch.int32).to(dev)
    acc = torch.ones(bs, dtype=torch.int32, device=dev)
    slots, conv_state = slots.to(dev), conv_state.to(dev)

    rows = SimpleNamespace(hidden_states_B_C=xbc, conv_state=conv_state.clone(), conv_weight=conv_w, conv_bias=None,
                           activation="silu", state_indices=slots, query_start_loc=qsl, num_accepted_tokens=acc,
                           num_heads=heads, head_dim=head_dim, n_groups=groups, ssm_state_size=dstate,
                           ssm_state=ssm.clone(), dt=dt, A=A, D=D, dt_bias=bias, layer_name="layers.1.mixer",
                           out=torch.zeros(tokens, heads * head_dim, dtype=torch.bfloat16, device=dev))
    set_stage(SimpleNamespace(ancestors=anc, parents=parents, state_slots={}))
    try:
        TreeVerify().forward_mamba2_spec_rows(rows)
        torch.cuda.synchronize()
    finally:
        set_stage(None)

    cs2, ssm2 = conv_state.clone(), ssm.clone()
    out2 = torch.zeros(tokens, heads, head_dim, dtype=torch.bfloat16, device=dev)
    conv = torch.empty(tokens, dim, dtype=torch.bfloat16, device=dev)
    gdn_tree_conv1d_update(xbc.t()[None], cs2, conv_w, None, "silu", slots[:, 0].contiguous(), None, None, anc,
                           pad_slot_id=0, out=conv.t()[None], num_accepted_tokens=acc, query_start_loc=qsl)
    x, B, C = (t.contiguous() for t in conv.split([heads * head_dim, groups * dstate, groups * dstate], dim=-1))
    kw = dict(state_indices=slots, parents=parents, query_start_loc=qsl, num_accepted_tokens=acc, pad_slot_id=0)
    mamba2_tree_state_update(ssm2, x.view(tokens, heads, head_dim), dt, A, B.view(tokens, groups, dstate),
                             C.view(tokens, groups, dstate), D, bias, out2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(rows.out.view_as(out2), out2) and torch.equal(rows.ssm_state, ssm2)
    assert torch.equal(rows.conv_state, cs2)
    s_want, o_want = ssm.cpu(), torch.zeros(tokens, heads, head_dim, dtype=torch.bfloat16)
    om.mamba2_tree_state_update(s_want, x.cpu().view(tokens, heads, head_dim), dt.cpu(), A.cpu(),
                                B.cpu().view(tokens, groups, dstate), C.cpu().view(tokens, groups, dstate), D.cpu(),
                                bias.cpu(), o_want, **{k: v.cpu() if isinstance(v, torch.Tensor) else v
                                                       for k, v in kw.items()})
    torch.testing.assert_close(out2.cpu().float(), o_want.float(), atol=2e-2, rtol=1e-2)
    torch.testing.assert_close(ssm2.cpu(), s_want, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("shape,bs", [("tp1", 10), ("super-tp4", 40)])
def test_nontemporal_state_stores(dev, shape, bs):
    """Launches whose stored states exceed the 256 MB last-level cache (320 MB here: 10 requests x 16 nodes at Nano
    TP1 in fp32, 40 requests at Super TP4 with a bf16 pool) store them with the nontemporal buffer-store path.
    Random 16-node trees, accepted counts, and one request with a pad slot mid-tree, which keeps the index-order walk:
    its nodes reload parent states that were stored nontemporally in the same launch. The bf16 pool is held to the
    reference test's 16-bit tolerances (a state's last bit can round either way where the fp32 arithmetic differs in
    its last bit, and 640 trees carry such flips on); the fp32 pool to the fp32 ones."""
    announce(f"mamba2 nontemporal state stores {shape} bs={bs}")
    rng = random.Random(81 + bs)
    trees = [_tree("random", 16, rng) for _ in range(bs)]
    accepted = [1 + rng.randrange(4) for _ in range(bs)]
    _case(dev, shape, trees, 81, pads=[(1, 7)], accepted=accepted, ref_tol=SHAPES[shape][4] != torch.float32)
