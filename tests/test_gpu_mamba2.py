"""The Mamba2 tree state update on the GPU against the oracle (kernels/mamba2_tree.py:41-240): the reference test's
per-rank shapes (tests/test_mamba2_tree_verify_gpu.py:33-38: Nemotron 3 Nano at TP1 / TP4 with fp32 SSM states,
Nemotron 3.5 Super at TP4 with a bf16 state pool), chains and random trees, accepted counts, pad slots, dstate 64 and
256, fp16 inputs. Outputs within 2e-2 abs / 1e-2 rel (16-bit outputs); fp32 states within 1e-5 abs / 1e-4 rel, 16-bit
pool states within 1e-2."""

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


def _case(dev, shape, trees, seed, in_dtype=torch.bfloat16, pads=(), accepted=None):
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


def test_accepted_counts_pads_and_ragged_requests(dev):
    """Row 0 of each request from slots[b, accepted - 1]; pad slots neither written nor read (zeros); an empty
    request between two others."""
    announce("mamba2 accepted pads ragged")
    rng = random.Random(5)
    trees = [_tree("tree", 16, rng), [], _tree("tree", 9, rng)]
    # qsl of an empty request: the tree list holds an empty list; parents / slots rows are padded
    _case(dev, "tp4", trees, seed=9, pads=((0, 3), (2, 0)), accepted=[3, 1, 2])
