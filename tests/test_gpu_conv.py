"""The tree conv1d on the GPU against the oracle (kernels/gdn_tree_conv.py:402-497), both engines' layouts: outputs
within one 16-bit rounding (the SiLU's exp), windows and the rolled state bit for bit."""

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import conv as oc
from oracle.tables import window_codes
from workloads import GDN_B1, gdn_inputs

pytestmark = pytest.mark.gpu


def _close_out(got, want):
    torch.testing.assert_close(got.float(), want.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("width", [1, 2, 5, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sglang_layout_matches_oracle(dev, width, dtype):
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update

    announce(f"conv sglang width={width} {dtype}")
    gen = torch.Generator().manual_seed(width)
    rng = np.random.default_rng(width)
    batch, dim = 3, 40
    trees = [[0] + [int(rng.integers(0, n)) for n in range(1, width)] for _ in range(batch)]
    x = torch.randn(batch * width, dim, generator=gen).to(dtype)
    weight, bias = torch.randn(dim, 4, generator=gen).to(dtype), torch.randn(dim, generator=gen).to(dtype)
    state0 = torch.randn(5, dim, 3, generator=gen).to(dtype)
    idx = torch.tensor([3, -1, 1], dtype=torch.int32)  # request 1 is padding
    inter = torch.tensor([0, 1, 2], dtype=torch.int32)
    anc = torch.tensor([list(zip(*window_codes(t))) for t in trees], dtype=torch.int32).contiguous()
    xv = x.view(batch, width, dim).transpose(1, 2)
    w_want = torch.zeros(3, width, dim, 3, dtype=dtype)
    s_want = state0.clone()
    o_want = oc.gdn_tree_conv1d_update(xv, s_want, weight, bias, True, idx, w_want, inter, anc)

    xg = x.to(dev)
    s_got = state0.to(dev)
    w_got = torch.zeros(3, width, dim, 3, dtype=dtype, device=dev)
    o_got = gdn_tree_conv1d_update(xg.view(batch, width, dim).transpose(1, 2), s_got, weight.to(dev), bias.to(dev),
                                   True, idx.to(dev), w_got, inter.to(dev), anc.to(dev))
    torch.cuda.synchronize()
    for n in (0, 2):
        _close_out(o_got[n].cpu(), o_want[n])
        assert torch.equal(w_got[n].cpu(), w_want[n])
    assert torch.equal(s_got.cpu(), s_want)
    # the reference test's closed forms (tests/test_gdn_tree_conv.py:74-80)
    for n in (0, 2):
        nodes = x[n * width : (n + 1) * width]
        assert torch.equal(s_got[idx[n]].cpu(), torch.cat([state0[idx[n]], nodes.t()], dim=1)[:, -3:])
    assert torch.equal(s_got[[0, 2, 4]].cpu(), state0[[0, 2, 4]])


def test_vllm_layout_matches_oracle(dev):
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update

    announce("conv vllm packed")
    gen = torch.Generator().manual_seed(2)
    width, dim, state_len = 6, 24, 3 + 6
    trees = [[-1, 0, 0, 1, 2, 4], [-1, 0, 1], [-1]]
    qsl = torch.tensor([0, 6, 9, 10], dtype=torch.int32)
    x = torch.randn(10, dim, generator=gen).to(torch.bfloat16)
    weight, bias = torch.randn(dim, 4, generator=gen).to(torch.bfloat16), torch.randn(dim, generator=gen).to(torch.bfloat16)
    state0 = torch.randn(6, state_len, dim, generator=gen).to(torch.bfloat16).transpose(1, 2)  # vLLM's other layout
    slots = torch.tensor([4, 2, 0], dtype=torch.int32)  # request 2 is padding (null block 0)
    accepted = torch.tensor([1, 3, 1], dtype=torch.int32)
    anc = torch.zeros(4, 3, width, dtype=torch.int32)  # the stage is wider than the batch
    for n, t in enumerate(trees):
        anc[n, :, : len(t)] = torch.tensor(list(zip(*window_codes(t))), dtype=torch.int32)
    s_want = state0.clone()
    o_want = torch.zeros_like(x)
    oc.gdn_tree_conv1d_update(x.t()[None], s_want, weight, bias, "silu", slots, None, None, anc, pad_slot_id=0,
                              out=o_want.t()[None], num_accepted_tokens=accepted, query_start_loc=qsl)
    s_got = state0.to(dev)  # keeps the transposed strides
    o_got = torch.zeros(10, dim, dtype=torch.bfloat16, device=dev)
    gdn_tree_conv1d_update(x.to(dev).t()[None], s_got, weight.to(dev), bias.to(dev), "silu", slots.to(dev), None, None,
                           anc.to(dev), pad_slot_id=0, out=o_got.t()[None], num_accepted_tokens=accepted.to(dev),
                           query_start_loc=qsl.to(dev))
    torch.cuda.synchronize()
    _close_out(o_got.cpu(), o_want)
    assert torch.equal(s_got.cpu(), s_want)
    assert torch.equal(o_got[9].cpu(), torch.zeros(dim, dtype=torch.bfloat16))


@pytest.mark.parametrize("batch", [1, 8])
def test_gdn_layer_conv_matches_oracle(dev, batch):
    """The GDN layer's conv over the packed qkv channels (2 H K + HV V = 8192) with the seeded trees."""
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update

    announce(f"conv gdn layer batch={batch}")
    shape = type(GDN_B1)(batch, 16, 16, 32, 128, 128)
    inp = gdn_inputs(shape, seed=11)
    slots = inp["slots"][:, 0].contiguous()
    s_want = inp["conv_state"].clone()
    o_want = torch.zeros_like(inp["x"])
    oc.gdn_tree_conv1d_update(inp["x"].t()[None], s_want, inp["conv_weight"], None, "silu", slots, None, None,
                              inp["ancestors"], pad_slot_id=0, out=o_want.t()[None],
                              num_accepted_tokens=inp["num_accepted"], query_start_loc=inp["query_start_loc"])
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    o_got = torch.zeros_like(g["x"])
    gdn_tree_conv1d_update(g["x"].t()[None], g["conv_state"], g["conv_weight"], None, "silu", slots.to(dev), None, None,
                           g["ancestors"], pad_slot_id=0, out=o_got.t()[None], num_accepted_tokens=g["num_accepted"],
                           query_start_loc=g["query_start_loc"])
    torch.cuda.synchronize()
    _close_out(o_got.cpu(), o_want)
    assert torch.equal(g["conv_state"].cpu(), s_want)
