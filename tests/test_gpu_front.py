"""The GDN layer's tree-verify front on the GPU (vllm/gdn_tree_verify.py:55-106, ``TreeVerify.forward_spec_rows``):
the input projection's GEMM output as the only buffer, the conv reading its qkv columns and the recurrence its a / b
columns as token-strided views. The outputs, the state pool and the rolled conv window equal, bit for bit, those of
the same kernels on contiguous copies; the conv matches the oracle within one 16-bit rounding (2e-2 abs / 1e-2 rel)
with the window bit for bit, and the recurrence on the conv's q / k / v matches the oracle walk (outputs 2e-2 abs /
1e-2 rel in bf16, fp32 states 1e-5 abs / 1e-4 rel)."""

from types import SimpleNamespace

import pytest
import torch

from conftest import announce, assert_states_close
from oracle import conv as oc
from oracle import recurrence as orr
from workloads import GdnShape, gdn_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch", [1, 4])
def test_front_on_projection_views(dev, batch):
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.vllm.gdn_tree_verify import GDNSpecRows, TreeVerify
    from eagle_harness.vllm.verify_layout import set_stage

    announce(f"gdn front on projection views batch={batch}")
    shape = GdnShape(batch, 16, 4, 8, 128, 128)
    H, HV, K, V = shape.h, shape.hv, shape.k, shape.v
    inp = gdn_inputs(shape, seed=5 + batch)
    tokens, dim = batch * shape.width, inp["dim"]
    zdim = HV * V
    width_p = dim + zdim + 2 * HV  # [qkv | z | b | a], the layer's input projection

    cpu = torch.Generator().manual_seed(9 + batch)
    hidden = torch.randn(tokens, 256, generator=cpu).bfloat16().to(dev)
    w_in = (torch.randn(256, width_p, generator=cpu) / 16).bfloat16().to(dev)
    A_log = (torch.randn(HV, generator=cpu) * 0.5).to(dev)
    dt_bias = (torch.randn(HV, generator=cpu) * 0.5).to(dev)
    proj = hidden @ w_in
    mixed = proj[:, :dim]
    b = proj[:, dim + zdim : dim + zdim + HV]
    a = proj[:, dim + zdim + HV :]
    assert mixed.stride(0) == width_p and a.stride(0) == width_p  # views, no copies

    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    slots, qsl, accepted = g["slots"], g["query_start_loc"], g["num_accepted"]

    def fresh():
        return g["conv_state"].clone(), g["pool"].clone(), torch.zeros(tokens, HV * V, dtype=torch.bfloat16, device=dev)

    set_stage(SimpleNamespace(ancestors=g["ancestors"], parents=g["parent_table"], state_slots={}))
    try:
        cs, pool, out = fresh()
        rows = GDNSpecRows("layers.0.linear_attn", mixed, cs, g["conv_weight"], None, "silu", a, b, A_log, dt_bias,
                           pool, slots, qsl, accepted, out, H, K, HV, V)
        TreeVerify().forward_spec_rows(rows)
        torch.cuda.synchronize()
    finally:
        set_stage(None)

    # the same kernels on contiguous copies of the same values
    cs2, pool2, out2 = fresh()
    conv2 = torch.empty(tokens, dim, dtype=torch.bfloat16, device=dev)
    gdn_tree_conv1d_update(mixed.contiguous().t()[None], cs2, g["conv_weight"], None, "silu", slots[:, 0].contiguous(),
                           None, None, g["ancestors"], pad_slot_id=0, out=conv2.t()[None],
                           num_accepted_tokens=accepted, query_start_loc=qsl)
    q2, k2, v2 = (t.contiguous() for t in conv2.split([H * K, H * K, HV * V], dim=-1))
    gdn_tree_recurrent_update(A_log, dt_bias, q2.view(1, tokens, H, K), k2.view(1, tokens, H, K),
                              v2.view(1, tokens, HV, V), a.contiguous(), b.contiguous(), initial_state_source=pool2,
                              initial_state_indices=slots, cu_seqlens=qsl, intermediate_states_buffer=pool2,
                              intermediate_state_indices=slots, retrieve_parent_token=g["parent_table"],
                              num_accepted_tokens=accepted, pad_slot_id=0, out=out2.view(1, tokens, HV, V))
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(pool, pool2) and torch.equal(cs, cs2)

    # the oracle: the conv, then the walk on the kernel's own q / k / v
    s_c = inp["conv_state"].clone()
    o_c = torch.zeros(tokens, dim, dtype=torch.bfloat16)
    oc.gdn_tree_conv1d_update(mixed.cpu().t()[None], s_c, inp["conv_weight"], None, "silu", inp["slots"][:, 0], None,
                              None, inp["ancestors"], pad_slot_id=0, out=o_c.t()[None],
                              num_accepted_tokens=inp["num_accepted"], query_start_loc=inp["query_start_loc"])
    torch.testing.assert_close(conv2.cpu().float(), o_c.float(), atol=2e-2, rtol=1e-2)
    assert torch.equal(cs.cpu(), s_c)
    p_want = inp["pool"].clone()
    o_want = orr.gdn_tree_recurrent_update(
        A_log.cpu(), dt_bias.cpu(), q2.cpu().view(1, tokens, H, K), k2.cpu().view(1, tokens, H, K),
        v2.cpu().view(1, tokens, HV, V), a.cpu(), b.cpu(), initial_state_source=p_want,
        initial_state_indices=inp["slots"], cu_seqlens=inp["query_start_loc"], intermediate_states_buffer=p_want,
        intermediate_state_indices=inp["slots"], retrieve_parent_token=inp["parent_table"],
        num_accepted_tokens=inp["num_accepted"], pad_slot_id=0)
    torch.testing.assert_close(out.cpu().float().view(1, tokens, HV, V), o_want.float(), atol=2e-2, rtol=1e-2)
    assert_states_close(pool.cpu(), p_want)

