"""The verify round captured in a HIP graph and replayed: stage (tree tables), tree-verify attention, the GDN layer's
tree conv and snapshot walk, and the accepted-path state commit, at the batch-64 workload's heads with 8 requests.
Every replay starts from the same inputs (restored eagerly between replays, with the eager work the serving loop
would do in between) and must equal the eager round bit for bit; the eager round is checked against the oracle on
sampled requests (2e-2 abs / 1e-2 rel for bf16 outputs, 1e-5 abs / 1e-4 rel for fp32 states)."""

import pytest
import torch

from conftest import announce
from oracle import attention as oa
from oracle import recurrence as orr
from workloads import AttnShape, GdnShape, accept_paths, attention_inputs, gdn_inputs

pytestmark = pytest.mark.gpu


def test_captured_round_replays_equal_eager_round(dev):
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit
    from eagle_harness.vllm.verify_attention import verify_attention
    from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage

    announce("graph capture: stage + attention + conv + walk + commit, 8 requests")
    B, W = 8, 16
    att = attention_inputs(AttnShape(B, W, 24, 4, 256, 16, 200, 2500), seed=7, device=dev)
    gdn = gdn_inputs(GdnShape(B, W, 16, 32, 128, 128), seed=7, device=dev)
    assert att["parents"] == gdn["parents"]
    tokens = B * W
    store = TreeStore(B, W, dev)
    store.parents.copy_(torch.tensor(att["parents"], dtype=torch.int32))
    stage = VerifyStage(B, tokens, W, dev)
    chain = (att["context_lens"].to(torch.int64)[:, None] + torch.arange(W, device=dev)).reshape(-1)
    positions = chain.clone()
    idx = torch.arange(B, dtype=torch.int32, device=dev)
    qsl = att["query_start_loc"]
    path, plen = accept_paths(att["parents"], 7, W)
    path, plen = path.to(dev), plen.to(dev)
    commit = LinearStateCommit([(gdn["conv_state"], gdn["pool"])], [gdn["slots"]], dev)
    out = torch.empty_like(att["q"])
    mixed = torch.empty_like(gdn["x"])
    H, HV, K, V = 16, 32, 128, 128
    q4 = mixed[:, : H * K].view(1, tokens, H, K)
    k4 = mixed[:, H * K : 2 * H * K].view(1, tokens, H, K)
    v4 = mixed[:, 2 * H * K :].view(1, tokens, HV, V)
    rec = torch.empty(1, tokens, HV, V, dtype=torch.bfloat16, device=dev)
    slots0 = gdn["slots"][:, 0].contiguous()

    def round_():
        stage.stage(store, idx, qsl, qsl, positions, B, tokens, tree=True)
        verify_attention(att["q"], att["k_new"], att["v_new"], att["key_cache"], att["value_cache"],
                         att["block_table"], stage.context_lens[:B], qsl, stage.masks[:B], att["scale"], out,
                         max_query_len=W)
        gdn_tree_conv1d_update(gdn["x"].t()[None], gdn["conv_state"], gdn["conv_weight"], None, "silu", slots0, None,
                               None, stage.ancestors[:B], pad_slot_id=0, out=mixed.t()[None],
                               num_accepted_tokens=gdn["num_accepted"], query_start_loc=qsl)
        gdn_tree_recurrent_update(gdn["A_log"], gdn["dt_bias"], q4, k4, v4, gdn["a"], gdn["b"],
                                  initial_state_source=gdn["pool"], initial_state_indices=gdn["slots"],
                                  cu_seqlens=qsl, intermediate_states_buffer=gdn["pool"],
                                  intermediate_state_indices=gdn["slots"], retrieve_parent_token=stage.parents[:B],
                                  num_accepted_tokens=gdn["num_accepted"], pad_slot_id=0, out=rec)
        commit.commit(idx, path, plen)
        positions.copy_(chain)

    inputs = {"pool": gdn["pool"].clone(), "conv_state": gdn["conv_state"].clone()}

    def restore():
        gdn["pool"].copy_(inputs["pool"])
        gdn["conv_state"].copy_(inputs["conv_state"])
        positions.copy_(chain)
        for t in (out, mixed, rec):
            t.fill_(3.0)

    def results():
        return [t.clone() for t in (out, mixed, rec, gdn["pool"], gdn["conv_state"], stage.masks, stage.context_lens,
                                    positions)]

    restore()
    round_()
    torch.cuda.synchronize()
    want = results()

    # the eager round against the oracle: attention of every request, the walk of two (on the kernel's own q / k / v)
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in att.items()}
    a_want = oa.verify_attention(cpu["q"], cpu["k_new"], cpu["v_new"], cpu["key_cache"], cpu["value_cache"],
                                 cpu["block_table"], cpu["context_lens"], cpu["query_start_loc"], cpu["masks"],
                                 cpu["scale"], torch.empty_like(cpu["q"]), max_query_len=W)
    torch.testing.assert_close(want[0].cpu().float(), a_want.float(), atol=2e-2, rtol=1e-2)
    mixed_cpu = want[1].cpu()
    for r in (0, B - 1):
        sl = slice(r * W, (r + 1) * W)
        sub_slots = gdn["slots"][r : r + 1].cpu()
        pool = inputs["pool"].cpu()
        o = orr.gdn_tree_recurrent_update(
            gdn["A_log"].cpu(), gdn["dt_bias"].cpu(), mixed_cpu[sl, : H * K].reshape(1, W, H, K),
            mixed_cpu[sl, H * K : 2 * H * K].reshape(1, W, H, K), mixed_cpu[sl, 2 * H * K :].reshape(1, W, HV, V),
            gdn["a"][sl].cpu(), gdn["b"][sl].cpu(), initial_state_source=pool, initial_state_indices=sub_slots,
            cu_seqlens=torch.tensor([0, W], dtype=torch.int32), intermediate_states_buffer=pool,
            intermediate_state_indices=sub_slots, retrieve_parent_token=gdn["parent_table"][r : r + 1].cpu(),
            num_accepted_tokens=gdn["num_accepted"][r : r + 1].cpu(), pad_slot_id=0)
        torch.testing.assert_close(want[2][:, sl].cpu().float(), o.float(), atol=2e-2, rtol=1e-2)

    graph = torch.cuda.CUDAGraph()
    restore()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        round_()
    for rep in range(3):
        restore()
        torch.zeros(1 << 20, device=dev).sum().item()  # eager work and a synchronisation between replays
        graph.replay()
        torch.cuda.synchronize()
        got = results()
        for i, (g, w) in enumerate(zip(got, want)):
            assert torch.equal(g, w), f"replay {rep}: result {i} differs from the eager round"
