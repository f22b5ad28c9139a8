"""The quantized hybrid verify round at batch 512 x 16-node trees, composed as one round on the GPU and checked
against the oracle: the verify stage, fp8-e4m3 tree attention (per-(page, KV head) scales, prefixes U[512, 4096]),
three GDN layers (tree conv, then the snapshot walk on views of the conv output, fp32 states, vLLM per-row slots),
greedy targets over 8192 x 151936 bf16 logits, the tree walk, and the accepted-path commit of the three layers
(vllm/verify_attention.py:142-207, kernels/gdn_tree_recurrence.py:562-706, vllm/tree_accept.py:45-83,
vllm/gdn_tree_verify.py:289-322).

Checked: the stage tables of every request bit for bit; attention on sampled requests (2e-2 abs / 1e-2 rel against
the dequantised oracle); every layer's conv output and walk output on sampled requests (the same 16-bit tolerance)
and their fp32 snapshots (1e-4 relative); the targets against ``torch.argmax`` bit for bit; the walk of all 512
requests against the oracle walk bit for bit; the commit of every request and layer against the snapshots and
windows taken just before it, bit for bit."""

import numpy as np
import pytest
import torch

from conftest import announce, assert_states_close
from oracle import accept as oacc
from oracle import conv as oc
from oracle import recurrence as orr
from oracle import tables as ot
from test_gpu_configs import _attention_subset, _close16, _gdn_subset
from workloads import ATTN_B512_FP8, GdnShape, attention_inputs, gdn_inputs

pytestmark = pytest.mark.gpu


def test_quantized_hybrid_round_b512(dev):
    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit
    from eagle_harness.vllm.tree_accept import accept_tree, greedy_targets
    from eagle_harness.vllm.verify_attention import verify_attention
    from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage

    announce("round 5: b512 stage + fp8 attention + 3 GDN layers + argmax + walk + commit")
    shape = GdnShape(512, 16, 16, 32, 128, 128)
    B, W, H, HV, K, V, vocab = shape.batch, shape.width, shape.h, shape.hv, shape.k, shape.v, 151936
    tokens = B * W
    att = attention_inputs(ATTN_B512_FP8, seed=31, device=dev, fp8=True, gen_device=dev)
    layers = [gdn_inputs(shape, seed=31, device=dev, layout="vllm", gen_device=dev) for _ in range(3)]
    assert all(g["parents"] == att["parents"] for g in layers)
    rng = np.random.default_rng(31)
    reqs = sorted({0, B - 1, *map(int, rng.choice(B, 4, replace=False))})
    subs = [_gdn_subset(g, reqs, W) for g in layers]  # the sampled requests' slots before anything runs

    store = TreeStore(B, W, dev)
    store.parents.copy_(torch.tensor(att["parents"], dtype=torch.int32))
    stage = VerifyStage(B, tokens, W, dev)
    chain = (att["context_lens"].to(torch.int64)[:, None] + torch.arange(W, device=dev)).reshape(-1)
    positions = chain.clone()
    idx = torch.arange(B, dtype=torch.int32, device=dev)
    qsl = att["query_start_loc"]
    attn_out = torch.full_like(att["q"], 7.0)
    convs = [torch.empty_like(g["x"]) for g in layers]
    recs = [torch.empty(1, tokens, HV, V, dtype=torch.bfloat16, device=dev) for _ in layers]
    gen = torch.Generator(device=dev).manual_seed(31)
    logits = torch.randn(tokens, vocab, device=dev, generator=gen).bfloat16()
    target = torch.empty(tokens, dtype=torch.int64, device=dev)
    # drafts: a node's draft is its parent's target at 80 % of the nodes, so accepted paths run several rows deep
    want_target = torch.argmax(logits, dim=-1)
    par = torch.tensor(att["parents"], dtype=torch.int64, device=dev)
    from_parent = want_target[(torch.arange(B, device=dev)[:, None] * W + par.clamp(min=0)).reshape(-1)]
    agree = torch.rand(tokens, device=dev, generator=gen) < 0.8
    drafted = torch.where(agree, from_parent, torch.randint(0, vocab, (tokens,), device=dev, generator=gen))
    commit = LinearStateCommit([(g["conv_state"], g["pool"]) for g in layers], [g["slots"] for g in layers], dev)

    # ---- the round -------------------------------------------------------------------------------------------------
    stage.stage(store, idx, qsl, qsl, positions, B, tokens, tree=True)
    verify_attention(att["q"], att["k_new"], att["v_new"], att["key_cache"], att["value_cache"], att["block_table"],
                     stage.context_lens[:B], qsl, stage.masks[:B], att["scale"], attn_out, max_query_len=W,
                     k_scale=att["k_scale"], v_scale=att["v_scale"])
    for g, conv_out, rec_out in zip(layers, convs, recs):
        gdn_tree_conv1d_update(g["x"].t()[None], g["conv_state"], g["conv_weight"], None, "silu",
                               g["slots"][:, 0].contiguous(), None, None, stage.ancestors[:B], pad_slot_id=0,
                               out=conv_out.t()[None], num_accepted_tokens=g["num_accepted"], query_start_loc=qsl)
        gdn_tree_recurrent_update(g["A_log"], g["dt_bias"], conv_out[:, : H * K].view(1, tokens, H, K),
                                  conv_out[:, H * K : 2 * H * K].view(1, tokens, H, K),
                                  conv_out[:, 2 * H * K :].view(1, tokens, HV, V), g["a"], g["b"],
                                  initial_state_source=g["pool"], initial_state_indices=g["slots"], cu_seqlens=qsl,
                                  intermediate_states_buffer=g["pool"], intermediate_state_indices=g["slots"],
                                  retrieve_parent_token=stage.parents[:B], num_accepted_tokens=g["num_accepted"],
                                  pad_slot_id=0, out=rec_out)
    greedy_targets(logits, out=target)
    sampled, num_sampled = accept_tree(target, drafted, qsl, idx, store.parents, store)
    torch.cuda.synchronize()
    # what the commit must move: each request's accepted node's snapshot and its window, per layer
    path, plen = store.path.cpu(), store.path_len.cpu()
    last = path[torch.arange(B), (plen - 1).long()]
    want_states, want_windows = [], []
    for g in layers:
        slots = g["slots"].cpu()
        want_states.append(g["pool"][slots[torch.arange(B), last.long()].long().to(dev)].clone())
        win = g["conv_state"][g["slots"][:, 0].long()].clone()
        moved = win.clone()
        for b in range(B):
            for j in range(1, int(plen[b])):
                moved[b, :, 2 + j] = win[b, :, 2 + int(path[b, j])]
        want_windows.append(moved)
    snaps = [g["pool"][sub["old_slots"].flatten().long().to(dev)].cpu() for g, sub in zip(layers, subs)]
    commit.commit(idx, store.path, store.path_len)
    positions.copy_(chain)
    torch.cuda.synchronize()

    # ---- the stage --------------------------------------------------------------------------------------------------
    o = dict(stage_parents=np.zeros((B, W), np.int32), stage_anc=np.zeros((B, 3, W), np.int32),
             stage_mask=np.ones((B, W), np.int64), context_lens=np.zeros(B, np.int32),
             slot_parents=np.zeros((B, W), np.int32), slot_depths=np.zeros((B, W), np.int32))
    pos = chain.cpu().numpy().copy()
    qsl_np = qsl.cpu().numpy()
    ot.stage_tree(np.array(att["parents"], np.int32), np.arange(B), qsl_np, qsl_np, pos, o["stage_parents"],
                  o["stage_anc"], o["stage_mask"], o["context_lens"], o["slot_parents"], o["slot_depths"], B, W, True)
    assert stage.masks[:B].cpu().numpy().tolist() == o["stage_mask"].tolist()
    assert stage.ancestors[:B].cpu().numpy().tolist() == o["stage_anc"].tolist()
    assert stage.context_lens[:B].cpu().numpy().tolist() == o["context_lens"].tolist()
    assert torch.equal(stage.context_lens[:B].cpu(), att["context_lens"].cpu())

    # ---- fp8 attention on the sampled requests -----------------------------------------------------------------------
    assert bool(torch.isfinite(attn_out.float()).all())
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in att.items()}
    rows, want = _attention_subset(cpu, reqs)
    _close16(attn_out.cpu()[rows], want)

    # ---- the three GDN layers on the sampled requests ----------------------------------------------------------------
    n = len(reqs)
    for layer, (g, sub, conv_out, rec_out) in enumerate(zip(layers, subs, convs, recs)):
        s_conv = sub["conv_state"].clone()
        o_conv = torch.zeros(n * W, g["dim"], dtype=torch.bfloat16)
        oc.gdn_tree_conv1d_update(sub["x"].t()[None], s_conv, g["conv_weight"].cpu(), None, "silu",
                                  sub["slots"][:, 0], None, None, sub["ancestors"], pad_slot_id=0,
                                  out=o_conv.t()[None], num_accepted_tokens=sub["num_accepted"],
                                  query_start_loc=sub["query_start_loc"])
        mixed = conv_out.cpu()[sub["rows"]]
        _close16(mixed, o_conv)
        pool = sub["pool"].clone()
        o_walk = orr.gdn_tree_recurrent_update(
            g["A_log"].cpu(), g["dt_bias"].cpu(), mixed[:, : H * K].reshape(1, n * W, H, K),
            mixed[:, H * K : 2 * H * K].reshape(1, n * W, H, K), mixed[:, 2 * H * K :].reshape(1, n * W, HV, V),
            sub["a"], sub["b"], initial_state_source=pool, initial_state_indices=sub["slots"],
            cu_seqlens=sub["query_start_loc"], intermediate_states_buffer=pool,
            intermediate_state_indices=sub["slots"], retrieve_parent_token=sub["parent_table"],
            num_accepted_tokens=sub["num_accepted"], pad_slot_id=0)
        _close16(rec_out.cpu()[0, sub["rows"]], o_walk[0])
        assert_states_close(snaps[layer], pool[sub["slots"].flatten().long()])

    # ---- greedy targets and the walk -----------------------------------------------------------------------------------
    assert torch.equal(target, want_target)
    path_o, plen_o = torch.zeros(B, W, dtype=torch.int32), torch.ones(B, dtype=torch.int32)
    sampled_o, num_o = oacc.accept_tree(want_target.cpu(), drafted.cpu(), qsl.cpu(), idx.cpu(),
                                        torch.tensor(att["parents"], dtype=torch.int32), path_o, plen_o, W)
    assert torch.equal(num_sampled.cpu(), num_o) and torch.equal(plen, plen_o)
    assert float(plen_o.float().mean()) > 2.0  # the drafts are accepted past the root
    for b in range(B):
        k = int(num_o[b])
        assert torch.equal(path[b, :k], path_o[b, :k])
        assert torch.equal(sampled[b, :k].cpu(), sampled_o[b, :k])

    # ---- the commit of the three layers -------------------------------------------------------------------------------
    dst = (plen - 1).long()
    for g, ws, ww in zip(layers, want_states, want_windows):
        slots = g["slots"].cpu()
        moved = last != dst  # requests whose accepted node is not already in the resume slot
        dst_slots = slots[torch.arange(B), dst].long()
        assert torch.equal(g["pool"][dst_slots[moved].to(dev)], ws[moved.to(dev)])
        assert torch.equal(g["conv_state"][g["slots"][:, 0].long()], ww)
