#!/usr/bin/env python
"""Benchmark of the draft-tree verify hot path on one MI355X: verified tree tokens/s of one verify round.

A step is one pass of the hot path over one batch of synthetic input, resident in HBM before the timed region:

  1. verify stage (tree masks, depths, window codes, context lengths, depth positions);
  2. tree-verify attention: batch 64, 16-node seeded trees, 24 query / 4 KV heads, D 256, bf16 paged KV (page 16,
     permuted page tables), prefixes U[1024, 8192];
  3. one GDN layer at the same batch: tree conv1d over the 8192 qkv channels, the gated delta rule walk with every
     node's fp32 state snapshot (16 key / 32 value heads, K = V = 128), and the accepted-path commit (window
     compaction, state move) for seeded accept lengths U[1, 12].

``value`` = 64 x 16 verified tokens per step / step time. The JSON line also carries the dominant kernel's
roofline (algorithmic HBM bytes per launch / its HIP-event duration, against MI355X's 8 TB/s), the CPU baseline
(the oracle, timed on a bounded sample on this host's cores) and the records contract's chunk form per layer at
1 / 4 / 16 / 32 requests beside the reference's published times (``--records-only`` prints just that). ``--calibrate-copy`` instead times a plain 1 GiB
device copy (the reference kernel for the rocprofv3 FETCH_SIZE / WRITE_SIZE scale) and a 2 GiB fill (the write
ceiling).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "eagle-4_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s (published)
METRIC = "verified tree tokens/s (tree-attn+GDN) at B=64, T=16; % of HBM roofline"


def _gdn_layer_bytes(B: int, W: int, H: int, HV: int, K: int, V: int, dim: int, path_len, path_last) -> dict:
    """Algorithmic bytes of one GDN layer's verify (conv, snapshot walk) and of its accepted-path commit."""
    state = HV * K * V * 4
    tokens = B * W
    conv = tokens * dim * 2 * 2 + B * dim * 3 * 2 + B * dim * (W + 2) * 2 + dim * 4 * 2
    rec = (B * state + tokens * state + tokens * H * K * 2 * 2 + tokens * HV * V * 2 + tokens * HV * 2 * 2
           + tokens * HV * V * 2 + tokens * 4)
    moved = sum(1 for n, last in zip(path_len, path_last) if last != n - 1)
    commit = moved * 2 * state + sum(2 * max(n - 1, 0) for n in path_len) * dim * 2
    return {"conv": conv, "recurrence": rec, "commit": commit}


def _algorithmic_bytes(B, W, att, gdn, ctx, path_len, path_last):
    """Bytes each kernel must move at least (every element once; re-reads and partials not counted)."""
    import math

    tokens = B * W
    kv = sum(int(L) for L in ctx) * att["hkv"] * att["d"] * 2 * 2
    pages = sum(math.ceil(int(L) / att["page"]) for L in ctx) * 4
    attn = kv + pages + tokens * att["hq"] * att["d"] * 2 * 2 + tokens * att["hkv"] * att["d"] * 2 * 2 + B * W * 8
    layer = _gdn_layer_bytes(B, W, gdn["h"], gdn["hv"], gdn["k"], gdn["v"], gdn["dim"], path_len, path_last)
    stage = B * W * (4 + 12 + 8 + 8 + 8) + B * 4
    return {"stage": stage, "attention": attn, **layer}


def _cpu_baseline(work, sample: int, seconds: float) -> dict:
    """The oracle (torch on the host CPU) over the first ``sample`` requests of the workload, in whole passes until
    ``seconds`` have gone by (at least one pass)."""
    import torch

    from oracle import attention as oa
    from oracle import commit as ocm
    from oracle import conv as oc
    from oracle import recurrence as orr

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    W, B = work["W"], sample
    a, g = work["attn_cpu"], work["gdn_cpu"]
    HK = g["H"] * g["K"]
    tokens = B * W

    def one_pass():
        out = torch.empty_like(a["q"])
        oa.verify_attention(a["q"], a["k_new"], a["v_new"], a["key_cache"], a["value_cache"], a["block_table"],
                            a["context_lens"], a["query_start_loc"], a["masks"], a["scale"], out, max_query_len=W)
        conv_out = torch.empty_like(g["x"])
        oc.gdn_tree_conv1d_update(g["x"].t()[None], g["conv_state"], g["conv_weight"], None, "silu",
                                  g["slots"][:, 0].contiguous(), None, None, g["ancestors"], pad_slot_id=0,
                                  out=conv_out.t()[None], num_accepted_tokens=g["num_accepted"],
                                  query_start_loc=g["query_start_loc"])
        q = conv_out[:, :HK].reshape(1, tokens, g["H"], g["K"])
        k = conv_out[:, HK : 2 * HK].reshape(1, tokens, g["H"], g["K"])
        v = conv_out[:, 2 * HK :].reshape(1, tokens, g["HV"], g["V"])
        orr.gdn_tree_recurrent_update(g["A_log"], g["dt_bias"], q, k, v, g["a"], g["b"],
                                      initial_state_source=g["pool"], initial_state_indices=g["slots"],
                                      cu_seqlens=g["query_start_loc"], intermediate_states_buffer=g["pool"],
                                      intermediate_state_indices=g["slots"], retrieve_parent_token=g["parent_table"],
                                      num_accepted_tokens=g["num_accepted"], pad_slot_id=0)
        ocm.linear_state_commit([g["conv_state"]], [g["pool"]], [g["slots"]], torch.arange(B, dtype=torch.int32),
                                g["path"], g["path_len"])

    t0 = time.perf_counter()
    passes = 0
    while passes == 0 or time.perf_counter() - t0 < seconds:
        one_pass()
        passes += 1
    dt = time.perf_counter() - t0
    return {"value": passes * tokens / dt, "unit": "verified tree tokens/s", "cores": threads, "kind": "port",
            "sample": f"{sample} of 64 requests x 16 nodes through the CPU oracle (stage-free: attention, tree conv, "
                      f"GDN walk with fp32 snapshots, commit), {passes} passes in {dt:.1f} s on {threads} host threads"}


# The reference's published MI355X figures for the records chunk form (FlyDSL, per layer, TP1 H16/HV48, K = V = 128,
# 16-node trees, bf16 pool; eagle_harness/kernels/gdn_tree_chunk_flydsl.py:25-27), microseconds by request count.
RECORDS_PUBLISHED_US = {1: 10.5, 4: 11.9, 16: 23.8, 32: 34.7}


EAGER = False  # --eager: rows are called without graph capture, so a counter run sees every dispatch


def _time_graph(fn, steps: int, reps: int = 5) -> float:
    """Microseconds per call of ``fn``: a HIP graph of ``reps`` calls, replayed ``steps`` times between events on the
    launch stream, best of 3 (with ``EAGER``: ``steps`` plain calls, launch gaps included)."""
    import torch

    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    if EAGER:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / (steps * reps))
    return best


def _row(us: float, nbytes: int | None = None, **extra) -> dict:
    r = {"us": round(us, 2)}
    if nbytes:
        r.update(bytes=nbytes, GBps=round(nbytes / (us * 1e-6) / 1e9, 1),
                 frac_of_hbm_peak=round(nbytes / (us * 1e-6) / HBM_PEAK, 3))
    r.update(extra)
    return r


def _rows(steps: int) -> dict:
    """The rows and configurations the step does not contain, each timed like the step's parts: the accept path at
    batch 512 x 16 over a 151936-token vocab (argmax, tree walk), the bs1 accept tail, the tail-mask words, fp8 verify
    attention at batch 512, the GDN walk at batch 1 and 256, fp32 and bf16 attention at batch 1, the rounded records
    path replay and commit, vLLM's round commit (KV compaction, chainize), draft-row attention, the GDN layer front
    on projection views and the Mamba2 tree state update. Algorithmic bytes
    count every element once."""
    import math

    import numpy as np
    import torch

    from eagle_harness.kernels.accept_tail import accept_tail
    from eagle_harness.kernels.gdn_tree import gdn_tree_ancestors
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_commit, gdn_tree_records_update
    from eagle_harness.kernels.verify_prep import tree_tail_words
    from eagle_harness.vllm.tree_accept import accept_tree, greedy_targets
    from eagle_harness.vllm.verify_attention import verify_attention
    from eagle_harness.vllm.verify_layout import TreeStore
    from workloads import (ATTN_B1, ATTN_B512_FP8, GDN_B1, GDN_B256, attention_inputs, gdn_inputs, records_inputs,
                           seeded_tree, tree_links)

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)
    rows = {}

    # a9: greedy targets and the tree walk at batch 512 x 16 rows, vocab 151936 (bf16 logits, 2.49 GB)
    B, W, vocab = 512, 16, 151936
    logits = torch.randn(B * W, vocab, device=dev, generator=gen).bfloat16()
    target = torch.empty(B * W, dtype=torch.int64, device=dev)
    us = _time_graph(lambda: greedy_targets(logits, out=target), steps)
    rows["a9_argmax_b512x16_vocab151936_bf16"] = _row(us, logits.numel() * 2 + B * W * 8)
    rng = np.random.default_rng(11)
    trees = [seeded_tree(rng, W) for _ in range(B)]
    parents = torch.tensor(trees, dtype=torch.int32, device=dev)
    drafted = torch.randint(0, vocab, (B * W,), device=dev, generator=gen)
    cu = torch.arange(0, B * W + 1, W, dtype=torch.int32, device=dev)
    idx = torch.arange(B, dtype=torch.int32, device=dev)
    store = TreeStore(B, W, dev)
    us = _time_graph(lambda: accept_tree(target, drafted, cu, idx, parents, store), steps)
    rows["a9_accept_tree_walk_b512x16"] = _row(us, B * W * (8 + 8 + 4 + 8) + B * (4 + W * 4 + 4))
    del logits

    # a10: the bs1 accept tail over a 16-node tree (one workgroup: latency)
    t1 = seeded_tree(rng, W)
    nxt, sib = tree_links(t1, W)
    tail_args = (target[:W].clone(), drafted[:W].clone(), torch.arange(W, device=dev)[None],
                 torch.tensor([nxt], device=dev), torch.tensor([sib], device=dev), torch.tensor([4096], device=dev),
                 torch.arange(W, device=dev) + 5000, torch.zeros(2, 8192, dtype=torch.int32, device=dev),
                 torch.tensor([1], device=dev))
    us = _time_graph(lambda: accept_tail(*tail_args, 12), steps)
    rows["a10_accept_tail_bs1_w16"] = _row(us)

    # a8: tail-mask words of a 16-row verify over an 8192-slot KV
    mask = torch.randint(0, 2, (W * 8192,), device=dev, generator=gen).bool()
    committed = torch.tensor([8192 - W], dtype=torch.int64, device=dev)
    tail = torch.zeros(W + 1, dtype=torch.int64, device=dev)
    us = _time_graph(lambda: tree_tail_words(mask, committed, tail, W), steps)
    rows["a8_tail_words_w16"] = _row(us)

    # next row (f) 2: vLLM's round commit at batch 64 x 16 rows — the accepted rows' KV (4 KV heads, D 256 bf16, K and
    # V adjacent, page 16) moved in 4 full-attention layers, and chainize
    from eagle_harness.vllm.round_commit import KvCompactor, chainize
    from workloads import accept_paths

    Bc, Wc, Hc, Dc, page, Lc = 64, 16, 4, 256, 16, 4
    trees_c = [seeded_tree(rng, Wc) for _ in range(Bc)]
    path_c, plen_c = accept_paths(trees_c, 7, Wc)
    ctx_c = torch.tensor(rng.integers(1024, 8192, Bc), dtype=torch.int32)
    blocks_per = [(int(c) + Wc + page - 1) // page for c in ctx_c]
    max_b = max(blocks_per)
    perm = torch.tensor(rng.permutation(sum(blocks_per)), dtype=torch.int32)
    table_c = torch.zeros(Bc, max_b, dtype=torch.int32)
    off = 0
    for b, nb in enumerate(blocks_per):
        table_c[b, :nb] = perm[off : off + nb]
        off += nb
    caches_c = [torch.empty(sum(blocks_per), Hc, page, 2 * Dc, dtype=torch.bfloat16, device=dev) for _ in range(Lc)]
    qsl_c = torch.arange(0, Bc * Wc + 1, Wc, dtype=torch.int32, device=dev)
    seq_c = (ctx_c + Wc).to(dev)
    idx_c = torch.arange(Bc, dtype=torch.int32, device=dev)
    compactor = KvCompactor(caches_c, [table_c.to(dev)] * Lc, [page] * Lc, dev)
    path_d, plen_d = path_c.to(dev), plen_c.to(dev)
    us = _time_graph(lambda: compactor.compact(idx_c, qsl_c, qsl_c, seq_c, path_d, plen_d), steps)
    moved = sum(sum(1 for j in range(1, int(plen_c[b])) if int(path_c[b, j]) != j) for b in range(Bc))
    rows["kv_compaction_b64x16_4layers"] = _row(us, moved * Lc * Hc * 2 * Dc * 2 * 2)
    ids_c = torch.zeros(Bc * Wc, dtype=torch.int64, device=dev)
    pos_c = torch.zeros_like(ids_c)
    src_c = torch.arange(Bc * Wc, dtype=torch.int64, device=dev)
    sampled_c = torch.zeros(Bc, Wc, dtype=torch.int64, device=dev)
    us = _time_graph(lambda: chainize(ids_c, pos_c, src_c, idx_mapping=idx_c, query_start_loc=qsl_c,
                                      cu_num_logits=qsl_c, seq_lens=seq_c, path=path_d, path_len=plen_d,
                                      sampled=sampled_c, width=Wc), steps)
    rows["chainize_b64x16"] = _row(us)
    del caches_c

    # next row (f) 3: draft-row attention, a draft step (4 frontier rows, step 7) at batch 64 over a 4096-key window of
    # 8192 committed keys, 32 query / 8 KV heads, D 128 bf16, slot-major cache through a permuted token table
    from eagle_harness.kernels.row_attention import RowsLaunch, rows_attention, rows_padded

    Br, rr, stp, win, Lr, Hq, Hk, Dr = 64, 4, 7, 4096, 8192, 32, 8, 128
    nslot = Br * (Lr + rr * stp)
    k_r = torch.randn(nslot, Hk, Dr, device=dev, generator=gen).bfloat16()
    v_r = torch.randn(nslot, Hk, Dr, device=dev, generator=gen).bfloat16()
    tab_r = torch.randperm(nslot, device=dev, generator=gen).to(torch.int32).view(Br, Lr + rr * stp)
    anc_r = tab_r[:, Lr:].reshape(Br, rr, stp).contiguous()
    q_r = torch.randn(Br * rr, Hq, Dr, device=dev, generator=gen).bfloat16()
    out_r = torch.empty_like(q_r)
    sp = 8
    npart = Br * Hq * (sp + 1) * rows_padded(rr)
    po, pl = torch.empty(npart, Dr, device=dev), torch.empty(npart, device=dev)
    seq_r = torch.full((Br,), Lr, dtype=torch.int32, device=dev)
    us = _time_graph(lambda: rows_attention(q_r, k_r, v_r, out_r, po, pl, tab_r, seq_r, anc_r, rows_per_request=rr,
                                            step=stp, window=win, scale=Dr**-0.5,
                                            launch=RowsLaunch(splits=sp, block_n=32)), steps)
    rows["row_attention_step7_b64_window4096_d128"] = _row(us, Br * Hk * (win + rr * stp) * Dr * 2 * 2
                                                           + Br * (win + rr * stp) * 4 + 2 * q_r.numel() * 2)
    del k_r, v_r

    # next row (f) 1: the GDN layer front at the step's layer (B64 T16, H16/HV32, K = V = 128, fp32 states): the conv
    # and the walk reading token-strided views of one [qkv | z | b | a] projection buffer, no split or copy kernels
    from types import SimpleNamespace

    from eagle_harness.vllm.gdn_tree_verify import GDNSpecRows, TreeVerify
    from eagle_harness.vllm.verify_layout import set_stage
    from workloads import GDN_B64

    g = gdn_inputs(GDN_B64, seed=4, device=dev, layout="vllm", gen_device=dev)
    Bf, Wf, H, HV, K, V = GDN_B64.batch, GDN_B64.width, GDN_B64.h, GDN_B64.hv, GDN_B64.k, GDN_B64.v
    tokens, dim = Bf * Wf, g["dim"]
    proj = torch.randn(tokens, dim + HV * V + 2 * HV, device=dev, generator=gen).bfloat16()
    front_rows = GDNSpecRows("layers.0.linear_attn", proj[:, :dim], g["conv_state"], g["conv_weight"], None, "silu",
                             proj[:, dim + HV * V + HV :], proj[:, dim + HV * V : dim + HV * V + HV], g["A_log"],
                             g["dt_bias"], g["pool"], g["slots"], g["query_start_loc"], g["num_accepted"],
                             torch.empty(tokens, HV * V, dtype=torch.bfloat16, device=dev), H, K, HV, V)
    set_stage(SimpleNamespace(ancestors=g["ancestors"], parents=g["parent_table"], state_slots={}))
    try:
        us = _time_graph(lambda: TreeVerify().forward_spec_rows(front_rows), steps)
    finally:
        set_stage(None)
    state = HV * K * V * 4
    conv_b = tokens * dim * 2 * 2 + Bf * dim * 3 * 2 + Bf * dim * (Wf + 2) * 2 + dim * 4 * 2
    rec_b = (Bf * state + tokens * state + tokens * H * K * 2 * 2 + tokens * HV * V * 2 + tokens * HV * 2 * 2
             + tokens * HV * V * 2 + tokens * 4)
    rows["gdn_front_views_b64x16"] = _row(us, conv_b + rec_b)
    del g, proj, front_rows

    # next row (f) 4: the Mamba2 tree state update at Nemotron 3 Nano's TP1 layer (64 heads x 64 x 128 state, 8
    # groups, fp32 state pool), batch 64 x 16-node seeded trees, one state slot per row
    from eagle_harness.kernels.mamba2_tree import mamba2_tree_state_update

    Bm, Wm, Hm, Pm, Gm, Nm = 64, 16, 64, 64, 8, 128
    tm = Bm * Wm
    rng_m = np.random.default_rng(8)
    par_m = torch.tensor([seeded_tree(rng_m, Wm) for _ in range(Bm)], dtype=torch.int32, device=dev)
    slots_m = (1 + torch.arange(Bm * Wm, dtype=torch.int32, device=dev)).view(Bm, Wm)
    st_m = torch.randn(1 + Bm * Wm, Hm, Pm, Nm, device=dev, generator=gen) * 0.1
    x_m = torch.randn(tm, Hm, Pm, device=dev, generator=gen).bfloat16()
    dt_m = torch.randn(tm, Hm, device=dev, generator=gen).bfloat16()
    bc_m = torch.randn(tm, 2, Gm, Nm, device=dev, generator=gen).bfloat16()
    A_m, D_m, bias_m = -torch.rand(Hm, device=dev), torch.randn(Hm, device=dev), torch.randn(Hm, device=dev)
    o_m = torch.empty_like(x_m)
    qsl_m = torch.arange(0, tm + 1, Wm, dtype=torch.int32, device=dev)
    us = _time_graph(lambda: mamba2_tree_state_update(st_m, x_m, dt_m, A_m, bc_m[:, 0], bc_m[:, 1], D_m, bias_m, o_m,
                                                      state_indices=slots_m, parents=par_m, query_start_loc=qsl_m),
                     steps)
    state_m = Hm * Pm * Nm * 4
    rows["mamba2_tree_b64x16_nano_tp1"] = _row(us, Bm * state_m + tm * state_m + tm * (2 * Hm * Pm * 2 + 2 * Gm * Nm * 2
                                                                                      + Hm * 2 + 8))
    del st_m

    # a6: fp8-e4m3 pages with per-(page, KV head) scales at batch 512 (Hq24/Hkv4, D256, prefixes U[512, 4096])
    for name, shape, fp8, dtype in (("a6_attention_fp8_b512_d256", ATTN_B512_FP8, True, torch.bfloat16),
                                    ("a6_attention_fp32_b1_d128", ATTN_B1, False, torch.float32),
                                    ("a6_attention_bf16_b1_d128", ATTN_B1, False, torch.bfloat16)):
        x = attention_inputs(shape, seed=3, device=dev, dtype=dtype, fp8=fp8, gen_device=dev)
        out = torch.empty_like(x["q"])
        kw = dict(k_scale=x["k_scale"], v_scale=x["v_scale"]) if fp8 else {}

        def attn():
            verify_attention(x["q"], x["k_new"], x["v_new"], x["key_cache"], x["value_cache"], x["block_table"],
                             x["context_lens"], x["query_start_loc"], x["masks"], x["scale"], out,
                             max_query_len=shape.width, **kw)

        us = _time_graph(attn, steps)
        ctx = x["context_lens"].tolist()
        tokens = shape.batch * shape.width
        esz = 1 if fp8 else x["key_cache"].element_size()
        qsz = x["q"].element_size()
        nbytes = (sum(ctx) * shape.hkv * shape.d * 2 * esz + tokens * shape.hq * shape.d * 2 * qsz
                  + tokens * shape.hkv * shape.d * 2 * qsz + sum(math.ceil(L / shape.page) for L in ctx) * 4
                  + (sum(math.ceil(L / shape.page) for L in ctx) * shape.hkv * 4 * 2 if fp8 else 0))
        rows[name] = _row(us, nbytes)
        del x, out

    # a4: the snapshot walk at batch 1 and 256 (H16/HV32, K = V = 128, fp32 states, per-row slots)
    for name, shape in (("a4_walk_b1", GDN_B1), ("a4_walk_b256", GDN_B256)):
        g = gdn_inputs(shape, seed=2, device=dev, layout="vllm", gen_device=dev)
        o = torch.empty_like(g["v"])

        def walk():
            gdn_tree_recurrent_update(g["A_log"], g["dt_bias"], g["q"], g["k"], g["v"], g["a"], g["b"],
                                      initial_state_source=g["pool"], initial_state_indices=g["slots"],
                                      cu_seqlens=g["query_start_loc"], intermediate_states_buffer=g["pool"],
                                      intermediate_state_indices=g["slots"], retrieve_parent_token=g["parent_table"],
                                      num_accepted_tokens=g["num_accepted"], pad_slot_id=0, out=o)

        us = _time_graph(walk, steps)
        Bq, Wq, H, HV, K, V = shape.batch, shape.width, shape.h, shape.hv, shape.k, shape.v
        state = HV * K * V * 4
        tokens = Bq * Wq
        nbytes = (Bq * state + tokens * state + tokens * H * K * 2 * 2 + tokens * HV * V * 2 * 2
                  + tokens * HV * 2 * 2 + tokens * 4)
        rows[name] = _row(us, nbytes)
        del g, o

    # a5: the rounded path replay (bf16 pool) and the commit of one accepted node per request, at 1 and 32 requests
    for Bq in (1, 32):
        x = records_inputs(Bq, seed=Bq, device=dev)
        Wq = x["width"]
        # the path table as the engine derives it: sglang links -> gdn_tree_ancestors (the a2 kernel)
        links = [tree_links(p, Wq) for p in x["trees"]]
        nxt_t = torch.tensor([lk[0] for lk in links], dtype=torch.int64, device=dev)
        sib_t = torch.tensor([lk[1] for lk in links], dtype=torch.int64, device=dev)
        par_t = torch.empty(Bq, Wq, dtype=torch.int64, device=dev)
        anc_t = torch.empty(Bq, 3, Wq, dtype=torch.int32, device=dev)
        paths = torch.zeros(Bq, Wq, 2 + Wq, dtype=torch.int32, device=dev)
        gdn_tree_ancestors(nxt_t, sib_t, par_t, x["state_indices"], Wq, anc_t, x["query_start_loc"], paths)

        def replay():
            gdn_tree_records_update(x["A_log"], x["dt_bias"], x["q"], x["k"], x["v"], x["a"], x["b"],
                                    state=x["state"], state_indices=x["state_indices"],
                                    query_start_loc=x["query_start_loc"], parent=x["parent"], tree_paths=paths,
                                    records=x["records"], record_indices=x["record_indices"], width=Wq)

        us = _time_graph(replay, steps)
        HV, K, V = 48, 128, 128
        nbytes = (Bq * HV * V * K * 2 + Bq * Wq * 16 * K * 2 * 2 + Bq * Wq * HV * V * 2 * 2 + Bq * Wq * HV * 4
                  + Bq * Wq * HV * (V + K + 1) * 4)
        rows[f"a5_path_replay_bf16_b{Bq}"] = _row(us, nbytes)
        steps_c = torch.full((Bq,), Wq - 1, dtype=torch.int32, device=dev)
        state5 = x["state"][None]
        us = _time_graph(lambda: gdn_tree_records_commit(state5, x["records"][None], x["state_indices"],
                                                         x["record_indices"], steps_c, x["parent"], True), steps)
        rows[f"a5_commit_bf16_b{Bq}"] = _row(us, Bq * HV * V * K * 2 * 2)
        del x
    return rows


def _records_chunk(steps: int) -> dict:
    """The records contract's chunk form (one GDN layer's verify writing replay records) at 1 / 4 / 16 / 32 requests:
    the time per call of a HIP graph of 5 calls, best of 3 replays of ``steps`` graphs."""
    import torch

    from eagle_harness.kernels.gdn_tree_records import gdn_tree_chunk_update
    from workloads import RECORDS_BATCHES, records_inputs

    dev = torch.device("cuda:0")
    us = {}
    for batch in RECORDS_BATCHES:
        x = records_inputs(batch, seed=batch, device=dev)

        def call():
            gdn_tree_chunk_update(x["A_log"], x["dt_bias"], x["q"], x["k"], x["v"], x["a"], x["b"], state=x["state"],
                                  state_indices=x["state_indices"], query_start_loc=x["query_start_loc"],
                                  parent=x["parent"], records=x["records"], record_indices=x["record_indices"],
                                  width=x["width"])

        us[batch] = _time_graph(call, steps)
        del x
    return {"workload": "GDN records chunk form per layer: H16/HV48 K=V=128, 16-node trees, bf16 pool, bf16 q/k/v",
            "us_per_call": us, "reference_published_us": RECORDS_PUBLISHED_US,
            "speedup_vs_reference": {b: RECORDS_PUBLISHED_US[b] / us[b] for b in us}}


def _time_round(fn, steps: int) -> float:
    """Microseconds per call of ``fn`` (a whole round): a HIP graph of one call, replayed ``steps`` times between
    events, best of 3. One call per graph, so no part is timed against its own warm caches."""
    return _time_graph(fn, steps, reps=1)


def _configs(steps: int) -> dict:
    """The configurations beside the metric's step, each timed as whole rounds: the GDN layer at batch 256 (conv,
    snapshot walk, accepted-path commit), the quantized hybrid round at batch 512 (stage, fp8 attention, three GDN
    layers, greedy targets over 151936 tokens, tree walk, commit of the three layers), and the records contract's
    chunk form at batch 64 and 512 with the same heads (bf16 and fp32 pools)."""
    import math

    import numpy as np
    import torch

    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_chunk_update
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit
    from eagle_harness.vllm.tree_accept import accept_tree, greedy_targets
    from eagle_harness.vllm.verify_attention import verify_attention
    from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage
    from workloads import ATTN_B512_FP8, GDN_B256, GdnShape, accept_paths, attention_inputs, gdn_inputs, records_inputs

    dev = torch.device("cuda:0")
    out = {}

    def layer(g, conv_out, rec_out, parents_tab, ancestors):
        tokens = conv_out.shape[0]
        H, K = g["q"].shape[2], g["q"].shape[3]
        HV, V = g["v"].shape[2], g["v"].shape[3]
        gdn_tree_conv1d_update(g["x"].t()[None], g["conv_state"], g["conv_weight"], None, "silu",
                               g["slots0"], None, None, ancestors, pad_slot_id=0, out=conv_out.t()[None],
                               num_accepted_tokens=g["num_accepted"], query_start_loc=g["query_start_loc"])
        gdn_tree_recurrent_update(g["A_log"], g["dt_bias"], conv_out[:, : H * K].view(1, tokens, H, K),
                                  conv_out[:, H * K : 2 * H * K].view(1, tokens, H, K),
                                  conv_out[:, 2 * H * K :].view(1, tokens, HV, V), g["a"], g["b"],
                                  initial_state_source=g["pool"], initial_state_indices=g["slots"],
                                  cu_seqlens=g["query_start_loc"], intermediate_states_buffer=g["pool"],
                                  intermediate_state_indices=g["slots"], retrieve_parent_token=parents_tab,
                                  num_accepted_tokens=g["num_accepted"], pad_slot_id=0, out=rec_out)

    # configuration 4: one GDN layer at batch 256 x 16 (conv, walk, commit of seeded accepted paths U[1, 12])
    sh = GDN_B256
    g = gdn_inputs(sh, seed=6, device=dev, layout="vllm", gen_device=dev)
    g["slots0"] = g["slots"][:, 0].contiguous()
    tokens = sh.batch * sh.width
    conv_out = torch.empty_like(g["x"])
    rec_out = torch.empty(1, tokens, sh.hv, sh.v, dtype=torch.bfloat16, device=dev)
    path, plen = accept_paths(g["parents"], 6, sh.width)
    last = [int(path[b, int(plen[b]) - 1]) for b in range(sh.batch)]
    path_d, plen_d = path.to(dev), plen.to(dev)
    idx = torch.arange(sh.batch, dtype=torch.int32, device=dev)
    commit = LinearStateCommit([(g["conv_state"], g["pool"])], [g["slots"]], dev)

    def round4():
        layer(g, conv_out, rec_out, g["parent_table"], g["ancestors"])
        commit.commit(idx, path_d, plen_d)

    us = _time_round(round4, steps)
    nb = _gdn_layer_bytes(sh.batch, sh.width, sh.h, sh.hv, sh.k, sh.v, g["dim"], plen.tolist(), last)
    total = sum(nb.values())
    out["cfg4_gdn_layer_b256x16"] = _row(us, total, verified_tree_tokens_per_s=tokens / (us * 1e-6), parts=nb)
    del g, conv_out, rec_out, commit

    # configuration 5: the quantized hybrid round at batch 512 x 16: stage, one fp8-e4m3 attention layer (prefixes
    # U[512, 4096], per-(page, KV head) scales), three GDN layers (conv + walk), greedy targets over 151936 tokens,
    # the tree walk and the commit of the three layers' accepted states
    sh5 = GdnShape(512, 16, 16, 32, 128, 128)
    W5, B5, vocab = sh5.width, sh5.batch, 151936
    att = attention_inputs(ATTN_B512_FP8, seed=9, device=dev, fp8=True, gen_device=dev)
    layers = []
    for li in range(3):
        gl = gdn_inputs(sh5, seed=9, device=dev, layout="vllm", gen_device=dev)  # the same trees as the attention
        gl["slots0"] = gl["slots"][:, 0].contiguous()
        layers.append(gl)
    assert layers[0]["parents"] == att["parents"]
    tokens5 = B5 * W5
    store = TreeStore(B5, W5, dev)
    store.parents.copy_(torch.tensor(att["parents"], dtype=torch.int32))
    stage = VerifyStage(B5, tokens5, W5, dev)
    chain = (att["context_lens"].to(torch.int64)[:, None] + torch.arange(W5, device=dev)).reshape(-1)
    positions = chain.clone()
    idx5 = torch.arange(B5, dtype=torch.int32, device=dev)
    qsl5 = att["query_start_loc"]
    attn_out = torch.empty_like(att["q"])
    conv5 = torch.empty_like(layers[0]["x"])
    rec5 = torch.empty(1, tokens5, sh5.hv, sh5.v, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(9)
    logits = torch.randn(tokens5, vocab, device=dev, generator=gen).bfloat16()
    target = torch.empty(tokens5, dtype=torch.int64, device=dev)
    # a node's draft equals its parent's target at 80 % of the nodes (the walk accepts a child whose draft is the
    # target of the row it hangs from): accepted paths of a few rows
    greedy_targets(logits, out=target)
    par = torch.tensor(att["parents"], dtype=torch.int64, device=dev)
    from_parent = target[(torch.arange(B5, device=dev)[:, None] * W5 + par.clamp(min=0)).reshape(-1)]
    agree = torch.rand(tokens5, device=dev, generator=gen) < 0.8
    drafted = torch.where(agree, from_parent, torch.randint(0, vocab, (tokens5,), device=dev, generator=gen))
    commit5 = LinearStateCommit([(gl["conv_state"], gl["pool"]) for gl in layers], [gl["slots"] for gl in layers], dev)

    def round5():
        stage.stage(store, idx5, qsl5, qsl5, positions, B5, tokens5, tree=True)
        verify_attention(att["q"], att["k_new"], att["v_new"], att["key_cache"], att["value_cache"],
                         att["block_table"], stage.context_lens[:B5], qsl5, stage.masks[:B5], att["scale"], attn_out,
                         max_query_len=W5, k_scale=att["k_scale"], v_scale=att["v_scale"])
        for gl in layers:
            layer(gl, conv5, rec5, stage.parents[:B5], stage.ancestors[:B5])
        greedy_targets(logits, out=target)
        accept_tree(target, drafted, qsl5, idx5, store.parents, store)
        commit5.commit(idx5, store.path, store.path_len)
        positions.copy_(chain)

    us = _time_round(round5, steps)
    ctx = att["context_lens"].tolist()
    pages = sum(math.ceil(L / 16) for L in ctx)
    attn_b = (sum(ctx) * 4 * 256 * 2 + pages * 4 * 4 * 2 + pages * 4 + tokens5 * 24 * 256 * 2 * 2
              + tokens5 * 4 * 256 * 2 * 2)
    plen5 = store.path_len.cpu().tolist()
    last5 = [int(store.path[b, plen5[b] - 1]) for b in range(B5)]
    nb5 = _gdn_layer_bytes(B5, W5, sh5.h, sh5.hv, sh5.k, sh5.v, layers[0]["dim"], plen5, last5)
    parts5 = {"attention_fp8": attn_b, "gdn_layers_x3": 3 * (nb5["conv"] + nb5["recurrence"]),
              "logits_argmax": logits.numel() * 2 + tokens5 * 8, "commit_x3": 3 * nb5["commit"]}
    out["cfg5_hybrid_round_b512x16"] = _row(us, sum(parts5.values()), verified_tree_tokens_per_s=tokens5 / (us * 1e-6),
                                            parts=parts5, accepted_mean=float(np.mean(plen5)))
    del att, layers, logits, commit5

    # the records contract (no per-node snapshots) at the same heads, batch 64 and 512: the chunk form per layer
    for B in (64, 512):
        for pool_dtype, pname in ((torch.bfloat16, "bf16"), (torch.float32, "fp32")):
            x = records_inputs(B, seed=B, device=dev, pool_dtype=pool_dtype, heads=16, value_heads=32)

            def chunk():
                gdn_tree_chunk_update(x["A_log"], x["dt_bias"], x["q"], x["k"], x["v"], x["a"], x["b"],
                                      state=x["state"], state_indices=x["state_indices"],
                                      query_start_loc=x["query_start_loc"], parent=x["parent"], records=x["records"],
                                      record_indices=x["record_indices"], width=x["width"])

            us = _time_round(chunk, steps)
            Wr, HV, K, V = x["width"], 32, 128, 128
            esz = 2 if pool_dtype == torch.bfloat16 else 4
            nbytes = (B * HV * V * K * esz + B * Wr * HV * (V + K + 1) * 4 + B * Wr * 16 * K * 2 * 2
                      + B * Wr * HV * V * 2 * 2 + B * Wr * HV * 2 * 2)
            out[f"records_chunk_b{B}x16_h16_hv32_{pname}_pool"] = _row(us, nbytes)
            del x
    return out


def _cpu_configs(seconds: float) -> dict:
    """The oracle (torch on this host's cores) over the configurations, each timed in whole passes for at least
    ``seconds`` (one pass at least, after an untimed one): configurations 1-4 whole (attention fp32 at batch 1, the
    GDN layer with conv, walk and commit at batch 1, bf16 attention at batch 64, the GDN layer at batch 256), and
    configuration 5, the quantized hybrid round at batch 512, layer by layer on a sample of 32 of its requests (fp8
    attention, three GDN layers through one reused state pool, greedy targets over 151936 tokens, the walk, the commit
    of the three layers), its tokens/s extrapolated linearly (the oracle's cost is linear in requests; the whole
    round's 3 x 17 GB of snapshots and 2.5 GB of logits are left out)."""
    import dataclasses
    import platform

    import torch

    from oracle import accept as oacc
    from oracle import attention as oa
    from oracle import commit as ocm
    from oracle import conv as oc
    from oracle import recurrence as orr
    from workloads import (ATTN_B1, ATTN_B64, ATTN_B512_FP8, GDN_B1, GDN_B256, GdnShape, accept_paths,
                           attention_inputs, gdn_inputs)

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass

    def timed(fn):
        fn()  # one untimed pass: first-touch allocations and thread-pool start
        t0 = time.perf_counter()
        passes = 0
        while passes == 0 or time.perf_counter() - t0 < seconds:
            fn()
            passes += 1
        return (time.perf_counter() - t0) / passes

    def attention_pass(a, width, **kw):
        return lambda: oa.verify_attention(a["q"], a["k_new"], a["v_new"], a["key_cache"], a["value_cache"],
                                           a["block_table"], a["context_lens"], a["query_start_loc"], a["masks"],
                                           a["scale"], torch.empty_like(a["q"]), max_query_len=width, **kw)

    def gdn_pass(g, shape, path, plen):
        """Conv, walk and commit of one layer. Passes after the first start from the states the commit left (the
        cost of a pass does not depend on them)."""
        tokens, HK = shape.batch * shape.width, shape.h * shape.k
        slots0 = g["slots"][:, 0].contiguous()

        def run():
            conv_out = torch.empty_like(g["x"])
            oc.gdn_tree_conv1d_update(g["x"].t()[None], g["conv_state"], g["conv_weight"], None, "silu", slots0, None,
                                      None, g["ancestors"], pad_slot_id=0, out=conv_out.t()[None],
                                      num_accepted_tokens=g["num_accepted"], query_start_loc=g["query_start_loc"])
            orr.gdn_tree_recurrent_update(g["A_log"], g["dt_bias"], conv_out[:, :HK].reshape(1, tokens, shape.h, shape.k),
                                          conv_out[:, HK : 2 * HK].reshape(1, tokens, shape.h, shape.k),
                                          conv_out[:, 2 * HK :].reshape(1, tokens, shape.hv, shape.v), g["a"], g["b"],
                                          initial_state_source=g["pool"], initial_state_indices=g["slots"],
                                          cu_seqlens=g["query_start_loc"], intermediate_states_buffer=g["pool"],
                                          intermediate_state_indices=g["slots"],
                                          retrieve_parent_token=g["parent_table"],
                                          num_accepted_tokens=g["num_accepted"], pad_slot_id=0)
            ocm.linear_state_commit([g["conv_state"]], [g["pool"]], [g["slots"]],
                                    torch.arange(shape.batch, dtype=torch.int32), path, plen)

        return run

    out = {"cores": threads, "cpu_model": model, "kind": "port"}
    for name, shape, dtype in (("cfg1_attention_fp32_b1", ATTN_B1, torch.float32),
                               ("cfg3_attention_bf16_b64", ATTN_B64, torch.bfloat16)):
        a = attention_inputs(shape, seed=0, dtype=dtype)
        s = timed(attention_pass(a, shape.width))
        out[name] = {"ms_per_pass": s * 1e3, "requests": shape.batch,
                     "verified_tree_tokens_per_s": shape.batch * shape.width / s}
        del a
    for name, shape in (("cfg2_gdn_layer_b1", GDN_B1), ("cfg4_gdn_layer_b256", GDN_B256)):
        g = gdn_inputs(shape, seed=0, layout="vllm")
        path, plen = accept_paths(g["parents"], 0, shape.width)
        s = timed(gdn_pass(g, shape, path, plen))
        out[name] = {"ms_per_pass": s * 1e3, "requests": shape.batch,
                     "verified_tree_tokens_per_s": shape.batch * shape.width / s}
        del g

    # configuration 5 on a sample of its requests, layer by layer
    sample, B5, vocab = 32, ATTN_B512_FP8.batch, 151936
    shape_a = dataclasses.replace(ATTN_B512_FP8, batch=sample)
    shape_g = GdnShape(sample, 16, 16, 32, 128, 128)
    W = shape_a.width
    a = attention_inputs(shape_a, seed=9, fp8=True)
    g = gdn_inputs(shape_g, seed=9, layout="vllm")  # one state pool, reused by the three layers
    path, plen = accept_paths(g["parents"], 9, W)
    gen = torch.Generator().manual_seed(9)
    logits = torch.randn(sample * W, vocab, generator=gen).bfloat16()
    drafted = torch.randint(0, vocab, (sample * W,), generator=gen)
    cu = torch.arange(0, sample * W + 1, W, dtype=torch.int32)
    idx = torch.arange(sample, dtype=torch.int32)
    parents = torch.tensor(a["parents"], dtype=torch.int32)
    attn = attention_pass(a, W, k_scale=a["k_scale"], v_scale=a["v_scale"])
    layer = gdn_pass(g, shape_g, path, plen)

    def round5():
        attn()
        for _ in range(3):
            layer()
        target = oacc.argmax_rows(logits)
        oacc.accept_tree(target, drafted, cu, idx, parents, torch.zeros(sample, W, dtype=torch.int32),
                         torch.ones(sample, dtype=torch.int32), W)

    s = timed(round5)
    out["cfg5_hybrid_round_b512"] = {
        "ms_per_pass": s * 1e3, "requests": sample, "of_requests": B5,
        "verified_tree_tokens_per_s": sample * W / s,
        "sample": f"{sample} of {B5} requests, the round's parts layer by layer (three GDN layers through one state "
                  "pool); tokens/s extrapolated linearly in requests"}
    return out


def _calibrate_copy(steps: int) -> None:
    import torch

    dev = torch.device("cuda:0")
    n = 1 << 30
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "ms": dt * 1e3,
                      "GB/s (read+write)": 2 * n / dt / 1e9}), flush=True)
    # the write ceiling: a 2 GiB fill (the GDN walk's snapshot stores are ~2.2 GB of writes per step)
    big = torch.empty(2 * n // 4, dtype=torch.float32, device=dev)
    del src, dst
    for _ in range(2):
        big.fill_(1.0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        big.fill_(1.0)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"calibration": "device fill", "bytes_written": 2 * n, "ms": dt * 1e3,
                      "GB/s (write)": 2 * n / dt / 1e9}), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the GPU takes ~30 step replays (~25 ms) to reach its steady step time (the first 10 run ~8 % slower)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--chunk", type=int, default=0, help="attention context keys per split (0: the library's)")
    ap.add_argument("--cpu-sample", type=int, default=64, help="requests in the CPU baseline's sample (0: skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="the CPU baseline runs whole passes this long")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--records-only", action="store_true", help="time only the records chunk form and print it")
    ap.add_argument("--rows-only", action="store_true", help="time only the rows outside the step and print them")
    ap.add_argument("--step-only", action="store_true",
                    help="time only the verify step (no records chunk, rows or configurations); for quick comparisons")
    ap.add_argument("--configs-only", action="store_true", help="time only the configuration rounds and print them")
    ap.add_argument("--cpu-configs", type=float, default=0.5,
                    help="seconds per configuration for the oracle's CPU times of configurations 1-5 (negative: skip)")
    ap.add_argument("--eager", action="store_true",
                    help="rows, records and configurations without graph capture (for counter runs); times include "
                         "launch gaps")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU (--gpus 1): the verify path needs no collective; a sharded deployment runs "
              "one such process per GPU on its share of the requests and heads.", file=sys.stderr)
        return 2
    import torch

    if args.calibrate_copy:
        _calibrate_copy(args.steps)
        return 0
    if args.records_only:
        print(json.dumps({"records_chunk": _records_chunk(args.steps)}), flush=True)
        return 0
    if args.rows_only:
        print(json.dumps({"rows": _rows(args.steps)}), flush=True)
        return 0
    if args.configs_only:
        print(json.dumps({"configs": _configs(args.steps)}), flush=True)
        return 0

    from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
    from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
    from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit
    from eagle_harness.vllm.verify_attention import verify_attention
    from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage
    from workloads import ATTN_B64, GDN_B64, accept_paths, attention_inputs, gdn_inputs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, W = ATTN_B64.batch, ATTN_B64.width
    seed = 0
    att = attention_inputs(ATTN_B64, seed=seed, device=dev, gen_device=dev)
    gdn = gdn_inputs(GDN_B64, seed=seed, device=dev, layout="vllm", gen_device=dev)
    parents = att["parents"]
    assert parents == gdn["parents"]  # one tree per request drives both layers
    tokens = B * W
    store = TreeStore(B, W, dev)
    store.parents.copy_(torch.tensor(parents, dtype=torch.int32))
    stage = VerifyStage(B, tokens, W, dev)
    chain_pos = (att["context_lens"].to(torch.int64)[:, None] + torch.arange(W, device=dev)).reshape(-1)
    positions = chain_pos.clone()
    idx = torch.arange(B, dtype=torch.int32, device=dev)
    qsl = att["query_start_loc"]
    path, path_len = accept_paths(parents, seed, W)
    path_last = [int(path[b, int(path_len[b]) - 1]) for b in range(B)]
    path_d, path_len_d = path.to(dev), path_len.to(dev)
    commit = LinearStateCommit([(gdn["conv_state"], gdn["pool"])], [gdn["slots"]], dev)
    out = torch.empty_like(att["q"])
    conv_out = torch.empty_like(gdn["x"])
    H, HV, K, V = GDN_B64.h, GDN_B64.hv, GDN_B64.k, GDN_B64.v
    HK = H * K
    q4 = conv_out[:, :HK].view(1, tokens, H, K)
    k4 = conv_out[:, HK : 2 * HK].view(1, tokens, H, K)
    v4 = conv_out[:, 2 * HK :].view(1, tokens, HV, V)
    rec_out = torch.empty(1, tokens, HV, V, dtype=torch.bfloat16, device=dev)
    slots0 = gdn["slots"][:, 0].contiguous()

    # the CPU baseline's sample: the first requests, copied before any step mutates the states
    work = None
    if args.cpu_sample > 0:
        S = args.cpu_sample
        a_cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in att.items()}
        a_cpu.update(q=a_cpu["q"][: S * W], k_new=a_cpu["k_new"][: S * W], v_new=a_cpu["v_new"][: S * W],
                     block_table=a_cpu["block_table"][:S], context_lens=a_cpu["context_lens"][:S],
                     query_start_loc=a_cpu["query_start_loc"][: S + 1], masks=a_cpu["masks"][:S])
        nslot = 1 + S * (W + 1)
        g_cpu = dict(x=gdn["x"][: S * W].cpu(), conv_state=gdn["conv_state"][:nslot].cpu(),
                     conv_weight=gdn["conv_weight"].cpu(), slots=gdn["slots"][:S].cpu(),
                     ancestors=gdn["ancestors"][:S].cpu(), num_accepted=gdn["num_accepted"][:S].cpu(),
                     query_start_loc=gdn["query_start_loc"][: S + 1].cpu(), A_log=gdn["A_log"].cpu(),
                     dt_bias=gdn["dt_bias"].cpu(), a=gdn["a"][: S * W].cpu(), b=gdn["b"][: S * W].cpu(),
                     pool=gdn["pool"][:nslot].cpu(), parent_table=gdn["parent_table"][:S].cpu(), path=path[:S],
                     path_len=path_len[:S], H=H, HV=HV, K=K, V=V)
        work = dict(W=W, attn_cpu=a_cpu, gdn_cpu=g_cpu)

    names = ["stage", "attention", "conv", "recurrence", "commit"]

    def run_stage():
        stage.stage(store, idx, qsl, qsl, positions, B, tokens, tree=True)

    def run_attention():
        verify_attention(att["q"], att["k_new"], att["v_new"], att["key_cache"], att["value_cache"],
                         att["block_table"], stage.context_lens[:B], qsl, stage.masks[:B], att["scale"], out,
                         max_query_len=W, chunk=args.chunk)

    def run_conv():
        gdn_tree_conv1d_update(gdn["x"].t()[None], gdn["conv_state"], gdn["conv_weight"], None, "silu", slots0, None,
                               None, stage.ancestors[:B], pad_slot_id=0, out=conv_out.t()[None],
                               num_accepted_tokens=gdn["num_accepted"], query_start_loc=qsl)

    def run_recurrence():
        gdn_tree_recurrent_update(gdn["A_log"], gdn["dt_bias"], q4, k4, v4, gdn["a"], gdn["b"],
                                  initial_state_source=gdn["pool"], initial_state_indices=gdn["slots"],
                                  cu_seqlens=qsl, intermediate_states_buffer=gdn["pool"],
                                  intermediate_state_indices=gdn["slots"], retrieve_parent_token=stage.parents[:B],
                                  num_accepted_tokens=gdn["num_accepted"], pad_slot_id=0, out=rec_out)

    def run_commit():
        commit.commit(idx, path_d, path_len_d)
        stage.restore_positions(positions, tokens)  # the chain positions back (the stage rewrote them to depths)

    parts = dict(stage=run_stage, attention=run_attention, conv=run_conv, recurrence=run_recurrence,
                 commit=run_commit)

    def step():
        for n in names:
            parts[n]()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # A step is replayed as one HIP graph (the launches of a verify round, as a serving loop issues them), so the
    # timing is the GPU's, not the host's Python; graphs are timed between events on the replay stream.
    def graph_of(fn, reps=1):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        return g

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    # A part's time is what it adds to the step: T(step) - T(step without it), both one graph replayed back to back
    # (the positions copy stays in every variant, so the stage always reads the same positions). Every kernel so runs
    # between the kernels it has in the step, with the caches they leave: replayed alone, a kernel finds its own inputs
    # in the 256 MB last-level cache (the walk runs ~50 us faster alone), and split into one graph per part, the
    # dispatch gaps between the graphs let the cache write back the previous part's dirty lines (~30 us for the walk).
    # Graph-launch overhead cancels in the difference.
    def without(skip):
        def run():
            for n in names:
                if n == skip:
                    continue
                if n == "commit":
                    commit.commit(idx, path_d, path_len_d)  # the commit part without its positions copy
                else:
                    parts[n]()
            stage.restore_positions(positions, tokens)
        return run

    timing = "hip-graph replay"
    try:
        g_step = graph_of(step)
        g_less = {n: graph_of(without(n)) for n in names}
        # The parts first (each variant replayed back to back against the whole step), then the headline: W
        # warm-up replays and exactly K timed ones. A GPU coming out of idle runs its first hundred or so step
        # replays up to ~5 % slower while its clocks ramp: the parts are timed after 100 untimed replays, and the
        # K timed steps come after them, in the steady state a serving loop runs in.
        reps = max(args.steps, 30)
        for _ in range(100):
            g_step.replay()
        t_step = timed(g_step.replay, reps)
        per = {n: t_step - timed(g_less[n].replay, reps) for n in names}
        for _ in range(args.warmup):
            g_step.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g_step.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    except RuntimeError as err:  # capture unavailable: eager launches (host time between launches included)
        timing = f"eager ({err.__class__.__name__}: graph capture failed)"
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per = {n: timed(parts[n], args.steps) for n in names}
    ctx = att["context_lens"].cpu().tolist()
    nbytes = _algorithmic_bytes(B, W, dict(hq=ATTN_B64.hq, hkv=ATTN_B64.hkv, d=ATTN_B64.d, page=ATTN_B64.page),
                                dict(h=H, hv=HV, k=K, v=V, dim=gdn["dim"]), ctx, path_len.tolist(), path_last)
    kernels = {n: {"ms": per[n], "bytes": nbytes[n], "GB/s": nbytes[n] / (per[n] * 1e-3) / 1e9,
                   "frac_of_hbm_peak": nbytes[n] / (per[n] * 1e-3) / HBM_PEAK} for n in names}
    dominant = max(names, key=lambda n: per[n])
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(dominant, {}).get("bytes_per_launch")
    achieved = nbytes[dominant] / (per[dominant] * 1e-3)
    step_bytes = sum(nbytes.values())
    result = {
        "metric": METRIC,
        "value": tokens * args.steps / wall,
        "unit": "verified tree tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded trees, prefixes, pages and tensors; random-init layer parameters)",
        "config": {
            "workload": "tree-verify attention (B64 T16, Hq24/Hkv4 D256 bf16, page 16, L~U[1024,8192]) + one GDN "
                        "layer (tree conv1d + snapshot walk H16/HV32 K=V=128 fp32 states + accepted-path commit)",
            "batch": B, "tree_nodes": W, "attention_chunk": args.chunk,
            "step_hbm_bytes": step_bytes, "step_frac_of_hbm_roofline": step_bytes / (wall / args.steps) / HBM_PEAK,
            "timing": timing, "parts_sum_ms": sum(per.values()),
        },
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK, "traffic": traffic},
        "kernels": kernels,
        "cpu_baseline": _cpu_baseline(work, args.cpu_sample, args.cpu_seconds) if work is not None else None,
    }
    print(f"[bench] step {wall / args.steps * 1e3:.3f} ms", file=sys.stderr, flush=True)
    if not args.step_only:
        result["records_chunk"] = _records_chunk(args.steps)
        print("[bench] records chunk timed", file=sys.stderr, flush=True)
        result["rows"] = _rows(args.steps)
        print("[bench] rows timed", file=sys.stderr, flush=True)
        result["configs"] = _configs(args.steps)
        print("[bench] configuration rounds timed", file=sys.stderr, flush=True)
        if args.cpu_configs >= 0:
            result["cpu_configs"] = _cpu_configs(args.cpu_configs)
            print("[bench] CPU configurations timed", file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
