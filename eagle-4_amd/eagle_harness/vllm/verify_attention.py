"""Tree-verify attention of a verify forward's full-attention layers (vllm/verify_attention.py), engine-free.

A request's ``W`` verify rows attend to its committed context in the paged KV cache (the same keys for every row)
and to their own tree ancestors among the ``W`` new tokens. Every kernel reads each K / V tile once for all ``G x W``
rows of a KV head (``G`` query heads per KV head); the reference's grid is per query head and reads it ``G`` times.
Three schedules (``csrc/``):

- ``verify_attention_stream.hip`` (default for 16-bit and fp8 pages, up to 1024 requests): a persistent grid of one
  workgroup per resident slot takes equal contiguous shares of all (request, KV head, row group) tiles of 32 keys
  (64 fp8 keys), streamed into LDS by producer waves; segments cut by a share boundary leave fp32 partials that a
  second kernel merges by their log-sum-exp.
- ``verify_attention.hip`` (more requests, a caller-chosen ``chunk``, or a single request whose block table holds at
  most 4096 keys, in 96-key splits): one workgroup per (context split, KV head, request), then the same merge.
- ``verify_attention_f32.hip``: fp32 rows over fp32 pages (the reference test's dtype).

The cache may be bf16 / fp16, or fp8-e4m3 (OCP) with one fp32 scale per (page, KV head) for keys (``k_scale``) and
values (``v_scale``), dequantised inside the kernels: new function relative to the reference, whose vLLM backend
refuses quantized caches (vllm/tree_attention.py:69-70); :mod:`eagle_harness.vllm.tree_attention` routes such caches
here.
"""

from __future__ import annotations

from typing import Optional

import torch

from eagle_harness.kernels import _native

def verify_attention(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    masks: torch.Tensor,
    scale: float,
    out: torch.Tensor,
    *,
    max_query_len: int,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    chunk: int = 0,
    no_alloc: bool = False,
) -> torch.Tensor:
    """Tree verify attention into ``out`` ``[tokens, Hq, D]`` (rows past the last request's are left alone;
    vllm/verify_attention.py:142-207).

    ``q`` ``[tokens, Hq, D]``; ``k_new`` / ``v_new`` ``[tokens, Hkv, D]`` the new tokens' keys and values;
    ``key_cache`` / ``value_cache`` ``[blocks, page, Hkv, D]`` views of the paged cache, which holds each request's
    first ``context_lens[b]`` tokens through ``block_table[b]``; ``masks[b, r]`` has bit ``j`` set iff new token
    ``j`` is row ``r`` or one of its ancestors. Every request has at most ``max_query_len`` (<= 64) rows.
    ``k_scale`` / ``v_scale``: fp32 ``[blocks, Hkv]`` scales of an fp8-e4m3 cache. ``chunk``: context keys per split
    of the split-context schedule (a multiple of 32; 0 lets the library choose: the streamed schedule where it applies,
    the split one for a single short request). ``no_alloc``: allocate nothing; the split partials go to the
    library's static per-GPU buffer (``eagle4_verify_attention_static``, 64 MiB), and a launch needing more raises
    ValueError before anything runs. Every such call on one GPU shares that buffer: calls overlapping in time race.
    """
    num_reqs = query_start_loc.shape[0] - 1
    heads, head_dim = q.shape[1], q.shape[2]
    fp8 = key_cache.dtype == torch.float8_e4m3fn
    if fp8 and (k_scale is None or v_scale is None):
        raise ValueError("an fp8-e4m3 cache needs k_scale and v_scale ([blocks, Hkv] fp32)")
    if fp8 and (k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32):
        raise ValueError("k_scale / v_scale must be fp32")
    if value_cache.dtype != key_cache.dtype:
        raise _native.NotCovered(f"key_cache is {key_cache.dtype} but value_cache is {value_cache.dtype}")
    if fp8:
        blocks, kv_heads = key_cache.shape[0], key_cache.shape[2]
        for name, sc in (("k_scale", k_scale), ("v_scale", v_scale)):
            if sc.dim() != 2 or sc.shape[0] < blocks or sc.shape[1] < kv_heads or sc.device != key_cache.device:
                raise ValueError(f"{name} must be [blocks >= {blocks}, Hkv >= {kv_heads}] fp32 on the cache's device, "
                                 f"got {tuple(sc.shape)}")
    if block_table.dtype != torch.int32:
        raise _native.NotCovered("the block table must be int32")
    for name, t in (("q", q), ("k_new", k_new), ("v_new", v_new), ("out", out), ("key_cache", key_cache),
                    ("value_cache", value_cache)):
        if t.stride(-1) != 1:
            raise _native.NotCovered(f"{name} must have a unit stride over the head dim")
    if masks.stride(1) != 1 or masks.dtype != torch.int64:
        raise _native.NotCovered("masks must be int64 with unit row stride")
    args = _native.AttnArgs(
        q=q.data_ptr(),
        stride_qt=q.stride(0),
        stride_qh=q.stride(1),
        k_new=k_new.data_ptr(),
        stride_knt=k_new.stride(0),
        stride_knh=k_new.stride(1),
        v_new=v_new.data_ptr(),
        stride_vnt=v_new.stride(0),
        stride_vnh=v_new.stride(1),
        key_cache=key_cache.data_ptr(),
        stride_kb=key_cache.stride(0),
        stride_ks=key_cache.stride(1),
        stride_kh=key_cache.stride(2),
        value_cache=value_cache.data_ptr(),
        stride_vb=value_cache.stride(0),
        stride_vs=value_cache.stride(1),
        stride_vh=value_cache.stride(2),
        k_scale=_native.ptr(k_scale),
        stride_ksb=k_scale.stride(0) if fp8 else 0,
        stride_ksh=k_scale.stride(1) if fp8 else 0,
        v_scale=_native.ptr(v_scale),
        stride_vsb=v_scale.stride(0) if fp8 else 0,
        stride_vsh=v_scale.stride(1) if fp8 else 0,
        block_table=_native.itab(block_table),
        context_lens=_native.itab(context_lens),
        query_start_loc=_native.itab(query_start_loc),
        masks=masks.data_ptr(),
        stride_mask=masks.stride(0),
        out=out.data_ptr(),
        stride_ot=out.stride(0),
        stride_oh=out.stride(1),
        workspace=None,
        workspace_bytes=0,
        scale=scale,
        num_reqs=num_reqs,
        Hq=heads,
        Hkv=key_cache.shape[2],
        D=head_dim,
        page=key_cache.shape[1],
        max_query_len=max_query_len,
        max_blocks=block_table.shape[1],
        dtype=_native.dtype_code(q.dtype),
        cache_dtype=_native.dtype_code(key_cache.dtype),
        chunk=chunk,
    )
    if q.dtype != out.dtype or q.dtype != k_new.dtype or q.dtype != v_new.dtype:
        raise _native.NotCovered("q, k_new, v_new and out must share a dtype (bf16, fp16, or fp32 over fp32 pages)")
    lib = _native.library()
    if no_alloc:
        _native.launch("eagle4_verify_attention_static", args, q.device)
        return out
    need = lib.eagle4_verify_attention_workspace(args)
    if need < 0:
        raise _native.NotCovered("eagle4_amd: verify_attention does not cover this launch (shape, dtype or layout)")
    workspace = None
    if need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)  # the torch caching allocator's
        args.workspace = workspace.data_ptr()
        args.workspace_bytes = need
    _native.launch("eagle4_verify_attention", args, q.device)
    return out
