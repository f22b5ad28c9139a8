"""Tree-verify attention over a paged KV cache, restated on the CPU (oracle; test infrastructure only).

Follows ``verify_attention`` (vllm/verify_attention.py:4-11, 58-139, 142-207) as its dense equivalent: row ``r`` of
request ``b`` attends to the ``context_lens[b]`` committed keys of the request's pages (all visible) and to the new
tokens ``j`` whose bit is set in ``masks[b, r]``; softmax in fp32. The reference's split-KV partials and log-sum-exp
merge compute this same softmax (the merge is exact up to fp32 rounding); it rounds P to the value dtype before
P @ V (kernels/online_softmax.py:23), which the tolerance of the checks covers.

fp8: the reference has no quantized tree attention (vllm/tree_attention.py:69-70); the cache format added here is
OCP float8_e4m3fn (max 448) with one fp32 scale per (page, kv head) for keys and one for values, quantized with
``scale = amax / 448`` and round-to-nearest-even, saturating. Its oracle is quantize -> dequantize -> the dense
attention above.
"""

from __future__ import annotations

from typing import Optional

import torch

FP8_MAX = 448.0


def quantize_fp8_pages(cache: torch.Tensor):
    """Per-(page, kv head) amax quantization of a ``[blocks, page, Hkv, D]`` cache to float8_e4m3fn.

    Returns (fp8 cache, fp32 scales [blocks, Hkv]); an all-zero page gets scale 1."""
    amax = cache.float().abs().amax(dim=(1, 3))  # [blocks, Hkv]
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    scaled = cache.float() / scale[:, None, :, None]
    q = scaled.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale.float()


def dequantize_fp8_pages(cache_fp8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 values of a float8_e4m3fn ``[blocks, page, Hkv, D]`` cache with scales ``[blocks, Hkv]``."""
    return cache_fp8.float() * scale[:, None, :, None]


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
) -> torch.Tensor:
    """The reference signature (vllm/verify_attention.py:142-156, plus ``k_scale`` / ``v_scale`` for fp8 caches) on
    CPU tensors; writes each request's rows of ``out`` and leaves rows past the batch alone (:157)."""
    num_reqs = query_start_loc.shape[0] - 1
    page = key_cache.shape[1]
    hq, hkv = q.shape[1], key_cache.shape[2]
    group = hq // hkv
    for b in range(num_reqs):
        start = int(query_start_loc[b])
        w = int(query_start_loc[b + 1]) - start
        if w <= 0:
            continue
        c = int(context_lens[b])
        pos = torch.arange(c)
        blocks = block_table[b, pos // page].long()
        slots = pos % page
        ctx_k = key_cache[blocks, slots].float()  # [c, Hkv, D]
        ctx_v = value_cache[blocks, slots].float()
        if k_scale is not None:
            ctx_k = ctx_k * k_scale[blocks][:, :, None]
            ctx_v = ctx_v * v_scale[blocks][:, :, None]
        keys = torch.cat([ctx_k, k_new[start : start + w].float()])
        values = torch.cat([ctx_v, v_new[start : start + w].float()])
        keys = keys.repeat_interleave(group, 1)
        values = values.repeat_interleave(group, 1)
        qr = q[start : start + w].float()
        scores = torch.einsum("qhd,khd->hqk", qr, keys) * scale
        row_mask = masks[b, :w].tolist()
        tree_visible = torch.tensor([[bool((row_mask[r] >> j) & 1) for j in range(w)] for r in range(w)])
        visible = torch.cat([torch.ones(w, c, dtype=torch.bool), tree_visible], 1)
        scores = scores.masked_fill(~visible, float("-inf"))
        probs = scores.softmax(-1)
        out[start : start + w] = torch.einsum("hqk,khd->qhd", probs, values).to(out.dtype)
    return out
