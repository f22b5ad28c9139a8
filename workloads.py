"""Seeded synthetic inputs of the verify hot path's workloads (trees, paged KV, GDN layers), for tests and bench.py.

Tree rule (every workload): node 0 is the root (the child of the last prefix token); node i > 0 takes a parent drawn
uniformly from the nodes j < i that have fewer than 4 children and depth below 12 (top-k <= 4, depth <= 12). Rows are
parent first. Everything is drawn from ``numpy.random.default_rng(seed)`` (trees, lengths, page permutations) and
``torch.Generator`` (tensors), so a seed fixes a workload.

Workloads by name:

- ``attn_b1_l512_fp32``: tree-verify attention, batch 1, 16 nodes, prefix 512, 16 query / 4 KV heads, D 128,
  Q/K/V ~ N(0,1)*0.5 (fp32: the oracle's CPU case; the GPU runs it in bf16);
- ``gdn_b1``: GDN tree recurrence + conv, batch 1, 16 nodes, 16 key / 32 value heads, K = V = 128;
- ``attn_b64``: batch 64, 16 nodes, page 16 with permuted page tables, prefixes U[1024, 8192], 24 / 4 heads, D 256,
  bf16;
- ``gdn_b256``: batch 256 x 16 nodes of the ``gdn_b1`` heads, with the accepted-path commit (accept lengths
  U[1, 12]);
- ``hybrid_b512``: 4 layers (3 GDN : 1 attention, fp8-e4m3 KV with per-(page, KV head) scales, prefixes
  U[512, 4096]) at batch 512 and the greedy accept over vocab 151936.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

MAX_CHILDREN = 4
MAX_DEPTH = 12


def seeded_tree(rng: np.random.Generator, width: int = 16) -> list[int]:
    """Parents of a ``width``-node tree by the rule above (parents[0] = -1)."""
    parents, depth, children = [-1], [0], [0]
    for _ in range(1, width):
        ok = [j for j in range(len(parents)) if children[j] < MAX_CHILDREN and depth[j] < MAX_DEPTH]
        p = int(ok[int(rng.integers(len(ok)))])
        parents.append(p)
        depth.append(depth[p] + 1)
        children[p] += 1
        children.append(0)
    return parents


def tree_depths(parents: list[int]) -> list[int]:
    d = []
    for p in parents:
        d.append(0 if p < 0 else d[p] + 1)
    return d


def tree_masks(parents: list[int]) -> list[int]:
    """Ancestor-or-self masks as signed int64 (bit j: row j is the row or one of its ancestors)."""
    out: list[int] = []
    for r, p in enumerate(parents):
        m = (1 << r) | (out[p] & ((1 << 64) - 1) if p >= 0 else 0)
        out.append(m - (1 << 64) if m >= 1 << 63 else m)
    return out


def window_codes(parents: list[int]) -> list[list[int]]:
    anc = [[-1, -2, -3]]
    for node in range(1, len(parents)):
        p = parents[node]
        anc.append([p, anc[p][0], anc[p][1]])
    return anc


def tree_links(parents: list[int], width: int) -> tuple[list[int], list[int]]:
    """First-child / next-sibling links of a parent-first tree (children in row order; sglang's form), -1 padded."""
    first = [-1] * width
    sibling = [-1] * width
    last: dict[int, int] = {}
    for node in range(1, len(parents)):
        p = parents[node]
        if p in last:
            sibling[last[p]] = node
        else:
            first[p] = node
        last[p] = node
    return first, sibling


def root_path(parents: list[int], node: int) -> list[int]:
    path = []
    while node >= 0:
        path.append(node)
        node = parents[node]
    return path[::-1]


def committed_path(parents: list[int], accept_len: int) -> list[int]:
    """The accepted path of a synthetic accept length: the root path of the lowest-index node at depth
    ``min(accept_len - 1, max depth)``."""
    d = tree_depths(parents)
    target = min(accept_len - 1, max(d))
    node = next(i for i, di in enumerate(d) if di == target)
    return root_path(parents, node)


# ---------------------------------------------------------------------------------------------------------------------
@dataclass
class AttnShape:
    batch: int
    width: int
    hq: int
    hkv: int
    d: int
    page: int
    lmin: int
    lmax: int


ATTN_B1 = AttnShape(1, 16, 16, 4, 128, 16, 512, 512)
ATTN_B64 = AttnShape(64, 16, 24, 4, 256, 16, 1024, 8192)
ATTN_B512_FP8 = AttnShape(512, 16, 24, 4, 256, 16, 512, 4096)


def attention_inputs(shape: AttnShape, seed: int, device="cpu", dtype=torch.bfloat16, fp8: bool = False,
                     scale_qkv: float = 0.5, gen_device="cpu") -> dict:
    """Inputs of ``verify_attention`` for a workload: seeded trees, prefix lengths, a permuted page table over all
    pages plus one spare page (never read), Q/K/V ~ N(0,1) * ``scale_qkv`` (fp8 caches: N(0,1), quantized per
    (page, KV head) with amax / 448)."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=gen_device).manual_seed(seed)
    B, W = shape.batch, shape.width
    parents = [seeded_tree(rng, W) for _ in range(B)]
    lens = rng.integers(shape.lmin, shape.lmax + 1, size=B)
    blocks_per = [math.ceil(int(L) / shape.page) for L in lens]
    max_blocks = max(max(blocks_per), 1)
    num_blocks = sum(blocks_per) + 1
    perm = torch.from_numpy(rng.permutation(num_blocks).astype(np.int32))
    table = torch.full((B, max_blocks), int(perm[-1]), dtype=torch.int32)  # unused entries: the spare page
    off = 0
    for b, nb in enumerate(blocks_per):
        table[b, :nb] = perm[off : off + nb]
        off += nb
    tokens = B * W
    rnd = lambda *sz: torch.randn(*sz, generator=gen, device=gen_device)  # noqa: E731
    q = (rnd(tokens, shape.hq, shape.d) * scale_qkv).to(dtype)
    k_new = (rnd(tokens, shape.hkv, shape.d) * scale_qkv).to(dtype)
    v_new = (rnd(tokens, shape.hkv, shape.d) * scale_qkv).to(dtype)
    kscale = 1.0 if fp8 else scale_qkv
    key_cache = rnd(num_blocks, shape.page, shape.hkv, shape.d) * kscale
    value_cache = rnd(num_blocks, shape.page, shape.hkv, shape.d) * kscale
    out = dict(parents=parents, context_lens=torch.tensor(lens, dtype=torch.int32), block_table=table, q=q,
               k_new=k_new, v_new=v_new, query_start_loc=torch.arange(0, tokens + 1, W, dtype=torch.int32),
               masks=torch.tensor([tree_masks(p) for p in parents], dtype=torch.int64), scale=shape.d**-0.5,
               max_query_len=W)
    if fp8:
        from_q = _quantize_fp8_pages
        out["key_cache"], out["k_scale"] = from_q(key_cache)
        out["value_cache"], out["v_scale"] = from_q(value_cache)
    else:
        out["key_cache"], out["value_cache"] = key_cache.to(dtype), value_cache.to(dtype)
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in out.items()}


def _quantize_fp8_pages(cache: torch.Tensor):
    """float8_e4m3fn pages with one fp32 scale per (page, KV head): scale = amax / 448 (1 for an all-zero page)."""
    amax = cache.float().abs().amax(dim=(1, 3))
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (cache.float() / scale[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale.float()


# ---------------------------------------------------------------------------------------------------------------------
@dataclass
class GdnShape:
    batch: int
    width: int
    h: int
    hv: int
    k: int
    v: int


GDN_B1 = GdnShape(1, 16, 16, 32, 128, 128)
GDN_B64 = GdnShape(64, 16, 16, 32, 128, 128)
GDN_B256 = GdnShape(256, 16, 16, 32, 128, 128)


def gdn_inputs(shape: GdnShape, seed: int, device="cpu", layout: str = "vllm", state_dtype=torch.float32,
               in_dtype=torch.bfloat16, history: int = 3, gen_device="cpu") -> dict:
    """A GDN layer's tree verify inputs.

    q/k ~ N(0,1) (the kernel L2-normalizes them), v ~ N(0,1), a and b ~ N(0,1) with A_log = dt_bias = 0 (so
    g = -softplus(a), beta = sigmoid(b)), initial states ~ N(0, 0.02^2). The conv part: x ~ N(0,1) over the qkv
    channels (2 H K + HV V), weights ~ N(0, 0.3^2), no bias, SiLU, a seeded 3-column history.

    ``layout`` "vllm": one state slot per verify row in the pool (the request's state at column ``accept - 1`` of its
    slot row, here accept = 1), conv window in slot column 0; "sglang": a state pool with one slot per request and a
    [requests, steps, HV, V, K] snapshot scratch.
    """
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=gen_device).manual_seed(seed + 1)
    B, W, H, HV, K, V = shape.batch, shape.width, shape.h, shape.hv, shape.k, shape.v
    parents = [seeded_tree(rng, W) for _ in range(B)]
    tokens = B * W
    dim = 2 * H * K + HV * V
    x = torch.randn(device=gen_device, size=(tokens, dim,), generator=gen).to(in_dtype)  # the packed projection, token-major
    conv_w = (torch.randn(device=gen_device, size=(dim, 4,), generator=gen) * 0.3).to(in_dtype)
    q = torch.randn(device=gen_device, size=(1, tokens, H, K,), generator=gen).to(in_dtype)
    k = torch.randn(device=gen_device, size=(1, tokens, H, K,), generator=gen).to(in_dtype)
    v = torch.randn(device=gen_device, size=(1, tokens, HV, V,), generator=gen).to(in_dtype)
    a = torch.randn(device=gen_device, size=(tokens, HV,), generator=gen).to(in_dtype)
    b = torch.randn(device=gen_device, size=(tokens, HV,), generator=gen).to(in_dtype)
    A_log = torch.zeros(HV, device=gen_device)
    dt_bias = torch.zeros(HV, device=gen_device)
    par = torch.tensor(parents, dtype=torch.int32)
    anc = torch.tensor([list(zip(*window_codes(p))) for p in parents], dtype=torch.int32)  # [B, 3, W]
    qsl = torch.arange(0, tokens + 1, W, dtype=torch.int32)
    out = dict(parents=parents, parent_table=par, ancestors=anc.contiguous(), query_start_loc=qsl, x=x,
               conv_weight=conv_w, q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt_bias=dt_bias, dim=dim)
    if layout == "vllm":
        # slots[b] = W + 1 per-row slots (row i -> slot 1 + b (W + 1) + i); slot 0 is the null block
        slots = (1 + torch.arange(B * (W + 1), dtype=torch.int32)).view(B, W + 1)
        pool = torch.zeros(1 + B * (W + 1), HV, V, K, dtype=state_dtype, device=gen_device)
        init = torch.randn(device=gen_device, size=(B, HV, V, K,), generator=gen) * 0.02
        pool[slots[:, 0].long()] = init.to(state_dtype)
        conv_state = torch.zeros(1 + B * (W + 1), dim, history + W, dtype=in_dtype, device=gen_device)
        conv_state[slots[:, 0].long(), :, :3] = torch.randn(device=gen_device, size=(B, dim, 3,), generator=gen).to(in_dtype)
        out.update(slots=slots, pool=pool, num_accepted=torch.ones(B, dtype=torch.int32), conv_state=conv_state)
    else:
        pool = (torch.randn(device=gen_device, size=(B + 1, HV, V, K,), generator=gen) * 0.02).to(state_dtype)
        scratch = torch.zeros(B, W, HV, V, K, dtype=state_dtype, device=gen_device)
        conv_state = torch.randn(device=gen_device, size=(B + 1, dim, 3,), generator=gen).to(in_dtype)
        out.update(pool=pool, state_indices=torch.arange(1, B + 1, dtype=torch.int32), scratch=scratch,
                   scratch_indices=torch.arange(B, dtype=torch.int32), conv_state=conv_state,
                   windows=torch.zeros(B, W, dim, 3, dtype=in_dtype, device=gen_device))
    return {kk: (vv.to(device) if isinstance(vv, torch.Tensor) else vv) for kk, vv in out.items()}


# The records contract's chunk form at the 27B-class TP1 layer (16 key / 48 value heads, K = V = 128), 16-node trees.
RECORDS_BATCHES = (1, 4, 16, 32)


def records_inputs(batch: int, seed: int, device="cpu", pool_dtype=torch.bfloat16, heads: int = 16,
                   value_heads: int = 48, dk: int = 128, dv: int = 128, width: int = 16) -> dict:
    """Inputs of one GDN layer's records verify: ``batch`` seeded ``width``-node trees, q/k/v/a/b ~ N(0,1) (bf16),
    A_log = dt_bias = 0, a pool of ``batch + 1`` slots ~ N(0, 0.02^2) (request n reads slot n + 1), records
    [batch, width, HV, V + K + 4] fp32 (request n writes row n)."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    tokens = batch * width
    trees = [seeded_tree(rng, width) for _ in range(batch)]

    def r(*shape):
        return torch.randn(*shape, device=device, generator=gen)

    return dict(
        q=r(1, tokens, heads, dk).bfloat16(), k=r(1, tokens, heads, dk).bfloat16(),
        v=r(1, tokens, value_heads, dv).bfloat16(), a=r(tokens, value_heads).bfloat16(),
        b=r(tokens, value_heads).bfloat16(), A_log=torch.zeros(value_heads, device=device),
        dt_bias=torch.zeros(value_heads, device=device), state=(r(batch + 1, value_heads, dv, dk) * 0.02).to(pool_dtype),
        state_indices=torch.arange(1, batch + 1, dtype=torch.int32, device=device),
        query_start_loc=torch.arange(0, tokens + 1, width, dtype=torch.int32, device=device),
        parent=torch.tensor(trees, dtype=torch.int32, device=device),
        records=torch.zeros(batch, width, value_heads, dv + dk + 4, device=device),
        record_indices=torch.arange(batch, dtype=torch.int32, device=device), width=width, trees=trees)


def accept_paths(parents_list: list[list[int]], seed: int, width: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Seeded accept lengths U[1, 12] -> (path [B, W] int32, path_len [B] int32) of the committed node's root path."""
    rng = np.random.default_rng(seed + 7)
    B = len(parents_list)
    path = torch.zeros(B, width, dtype=torch.int32)
    plen = torch.zeros(B, dtype=torch.int32)
    for b, parents in enumerate(parents_list):
        p = committed_path(parents, int(rng.integers(1, 13)))
        path[b, : len(p)] = torch.tensor(p, dtype=torch.int32)
        plen[b] = len(p)
    return path, plen
