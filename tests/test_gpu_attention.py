"""Tree-verify attention on the GPU against the dense oracle (vllm/verify_attention.py:142-207): bf16 / fp16 paged
caches, GQA, ragged trees, single and multi-split contexts, fp8-e4m3 pages with per-(page, KV head) scales, and rows
past the batch left untouched. Tolerance: 2e-2 absolute, 1e-2 relative (bf16 outputs)."""

import pytest
import torch

from conftest import announce
from oracle import attention as oa
from oracle.tables import tree_masks
from workloads import ATTN_B1, AttnShape, attention_inputs

pytestmark = pytest.mark.gpu


def _run(dev, inp, dtype, chunk=0, fp8=False):
    from eagle_harness.vllm.verify_attention import verify_attention

    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = torch.full_like(g["q"], 7.0)
    kw = dict(k_scale=g["k_scale"], v_scale=g["v_scale"]) if fp8 else {}
    verify_attention(g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"],
                     g["context_lens"], g["query_start_loc"], g["masks"], g["scale"], out,
                     max_query_len=g["max_query_len"], chunk=chunk, **kw)
    torch.cuda.synchronize()
    return out.cpu()


def _want(inp, fp8=False):
    out = torch.full_like(inp["q"], 7.0)
    kw = dict(k_scale=inp["k_scale"], v_scale=inp["v_scale"]) if fp8 else {}
    return oa.verify_attention(inp["q"], inp["k_new"], inp["v_new"], inp["key_cache"], inp["value_cache"],
                               inp["block_table"], inp["context_lens"], inp["query_start_loc"], inp["masks"],
                               inp["scale"], out, max_query_len=inp["max_query_len"], **kw)


def _inputs(contexts, parents, heads, kv_heads, d, page, dtype, seed):
    """Paged caches with permuted blocks, draft rows, and the trees' ancestor masks; two spare rows past the batch."""
    gen = torch.Generator().manual_seed(seed)
    num_reqs = len(contexts)
    widths = [len(p) for p in parents]
    width = max(max(widths), 1)
    max_blocks = max(c // page + 1 for c in contexts) + 1
    num_blocks = num_reqs * max_blocks + 3
    kv = torch.randn(num_blocks, page, kv_heads, 2 * d, generator=gen).to(dtype)
    key_cache, value_cache = kv[..., :d], kv[..., d:]
    table = torch.randperm(num_blocks, generator=gen)[: num_reqs * max_blocks].view(num_reqs, max_blocks).int()
    tokens = sum(widths)
    return dict(
        q=torch.randn(tokens + 2, heads, d, generator=gen).to(dtype),
        k_new=torch.randn(tokens + 2, kv_heads, d, generator=gen).to(dtype),
        v_new=torch.randn(tokens + 2, kv_heads, d, generator=gen).to(dtype),
        key_cache=key_cache, value_cache=value_cache, block_table=table,
        context_lens=torch.tensor(contexts, dtype=torch.int32),
        query_start_loc=torch.tensor([0] + [sum(widths[: i + 1]) for i in range(num_reqs)], dtype=torch.int32),
        masks=torch.tensor([tree_masks(p, width) if p else [0] * width for p in parents], dtype=torch.int64),
        scale=d**-0.5, max_query_len=width,
    )


def _random_parents(gen, width):
    return [-1] + [int(torch.randint(0, r, (1,), generator=gen)) for r in range(1, width)] if width else []


def _close(got, want):
    torch.testing.assert_close(got.float(), want.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize(
    "contexts, parents, heads, kv_heads, d, page",
    [
        ([300], [[-1, 0, 0, 1, 1, 2, 3]], 6, 1, 64, 16),
        ([5, 700, 0], [[-1, 0, 1], [-1, 0, 0, 1, 2, 2, 3, 4, 5], [-1, 0]], 4, 2, 32, 32),
        ([129], [[-1] + [r - 1 for r in range(1, 24)]], 6, 1, 64, 16),
        ([1500, 2], [[-1, 0, 0, 1], [-1, 0]], 8, 2, 128, 16),
        ([1000], [[-1, 0, 1, 1, 3, 0]], 12, 2, 256, 48),  # a page size that is not a power of two
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_matches_dense_oracle(dev, contexts, parents, heads, kv_heads, d, page, dtype):
    """The reference test's cases (tests/test_verify_attention.py:31-92) plus wider heads and pages."""
    announce(f"attention contexts={contexts} heads={heads}/{kv_heads} d={d} page={page} {dtype}")
    inp = _inputs(contexts, parents, heads, kv_heads, d, page, dtype, seed=len(contexts) * 100 + heads)
    tokens = sum(len(p) for p in parents)
    want = _want(inp)
    for chunk in (0, 64, 256):  # one split, many splits, the default
        got = _run(dev, inp, dtype, chunk=chunk)
        _close(got[:tokens], want[:tokens])
        assert torch.equal(got[tokens:], torch.full_like(got[tokens:], 7.0))  # rows past the batch untouched


@pytest.mark.parametrize(
    "contexts, parents, heads, kv_heads, d, page",
    [
        ([300], [[-1, 0, 0, 1, 1, 2, 3]], 6, 1, 64, 16),
        ([5, 700, 0], [[-1, 0, 1], [-1, 0, 0, 1, 2, 2, 3, 4, 5], [-1, 0]], 4, 2, 32, 32),
        ([1500, 2], [[-1, 0, 0, 1], [-1, 0]], 8, 2, 128, 16),
        ([1000], [[-1, 0, 1, 1, 3, 0]], 12, 2, 256, 48),  # a page size that is not a power of two
        ([777, 64], [[-1, 0, 0, 2], [-1, 0, 1]], 6, 2, 256, 2),  # pages smaller than a load instruction's rows
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_matches_dense_oracle(dev, contexts, parents, heads, kv_heads, d, page, dtype):
    """fp8-e4m3 pages (per-(page, KV head) scales) on both schedules: the streamed one (the library's split) and the
    split-context one (a caller-chosen split of 64 or 256 keys)."""
    from workloads import _quantize_fp8_pages

    announce(f"attention fp8 contexts={contexts} heads={heads}/{kv_heads} d={d} page={page} {dtype}")
    inp = _inputs(contexts, parents, heads, kv_heads, d, page, dtype, seed=len(contexts) * 100 + heads + 7)
    inp["key_cache"], inp["k_scale"] = _quantize_fp8_pages(inp["key_cache"].float() * 3.0)
    inp["value_cache"], inp["v_scale"] = _quantize_fp8_pages(inp["value_cache"].float() * 0.5)
    tokens = sum(len(p) for p in parents)
    want = _want(inp, fp8=True)
    for chunk in (0, 64, 256):
        got = _run(dev, inp, dtype, chunk=chunk, fp8=True)
        _close(got[:tokens], want[:tokens])
        assert torch.equal(got[tokens:], torch.full_like(got[tokens:], 7.0))


@pytest.mark.parametrize(
    "contexts, parents, heads, kv_heads, d, page",
    [
        ([300], [[-1, 0, 0, 1, 1, 2, 3]], 6, 1, 64, 16),
        ([5, 700, 0], [[-1, 0, 1], [-1, 0, 0, 1, 2, 2, 3, 4, 5], [-1, 0]], 4, 2, 32, 32),
        ([129], [[-1] + [r - 1 for r in range(1, 24)]], 6, 1, 64, 16),
        ([1500, 2], [[-1, 0, 0, 1], [-1, 0]], 8, 2, 128, 16),
        ([1000], [[-1, 0, 1, 1, 3, 0]], 12, 2, 256, 48),
    ],
)
def test_fp32_matches_dense_oracle(dev, contexts, parents, heads, kv_heads, d, page):
    """fp32 rows over fp32 pages (the reference's own test dtype): single and multi-split requests, ragged trees;
    tolerance 1e-4 (fp32 sums in another order)."""
    announce(f"attention fp32 contexts={contexts} heads={heads}/{kv_heads} d={d} page={page}")
    inp = _inputs(contexts, parents, heads, kv_heads, d, page, torch.float32, seed=len(contexts) * 100 + heads + 3)
    tokens = sum(len(p) for p in parents)
    got = _run(dev, inp, torch.float32)
    torch.testing.assert_close(got[:tokens], _want(inp)[:tokens], atol=1e-4, rtol=1e-4)
    assert torch.equal(got[tokens:], torch.full_like(got[tokens:], 7.0))


def test_fp32_b1_l512_workload(dev):
    """The oracle's CPU case as is: batch 1, 16 seeded nodes, prefix 512, 16 / 4 heads, D 128, fp32."""
    announce("attention b1 l512 fp32")
    inp = attention_inputs(ATTN_B1, seed=1, dtype=torch.float32)
    torch.testing.assert_close(_run(dev, inp, torch.float32), _want(inp), atol=1e-4, rtol=1e-4)


def test_b1_l512_workload(dev):
    """Batch 1, 16 seeded nodes, prefix 512, 16 / 4 heads, D 128 (the oracle's fp32 CPU case, run in bf16)."""
    announce("attention b1 l512")
    inp = attention_inputs(ATTN_B1, seed=1, dtype=torch.bfloat16)
    _close(_run(dev, inp, torch.bfloat16), _want(inp))


@pytest.mark.parametrize("chunk", [0, 512])
def test_b64_heads_short_batch(dev, chunk):
    """The batch-64 workload's heads (24 / 4, D 256, page 16, permuted pages) at 6 requests with long prefixes."""
    announce(f"attention d256 6 requests chunk={chunk}")
    shape = AttnShape(6, 16, 24, 4, 256, 16, 1024, 4000)
    inp = attention_inputs(shape, seed=4, dtype=torch.bfloat16)
    _close(_run(dev, inp, torch.bfloat16, chunk=chunk), _want(inp))


@pytest.mark.parametrize("chunk", [0, 256])
def test_fp8_pages_match_dequantized_oracle(dev, chunk):
    """fp8-e4m3 pages with per-(page, KV head) scales, dequantized in the tile loads; oracle: dequantize, then the
    dense attention."""
    announce(f"attention fp8 chunk={chunk}")
    shape = AttnShape(4, 16, 24, 4, 256, 16, 300, 1800)
    inp = attention_inputs(shape, seed=8, dtype=torch.bfloat16, fp8=True)
    _close(_run(dev, inp, torch.bfloat16, chunk=chunk, fp8=True), _want(inp, fp8=True))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_dequant_is_ocp_e4m3(dev, dtype):
    """Every one of the 256 fp8 codes dequantizes as torch's float8_e4m3fn (OCP): one page whose keys and values
    are the codes, attended by a single row with a one-hot query, reads them back exactly (16-bit outputs)."""
    announce(f"attention fp8 code table {dtype}")
    d, page = 64, 16
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]  # NaN codes stay out
    n = codes.numel()
    keys = n // d + 1
    pages = (keys + page - 1) // page
    cache = torch.zeros(pages * page * d, dtype=torch.uint8)
    cache[:n] = codes
    cache = cache.view(torch.float8_e4m3fn).view(pages, page, 1, d)
    value = cache.clone()
    scale = torch.ones(pages, 1)
    want_vals = value.float().view(pages * page, d)
    # one row attends to exactly one context key through a dominant score: q along a key the others do not have
    from eagle_harness.vllm.verify_attention import verify_attention

    for kpos in range(keys):
        kc = torch.zeros(pages * page, d)
        kc[kpos, 0] = 448.0
        key_cache = kc.to(torch.float8_e4m3fn).view(pages, page, 1, d)
        q = torch.zeros(1, 1, d, dtype=dtype)
        q[0, 0, 0] = 1.0
        out = torch.zeros(1, 1, d, dtype=dtype, device=dev)
        verify_attention(q.to(dev), torch.zeros(1, 1, d, dtype=dtype, device=dev),
                         torch.zeros(1, 1, d, dtype=dtype, device=dev), key_cache.to(dev), value.to(dev),
                         torch.arange(pages, dtype=torch.int32, device=dev)[None], torch.tensor([keys], dtype=torch.int32, device=dev),
                         torch.tensor([0, 1], dtype=torch.int32, device=dev), torch.ones(1, 1, dtype=torch.int64, device=dev),
                         1.0, out, max_query_len=1, k_scale=scale.to(dev), v_scale=scale.to(dev))
        torch.cuda.synchronize()
        torch.testing.assert_close(out[0, 0].cpu().float(), want_vals[kpos].to(dtype).float(), atol=0, rtol=0)


def test_ragged_batch_with_empty_requests(dev):
    """40 requests: contexts 0..2500, tree widths 0..24 (empty requests between others), heads 8 / 2, D 128: the
    streamed schedule's shares cut segments anywhere, so direct and merged rows both occur."""
    announce("attention ragged 40 requests")
    gen = torch.Generator().manual_seed(11)
    contexts = [int(x) for x in torch.randint(0, 2500, (40,), generator=gen)]
    contexts[3] = 0
    widths = [int(x) for x in torch.randint(0, 25, (40,), generator=gen)]
    widths[0], widths[7], widths[39] = 0, 1, 0
    parents = [_random_parents(gen, w) for w in widths]
    inp = _inputs(contexts, parents, 8, 2, 128, 16, torch.bfloat16, seed=12)
    tokens = sum(widths)
    got = _run(dev, inp, torch.bfloat16)
    _close(got[:tokens], _want(inp)[:tokens])
    assert torch.equal(got[tokens:], torch.full_like(got[tokens:], 7.0))


def test_one_long_request_spans_every_group(dev):
    """One request with a 60000-key context (heads 8 / 1, D 128): its single segment is cut into one piece per
    workgroup, all merged."""
    announce("attention one request l60000")
    parents = [[-1, 0, 0, 1, 2, 2, 5, 6]]
    inp = _inputs([60000], parents, 8, 1, 128, 16, torch.bfloat16, seed=13)
    _close(_run(dev, inp, torch.bfloat16)[:8], _want(inp)[:8])


def test_more_requests_than_the_streamed_schedule_holds(dev):
    """1030 requests (above the streamed schedule's 1024) take the split-context schedule with 16-bit pages."""
    announce("attention 1030 requests")
    gen = torch.Generator().manual_seed(14)
    contexts = [int(x) for x in torch.randint(0, 90, (1030,), generator=gen)]
    parents = [_random_parents(gen, int(w)) for w in torch.randint(1, 4, (1030,), generator=gen)]
    inp = _inputs(contexts, parents, 2, 1, 32, 16, torch.bfloat16, seed=15)
    tokens = sum(len(p) for p in parents)
    _close(_run(dev, inp, torch.bfloat16)[:tokens], _want(inp)[:tokens])
