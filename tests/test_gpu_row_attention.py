"""Draft-row attention on the GPU against the oracle (kernels/row_attention.py): the reference tests' scenarios
(tests/test_row_attention_gpu.py:99-200: draft steps 1-11 over windows 0 / 96 / 2048 with random ancestor slots,
extend rows of widths 1-16 over their causal windows, the 4096-key window boundary at lengths 4095-8192), GQA groups,
a packed paged cache, fp16, and splits that leave some of them without keys. bf16 outputs within 2e-2 (the
reference's own bound)."""

import pytest
import torch

from conftest import announce
from oracle import row_attention as ora

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)


def _run(dev, q, keys, values, table, seq_lens, ancestors, *, rows, step, window, splits, table_rows=None,
         table_page=1):
    from eagle_harness.kernels.row_attention import RowsLaunch, rows_attention, rows_padded

    bs, heads, D = q.shape[0] // rows, q.shape[1], q.shape[2]
    n = bs * heads * (splits + 1) * rows_padded(rows)
    out = torch.empty_like(q)
    part_out = torch.empty(n, D, dtype=torch.float32, device=dev)
    part_lse = torch.empty(n, dtype=torch.float32, device=dev)
    rows_attention(q, keys, values, out, part_out, part_lse, table, seq_lens, ancestors, rows_per_request=rows,
                   step=step, window=window, scale=D**-0.5, launch=RowsLaunch(splits=splits, block_n=32),
                   table_rows=table_rows, table_page=table_page)
    torch.cuda.synchronize()
    return out


def _check(got, q, keys, values, table, seq_lens, ancestors, **kw):
    want = ora.rows_attention(q.cpu(), keys.cpu(), None if values is None else values.cpu(), table.cpu(),
                              seq_lens.cpu(), None if ancestors is None else ancestors.cpu(),
                              scale=q.shape[-1] ** -0.5, **kw)
    torch.testing.assert_close(got.cpu().float(), want.float(), **TOL)


def _inputs(dev, seed, bs, rows, heads, kv_heads, D, low, high, dtype=torch.bfloat16):
    gen = torch.Generator(device=dev).manual_seed(seed)
    table = torch.randperm(8 * 4096, device=dev, generator=gen).to(torch.int32).view(8, 4096)
    req = torch.tensor([5, 0, 3][:bs], dtype=torch.int64, device=dev)
    seq = torch.randint(low, high, (bs,), device=dev, generator=gen)
    k = torch.randn(8 * 4096, kv_heads, D, device=dev, generator=gen).to(dtype)
    v = torch.randn(8 * 4096, kv_heads, D, device=dev, generator=gen).to(dtype)
    q = torch.randn(bs * rows, heads, D, device=dev, generator=gen).to(dtype)
    return gen, table, req, seq, k, v, q


@pytest.mark.parametrize("window,low,high", [(0, 40, 300), (96, 40, 300), (2048, 2500, 3900)])
@pytest.mark.parametrize("bs,step", [(1, 1), (1, 5), (3, 7), (2, 11)])
def test_tree_rows_attend_window_and_ancestors(dev, bs, step, window, low, high):
    announce(f"row attention draft step bs={bs} step={step} window={window}")
    rows, depth = 4, 12
    gen, table, req, seq, k, v, q = _inputs(dev, bs * 1000 + step + window, bs, rows, 3, 3, 128, low, high)
    anc = torch.randint(0, 8 * 4096, (bs, rows, depth), dtype=torch.int32, device=dev, generator=gen)
    kw = dict(rows_per_request=rows, step=step, window=window, table_rows=req)
    got = _run(dev, q, k, v, table, seq, anc, rows=rows, step=step, window=window, splits=8, table_rows=req)
    _check(got, q, k, v, table, seq, anc, **kw)


@pytest.mark.parametrize("window,low,high", [(0, 40, 300), (96, 40, 300), (2048, 2500, 3900)])
@pytest.mark.parametrize("bs,width", [(1, 16), (3, 16), (1, 8), (2, 1)])
def test_extend_rows_attend_their_causal_window(dev, bs, width, window, low, high):
    announce(f"row attention extend bs={bs} width={width} window={window}")
    _, table, req, seq, k, v, q = _inputs(dev, bs * 7 + window + width, bs, width, 3, 3, 128, low, high)
    kw = dict(rows_per_request=width, step=0, window=window, table_rows=req)
    got = _run(dev, q, k, v, table, seq, None, rows=width, step=0, window=window, splits=8, table_rows=req)
    _check(got, q, k, v, table, seq, None, **kw)


@pytest.mark.parametrize("heads", [8, 32])
@pytest.mark.parametrize("length", [4095, 4096, 4100, 8192])
@pytest.mark.parametrize("step", [0, 7])
def test_window_boundary(dev, heads, length, step):
    """The reference's Nemotron boundary case: a 4096-key window around lengths 4095 .. 8192."""
    announce(f"row attention window boundary heads={heads} length={length} step={step}")
    window, D = 4096, 128
    rows = 4 if step else 16
    gen = torch.Generator(device=dev).manual_seed(length + heads + step)
    slots = length + rows * max(step, 1)
    table = torch.randperm(slots, device=dev, generator=gen).to(torch.int32).unsqueeze(0)
    req = torch.zeros(1, device=dev, dtype=torch.int64)
    seq = torch.tensor([length], device=dev, dtype=torch.int64)
    q = torch.randn(rows, heads, D, device=dev, generator=gen).bfloat16()
    k = torch.randn(slots, heads, D, device=dev, generator=gen).bfloat16()
    v = torch.randn(slots, heads, D, device=dev, generator=gen).bfloat16()
    anc = table[:, length:].reshape(1, rows, step).contiguous() if step else None
    got = _run(dev, q, k, v, table, seq, anc, rows=rows, step=step, window=window, splits=16, table_rows=req)
    _check(got, q, k, v, table, seq, anc, rows_per_request=rows, step=step, window=window, table_rows=req)


@pytest.mark.parametrize("step", [0, 3])
@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.float16), (256, torch.bfloat16)])
def test_gqa_packed_paged_cache(dev, step, D, dtype):
    """8 query heads over 2 KV heads, K and V packed in one paged cache (pages of 16 slots, a table of 64-slot
    blocks), no table_rows; more splits than the shorter requests have keys."""
    announce(f"row attention gqa packed paged D={D} {dtype} step={step}")
    gen = torch.Generator(device=dev).manual_seed(D + step)
    bs, rows, heads, kvh, page, tpage = 3, 5, 8, 2, 16, 64
    nslots = 4096
    cache = torch.randn(nslots // page, page, kvh, 2 * D, device=dev, generator=gen).to(dtype)
    table = torch.randperm(nslots // tpage, device=dev, generator=gen).to(torch.int32)[: 3 * 20].view(3, 20)
    seq = torch.tensor([33, 700, 1200], device=dev)
    q = torch.randn(bs * rows, heads, D, device=dev, generator=gen).to(dtype)
    anc = torch.randint(0, nslots, (bs, rows, 6), dtype=torch.int32, device=dev, generator=gen) if step else None
    got = _run(dev, q, cache, None, table, seq, anc, rows=rows, step=step, window=512, splits=32, table_page=tpage)
    _check(got, q, cache, None, table, seq, anc, rows_per_request=rows, step=step, window=512, table_page=tpage)


@pytest.mark.parametrize("length", [17, 33, 64, 65, 97, 129, 161, 200])
@pytest.mark.parametrize("step", [0, 9])
def test_every_ring_depth_of_a_split(dev, length, step):
    """One split over the whole context, so the split's tile count is ceil(length / 32): 1 .. 7 tiles take every
    prologue and wait count of the kernel's three-stage ring (loads two tiles ahead, lookups two further). At step 9
    the ancestors' split holds 16 rows x 12 columns (6 tiles); the table is paged (16 slots per entry)."""
    announce(f"row attention ring depths length={length} step={step}")
    rows, depth, heads, D, tpage = (16, 12, 4, 128, 16) if step else (8, 1, 4, 128, 16)
    gen = torch.Generator(device=dev).manual_seed(length * 10 + step)
    nslots = 64 * tpage
    table = torch.randperm(64, device=dev, generator=gen).to(torch.int32).view(2, 32)
    req = torch.tensor([1], dtype=torch.int64, device=dev)
    seq = torch.tensor([length], device=dev)
    k = torch.randn(nslots, heads, D, device=dev, generator=gen).bfloat16()
    v = torch.randn(nslots, heads, D, device=dev, generator=gen).bfloat16()
    q = torch.randn(rows, heads, D, device=dev, generator=gen).bfloat16()
    anc = torch.randint(0, nslots, (1, rows, depth), dtype=torch.int32, device=dev, generator=gen) if step else None
    kw = dict(rows_per_request=rows, step=step, window=0, table_rows=req, table_page=tpage)
    got = _run(dev, q, k, v, table, seq, anc, rows=rows, step=step, window=0, splits=1, table_rows=req,
               table_page=tpage)
    _check(got, q, k, v, table, seq, anc, **kw)


@pytest.mark.parametrize("step", [1, 4])
def test_masked_ancestor_columns_read_no_unwritten_slot(dev, step):
    """A draft step's ancestor split has max_depth columns per row, of which the first ``step`` are the row's
    ancestors; the masked columns past them must not read a slot nobody wrote. KV slot 0 holds NaN (as a null block
    of a cache that is not zero-filled would) and no window key or ancestor uses it: the outputs stay finite and equal
    the oracle's."""
    announce(f"row attention masked ancestors with a NaN slot 0, step={step}")
    bs, rows, depth, heads, D = 2, 4, 12, 3, 128
    gen = torch.Generator(device=dev).manual_seed(77 + step)
    nslots = 8 * 4096
    table = (torch.randperm(nslots - 8, device=dev, generator=gen) + 8).to(torch.int32).view(8, 4095)
    req = torch.tensor([5, 2], dtype=torch.int64, device=dev)
    seq = torch.randint(40, 300, (bs,), device=dev, generator=gen)
    k = torch.randn(nslots, heads, D, device=dev, generator=gen).bfloat16()
    v = torch.randn(nslots, heads, D, device=dev, generator=gen).bfloat16()
    k[0], v[0] = float("nan"), float("nan")
    q = torch.randn(bs * rows, heads, D, device=dev, generator=gen).bfloat16()
    anc = torch.randint(1, nslots, (bs, rows, depth), dtype=torch.int32, device=dev, generator=gen)
    got = _run(dev, q, k, v, table, seq, anc, rows=rows, step=step, window=96, splits=8, table_rows=req)
    assert torch.isfinite(got.float()).all()
    _check(got, q, k, v, table, seq, anc, rows_per_request=rows, step=step, window=96, table_rows=req)
