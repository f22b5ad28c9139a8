"""Pins of the CPU oracle of draft-row attention (oracle/row_attention.py): the key ranges the reference tests state
(tests/test_row_attention_gpu.py:99-156: a draft step's window [max(len - window, 0), len) plus the row's ancestors;
an extend row's [max(pos - window + 1, 0), pos]) through zero queries, whose output is the mean of exactly the visible
values; a lone ancestor's value; extend rows over a whole contiguous context = torch's causal
scaled_dot_product_attention; and GQA heads reading their group's KV head."""

import torch

from oracle import row_attention as ora


def _cache(n, heads, d, seed):
    return torch.randn(n, heads, d, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def test_zero_queries_average_exactly_the_visible_values():
    n, heads, d = 64, 2, 4
    k, v = _cache(n, heads, d, 1), _cache(n, heads, d, 2)
    table = torch.randperm(n, generator=torch.Generator().manual_seed(3)).to(torch.int32).view(1, n)
    rows = 3
    q = torch.zeros(rows, heads, d, dtype=torch.float64)
    anc = torch.tensor([[[7, 9, 11], [5, 0, 0], [40, 41, 0]]], dtype=torch.int32)
    for window, length in ((0, 20), (8, 20), (8, 5), (16, 30)):
        for step in (0, 1, 2):
            out = ora.rows_attention(q, k, v, table, torch.tensor([length]), anc if step else None,
                                     rows_per_request=rows, step=step, window=window, scale=1.0)
            for t in range(rows):
                if step:  # the reference test's key list: [start, length) of the table, then the row's ancestors
                    start = max(length - window, 0) if window > 0 else 0
                    slots = table[0, start:length].tolist() + anc[0, t, :step].tolist()
                else:
                    pos = length + t
                    start = max(pos - window + 1, 0) if window > 0 else 0
                    slots = table[0, start : pos + 1].tolist()
                torch.testing.assert_close(out[t], v[slots].mean(0), rtol=0, atol=1e-12)


def test_a_lone_ancestor_returns_its_value():
    """Nothing committed (seq_len 0) and one ancestor: the output is that slot's value row."""
    k, v = _cache(16, 1, 8, 4), _cache(16, 1, 8, 5)
    q = torch.randn(1, 1, 8, dtype=torch.float64)
    out = ora.rows_attention(q, k, v, torch.zeros(1, 4, dtype=torch.int32), torch.tensor([0]),
                             torch.tensor([[[13]]], dtype=torch.int32), rows_per_request=1, step=1, window=0,
                             scale=0.3)
    torch.testing.assert_close(out[0, 0], v[13, 0], rtol=0, atol=0)


def test_extend_rows_equal_causal_sdpa():
    """A contiguous table, no window: row j at seq_len + j over keys 0 .. seq_len + j is causal attention."""
    length, W, heads, d = 12, 4, 2, 8
    n = length + W
    k, v = _cache(n, heads, d, 6), _cache(n, heads, d, 7)
    q = torch.randn(W, heads, d, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    table = torch.arange(n, dtype=torch.int32).view(1, n)
    out = ora.rows_attention(q, k, v, table, torch.tensor([length]), None, rows_per_request=W, step=0, window=0,
                             scale=d**-0.5)
    mask = torch.arange(n)[None, :] <= (length + torch.arange(W))[:, None]
    want = torch.nn.functional.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                                            attn_mask=mask)
    torch.testing.assert_close(out, want.transpose(0, 1), rtol=1e-10, atol=1e-10)


def test_gqa_heads_read_their_group_and_packed_paged_caches_agree():
    """Query heads 2 h, 2 h + 1 read KV head h; a packed, paged cache (K then V in one row, pages of 4 slots) gives
    what separate slot-major caches give."""
    n, kvh, d, page = 32, 2, 4, 4
    k, v = _cache(n, kvh, d, 9), _cache(n, kvh, d, 10)
    q = torch.randn(2, 4, d, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    table = torch.tensor([[3, 1, 6, 0, 2, 7, 4, 5]], dtype=torch.int32)
    kw = dict(rows_per_request=2, step=0, window=6, scale=0.5, table_page=page)
    out = ora.rows_attention(q, k, v, table, torch.tensor([9]), None, **kw)
    packed = torch.cat([k, v], -1).view(n // page, page, kvh, 2 * d)
    torch.testing.assert_close(ora.rows_attention(q, packed, None, table, torch.tensor([9]), None, **kw), out,
                               rtol=0, atol=0)
    for h in range(4):
        one = ora.rows_attention(q[:, h : h + 1], k[:, h // 2 : h // 2 + 1], v[:, h // 2 : h // 2 + 1], table,
                                 torch.tensor([9]), None, **kw)
        torch.testing.assert_close(one[:, 0], out[:, h], rtol=0, atol=0)
