"""The allocation-free tree-verify attention entry (``eagle4_verify_attention_static``) against the regular one.

Both run the same kernels; only where the split partials live differs (the library's static per-GPU buffer instead of
a caller workspace), so the outputs must be equal bit for bit. Two calls in a row, the second smaller than the first,
so the second reads a buffer that still holds the first call's partials. A launch whose partials exceed the buffer
is refused before anything runs, and no call allocates through torch's allocator."""

import pytest
import torch

from conftest import announce
from workloads import AttnShape, attention_inputs

pytestmark = pytest.mark.gpu


def _run(dev, inp, no_alloc, fp8=False):
    from eagle_harness.vllm.verify_attention import verify_attention

    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = torch.full_like(g["q"], 7.0)
    kw = dict(k_scale=g["k_scale"], v_scale=g["v_scale"]) if fp8 else {}
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0)
    verify_attention(g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"],
                     g["context_lens"], g["query_start_loc"], g["masks"], g["scale"], out,
                     max_query_len=g["max_query_len"], no_alloc=no_alloc, **kw)
    torch.cuda.synchronize()
    allocated = torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0) - before
    return out.cpu(), allocated


@pytest.mark.parametrize("fp8", [False, True])
def test_static_entry_matches_regular_entry_on_two_calls(dev, fp8):
    """A 24-request batch with long prefixes, then a 3-request batch with short ones (D 256, 24 / 4 heads)."""
    for n, (batch, lmin, lmax) in enumerate(((24, 1024, 6000), (3, 100, 900))):
        announce(f"attention no-alloc call {n} batch={batch} fp8={fp8}")
        inp = attention_inputs(AttnShape(batch, 16, 24, 4, 256, 16, lmin, lmax), seed=40 + n, fp8=fp8)
        want, _ = _run(dev, inp, no_alloc=False, fp8=fp8)
        got, allocated = _run(dev, inp, no_alloc=True, fp8=fp8)
        assert allocated == 0
        assert torch.equal(got, want)


def test_static_entry_refuses_a_launch_beyond_its_buffer(dev):
    """1000 requests of 16 rows: their partials need more than the static buffer holds, so the entry raises and
    leaves ``out`` untouched."""
    from eagle_harness.kernels import _native
    from eagle_harness.vllm.verify_attention import verify_attention

    announce("attention no-alloc refusal")
    inp = attention_inputs(AttnShape(1000, 16, 24, 4, 256, 16, 16, 64), seed=44)
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = torch.full_like(g["q"], 7.0)
    with pytest.raises(ValueError, match="static buffer"):
        verify_attention(g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"],
                         g["context_lens"], g["query_start_loc"], g["masks"], g["scale"], out,
                         max_query_len=g["max_query_len"], no_alloc=True)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    assert _native.library().eagle4_verify_attention_static_bytes() == 64 << 20
