"""The allocation-free tree-verify attention entry (``eagle4_verify_attention_static``) against the regular one.

Both run the same kernels; only where the split partials live differs (the library's static per-GPU buffer instead of
a caller workspace), so the outputs must be equal bit for bit. Two calls in a row, the second smaller than the first,
so the second reads a buffer that still holds the first call's partials; a 512-request fp8 call (the partial slots
are numbered per workgroup, so any batch of the streamed schedule fits the buffer); a launch whose partials exceed
the buffer is refused before anything runs; no call allocates through torch's allocator; and in a fresh process the
first call of all is made under HIP graph capture, its replays equal to the regular entry's output."""

import os
import subprocess
import sys

import pytest
import torch

from conftest import announce
from workloads import ATTN_B512_FP8, AttnShape, attention_inputs

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(dev, g, no_alloc, fp8=False):
    from eagle_harness.vllm.verify_attention import verify_attention

    out = torch.full_like(g["q"], 7.0)
    kw = dict(k_scale=g["k_scale"], v_scale=g["v_scale"]) if fp8 else {}
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0)
    verify_attention(g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"],
                     g["context_lens"], g["query_start_loc"], g["masks"], g["scale"], out,
                     max_query_len=g["max_query_len"], no_alloc=no_alloc, **kw)
    torch.cuda.synchronize()
    allocated = torch.cuda.memory_stats(dev).get("allocation.all.allocated", 0) - before
    return out, allocated


@pytest.mark.parametrize("fp8", [False, True])
def test_static_entry_matches_regular_entry_on_two_calls(dev, fp8):
    """A 24-request batch with long prefixes, then a 3-request batch with short ones (D 256, 24 / 4 heads)."""
    for n, (batch, lmin, lmax) in enumerate(((24, 1024, 6000), (3, 100, 900))):
        announce(f"attention no-alloc call {n} batch={batch} fp8={fp8}")
        inp = attention_inputs(AttnShape(batch, 16, 24, 4, 256, 16, lmin, lmax), seed=40 + n, fp8=fp8)
        g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
        want, _ = _run(dev, g, no_alloc=False, fp8=fp8)
        got, allocated = _run(dev, g, no_alloc=True, fp8=fp8)
        assert allocated == 0
        assert torch.equal(got, want)


def test_static_entry_covers_512_fp8_requests(dev):
    """The quantized hybrid round's attention: 512 requests x 16 rows over fp8 pages, prefixes U[512, 4096]."""
    announce("attention no-alloc batch 512 fp8")
    g = attention_inputs(ATTN_B512_FP8, seed=45, fp8=True, device=dev, gen_device=dev)
    want, _ = _run(dev, g, no_alloc=False, fp8=True)
    got, allocated = _run(dev, g, no_alloc=True, fp8=True)
    assert allocated == 0
    assert torch.equal(got, want)


def test_static_entry_refuses_a_launch_beyond_its_buffer(dev):
    """1100 requests with prefixes past one 1024-key split: more requests than the streamed schedule takes, and the
    split schedule's per-request partials need more than the static buffer holds, so the entry raises and leaves
    ``out`` untouched."""
    from eagle_harness.kernels import _native
    from eagle_harness.vllm.verify_attention import verify_attention

    announce("attention no-alloc refusal")
    g = attention_inputs(AttnShape(1100, 16, 24, 4, 256, 16, 1100, 1200), seed=44, device=dev, gen_device=dev)
    out = torch.full_like(g["q"], 7.0)
    with pytest.raises(ValueError, match="static buffer"):
        verify_attention(g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"],
                         g["context_lens"], g["query_start_loc"], g["masks"], g["scale"], out,
                         max_query_len=g["max_query_len"], no_alloc=True)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    assert _native.library().eagle4_verify_attention_static_bytes() == 64 << 20


CAPTURE_FIRST = r"""
import sys
import torch
from workloads import AttnShape, attention_inputs
from eagle_harness.vllm.verify_attention import verify_attention

dev = torch.device("cuda:0")
g = attention_inputs(AttnShape(16, 16, 24, 4, 256, 16, 1024, 4096), seed=46, device=dev, gen_device=dev)
out = torch.full_like(g["q"], 7.0)
args = (g["q"], g["k_new"], g["v_new"], g["key_cache"], g["value_cache"], g["block_table"], g["context_lens"],
        g["query_start_loc"], g["masks"], g["scale"])
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the library's first attention call in this process
    verify_attention(*args, out, max_query_len=16, no_alloc=True)
want = torch.full_like(out, 7.0)
verify_attention(*args, want, max_query_len=16)
torch.cuda.synchronize()
for replay in range(3):
    out.fill_(7.0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {replay} differs"
print("capture-first ok")
"""


def test_first_call_under_graph_capture():
    """A fresh process whose first no-alloc call is captured into a HIP graph: three replays, each with eager work and
    synchronisations between them, equal to the regular entry bit for bit."""
    announce("attention no-alloc first call under capture (subprocess)")
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([os.path.join(ROOT, "eagle-4_amd"), ROOT]))
    proc = subprocess.run([sys.executable, "-c", CAPTURE_FIRST], env=env, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "capture-first ok" in proc.stdout
