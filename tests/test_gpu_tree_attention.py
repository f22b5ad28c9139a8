"""The tree path of the full-attention backend on the GPU (vllm/tree_attention.py:29-88): a staged tree verify over
the backend's own ``[blocks, Hkv, page, 2 D]`` cache goes through ``TreeAttentionImpl.forward`` and matches the dense
oracle; fp8-e4m3 caches (which the reference's backend refuses, :69-70) are served with per-(page, KV head) scales
from the layer, or vLLM's per-tensor scales broadcast, against the dequantised oracle. Tolerance 2e-2 abs / 1e-2 rel
(bf16 outputs)."""

from types import SimpleNamespace

import pytest
import torch

from conftest import announce
from oracle import attention as oa
from workloads import AttnShape, attention_inputs

pytestmark = pytest.mark.gpu

SHAPE = AttnShape(5, 16, 24, 4, 256, 16, 200, 2500)


def _backend_cache(key_cache, value_cache):
    """[blocks, Hkv, page, 2 D] with K then V of a token adjacent: the layout the backend splits."""
    return torch.cat([key_cache, value_cache], dim=-1).transpose(1, 2).contiguous()


def _staged_forward(dev, inp, cache, layer, kv_cache_dtype):
    from eagle_harness.vllm.tree_attention import TreeAttentionImpl
    from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage, set_stage

    B, W = SHAPE.batch, SHAPE.width
    store = TreeStore(B, W, dev)
    store.parents.copy_(torch.tensor(inp["parents"], dtype=torch.int32))
    stage = VerifyStage(B, B * W, W, dev)
    qsl = inp["query_start_loc"].to(dev)
    positions = torch.cat([int(c) + torch.arange(W) for c in inp["context_lens"]]).to(dev)
    stage.stage(store, torch.arange(B, dtype=torch.int32, device=dev), qsl, qsl, positions, B, B * W, tree=True)
    meta = SimpleNamespace(num_actual_tokens=B * W, query_start_loc=qsl, max_query_len=W,
                           block_table=inp["block_table"].to(dev))
    impl = TreeAttentionImpl(SHAPE.hq, SHAPE.d, inp["scale"], SHAPE.hkv, kv_cache_dtype=kv_cache_dtype)
    out = torch.full((B * W + 3, SHAPE.hq, SHAPE.d), 7.0, dtype=torch.bfloat16, device=dev)
    set_stage(stage)
    try:
        impl.forward(layer, inp["q"].to(dev), inp["k_new"].to(dev), inp["v_new"].to(dev), cache, meta, out)
        torch.cuda.synchronize()
    finally:
        set_stage(None)
    return out.cpu()


def _want(inp, k_scale=None, v_scale=None):
    out = torch.full((SHAPE.batch * SHAPE.width + 3, SHAPE.hq, SHAPE.d), 7.0, dtype=torch.bfloat16)
    return oa.verify_attention(inp["q"], inp["k_new"], inp["v_new"], inp["key_cache"], inp["value_cache"],
                               inp["block_table"], inp["context_lens"], inp["query_start_loc"], inp["masks"],
                               inp["scale"], out, max_query_len=SHAPE.width, k_scale=k_scale, v_scale=v_scale)


def test_bf16_cache_through_the_backend(dev):
    announce("tree attention backend bf16")
    inp = attention_inputs(SHAPE, seed=31)
    got = _staged_forward(dev, inp, _backend_cache(inp["key_cache"], inp["value_cache"]).to(dev), SimpleNamespace(),
                          "auto")
    torch.testing.assert_close(got.float(), _want(inp).float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("scales", ["per_page", "per_tensor"])
def test_fp8_cache_through_the_backend(dev, scales):
    """uint8 storage of an fp8-e4m3 cache (vLLM's ``kv_cache_dtype="fp8"``) with the layer's scales."""
    announce(f"tree attention backend fp8 {scales}")
    inp = attention_inputs(SHAPE, seed=32, fp8=True)
    if scales == "per_tensor":  # one scale per tensor: requantize both caches with it
        k32 = oa.dequantize_fp8_pages(inp["key_cache"], inp["k_scale"])
        v32 = oa.dequantize_fp8_pages(inp["value_cache"], inp["v_scale"])
        ks, vs = float(k32.abs().max()) / 448.0, float(v32.abs().max()) / 448.0
        inp["key_cache"] = (k32 / ks).clamp(-448, 448).to(torch.float8_e4m3fn)
        inp["value_cache"] = (v32 / vs).clamp(-448, 448).to(torch.float8_e4m3fn)
        layer = SimpleNamespace(_k_scale=torch.tensor(ks, device=dev), _v_scale=torch.tensor(vs, device=dev))
        k_want, v_want = torch.full_like(inp["k_scale"], ks), torch.full_like(inp["v_scale"], vs)
    else:
        layer = SimpleNamespace(k_page_scale=inp["k_scale"].to(dev), v_page_scale=inp["v_scale"].to(dev))
        k_want, v_want = inp["k_scale"], inp["v_scale"]
    cache = _backend_cache(inp["key_cache"].view(torch.uint8), inp["value_cache"].view(torch.uint8)).to(dev)
    got = _staged_forward(dev, inp, cache, layer, "fp8")
    want = _want(inp, k_want, v_want)
    torch.testing.assert_close(got.float(), want.float(), atol=2e-2, rtol=1e-2)
    assert torch.equal(got[-3:], torch.full_like(got[-3:], 7.0))
