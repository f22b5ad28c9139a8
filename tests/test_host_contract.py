"""Host-side contract of the drop-in modules that needs no GPU: the errors the reference raises before any launch,
raised the same way (tests/test_rocm_dispatch.py:57-80, tests/test_verify_prep_gpu.py:35-37)."""

from types import SimpleNamespace

import pytest
import torch


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_records_require_rounded_paths(dtype):
    from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update

    with pytest.raises(ValueError, match="tree_paths.*low-precision"):
        gdn_tree_records_update(None, None, None, None, None, None, None, state=SimpleNamespace(dtype=dtype),
                                state_indices=None, query_start_loc=None, parent=None, tree_paths=None, records=None,
                                record_indices=None, width=16)


def test_tail_width_over_a_word_is_rejected():
    from eagle_harness.kernels.verify_prep import tree_tail_words

    with pytest.raises(ValueError, match="verify width 65"):
        tree_tail_words(None, None, None, width=65)


def test_fp8_cache_needs_its_scales():
    from eagle_harness.vllm.verify_attention import verify_attention

    cache = torch.zeros(2, 16, 1, 64, dtype=torch.float8_e4m3fn)
    q = torch.zeros(1, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="k_scale and v_scale"):
        verify_attention(q, q, q, cache, cache, torch.zeros(1, 2, dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
                         torch.tensor([0, 1], dtype=torch.int32), torch.ones(1, 1, dtype=torch.int64), 1.0, q,
                         max_query_len=1)


def test_front_without_a_stage_refuses():
    """A verify before the speculator staged its tables is an error, as in the reference (:169-173)."""
    from types import SimpleNamespace

    from eagle_harness.vllm.gdn_tree_verify import TreeVerify
    from eagle_harness.vllm.verify_layout import set_stage

    set_stage(None)
    with pytest.raises(RuntimeError, match="staged"):
        TreeVerify().forward_spec_rows(SimpleNamespace())


def test_tree_attention_routes_only_tree_verifies_to_the_kernels():
    """vllm/tree_attention.py:30-54: no stage, a stage that is not verifying, one query token per request or a
    draft layer take the plain path; with no plain path given that is an error, not another implementation."""
    from types import SimpleNamespace

    from eagle_harness.kernels._native import NotCovered
    from eagle_harness.vllm.tree_attention import TreeAttentionImpl
    from eagle_harness.vllm.verify_layout import set_stage

    calls = []
    impl = TreeAttentionImpl(8, 64, 0.125, 2, plain=lambda *a: calls.append(a) or "plain")
    meta = SimpleNamespace(max_query_len=16)
    stage = SimpleNamespace(verifying=True)
    cases = [(None, meta, SimpleNamespace()), (SimpleNamespace(verifying=False), meta, SimpleNamespace()),
             (stage, SimpleNamespace(max_query_len=1), SimpleNamespace()), (stage, None, SimpleNamespace()),
             (stage, meta, SimpleNamespace(is_draft_layer=True))]
    try:
        for st, md, layer in cases:
            set_stage(st)
            assert impl.forward(layer, None, None, None, None, md, None) == "plain"
        assert len(calls) == len(cases)
        set_stage(None)
        with pytest.raises(NotCovered, match="plain-path"):
            TreeAttentionImpl(8, 64, 0.125, 2).forward(SimpleNamespace(), None, None, None, None, meta, None)
    finally:
        set_stage(None)


def test_tree_attention_cache_views_and_scales():
    """The K / V halves of a [blocks, Hkv, page, 2 D] cache as [blocks, page, Hkv, D] views (no copies,
    vllm/tree_attention.py:73); per-tensor fp8 scales broadcast to every (page, KV head) with stride 0."""
    from eagle_harness.vllm.tree_attention import TreeAttentionImpl, TreeFlashAttentionBackend, _page_scales, split_kv_cache

    cache = torch.randn(5, 2, 16, 2 * 32)
    k, v = split_kv_cache(cache, 32)
    assert k.shape == v.shape == (5, 16, 2, 32) and k.data_ptr() == cache.data_ptr()
    assert torch.equal(k[3, 7, 1], cache[3, 1, 7, :32]) and torch.equal(v[3, 7, 1], cache[3, 1, 7, 32:])
    with pytest.raises(ValueError, match="2 \\* 64"):
        split_kv_cache(cache, 64)
    s = _page_scales(torch.tensor(0.25), 5, 2, torch.device("cpu"), "k_scale")
    assert s.shape == (5, 2) and s.stride() == (0, 0) and float(s[4, 1]) == 0.25
    page = torch.rand(5, 2)
    assert _page_scales(page, 5, 2, torch.device("cpu"), "k_scale") is page
    with pytest.raises(ValueError, match="one element"):
        _page_scales(torch.ones(3), 5, 2, torch.device("cpu"), "k_scale")
    assert TreeFlashAttentionBackend.get_name() == "CUSTOM"
    assert TreeFlashAttentionBackend.get_impl_cls() is TreeAttentionImpl


def test_fp8_tree_attention_needs_scales():
    from types import SimpleNamespace

    from eagle_harness.vllm.tree_attention import TreeAttentionImpl

    impl = TreeAttentionImpl(8, 64, 0.125, 2, kv_cache_dtype="fp8")
    cache = torch.zeros(3, 2, 16, 128, dtype=torch.uint8)
    meta = SimpleNamespace(num_actual_tokens=1, query_start_loc=torch.tensor([0, 1]), max_query_len=2)
    with pytest.raises(ValueError, match="k_scale and v_scale"):
        impl._forward_tree(None, None, None, cache, meta, None, None, None)


def test_verify_attention_refuses_mismatched_caches_and_short_scales():
    """A value cache of another dtype than the key cache, and fp8 scales with fewer rows or columns than the cache
    has pages / KV heads, are refused before any launch."""
    from eagle_harness.kernels._native import NotCovered
    from eagle_harness.vllm.verify_attention import verify_attention

    q = torch.zeros(1, 1, 64, dtype=torch.bfloat16)
    args = (torch.zeros(1, 2, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), torch.tensor([0, 1], dtype=torch.int32),
            torch.ones(1, 1, dtype=torch.int64), 1.0, q)
    with pytest.raises(NotCovered, match="value_cache"):
        verify_attention(q, q, q, torch.zeros(2, 16, 1, 64, dtype=torch.bfloat16),
                         torch.zeros(2, 16, 1, 64, dtype=torch.float16), *args, max_query_len=1)
    cache = torch.zeros(4, 16, 2, 64, dtype=torch.float8_e4m3fn)
    for ks in (torch.ones(3, 2), torch.ones(4, 1)):
        with pytest.raises(ValueError, match="k_scale must be"):
            verify_attention(q, q, q, cache, cache, *args, max_query_len=1, k_scale=ks, v_scale=torch.ones(4, 2))


def test_greedy_targets_refuses_a_wrong_out():
    from eagle_harness.vllm.tree_accept import greedy_targets

    logits = torch.zeros(4, 10, dtype=torch.bfloat16)
    for out in (torch.zeros(4, dtype=torch.int32), torch.zeros(3, dtype=torch.int64), torch.zeros(8, dtype=torch.int64)[::2]):
        with pytest.raises(ValueError, match="int64"):
            greedy_targets(logits, out=out)


def test_device_gate_without_a_gpu():
    """The launch gate on a machine without a ROCm GPU: a reason instead of an exception, and a launch raises
    UnsupportedHardware (a RuntimeError) before the library is touched."""
    from eagle_harness.kernels import _native

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert "not on a ROCm GPU" in _native.unsupported_reason(torch.device("cpu"))
    assert "no ROCm GPU" in _native.unsupported_reason(torch.device("cuda:0"))
    with pytest.raises(_native.UnsupportedHardware, match="ROCm GPU"):
        _native.launch("eagle4_stage_tree", _native.StageTreeArgs(), torch.device("cpu"))
    assert issubclass(_native.UnsupportedHardware, RuntimeError)
