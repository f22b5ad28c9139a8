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
