"""The reference-side binding a maintainer would add fills the C ABI's argument struct
exactly as this build's own launcher does.

The ``_launch_walk`` code block is taken from INTEGRATION.md as written and run against this package's
``gdn_tree_state_args`` (the reference's keys); the binding's ``launch`` records the struct instead of launching, so
no GPU is needed. Both slot-table layouts are covered: vLLM's per-row slots (with ``num_accepted_tokens`` and
``publish``) and sglang's per-request scratch rows.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _stub_source() -> str:
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    section = text[text.index("## 3. Binding the C ABI from the reference"):text.index("## 4.")]
    blocks = re.findall(r"```python\n(.*?)```", section, flags=re.S)
    found = [b for b in blocks if "def _launch_walk(" in b]
    assert len(found) == 1, "INTEGRATION.md section 3 must hold one _launch_walk block"
    return found[0]


def _fields(struct: ctypes.Structure) -> dict:
    out = {}
    for name, kind in struct._fields_:
        value = getattr(struct, name)
        if isinstance(value, ctypes.Structure):
            value = tuple(getattr(value, f) for f, _ in value._fields_)
        elif isinstance(value, float):
            value = round(value, 7)
        out[name] = value
    return out


def _inputs(layout: str):
    gen = torch.Generator().manual_seed(3)
    N, W, H, HV, K = 3, 5, 2, 4, 16
    tokens = N * W
    proj = torch.randn(tokens, 2 * H * K + HV * K + 8, generator=gen).to(torch.bfloat16)  # token-strided views
    q = proj[:, : H * K].view(1, tokens, H, K)
    k = proj[:, H * K : 2 * H * K].view(1, tokens, H, K)
    v = proj[:, 2 * H * K : 2 * H * K + HV * K].view(1, tokens, HV, K)
    ab = torch.randn(tokens, 2 * HV, generator=gen).to(torch.bfloat16)
    a, b = ab[:, :HV], ab[:, HV:]
    A_log, dt_bias = torch.randn(HV, generator=gen), torch.randn(HV, generator=gen)
    cu = torch.arange(0, tokens + 1, W, dtype=torch.int32)
    parents = torch.tensor([[-1, 0, 0, 1, 2]] * N, dtype=torch.int32)
    out = torch.empty(1, tokens, HV, K, dtype=torch.bfloat16)
    if layout == "vllm":
        pool = torch.zeros(1 + N * W, HV, K, K)
        slots = (1 + torch.arange(N * W, dtype=torch.int32)).view(N, W)
        state = dict(initial_state_source=pool, initial_state_indices=slots, intermediate_states_buffer=pool,
                     intermediate_state_indices=slots, num_accepted_tokens=torch.tensor([1, 2, 1], dtype=torch.int32),
                     publish=torch.zeros(N, W + 2, dtype=torch.int32), pad_slot_id=0)
    else:
        pool = torch.zeros(N + 1, HV, K, K)
        scratch = torch.zeros(N, W, HV, K, K)
        state = dict(initial_state_source=pool, initial_state_indices=torch.tensor([2, 0, 1], dtype=torch.int32),
                     intermediate_states_buffer=scratch,
                     intermediate_state_indices=torch.arange(N, dtype=torch.int32), num_accepted_tokens=None,
                     publish=None, pad_slot_id=-1)
    return dict(A_log=A_log, dt_bias=dt_bias, q=q, k=k, v=v, a=a, b=b, cu_seqlens=cu, parents=parents, out=out,
                H=H, HV=HV, K=K, V=K, **state)


@pytest.mark.parametrize("layout", ["vllm", "sglang"])
def test_reference_side_stub_fills_the_struct_as_the_overlay(monkeypatch, layout):
    from eagle_harness.kernels import _native
    from eagle_harness.kernels import gdn_tree_recurrence as rec

    seen = []
    monkeypatch.setattr(_native, "launch", lambda name, args, device: seen.append((name, _fields(args))))
    x = _inputs(layout)
    state = {k: x[k] for k in ("initial_state_source", "initial_state_indices", "num_accepted_tokens",
                               "intermediate_states_buffer", "intermediate_state_indices", "publish")}
    # the overlay's own launcher
    rec.gdn_tree_recurrent_update(x["A_log"], x["dt_bias"], x["q"], x["k"], x["v"], x["a"], x["b"],
                                  cu_seqlens=x["cu_seqlens"], retrieve_parent_token=x["parents"],
                                  pad_slot_id=x["pad_slot_id"], out=x["out"], **state)
    # the stub, as the reference's gdn_tree_recurrent_update would call it (kernels/gdn_tree_recurrence.py:651-693)
    namespace = {"gdn_tree_state_args": rec.gdn_tree_state_args}
    exec(compile(_stub_source(), "INTEGRATION.md", "exec"), namespace)
    q, k, v, a, b, out = x["q"], x["k"], x["v"], x["a"], x["b"], x["out"]
    common = dict(inputs=(q, k, v, a, b),
                  input_strides=(q.stride()[1], k.stride()[1], v.stride()[1], a.stride()[-2], b.stride()[-2]),
                  gate_params=(x["A_log"], x["dt_bias"], 1.0, 20.0), output=(out, out.stride(1)),
                  cu_seqlens=x["cu_seqlens"], scale=x["K"] ** -0.5, H=x["H"], HV=x["HV"], K=x["K"], V=x["V"],
                  BK=x["K"])
    fp32_state = state["intermediate_states_buffer"].dtype == torch.float32
    namespace["_launch_walk"](common, retrieve_parent_token=x["parents"], pad_slot_id=x["pad_slot_id"],
                              skip_chain_reload=fp32_state, **state)
    assert [name for name, _ in seen] == ["eagle4_gdn_tree_recurrent_update"] * 2
    ours, stub = seen[0][1], seen[1][1]
    assert stub == ours
    assert stub["row_slots"] == (layout == "vllm") and stub["N"] == 3
