"""The linear-attention layer hook of vLLM hybrid targets (vllm/gdn_tree_verify.py): the GDN and Mamba2 layers'
tree-verify front (``TreeVerify``, :55-148), the checks and factory the speculator and the plugin call
(``check_tree_verifiable``, ``create_extension``, :151-183) and the accepted-path commit of the layers' states
(``LinearStateCommit``, :186-322).

vLLM keeps one recurrent-state slot per verify row (``slots[b, i]``) and the request's conv window in slot
``slots[b, 0]``; the next step resumes from row / window offset ``num_accepted - 1``. The accepted rows of a tree are
not a prefix of the verify rows, so :class:`LinearStateCommit` moves them into chain order: the window columns of
the accepted path next to each other, and the last accepted row's recurrent state into row ``accepted - 1``. All
layers move in one gfx950 launch (``csrc/state_commit.hip``).

With vLLM installed, ``GDNSpecRows`` and the base class of :class:`TreeVerify` are vLLM's (``LinearAttnVerifyExtension``
through the installed eagle-harness's ``vllm.adapter``), so vLLM can use the extension :func:`create_extension`
returns; without vLLM they are this module's engine-free stand-ins, with the same fields.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from types import ModuleType
from typing import Any, Optional

import torch

from eagle_harness.kernels import _native
from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update
from eagle_harness.kernels.mamba2_tree import mamba2_tree_state_update
from eagle_harness.vllm.verify_layout import get_stage

# A padded request's state slot (vLLM's null block); the chain kernels skip it too.
NULL_BLOCK_ID = 0


def _vllm_verify_extension() -> Optional[ModuleType]:
    """vLLM's module of ``LinearAttnVerifyExtension`` and its row types, found by the installed eagle-harness's adapter
    (vllm/adapter.py:33-41); None when vLLM or the adapter is not installed."""
    try:
        from eagle_harness.vllm.adapter import verify_extension_module

        return verify_extension_module()
    except ModuleNotFoundError as err:
        if (err.name or "").startswith("vllm") or err.name == "eagle_harness.vllm.adapter":
            return None
        raise


def _vllm_conv_state_dim_first() -> Optional[bool]:
    """vLLM's choice of conv-state layout: True for ``[slots, dim, len]``, False for ``[slots, len, dim]``; None
    without vLLM."""
    try:
        from vllm.model_executor.layers.mamba.mamba_utils import is_conv_state_dim_first
    except ModuleNotFoundError as err:
        if (err.name or "").startswith("vllm"):
            return None
        raise
    return bool(is_conv_state_dim_first())


def _caches(layer: Any, dim_first: Optional[bool]) -> tuple[torch.Tensor, torch.Tensor]:
    """(window cache viewed as [slots, dim, state_len], state pool) of a layer.

    ``layer`` is either a (window, pool) pair whose window is already a [slots, dim, state_len] view, or a layer
    object with vLLM's ``kv_cache`` = (conv state, ssm state); the conv state of a layer object is in vLLM's layout,
    ``[slots, dim, len]`` when ``dim_first`` and ``[slots, len, dim]`` otherwise, and is viewed dim-first (its
    transpose, no copy), as vllm/gdn_tree_verify.py:261-265 does."""
    if isinstance(layer, (tuple, list)):
        conv, ssm = layer
        return conv, ssm
    conv, ssm = layer.kv_cache[0], layer.kv_cache[1]
    if dim_first is None:
        raise ValueError("LinearStateCommit: the conv-state layout of vLLM layer caches is unknown (vLLM is not "
                         "installed): pass dim_first=True for [slots, dim, len] caches, False for [slots, len, dim]")
    return (conv if dim_first else conv.transpose(-1, -2)), ssm


class LinearStateCommit:
    """Moves the accepted rows of a tree round into chain order in GDN layers, all layers in one launch.

    ``layers[i]``: layer ``i``'s (window cache viewed as [slots, dim, state_len], state pool [slots, ...]) pair, or a
    layer object with vLLM's ``kv_cache`` (conv state, ssm state); ``slots[i]``: its KV cache group's [reqs, S] int32
    state-slot table. ``dim_first`` gives the conv-state layout of layer objects (``[slots, dim, len]`` when True,
    ``[slots, len, dim]`` when False); None asks vLLM (``is_conv_state_dim_first``), and layer objects without vLLM
    and without ``dim_first`` are refused.
    """

    def __init__(self, layers: Sequence[Any], slots: Sequence[torch.Tensor], device: torch.device, *,
                 dim_first: Optional[bool] = None):
        self.num_layers = len(layers)
        self.device = device
        if not self.num_layers:
            return
        if dim_first is None and not all(isinstance(layer, (tuple, list)) for layer in layers):
            dim_first = _vllm_conv_state_dim_first()
        caches = [_caches(layer, dim_first) for layer in layers]
        first_conv, first_ssm = caches[0]
        for conv, ssm in caches:
            if conv.stride() != first_conv.stride() or conv.dtype != first_conv.dtype or ssm.stride() != first_ssm.stride():
                raise ValueError("the linear-attention layers must share one state layout")
            if ssm.dtype != first_ssm.dtype:
                raise ValueError("the linear-attention layers must share one state dtype")
        if any(s.dtype != torch.int32 for s in slots):
            raise ValueError("state slots must be int32")
        self.conv_dtype, self.ssm_dtype = first_conv.dtype, first_ssm.dtype
        self.conv_strides = first_conv.stride()
        self.dim = first_conv.shape[1]
        self.ssm_stride, self.ssm_numel = first_ssm.stride(0), first_ssm[0].numel()
        self.conv_ptrs = torch.tensor([c.data_ptr() for c, _ in caches], dtype=torch.uint64, device=device)
        self.ssm_ptrs = torch.tensor([s.data_ptr() for _, s in caches], dtype=torch.uint64, device=device)
        self.slots_ptrs = torch.tensor([s.data_ptr() for s in slots], dtype=torch.uint64, device=device)
        self.slots_strides = torch.tensor([s.stride(0) for s in slots], dtype=torch.int64, device=device)
        self._keep = (caches, list(slots))

    def commit(self, idx_mapping: torch.Tensor, path: torch.Tensor, path_len: torch.Tensor) -> None:
        """``path [state slots, W]`` / ``path_len [state slots]``: the accepted rows of each request, root first."""
        if not self.num_layers:
            return
        args = _native.StateCommitArgs(
            conv_ptrs=self.conv_ptrs.data_ptr(),
            ssm_ptrs=self.ssm_ptrs.data_ptr(),
            slots_ptrs=self.slots_ptrs.data_ptr(),
            slots_strides=self.slots_strides.data_ptr(),
            idx_mapping=_native.itab(idx_mapping),
            path=_native.itab(path),
            path_len=_native.itab(path_len),
            conv_stride_slot=self.conv_strides[0],
            conv_stride_dim=self.conv_strides[1],
            conv_stride_tok=self.conv_strides[2],
            ssm_stride_slot=self.ssm_stride,
            ssm_numel=self.ssm_numel,
            conv_dtype=_native.dtype_code(self.conv_dtype),
            ssm_dtype=_native.dtype_code(self.ssm_dtype),
            num_reqs=idx_mapping.shape[0],
            layers=self.num_layers,
            dim=self.dim,
        )
        _native.launch("eagle4_linear_state_commit", args, self.device)


_VLLM_EXTENSION = _vllm_verify_extension()

if _VLLM_EXTENSION is not None:
    GDNSpecRows = _VLLM_EXTENSION.GDNSpecRows
    LinearAttnVerifyExtension = _VLLM_EXTENSION.LinearAttnVerifyExtension
else:

    @dataclass
    class GDNSpecRows:
        """The speculative-decode rows a Qwen GDN layer hands its verify extension (vLLM's ``GDNSpecRows``, the fields
        vllm/gdn_tree_verify.py:65-106 reads). ``mixed_qkv`` ``[tokens, 2 H K + HV V]``, ``a`` / ``b`` ``[tokens, HV]``
        may be token-strided views of the layer's input projection; ``out`` ``[tokens, HV V]`` receives the recurrence
        output."""

        layer_name: str
        mixed_qkv: torch.Tensor
        conv_state: torch.Tensor
        conv_weight: torch.Tensor
        conv_bias: torch.Tensor | None
        activation: str | None
        a: torch.Tensor
        b: torch.Tensor
        A_log: torch.Tensor
        dt_bias: torch.Tensor
        ssm_state: torch.Tensor
        state_indices: torch.Tensor
        query_start_loc: torch.Tensor
        num_accepted_tokens: torch.Tensor
        out: torch.Tensor
        num_k_heads: int
        head_k_dim: int
        num_v_heads: int
        head_v_dim: int

    class LinearAttnVerifyExtension:
        """Engine-free stand-in for vLLM's verify-extension base class (vLLM is not installed)."""


class TreeVerify(LinearAttnVerifyExtension):
    """A GDN layer's tree-verify front (vllm/gdn_tree_verify.py:55-106): the tree conv over the layer's qkv projection,
    then the tree recurrence on q / k / v views of the conv output and a / b views of the projection. No split or copy
    kernel sits between the input projection's GEMM and the conv, nor between the conv and the recurrence: both gfx950
    kernels address token-strided inputs, and on one stream the conv starts as the GEMM ends."""

    def __init__(self, vllm_config: Any = None):
        self.vllm_config = vllm_config

    @staticmethod
    def _tree_conv(stage: Any, rows: Any, packed: torch.Tensor) -> torch.Tensor:
        """The width-4 tree conv of a layer's packed input ``packed`` [tokens, channels] (a token-strided view of the
        input projection is read in place) into a new [tokens, channels] tensor. Each request's history is the conv
        state of its slot column 0, read from column ``num_accepted - 1``; the stage's window codes name each row's
        three ancestors."""
        result = torch.empty(packed.shape, dtype=packed.dtype, device=packed.device)
        num_reqs = rows.query_start_loc.shape[0] - 1
        gdn_tree_conv1d_update(packed.t()[None], rows.conv_state, rows.conv_weight, rows.conv_bias, rows.activation,
                               conv_state_indices=rows.state_indices[:, 0], intermediate_conv_window=None,
                               intermediate_state_indices=None, tree_ancestors=stage.ancestors[:num_reqs],
                               pad_slot_id=NULL_BLOCK_ID, out=result.t()[None],
                               num_accepted_tokens=rows.num_accepted_tokens, query_start_loc=rows.query_start_loc)
        return result

    @staticmethod
    def _column_views(mixed: torch.Tensor, widths: Sequence[int]) -> list[torch.Tensor]:
        """Consecutive column blocks of ``mixed`` [tokens, sum(widths)] as views (no copies)."""
        views, col = [], 0
        for w in widths:
            views.append(mixed[:, col : col + w])
            col += w
        return views

    def forward_spec_rows(self, rows: GDNSpecRows) -> None:
        """Conv, then the gated delta rule walk over the stage's trees; the walk's snapshots go to the per-row
        slots ``rows.state_indices`` of ``rows.ssm_state`` and its output to ``rows.out``."""
        stage = _staged()
        mixed = self._tree_conv(stage, rows, rows.mixed_qkv)
        tokens = mixed.shape[0]
        kdim, vdim = rows.num_k_heads * rows.head_k_dim, rows.num_v_heads * rows.head_v_dim
        q, k, v = self._column_views(mixed, (kdim, kdim, vdim))
        per_head = lambda t, d: t.view(1, tokens, -1, d)  # noqa: E731  [1, tokens, heads, d], token-strided
        slot_rows = rows.state_indices
        publish = stage.state_slots.get(rows.layer_name)  # set for the one layer per KV cache group that publishes
        gdn_tree_recurrent_update(
            rows.A_log, rows.dt_bias, per_head(q, rows.head_k_dim), per_head(k, rows.head_k_dim),
            per_head(v, rows.head_v_dim), rows.a, rows.b,
            initial_state_source=rows.ssm_state, initial_state_indices=slot_rows,
            num_accepted_tokens=rows.num_accepted_tokens, cu_seqlens=rows.query_start_loc,
            intermediate_states_buffer=rows.ssm_state, intermediate_state_indices=slot_rows,
            retrieve_parent_token=stage.parents, pad_slot_id=NULL_BLOCK_ID,
            out=per_head(rows.out, rows.head_v_dim),
            publish=None if publish is None else publish[: slot_rows.shape[0]], gluon=True)

    def forward_mamba2_spec_rows(self, rows: Any) -> None:
        """A Mamba2 layer's decode rows (vllm/gdn_tree_verify.py:107-148): the tree conv over ``hidden_states_B_C``,
        then the tree selective state update on x / B / C views of the conv output. ``rows`` carries vLLM's
        ``Mamba2SpecRows`` fields (hidden_states_B_C, conv_state, conv_weight, conv_bias, activation, state_indices,
        query_start_loc, num_accepted_tokens, num_heads, head_dim, n_groups, ssm_state_size, ssm_state, dt, A, D,
        dt_bias, out, layer_name)."""
        stage = _staged()
        mixed = self._tree_conv(stage, rows, rows.hidden_states_B_C)
        tokens = mixed.shape[0]
        group_cols = rows.n_groups * rows.ssm_state_size
        x, B, C = self._column_views(mixed, (rows.num_heads * rows.head_dim, group_cols, group_cols))
        slot_rows = rows.state_indices
        mamba2_tree_state_update(
            rows.ssm_state, x.view(tokens, rows.num_heads, rows.head_dim), rows.dt, rows.A,
            B.view(tokens, rows.n_groups, rows.ssm_state_size), C.view(tokens, rows.n_groups, rows.ssm_state_size),
            rows.D, rows.dt_bias, rows.out.view(tokens, rows.num_heads, rows.head_dim), state_indices=slot_rows,
            parents=stage.parents, query_start_loc=rows.query_start_loc, num_accepted_tokens=rows.num_accepted_tokens,
            pad_slot_id=NULL_BLOCK_ID)
        publish = stage.state_slots.get(rows.layer_name)
        if publish is not None:  # the Mamba2 update has no publish argument: copy the slot rows in stream order
            publish[: slot_rows.shape[0]].copy_(slot_rows)


def _staged() -> Any:
    stage = get_stage()
    if stage is None:
        raise RuntimeError("eagle_harness: a linear-attention verify ran before the speculator staged its layout")
    return stage


def check_tree_verifiable(layers: Sequence[Any]) -> None:
    """Refuses a target with linear-attention layers that would not hand their rows to :class:`TreeVerify`
    (vllm/gdn_tree_verify.py:151-166): vLLM would run its own chain kernels on them and verify every tree as a
    chain. Qwen GDN layers always hand them over; Mamba2 mixers only where vLLM's extension base class declares the
    Mamba2 hook (``forward_mamba2_spec_rows``)."""
    from vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn import QwenGatedDeltaNetAttention
    from vllm.model_executor.layers.mamba.mamba_mixer2 import MambaMixer2

    served: list[type] = [QwenGatedDeltaNetAttention]
    if "forward_mamba2_spec_rows" in vars(LinearAttnVerifyExtension):
        served.append(MambaMixer2)
    refused = sorted({type(layer).__name__ for layer in layers if not isinstance(layer, tuple(served))})
    if refused:
        raise RuntimeError(
            f"eagle_harness: the tree verify does not reach the {', '.join(refused)} layers of this target with "
            f"this vLLM: only {', '.join(kind.__name__ for kind in served)} layers pass their rows to the verify "
            "extension (Mamba2 mixers need vLLM's LinearAttnVerifyExtension.forward_mamba2_spec_rows hook)")


def create_extension(vllm_config: Any) -> Optional[TreeVerify]:
    """The factory vLLM's speculative-method registry calls (``linear_attn_verify_extension``,
    vllm/gdn_tree_verify.py:176-183): a :class:`TreeVerify` when the method drafts trees, None when it drafts chains
    (node top-k 1), which vLLM verifies with its own kernels."""
    from eagle_harness.vllm.config import parse_method_config

    method = parse_method_config(vllm_config.speculative_config.method_config)
    return None if method.node_top_k == 1 else TreeVerify(vllm_config)
