"""The CUSTOM attention backend of the target's full-attention layers (vllm/tree_attention.py:29-98).

vLLM's ``TreeFlashAttentionImpl`` sends a layer's attention through :func:`verify_attention` when a tree verify is
staged and leaves every other forward (prefill, one query token per request, the draft's own layers) to
FlashAttention. Its ``_forward_tree`` splits the layer's cache into K / V views and refuses quantized caches
(:69-70). This module keeps the same decision and the same call:

- with vLLM importable, :class:`TreeFlashAttentionBackend` and :class:`TreeFlashAttentionImpl` derive from vLLM's
  FlashAttention backend and implementation, as the reference's do, so the plugin's registration string
  (``eagle_harness.vllm.tree_attention.TreeFlashAttentionBackend``) names a backend vLLM can load, and every forward
  that is not a tree verify is FlashAttention's own;
- :class:`TreeAttentionImpl` is the same forward without vLLM: it takes the plain-path implementation as ``plain``
  (any callable with the ``forward`` signature); without one, a forward that is not a tree verify raises instead of
  being computed some other way. Without vLLM, :class:`TreeFlashAttentionBackend` serves it;
- fp8 caches are served instead of refused: a cache of dtype ``float8_e4m3fn`` (or uint8 storage with
  ``kv_cache_dtype`` ``"fp8"`` / ``"fp8_e4m3"``) goes to the kernels with fp32 scales per (page, KV head). They come
  from ``k_scale`` / ``v_scale`` arguments, else from the layer's ``k_page_scale`` / ``v_page_scale`` attributes
  ([blocks, Hkv]), else from vLLM's per-tensor ``_k_scale`` / ``_v_scale``, broadcast to every (page, KV head) as a
  stride-0 view (no copy).

The cache layout is the one the reference's backend splits: ``kv_cache`` is ``[blocks, Hkv, page, 2 * D]`` with a
token's K and V adjacent in the last dimension; its ``transpose(1, 2)`` halves are the ``[blocks, page, Hkv, D]``
K and V views :func:`verify_attention` reads through their strides.
"""

from __future__ import annotations

from typing import Any, Callable, Optional

import torch

from eagle_harness.kernels import _native
from eagle_harness.vllm.verify_attention import verify_attention
from eagle_harness.vllm.verify_layout import get_stage

FP8_CACHE_DTYPES = ("fp8", "fp8_e4m3")


def split_kv_cache(kv_cache: torch.Tensor, head_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(key_cache, value_cache) ``[blocks, page, Hkv, D]`` views of a ``[blocks, Hkv, page, 2 * D]`` cache."""
    if kv_cache.dim() != 4 or kv_cache.shape[-1] != 2 * head_size:
        raise ValueError(f"kv_cache must be [blocks, Hkv, page, 2 * {head_size}], got {tuple(kv_cache.shape)}")
    both = kv_cache.transpose(1, 2)
    return both[..., :head_size], both[..., head_size:]


def _page_scales(value: Any, blocks: int, kv_heads: int, device: torch.device, name: str) -> torch.Tensor:
    """fp32 scales [blocks, Hkv]: a tensor of that shape as is; a one-element tensor or a float as a stride-0 view."""
    if isinstance(value, torch.Tensor) and value.dim() == 2:
        return value
    if isinstance(value, torch.Tensor):
        if value.numel() != 1:
            raise ValueError(f"{name}: a per-tensor scale must have one element, got {tuple(value.shape)}")
        one = value.reshape(1, 1).to(device=device, dtype=torch.float32)
    else:
        one = torch.full((1, 1), float(value), dtype=torch.float32, device=device)
    return one.expand(blocks, kv_heads)


def _vllm_flash_attention() -> tuple[Optional[type], Optional[type]]:
    """vLLM's (FlashAttentionBackend, FlashAttentionImpl); (None, None) when vLLM is not installed."""
    try:
        from vllm.v1.attention.backends.flash_attn import FlashAttentionBackend, FlashAttentionImpl
    except ModuleNotFoundError as err:
        if not (err.name or "").startswith("vllm"):
            raise
        return None, None
    return FlashAttentionBackend, FlashAttentionImpl


class _TreeForward:
    """The backend's forward (vllm/tree_attention.py:29-88): a staged tree verify with more than one query row per
    request, outside the draft's layers, goes to :func:`verify_attention`; every other forward to
    :meth:`_plain_forward`. Reads ``head_size``, ``scale`` and ``kv_cache_dtype`` from the implementation."""

    def _plain_forward(self, *args: Any) -> torch.Tensor:
        raise NotImplementedError

    def forward(self, layer: Any, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                attn_metadata: Any, output: torch.Tensor, output_scale: Optional[torch.Tensor] = None,
                output_block_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
        stage = get_stage()
        tree = (stage is not None and stage.verifying and attn_metadata is not None
                and attn_metadata.max_query_len > 1 and not getattr(layer, "is_draft_layer", False))
        if not tree:
            return self._plain_forward(layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                                       output_block_scale)
        k_scale = getattr(layer, "k_page_scale", None)
        v_scale = getattr(layer, "v_page_scale", None)
        if k_scale is None and hasattr(layer, "_k_scale"):
            k_scale, v_scale = layer._k_scale, layer._v_scale
        return self._forward_tree(query, key, value, kv_cache, attn_metadata, output, stage.masks,
                                  stage.context_lens, k_scale=k_scale, v_scale=v_scale)

    def _forward_tree(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                      attn_metadata: Any, output: torch.Tensor, masks: torch.Tensor, context_lens: torch.Tensor,
                      *, k_scale: Any = None, v_scale: Any = None) -> torch.Tensor:
        """The tree verify of ``attn_metadata.num_actual_tokens`` rows into ``output`` (vllm/tree_attention.py:
        56-88): ``context_lens`` are the staged committed lengths, ``masks`` the staged ancestor masks."""
        cache = kv_cache
        fp8 = cache.dtype == torch.float8_e4m3fn
        if cache.dtype == torch.uint8 and self.kv_cache_dtype in FP8_CACHE_DTYPES:
            cache, fp8 = cache.view(torch.float8_e4m3fn), True
        elif self.kv_cache_dtype not in ("auto",) + FP8_CACHE_DTYPES and cache.dtype not in (torch.bfloat16,
                                                                                              torch.float16):
            raise _native.NotCovered(f"kv_cache_dtype {self.kv_cache_dtype} ({cache.dtype}) is not covered")
        key_cache, value_cache = split_kv_cache(cache, self.head_size)
        scales = {}
        if fp8:
            if k_scale is None or v_scale is None:
                raise ValueError("an fp8 KV cache needs k_scale and v_scale (per (page, KV head) or per tensor)")
            blocks, kv_heads = key_cache.shape[0], key_cache.shape[2]
            scales = dict(k_scale=_page_scales(k_scale, blocks, kv_heads, cache.device, "k_scale"),
                          v_scale=_page_scales(v_scale, blocks, kv_heads, cache.device, "v_scale"))
        tokens = attn_metadata.num_actual_tokens
        num_reqs = attn_metadata.query_start_loc.shape[0] - 1
        verify_attention(query[:tokens], key[:tokens], value[:tokens], key_cache, value_cache,
                         attn_metadata.block_table, context_lens[:num_reqs], attn_metadata.query_start_loc, masks,
                         self.scale, output, max_query_len=attn_metadata.max_query_len, **scales)
        return output


class TreeAttentionImpl(_TreeForward):
    """The backend's implementation without vLLM. ``plain`` computes the forwards that are not tree verifies (the
    reference's ``super().forward``)."""

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 kv_cache_dtype: str = "auto", plain: Optional[Callable[..., torch.Tensor]] = None):
        self.num_heads, self.head_size, self.scale = num_heads, head_size, scale
        self.num_kv_heads, self.kv_cache_dtype, self.plain = num_kv_heads, kv_cache_dtype, plain

    def _plain_forward(self, *args: Any) -> torch.Tensor:
        if self.plain is None:
            raise _native.NotCovered("not a tree verify forward, and no plain-path implementation was given")
        return self.plain(*args)


_VllmBackend, _VllmImpl = _vllm_flash_attention()

if _VllmImpl is not None:

    class TreeFlashAttentionImpl(_TreeForward, _VllmImpl):
        """vLLM's FlashAttention implementation with the tree forward in front of it; vLLM constructs it as it
        constructs FlashAttention's."""

        def _plain_forward(self, *args: Any) -> torch.Tensor:
            return _VllmImpl.forward(self, *args)

    class TreeFlashAttentionBackend(_VllmBackend):
        """vLLM's FlashAttention backend under the name ``CUSTOM``, served by :class:`TreeFlashAttentionImpl`."""

        @staticmethod
        def get_name() -> str:
            return "CUSTOM"

        @staticmethod
        def get_impl_cls() -> type:
            return TreeFlashAttentionImpl

else:
    TreeFlashAttentionImpl = TreeAttentionImpl

    class TreeFlashAttentionBackend:
        """The backend name the plugin registers (vllm/tree_attention.py:91-98): ``CUSTOM``, served by
        :class:`TreeAttentionImpl` (vLLM is not installed)."""

        @staticmethod
        def get_name() -> str:
            return "CUSTOM"

        @staticmethod
        def get_impl_cls() -> type:
            return TreeAttentionImpl
