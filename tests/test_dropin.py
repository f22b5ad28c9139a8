"""The drop-in at the Python level: the reference's callers import the verify path from this overlay, unchanged.

A stand-in installation is written to a temporary directory:

- ``engines/``: a fake ``vllm`` and ``sglang`` holding only the classes and functions the callers import;
- ``installed/eagle_harness``: a fake installed eagle-harness. Its caller modules carry the reference callers' own
  import lines (each cited below); its modules that the overlay shadows raise at import, and its ``tree_accept``
  holds a ``TreeRejectionSampler`` whose walk goes through a "Triton" kernel that raises when launched.

A child interpreter runs with ``eagle-4_amd`` (the overlay) ahead of both on ``sys.path`` and checks that every
caller import resolves, every imported kernel entry is the overlay's, the plugin's registration strings load
vLLM-derived classes, and every launch the engine glue makes lands on a ``libeagle4_amd.so`` entry point (the
binding's ``launch`` is replaced by a recorder, so no GPU is needed). Nothing under ``/root/reference`` is read.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OVERLAY = os.path.join(ROOT, "eagle-4_amd")

SHADOWED = "raise AssertionError('the installed {name} ran: the overlay should have shadowed it')\n"

ENGINES = {
    "vllm/model_executor/layers/mamba/verify_extension.py": """
        from dataclasses import dataclass
        from typing import Any

        class LinearAttnVerifyExtension:
            def forward_spec_rows(self, rows):
                raise NotImplementedError

            def forward_mamba2_spec_rows(self, rows):
                raise NotImplementedError

        @dataclass
        class GDNSpecRows:
            layer_name: Any = None

        @dataclass
        class Mamba2SpecRows:
            layer_name: Any = None
        """,
    "vllm/model_executor/layers/mamba/mamba_utils.py": """
        import os

        def is_conv_state_dim_first():
            return os.environ.get("FAKE_VLLM_DIM_FIRST", "1") == "1"
        """,
    "vllm/model_executor/layers/mamba/gdn/qwen_gdn_linear_attn.py": "class QwenGatedDeltaNetAttention: pass\n",
    "vllm/model_executor/layers/mamba/mamba_mixer2.py": "class MambaMixer2: pass\n",
    "vllm/v1/attention/backends/flash_attn.py": """
        PLAIN_CALLS = []

        class FlashAttentionMetadata: pass

        class FlashAttentionImpl:
            def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes=None, sliding_window=None,
                         kv_cache_dtype="auto", **kwargs):
                self.num_heads, self.head_size, self.scale = num_heads, head_size, scale
                self.num_kv_heads, self.kv_cache_dtype = num_kv_heads, kv_cache_dtype

            def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                        output_block_scale=None):
                PLAIN_CALLS.append("flash_attention")
                return output

        class FlashAttentionBackend:
            @staticmethod
            def get_name():
                return "FLASH_ATTN"

            @staticmethod
            def get_impl_cls():
                return FlashAttentionImpl
        """,
    "vllm/v1/attention/backends/fa_utils.py": "def is_quantized_kv_cache(dtype): return dtype != 'auto'\n",
    "vllm/v1/worker/gpu/spec_decode/rejection_sampler.py": """
        class RejectionSampler:
            def __init__(self, sampler, spec_config, device):
                self.sampler, self.spec_config, self.device = sampler, spec_config, device
        """,
    "sglang/srt/layers/attention/linear/verify_extension.py": """
        class LinearAttnStateLayout: pass
        class LinearAttnVerifyExtension: pass
        class LinearAttnVerifyLayout: pass
        """,
}

INSTALLED = {
    "eagle_harness/__init__.py": "__version__ = '0.1.5'\n",
    "eagle_harness/compat.py": "from eagle_harness import __version__\n",  # compat.py:31
    "eagle_harness/kernels/arch.py": """
        INSTALLED = True

        def gdn_records_replay(device=None):
            return True
        """,
    "eagle_harness/kernels/online_softmax.py": "INSTALLED = True\n",
    "eagle_harness/vllm/adapter.py": """
        import importlib

        VERIFY_EXTENSION_MODULES = ("vllm.model_executor.layers.mamba.verify_extension",)

        def verify_extension_module():
            return importlib.import_module(VERIFY_EXTENSION_MODULES[0])
        """,
    "eagle_harness/vllm/config.py": """
        from types import SimpleNamespace

        METHOD_NAME = "eagle_harness"

        def parse_method_config(method_config):
            return SimpleNamespace(node_top_k=method_config["node_top_k"])
        """,
    # vllm/plugin.py:18-27
    "eagle_harness/vllm/plugin.py": """
        from eagle_harness.vllm.config import METHOD_NAME

        SPECULATOR = "eagle_harness.vllm.speculator:HarnessSpeculator"
        GDN_TREE_VERIFY = "eagle_harness.vllm.gdn_tree_verify:create_extension"
        TREE_ATTENTION = "eagle_harness.vllm.tree_attention.TreeFlashAttentionBackend"
        """,
    # vllm/speculator.py:53-58 (the verify path's lines)
    "eagle_harness/vllm/speculator.py": """
        from eagle_harness.vllm.gdn_tree_verify import LinearStateCommit, check_tree_verifiable
        from eagle_harness.vllm.round_commit import KvCompactor, chainize
        from eagle_harness.vllm.tree_accept import TreeRejectionSampler
        from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage, set_stage
        """,
    # vllm/draft_attention.py:20
    "eagle_harness/vllm/draft_attention.py":
        "from eagle_harness.kernels.row_attention import RowsLaunch, program_splits, rows_attention, rows_padded\n",
    # vllm/tree_accept.py: the engine glue around the walk (:41, :86-115, :129-229 in shape)
    "eagle_harness/vllm/tree_accept.py": """
        from vllm.v1.worker.gpu.spec_decode.rejection_sampler import RejectionSampler

        from eagle_harness.vllm.verify_layout import TreeStore, VerifyStage

        def _tree_accept_kernel(*args):
            raise AssertionError("the installed Triton walk was launched")

        def accept_tree(target, drafted, cu_num_logits, idx_mapping, parents, store):
            _tree_accept_kernel(target, drafted, cu_num_logits, idx_mapping, parents, store)

        def accepted_rows_first(expanded_idx_mapping, expanded_local_pos, store):
            raise AssertionError("the installed row map ran")

        class TreeRejectionSampler(RejectionSampler):
            def __init__(self, sampler, spec_config, device, store, stage):
                super().__init__(sampler, spec_config, device)
                self.store, self.stage = store, stage

            def _verify(self, target, drafted, cu_num_logits, idx_mapping, expanded_idx_mapping, expanded_local_pos):
                sampled, num_sampled = accept_tree(
                    target, drafted, cu_num_logits, idx_mapping, self.stage.slot_parents, self.store)
                rows = accepted_rows_first(expanded_idx_mapping, expanded_local_pos, self.store)
                return sampled, num_sampled, rows
        """,
    # sglang/gdn_tree_verify.py:27-37
    "eagle_harness/sglang/gdn_tree_verify.py": """
        from sglang.srt.layers.attention.linear.verify_extension import (
            LinearAttnStateLayout,
            LinearAttnVerifyExtension,
            LinearAttnVerifyLayout,
        )

        from eagle_harness.kernels import arch
        from eagle_harness.kernels.gdn_tree import gdn_tree_ancestors, gdn_tree_paths_buffer
        from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
        from eagle_harness.kernels.gdn_tree_recurrence import gdn_tree_recurrent_update

        def records_kernels():  # the lazy imports of :142 and :204
            from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_commit
            from eagle_harness.kernels.gdn_tree_records import gdn_tree_records_update
            return gdn_tree_records_update, gdn_tree_records_commit
        """,
    # sglang/mamba2_tree_verify.py:30-31
    "eagle_harness/sglang/mamba2_tree_verify.py": """
        from eagle_harness.kernels.gdn_tree import gdn_tree_ancestors
        from eagle_harness.kernels.gdn_tree_conv import gdn_tree_conv1d_update
        """,
    # sglang/verify_step.py:32
    "eagle_harness/sglang/verify_step.py":
        "from eagle_harness.kernels.accept_tail import Accepted, accept_tail, compact_rows\n",
    # sglang/verify_plan.py:24
    "eagle_harness/sglang/verify_plan.py": "from eagle_harness.kernels.verify_prep import MAX_TAIL_WIDTH, tree_tail_words\n",
    # sglang/worker.py:62
    "eagle_harness/sglang/worker.py": "from eagle_harness.kernels.accept_tail import warm_up as warm_up_accept_tail\n",
    # sglang/row_attention.py:28
    "eagle_harness/sglang/row_attention.py":
        "from eagle_harness.kernels.row_attention import RowsLaunch, rows_attention, rows_padded\n",
    # sglang/drafter.py:298 (a lazy import)
    "eagle_harness/sglang/drafter.py": """
        def tail_words():
            from eagle_harness.kernels.verify_prep import MAX_TAIL_WIDTH, tree_tail_words
            return MAX_TAIL_WIDTH, tree_tail_words
        """,
}
for _name in ("kernels/gdn_tree", "kernels/gdn_tree_conv", "kernels/gdn_tree_recurrence", "kernels/gdn_tree_records",
              "kernels/accept_tail", "kernels/verify_prep", "kernels/row_attention", "kernels/mamba2_tree",
              "vllm/gdn_tree_verify", "vllm/tree_attention", "vllm/verify_attention", "vllm/verify_layout",
              "vllm/round_commit"):
    INSTALLED[f"eagle_harness/{_name}.py"] = SHADOWED.format(name=_name)

# (caller module, name it imports, module that must define it in the overlay)
IMPORTS = [
    ("eagle_harness.vllm.speculator", n, "eagle_harness.vllm.gdn_tree_verify")
    for n in ("LinearStateCommit", "check_tree_verifiable")
] + [
    ("eagle_harness.vllm.speculator", n, "eagle_harness.vllm.round_commit") for n in ("KvCompactor", "chainize")
] + [
    ("eagle_harness.vllm.speculator", n, "eagle_harness.vllm.verify_layout") for n in ("TreeStore", "VerifyStage",
                                                                                      "set_stage")
] + [
    ("eagle_harness.vllm.draft_attention", n, "eagle_harness.kernels.row_attention")
    for n in ("RowsLaunch", "program_splits", "rows_attention", "rows_padded")
] + [
    ("eagle_harness.sglang.gdn_tree_verify", "gdn_tree_ancestors", "eagle_harness.kernels.gdn_tree"),
    ("eagle_harness.sglang.gdn_tree_verify", "gdn_tree_paths_buffer", "eagle_harness.kernels.gdn_tree"),
    ("eagle_harness.sglang.gdn_tree_verify", "gdn_tree_conv1d_update", "eagle_harness.kernels.gdn_tree_conv"),
    ("eagle_harness.sglang.gdn_tree_verify", "gdn_tree_recurrent_update", "eagle_harness.kernels.gdn_tree_recurrence"),
    ("eagle_harness.sglang.mamba2_tree_verify", "gdn_tree_ancestors", "eagle_harness.kernels.gdn_tree"),
    ("eagle_harness.sglang.mamba2_tree_verify", "gdn_tree_conv1d_update", "eagle_harness.kernels.gdn_tree_conv"),
    ("eagle_harness.sglang.verify_step", "Accepted", "eagle_harness.kernels.accept_tail"),
    ("eagle_harness.sglang.verify_step", "accept_tail", "eagle_harness.kernels.accept_tail"),
    ("eagle_harness.sglang.verify_step", "compact_rows", "eagle_harness.kernels.accept_tail"),
    ("eagle_harness.sglang.verify_plan", "MAX_TAIL_WIDTH", "eagle_harness.kernels.verify_prep"),
    ("eagle_harness.sglang.verify_plan", "tree_tail_words", "eagle_harness.kernels.verify_prep"),
    ("eagle_harness.sglang.worker", "warm_up_accept_tail", "eagle_harness.kernels.accept_tail"),
    ("eagle_harness.sglang.row_attention", "RowsLaunch", "eagle_harness.kernels.row_attention"),
    ("eagle_harness.sglang.row_attention", "rows_attention", "eagle_harness.kernels.row_attention"),
    ("eagle_harness.sglang.row_attention", "rows_padded", "eagle_harness.kernels.row_attention"),
]

CHILD = r'''
import importlib, json, os, sys
from types import SimpleNamespace

overlay, imports = sys.argv[1], json.loads(sys.argv[2])
out = {"imports": {}}


def under_overlay(module):
    return os.path.realpath(module.__file__).startswith(os.path.realpath(overlay) + os.sep)


for caller, name, source in imports:
    mod, src = importlib.import_module(caller), importlib.import_module(source)
    own = {"warm_up_accept_tail": "warm_up"}.get(name, name)
    out["imports"][f"{caller}:{name}"] = getattr(mod, name) is getattr(src, own) and under_overlay(src)

import eagle_harness
from eagle_harness.kernels import _native

out["version"] = eagle_harness.__version__
out["arch_installed"] = getattr(importlib.import_module("eagle_harness.sglang.gdn_tree_verify").arch, "INSTALLED", False)
out["online_softmax_installed"] = getattr(importlib.import_module("eagle_harness.kernels.online_softmax"), "INSTALLED",
                                          False)
importlib.import_module("eagle_harness.compat")
update, commit = importlib.import_module("eagle_harness.sglang.gdn_tree_verify").records_kernels()
rec = importlib.import_module("eagle_harness.kernels.gdn_tree_records")
out["records_lazy"] = update is rec.gdn_tree_records_update and commit is rec.gdn_tree_records_commit
mx, words = importlib.import_module("eagle_harness.sglang.drafter").tail_words()
out["drafter_lazy"] = words is importlib.import_module("eagle_harness.kernels.verify_prep").tree_tail_words

# every launch goes to the binding's launch: record the entry names instead of launching
calls = []
_native.launch = lambda name, args, device: calls.append(name)
_native.library = lambda: SimpleNamespace(eagle4_verify_attention_workspace=lambda args: 0)

import torch

plugin = importlib.import_module("eagle_harness.vllm.plugin")
mod_name, fn_name = plugin.GDN_TREE_VERIFY.split(":")
create_extension = getattr(importlib.import_module(mod_name), fn_name)
mod_name, _, cls_name = plugin.TREE_ATTENTION.rpartition(".")
backend = getattr(importlib.import_module(mod_name), cls_name)
ext_mod = importlib.import_module("vllm.model_executor.layers.mamba.verify_extension")
flash = importlib.import_module("vllm.v1.attention.backends.flash_attn")
gtv = importlib.import_module("eagle_harness.vllm.gdn_tree_verify")
ext = create_extension(SimpleNamespace(speculative_config=SimpleNamespace(method_config={"node_top_k": 4})))
out["extension"] = isinstance(ext, ext_mod.LinearAttnVerifyExtension) and type(ext) is gtv.TreeVerify
out["chain_extension_none"] = create_extension(
    SimpleNamespace(speculative_config=SimpleNamespace(method_config={"node_top_k": 1}))) is None
out["spec_rows_are_vllms"] = gtv.GDNSpecRows is ext_mod.GDNSpecRows
out["backend"] = (issubclass(backend, flash.FlashAttentionBackend) and backend.get_name() == "CUSTOM"
                  and issubclass(backend.get_impl_cls(), flash.FlashAttentionImpl))

qwen = importlib.import_module("vllm.model_executor.layers.mamba.gdn.qwen_gdn_linear_attn").QwenGatedDeltaNetAttention
mixer = importlib.import_module("vllm.model_executor.layers.mamba.mamba_mixer2").MambaMixer2
speculator = importlib.import_module("eagle_harness.vllm.speculator")
speculator.check_tree_verifiable([qwen(), mixer()])
try:
    speculator.check_tree_verifiable([qwen(), object()])
    out["refuses_unknown_layers"] = False
except RuntimeError as err:
    out["refuses_unknown_layers"] = "object" in str(err)

# the stage, the attention backend's two routes, the sampler's walk, the layer hook and the commit
dev = torch.device("cpu")
B, W, Hq, Hkv, D, page = 2, 4, 4, 2, 64, 16
store = speculator.TreeStore(B, W, dev)
stage = speculator.VerifyStage(B, B * W, W, dev)
idx = torch.arange(B, dtype=torch.int32)
qsl = torch.arange(0, B * W + 1, W, dtype=torch.int32)
positions = torch.arange(B * W, dtype=torch.int64) + 100
stage.stage(store, idx, qsl, qsl, positions, B, B * W, tree=True)
speculator.set_stage(stage)
stage.active = True
impl = backend.get_impl_cls()(Hq, D, D ** -0.5, Hkv, kv_cache_dtype="auto")
q = torch.zeros(B * W, Hq, D, dtype=torch.bfloat16)
kn = torch.zeros(B * W, Hkv, D, dtype=torch.bfloat16)
kv_cache = torch.zeros(8, Hkv, page, 2 * D, dtype=torch.bfloat16)
meta = SimpleNamespace(max_query_len=W, num_actual_tokens=B * W, query_start_loc=qsl,
                       block_table=torch.zeros(B, 4, dtype=torch.int32))
impl.forward(SimpleNamespace(), q, kn, kn, kv_cache, meta, torch.empty_like(q))
impl.forward(SimpleNamespace(), q, kn, kn, kv_cache, SimpleNamespace(max_query_len=1), torch.empty_like(q))
out["plain_route"] = flash.PLAIN_CALLS == ["flash_attention"]

sampler = speculator.TreeRejectionSampler(None, None, dev, store, stage)
tokens = torch.zeros(B * W, dtype=torch.int64)
sampled, num_sampled, rows = sampler._verify(tokens, tokens, qsl, idx, torch.arange(B).repeat_interleave(W),
                                             torch.arange(W).repeat(B))
out["row_map"] = rows.tolist() == list(range(B * W))  # path_len 0 everywhere: rows keep their place

H, HV, K = 2, 4, 16
dim = 2 * H * K + HV * K
slots = (1 + torch.arange(B * W, dtype=torch.int32)).view(B, W)
conv_state = torch.zeros(1 + B * W, dim, 3 + W, dtype=torch.bfloat16)
ssm = torch.zeros(1 + B * W, HV, K, K)
rows = ext_mod.GDNSpecRows()
for k, v in dict(layer_name="layers.0", mixed_qkv=torch.zeros(B * W, dim, dtype=torch.bfloat16),
                 conv_state=conv_state, conv_weight=torch.zeros(dim, 4, dtype=torch.bfloat16), conv_bias=None,
                 activation="silu", a=torch.zeros(B * W, HV, dtype=torch.bfloat16),
                 b=torch.zeros(B * W, HV, dtype=torch.bfloat16), A_log=torch.zeros(HV), dt_bias=torch.zeros(HV),
                 ssm_state=ssm, state_indices=slots, query_start_loc=qsl,
                 num_accepted_tokens=torch.ones(B, dtype=torch.int32),
                 out=torch.zeros(B * W, HV * K, dtype=torch.bfloat16), num_k_heads=H, head_k_dim=K, num_v_heads=HV,
                 head_v_dim=K).items():
    setattr(rows, k, v)
ext.forward_spec_rows(rows)

for dim_first in ("1", "0"):
    os.environ["FAKE_VLLM_DIM_FIRST"] = dim_first
    cache = conv_state if dim_first == "1" else conv_state.transpose(1, 2).contiguous()
    layer = SimpleNamespace(kv_cache=[cache, ssm])
    lsc = speculator.LinearStateCommit([layer, layer], [slots, slots], dev)
    want = cache.stride() if dim_first == "1" else (cache.stride(0), cache.stride(2), cache.stride(1))
    out[f"commit_dim_{dim_first}"] = lsc.dim == dim and tuple(lsc.conv_strides) == want
    lsc.commit(idx, store.path, store.path_len)

out["calls"] = calls
print(json.dumps(out))
'''


def _write_tree(base: str, files: dict) -> None:
    for rel, text in files.items():
        path = os.path.join(base, rel)
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(path, "w") as f:
            f.write(textwrap.dedent(text).lstrip("\n"))
    for here, dirs, names in os.walk(base):  # every directory a regular package
        if here != base and "__init__.py" not in names:
            open(os.path.join(here, "__init__.py"), "w").close()


def test_reference_callers_resolve_to_the_overlay(tmp_path):
    engines, installed = str(tmp_path / "engines"), str(tmp_path / "installed")
    _write_tree(engines, ENGINES)
    _write_tree(installed, INSTALLED)
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([OVERLAY, installed, engines]))
    proc = subprocess.run([sys.executable, "-c", CHILD, OVERLAY, json.dumps(IMPORTS)], env=env, cwd=str(tmp_path),
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    out = json.loads(proc.stdout.strip().splitlines()[-1])
    unresolved = [k for k, ok in out["imports"].items() if not ok]
    assert not unresolved, unresolved
    assert len(out["imports"]) == len(IMPORTS)
    assert out["version"] == "0.1.5"
    assert out["arch_installed"] and out["online_softmax_installed"]  # modules not built here stay the installed ones
    assert out["records_lazy"] and out["drafter_lazy"]
    assert out["extension"] and out["chain_extension_none"] and out["spec_rows_are_vllms"]
    assert out["backend"] and out["plain_route"] and out["refuses_unknown_layers"]
    assert out["row_map"] and out["commit_dim_1"] and out["commit_dim_0"]
    assert out["calls"] == [
        "eagle4_stage_tree",
        "eagle4_verify_attention",
        "eagle4_accept_tree",
        "eagle4_gdn_tree_conv1d_update",
        "eagle4_gdn_tree_recurrent_update",
        "eagle4_linear_state_commit",
        "eagle4_linear_state_commit",
    ]


def test_glue_without_an_installation_says_so():
    """Without an installed eagle-harness behind the overlay, the engine glue is refused with a reason, and the
    engine-free modules still import."""
    code = ("import sys\n"
            "from eagle_harness.vllm import tree_accept\n"
            "try:\n"
            "    tree_accept.TreeRejectionSampler\n"
            "except ImportError as err:\n"
            "    print('refused:', err)\n")
    proc = subprocess.run([sys.executable, "-c", code], env=dict(os.environ, PYTHONPATH=OVERLAY),
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "refused:" in proc.stdout and "installed eagle-harness" in proc.stdout
