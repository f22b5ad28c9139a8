"""ctypes binding of ``libeagle4_amd.so``, the gfx950 kernels of the verify hot path (``include/eagle4_amd.h``).

The library is loaded on first use from this directory (``EAGLE4_AMD_LIB`` overrides the path). It must have been
built (``python eagle-4_amd/build.py``): there is no other implementation to fall back to, so a missing library, a
"not covered" status or a HIP error raises. The argument structs below mirror the header field by field; their sizes
are checked against the library's own ``eagle4_args_size`` when it is loaded.

Conventions, as in the reference's native binding (kernels/native.py:28-41, kernels/candidate.py:23-28): every entry
returns 0 (launched), -1 (not covered: nothing launched) or a hipError_t; launches go to torch's current stream.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path
from typing import Optional

import torch

LIBRARY = Path(__file__).resolve().parent / "libeagle4_amd.so"

OK = 0
NOT_COVERED = -1
SCRATCH_TOO_SMALL = -2

BF16, F16, F32, FP8_E4M3, I32, I64, U8 = range(7)
_DTYPE_CODES = {
    torch.bfloat16: BF16,
    torch.float16: F16,
    torch.float32: F32,
    torch.float8_e4m3fn: FP8_E4M3,
    torch.int32: I32,
    torch.int64: I64,
    torch.uint8: U8,
    torch.bool: U8,
}

_i32, _i64, _f32, _ptr = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class NotCovered(NotImplementedError):
    """A shape, dtype or layout the gfx950 kernels do not cover (the library launched nothing)."""


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise NotCovered(f"dtype {dtype} is not covered by the gfx950 kernels") from None


def ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


class ITab(ctypes.Structure):
    _fields_ = [("ptr", _ptr), ("s0", _i64), ("s1", _i64), ("dtype", _i32), ("reserved", _i32)]


def itab(t: Optional[torch.Tensor]) -> ITab:
    """An integer table descriptor (int32 / int64, up to 2-D) of ``t``; a null descriptor for None."""
    if t is None:
        return ITab(None, 0, 0, I32, 0)
    if t.dtype not in (torch.int32, torch.int64):
        raise NotCovered(f"index tables must be int32 or int64, got {t.dtype}")
    s0 = t.stride(0) if t.ndim >= 1 else 0
    s1 = t.stride(1) if t.ndim >= 2 else 0
    return ITab(t.data_ptr(), s0, s1, dtype_code(t.dtype), 0)


def _fields(spec: str) -> list:
    """Fields from a compact spec: ``name:type`` pairs, type one of p (pointer), q (int64), i (int32), f (float),
    t (ITab)."""
    types = {"p": _ptr, "q": _i64, "i": _i32, "f": _f32, "t": ITab}
    out = []
    for item in spec.split():
        name, kind = item.split(":")
        out.append((name, types[kind]))
    return out


class StageTreeArgs(ctypes.Structure):
    _fields_ = _fields(
        "parents:t idx_mapping:t query_start_loc:t cu_num_logits:t positions:p stage_parents:p stage_anc:p "
        "stage_mask:p context_lens:p slot_parents:p slot_depths:p chain_positions:p num_reqs:i width:i tree:i "
        "num_tokens:i"
    )


class AncestorsArgs(ctypes.Structure):
    _fields_ = _fields(
        "next_token:t next_sibling:t parent_token:t conv_state_indices:t query_start_loc:t ancestors:p paths:p "
        "stride_paths_seq:q stride_paths_path:q batch:i width:i pad_slot_id:i reserved:i"
    )


class TailWordsArgs(ctypes.Structure):
    _fields_ = _fields("mask:p committed_len:t tail_bits:p width:i reserved:i")


class ConvArgs(ctypes.Structure):
    _fields_ = _fields(
        "x:p stride_x_seq:q stride_x_dim:q stride_x_token:q weight:p stride_w_dim:q stride_w_width:q bias:p "
        "conv_state:p stride_cs_seq:q stride_cs_dim:q stride_cs_tok:q conv_state_indices:t num_accepted:t "
        "query_start_loc:t window:p stride_win_seq:q stride_win_step:q stride_win_dim:q stride_win_win:q "
        "window_indices:t ancestors:p out:p stride_o_seq:q stride_o_dim:q stride_o_token:q batch:i dim:i seqlen:i "
        "state_len:i pad_slot_id:i silu:i dtype:i bias_dtype:i"
    )


class GdnArgs(ctypes.Structure):
    _fields_ = _fields(
        "q:p k:p v:p stride_q:q stride_k:q stride_v:q in_dtype:i gate_dtype:i a:p b:p stride_a:q stride_b:q "
        "A_log:p dt_bias:p A_log_dtype:i dt_bias_dtype:i softplus_beta:f softplus_threshold:f scale:f out_dtype:i "
        "out:p stride_o:q parents:t cu_seqlens:t h0_source:p stride_h0_source:q h0_dtype:i snap_dtype:i "
        "h0_indices:t num_accepted:t snap:p stride_snap_slot:q stride_snap_row:q snap_indices:t publish:p "
        "stride_publish:q num_slot_cols:i N:i H:i HV:i K:i V:i row_slots:i skip_chain_reload:i pad_slot_id:i"
    )


class RecordsArgs(ctypes.Structure):
    _fields_ = _fields(
        "q:p k:p v:p stride_q:q stride_k:q stride_v:q in_dtype:i gate_dtype:i a:p b:p stride_a:q stride_b:q "
        "A_log:p dt_bias:p A_log_dtype:i dt_bias_dtype:i scale:f out_dtype:i out:p stride_o:q state:p "
        "stride_state:q state_dtype:i path_replay:i state_indices:t query_start_loc:t parent:t tree_paths:t "
        "records:p stride_records_row:q record_indices:t rec:i width:i num_paths:i N:i H:i HV:i K:i V:i"
    )


class RecordsCommitArgs(ctypes.Structure):
    _fields_ = _fields(
        "state:p stride_state_layer:q stride_state_slot:q state_dtype:i round_state:i records:p "
        "stride_records_layer:q stride_records_row:q state_indices:t record_indices:t commit_steps:t parent:t "
        "n:i layers:i HV:i K:i V:i rec:i dmax:i reserved:i"
    )


class AttnArgs(ctypes.Structure):
    _fields_ = _fields(
        "q:p stride_qt:q stride_qh:q k_new:p stride_knt:q stride_knh:q v_new:p stride_vnt:q stride_vnh:q "
        "key_cache:p stride_kb:q stride_ks:q stride_kh:q value_cache:p stride_vb:q stride_vs:q stride_vh:q "
        "k_scale:p stride_ksb:q stride_ksh:q v_scale:p stride_vsb:q stride_vsh:q block_table:t context_lens:t "
        "query_start_loc:t masks:p stride_mask:q out:p stride_ot:q stride_oh:q workspace:p workspace_bytes:q "
        "scale:f num_reqs:i Hq:i Hkv:i D:i page:i max_query_len:i max_blocks:i dtype:i cache_dtype:i chunk:i"
    )


class ArgmaxArgs(ctypes.Structure):
    _fields_ = _fields("logits:p stride_row:q dtype:i rows:i vocab:i reserved:i out:p")


class AcceptTreeArgs(ctypes.Structure):
    _fields_ = _fields(
        "target:t drafted:t cu_num_logits:t idx_mapping:t parents:t sampled:p stride_sampled:q num_sampled:p "
        "path:p stride_path:q path_len:p num_reqs:i width:i"
    )


class AcceptTailArgs(ctypes.Structure):
    _fields_ = _fields(
        "target_predict:t candidates:t retrieve_index:t retrieve_next_token:t retrieve_next_sibling:t seq_lens:t "
        "out_cache_loc:t req_to_token:t req_pool_indices:t predict:p accept_index:p accept_lens:p new_seq_lens:p "
        "bonus:p committed_slots:p accepted_slots:p width:i depth:i"
    )


class CompactRowsArgs(ctypes.Structure):
    _fields_ = _fields(
        "src:p dst:p accept_index:t src_stride:q dst_stride:q row_bytes:q width:i depth:i"
    )


class StateCommitArgs(ctypes.Structure):
    _fields_ = _fields(
        "conv_ptrs:p ssm_ptrs:p slots_ptrs:p slots_strides:p idx_mapping:t path:t path_len:t conv_stride_slot:q "
        "conv_stride_dim:q conv_stride_tok:q ssm_stride_slot:q ssm_numel:q conv_dtype:i ssm_dtype:i num_reqs:i "
        "layers:i dim:i reserved:i"
    )


class CompactKvArgs(ctypes.Structure):
    _fields_ = _fields(
        "layer_ptrs:p table_ptrs:p table_strides:p table_block_sizes:p idx_mapping:t query_start_loc:t "
        "cu_num_logits:t seq_lens:t path:t path_len:t stride_block:q stride_head:q stride_slot:q block_size:i dim:i "
        "dtype:i num_reqs:i layers:i heads:i"
    )


class ChainizeArgs(ctypes.Structure):
    _fields_ = _fields(
        "idx_mapping:t query_start_loc:t cu_num_logits:t seq_lens:t path:t path_len:t sampled:t input_ids:p "
        "positions:p src_rows:p input_ids_dtype:i positions_dtype:i src_rows_dtype:i rows:i num_reqs:i reserved:i"
    )


class RowAttnArgs(ctypes.Structure):
    _fields_ = _fields(
        "q:p stride_q_row:q stride_q_head:q keys:p values:p k_stride_page:q k_stride_slot:q k_stride_head:q "
        "v_stride_page:q v_stride_slot:q v_stride_head:q out:p stride_o_row:q stride_o_head:q part_out:p part_lse:p "
        "part_rows:q table:p stride_table:q table_rows:t seq_lens:t ancestors:p max_depth:i table_page:i cache_page:i "
        "bs:i rows_per_request:i rows_padded:i heads:i kv_heads:i head_dim:i dtype:i step:i window:i splits:i scale:f"
    )


# entry name -> (args struct, index in eagle4_args_size)
class Mamba2Args(ctypes.Structure):
    _fields_ = _fields(
        "state:p stride_state_slot:q stride_state_head:q stride_state_dim:q x:p stride_x_tok:q stride_x_head:q dt:p "
        "stride_dt_tok:q stride_dt_head:q B:p stride_B_tok:q stride_B_group:q C:p stride_C_tok:q stride_C_group:q A:p "
        "D:p dt_bias:p out:p stride_out_tok:q stride_out_head:q slots:t parents:t num_accepted:t query_start_loc:t "
        "batch:i heads:i head_dim:i dstate:i groups:i state_dtype:i in_dtype:i dt_dtype:i param_dtype:i out_dtype:i "
        "dt_softplus:i pad_slot_id:i"
    )


ENTRIES = {
    "eagle4_stage_tree": (StageTreeArgs, 0),
    "eagle4_gdn_tree_ancestors": (AncestorsArgs, 1),
    "eagle4_tree_tail_words": (TailWordsArgs, 2),
    "eagle4_gdn_tree_conv1d_update": (ConvArgs, 3),
    "eagle4_gdn_tree_recurrent_update": (GdnArgs, 4),
    "eagle4_gdn_tree_records_update": (RecordsArgs, 5),
    "eagle4_gdn_tree_records_commit": (RecordsCommitArgs, 6),
    "eagle4_verify_attention": (AttnArgs, 7),
    "eagle4_verify_attention_static": (AttnArgs, 7),
    "eagle4_argmax_rows": (ArgmaxArgs, 8),
    "eagle4_accept_tree": (AcceptTreeArgs, 9),
    "eagle4_accept_tail": (AcceptTailArgs, 10),
    "eagle4_compact_rows": (CompactRowsArgs, 11),
    "eagle4_linear_state_commit": (StateCommitArgs, 12),
    "eagle4_compact_kv": (CompactKvArgs, 13),
    "eagle4_chainize": (ChainizeArgs, 14),
    "eagle4_row_attention": (RowAttnArgs, 15),
    "eagle4_mamba2_tree_state_update": (Mamba2Args, 16),
}
EXTRA_SYMBOLS = ("eagle4_verify_attention_workspace", "eagle4_verify_attention_static_bytes", "eagle4_version",
                 "eagle4_args_size", "eagle4_init")


@functools.lru_cache(maxsize=None)
def library() -> ctypes.CDLL:
    """The bound library; raises RuntimeError when it is missing or its structs disagree with this binding."""
    path = Path(os.environ.get("EAGLE4_AMD_LIB", LIBRARY))
    if not path.exists():
        raise RuntimeError(
            f"eagle4_amd: {path} is not built; run `python eagle-4_amd/build.py` (hipcc, gfx950). "
            "There is no non-native fallback."
        )
    lib = ctypes.CDLL(str(path))
    lib.eagle4_args_size.argtypes = [ctypes.c_int]
    lib.eagle4_args_size.restype = ctypes.c_int64
    lib.eagle4_version.restype = ctypes.c_char_p
    for name, (struct, which) in ENTRIES.items():
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.POINTER(struct), ctypes.c_void_p]
        fn.restype = ctypes.c_int
        native = lib.eagle4_args_size(which)
        if native != ctypes.sizeof(struct):
            raise RuntimeError(f"eagle4_amd: {struct.__name__} is {ctypes.sizeof(struct)} bytes here, {native} in {path}")
    lib.eagle4_verify_attention_workspace.argtypes = [ctypes.POINTER(AttnArgs)]
    lib.eagle4_verify_attention_workspace.restype = ctypes.c_int64
    lib.eagle4_verify_attention_static_bytes.argtypes = []
    lib.eagle4_verify_attention_static_bytes.restype = ctypes.c_int64
    lib.eagle4_init.argtypes = []
    lib.eagle4_init.restype = ctypes.c_int
    if torch.cuda.is_available():  # the static arrays' device addresses, looked up now rather than on a first call
        status = lib.eagle4_init()
        if status != OK:
            raise RuntimeError(f"eagle4_amd: eagle4_init failed with HIP error {status}")
    return lib


TARGET_ISA = "gfx950"


class UnsupportedHardware(RuntimeError):
    """The device cannot run the library's code objects (they are built for gfx950 only)."""


@functools.lru_cache(maxsize=None)
def _isa_of(index: int) -> tuple[str, str]:
    props = torch.cuda.get_device_properties(index)
    if torch.version.hip is None:
        return props.name, f"sm_{props.major}{props.minor}"
    return props.name, str(props.gcnArchName).partition(":")[0]


def unsupported_reason(device: torch.device) -> Optional[str]:
    """Why the kernels cannot run on ``device``, in one line; None when they can. A device is covered exactly when
    the ISA part of its target name (``gfx950`` of ``gfx950:sramecc+:xnack-``) is gfx950."""
    if device.type != "cuda":
        return f"tensors are on {device}, not on a ROCm GPU"
    if not torch.cuda.is_available():
        return "torch sees no ROCm GPU"
    name, isa = _isa_of(device.index if device.index is not None else torch.cuda.current_device())
    if isa != TARGET_ISA:
        return f"{name} is {isa or 'an unknown ISA'}, and libeagle4_amd.so holds {TARGET_ISA} (MI355X) code objects only"
    return None


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def launch(name: str, args: ctypes.Structure, device: torch.device) -> None:
    """Calls entry ``name`` on the current stream of ``device``; raises on anything but success."""
    reason = unsupported_reason(device)
    if reason is not None:
        raise UnsupportedHardware(f"eagle4_amd: {name} cannot run: {reason}")
    fn = getattr(library(), name)
    with torch.cuda.device(device):
        status = fn(ctypes.byref(args), ctypes.c_void_p(stream_of(device)))
    if status == NOT_COVERED:
        raise NotCovered(f"eagle4_amd: {name} does not cover this launch (shape, dtype or layout)")
    if status == SCRATCH_TOO_SMALL:
        raise ValueError(f"eagle4_amd: {name} needs more scratch than its static buffer holds "
                         f"({library().eagle4_verify_attention_static_bytes()} bytes); nothing was launched")
    if status != OK:
        raise RuntimeError(f"eagle4_amd: {name} failed with HIP error {status}")


# On a GPU machine the library is loaded (and its static arrays' device addresses looked up, eagle4_init) when this
# binding is imported, so that set-up never happens inside a caller's graph capture.
if torch.cuda.is_available() and Path(os.environ.get("EAGLE4_AMD_LIB", LIBRARY)).exists():
    library()
