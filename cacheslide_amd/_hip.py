"""ctypes binding of libcacheslide_hip.so (declared in include/cacheslide_hip.h).

Torch tensors are used only to own device memory and to name the current HIP
stream; every computation on them is a kernel of the library.  Loading fails
loudly when the library has not been built: there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import struct
from pathlib import Path

import torch

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libcacheslide_hip.so"

CS_F32, CS_F16, CS_BF16, CS_F64, CS_I32, CS_I64, CS_U8 = range(7)
DECODE_SCRATCH_BYTES = 64 << 20  # CS_DECODE_SCRATCH_BYTES
CS_OK, CS_EINVAL, CS_ELAUNCH, CS_EUNSUPPORTED, CS_ECAPACITY = range(5)

FLAG_Q_NONFINITE = 1 << 0
FLAG_K_NONFINITE = 1 << 1
FLAG_V_NONFINITE = 1 << 2
FLAG_QPOS_NEGATIVE = 1 << 3
FLAG_QPOS_DUPLICATE = 1 << 4
FLAG_KPOS_NEGATIVE = 1 << 5
FLAG_KPOS_DUPLICATE = 1 << 6
FLAG_KPOS_UNSORTED = 1 << 7
FLAG_LOGIT_NONFINITE = 1 << 8
FLAG_POS_INVALID = 1 << 9
FLAG_SCORE_NONFINITE = 1 << 10
FLAG_E_NONFINITE = 1 << 11
FLAG_POS_NONFINITE = 1 << 12
FLAG_BLOCK_INVALID = 1 << 13
FLAG_NO_KEY = 1 << 14
FLAG_CONTEXT_RANGE = 1 << 15
FLAG_PATH_NEGATIVE = 1 << 16
FLAG_PATH_AVAILABLE = 1 << 17
FLAG_PATH_INCREASING = 1 << 18
FLAG_PATH_GAP = 1 << 19
FLAG_ROW_LOST = 1 << 20
FLAG_ROWS_UNSORTED = 1 << 21
FLAG_ROW_INDEX = 1 << 22
FLAG_POLICY_GENERIC = 1 << 23
COPY_H2D, COPY_D2H, COPY_D2D = range(3)

_DTYPE_CODES = {
    torch.float32: CS_F32,
    torch.float16: CS_F16,
    torch.bfloat16: CS_BF16,
    torch.float64: CS_F64,
    torch.int32: CS_I32,
    torch.int64: CS_I64,
    torch.uint8: CS_U8,
    torch.bool: CS_U8,
}


class CsView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 6),
        ("stride", ctypes.c_int64 * 6),
    ]


class CsWcaUpdateArgs(ctypes.Structure):
    """cs_wca_update_args: one WCAState.update in one library call."""

    _fields_ = [
        ("cached_k", CsView), ("cached_v", CsView), ("recomputed_k", CsView),
        ("recomputed_v", CsView), ("fused_k", CsView), ("fused_v", CsView),
        ("rows", ctypes.c_void_p), ("computed", ctypes.c_void_p),
        ("a", ctypes.c_int64), ("n", ctypes.c_int64), ("budget", ctypes.c_int64),
        ("alpha", ctypes.c_void_p), ("deviation", ctypes.c_void_p),
        ("selected", ctypes.c_void_p), ("candidate", ctypes.c_void_p),
        ("removed_mask", ctypes.c_void_p), ("mandatory", ctypes.c_void_p),
        ("err", ctypes.c_void_p), ("norm", ctypes.c_void_p), ("next_alpha", ctypes.c_void_p),
        ("cosine", ctypes.c_void_p), ("used", ctypes.c_void_p), ("removed", ctypes.c_void_p),
        ("promoted", ctypes.c_void_p), ("scratch", ctypes.c_void_p), ("active", ctypes.c_void_p),
        ("flags", ctypes.c_void_p), ("counts", ctypes.c_void_p),
        ("epsilon", ctypes.c_double), ("threshold", ctypes.c_double),
        ("clamp", ctypes.c_int32), ("previous_layer", ctypes.c_int32), ("gate", ctypes.c_int32),
        ("distance_mode", ctypes.c_int32), ("abort_mask", ctypes.c_int32),
        ("clear_status", ctypes.c_int32), ("report", ctypes.c_void_p),
    ]


class CsWcaInitializeArgs(ctypes.Structure):
    """cs_wca_initialize_args: one WCAState.initialize in one library call."""

    _fields_ = [
        ("cached_k", CsView), ("recomputed_k", CsView),
        ("reused", ctypes.c_void_p), ("mandatory", ctypes.c_void_p), ("n", ctypes.c_int64),
        ("epsilon", ctypes.c_double), ("fraction", ctypes.c_double), ("clamp", ctypes.c_int32),
        ("clear_status", ctypes.c_int32), ("err", ctypes.c_void_p), ("norm", ctypes.c_void_p), ("alpha", ctypes.c_void_p),
        ("candidate", ctypes.c_void_p), ("selected", ctypes.c_void_p), ("removed", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p), ("promoted", ctypes.c_void_p), ("active", ctypes.c_void_p),
        ("flags", ctypes.c_void_p), ("counts", ctypes.c_void_p), ("report", ctypes.c_void_p),
    ]


# cs_wca_update_args from ``rows`` to ``report`` as bytes: two pointers, a, n,
# budget, seventeen pointers, epsilon, threshold, six int32 fields, report
WCA_UPDATE_TAIL = struct.Struct("<2q3q17q2d6iq")
assert WCA_UPDATE_TAIL.size == ctypes.sizeof(CsWcaUpdateArgs) - CsWcaUpdateArgs.rows.offset


class CsCcpeArgs(ctypes.Structure):
    _fields_ = [
        ("q", CsView),
        ("k", CsView),
        ("v", CsView),
        ("e", CsView),
        ("qpos", ctypes.c_void_p),
        ("kpos", ctypes.c_void_p),
        ("attn_mask", CsView),
        ("vis_mask", CsView),
        ("sel_rows", ctypes.c_void_p),
        ("fixed_keys", ctypes.c_void_p),
        ("fixed_pos", CsView),
        ("canonical", CsView),
        ("q_ord", ctypes.c_void_p),
        ("k_ord", ctypes.c_void_p),
        ("strict", ctypes.c_int32),
        ("chunk_rows", ctypes.c_int32),
        ("chunk_flags", ctypes.c_void_p),
        ("out", CsView),
        ("pos_out", CsView),
        ("flags", ctypes.c_void_p),
    ]


class CsKvSource(ctypes.Structure):
    _fields_ = [
        ("cache", ctypes.c_void_p),
        ("s_block", ctypes.c_int64),
        ("s_head", ctypes.c_int64),
        ("s_offset", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int64),
        ("block_table", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int64),
        ("bt_cols", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_s_batch", ctypes.c_int64),
        ("k_s_tok", ctypes.c_int64),
        ("k_s_head", ctypes.c_int64),
        ("v_s_batch", ctypes.c_int64),
        ("v_s_tok", ctypes.c_int64),
        ("v_s_head", ctypes.c_int64),
        ("slots", ctypes.c_void_p),
        ("slots_stride", ctypes.c_int64),
        ("side_k", ctypes.c_void_p),
        ("side_v", ctypes.c_void_p),
        ("side_s_row", ctypes.c_int64),
        ("side_s_head", ctypes.c_int64),
        ("side_rows", ctypes.c_int64),
        ("slots_cols", ctypes.c_int64),
    ]


class CsDecodeSharedArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_s_batch", ctypes.c_int64),
        ("q_s_head", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("hq", ctypes.c_int32),
        ("hkv", ctypes.c_int32),
        ("nk", ctypes.c_void_p),
        ("max_nk", ctypes.c_int32),
        ("kv", ctypes.POINTER(CsKvSource)),
        ("e", ctypes.c_void_p),
        ("max_positions", ctypes.c_int32),
        ("split", ctypes.c_int32),
        ("head_table", ctypes.c_void_p),
        ("head_items", ctypes.c_int32),
        ("head_blocks", ctypes.c_int32),
        ("head_nk", ctypes.c_void_p),
        ("head_qpos", ctypes.c_void_p),
        ("tail_table", ctypes.c_void_p),
        ("tail_stride", ctypes.c_int64),
        ("tail_cols", ctypes.c_int32),
        ("tail_nk", ctypes.c_void_p),
        ("tail_qpos", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("flags", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_VP = ctypes.POINTER(CsView)

# name -> (restype, argtypes); every symbol of include/cacheslide_hip.h.
SIGNATURES = {
    "cs_version": (ctypes.c_char_p, []),
    "cs_last_error": (ctypes.c_char_p, []),
    "cs_check_finite": (_I32, [_VP, _I32, _P, _P]),
    "cs_check_positions": (_I32, [_P, _I64, _I32, _P, _P]),
    "cs_check_bias_positions": (_I32, [_VP, _I64, _P, _P]),
    "cs_ccpe_attention": (_I32, [ctypes.POINTER(CsCcpeArgs), _P]),
    "cs_ccpe_prefill_policy_workspace_bytes": (_I64, [_I32, _I32, _I64]),
    "cs_ccpe_prefill_policy_bf16": (_I32, [ctypes.POINTER(CsCcpeArgs), _P, _I64, _P]),
    "cs_prepare_device": (_I32, []),
    "cs_cope_positional_bias": (_I32, [_VP, _VP, _VP, _VP, _P, _P]),
    "cs_contextual_positions": (_I32, [_VP, _VP, _I64, _VP, _P, _P]),
    "cs_ccpe_logits": (_I32, [_VP, _VP, _VP, _P, _P]),
    "cs_validate_contextual_path": (_I32, [_VP, _P, _P, _VP, ctypes.c_double, _P, _P]),
    "cs_selected_visibility": (_I32, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P]),
    "cs_isin": (_I32, [_P, _I64, _P, _I64, _P, _P]),
    "cs_canonical_substitute": (_I32, [_VP, _VP, _P, _P, _I64, _P, _P, _I64, _P]),
    "cs_ccpe_prefill_bf16": (
        _I32,
        [_P, _I64, _I64, _I64, _P, _I64, _I32, _I32, _I32, _I32, _P,
         ctypes.POINTER(CsKvSource), _P, _I32, _P, _P, _P],
    ),
    "cs_ccpe_decode_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32]),
    "cs_ccpe_decode_bf16": (
        _I32,
        [_P, _I64, _I64, _I32, _I32, _I32, _P, _I32, ctypes.POINTER(CsKvSource), _P,
         _I32, _I32, _P, _I64, _P, _P, _P],
    ),
    "cs_ccpe_decode_shared_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32]),
    "cs_ccpe_decode_shared_bf16": (_I32, [ctypes.POINTER(CsDecodeSharedArgs), _P, _I64, _P]),
    "cs_ccpe_decode_bf16_noalloc": (
        _I32,
        [_P, _I64, _I64, _I32, _I32, _I32, _P, _I32, ctypes.POINTER(CsKvSource), _P,
         _I32, _I32, _P, _P, _P],
    ),
    "cs_slot_scatter": (_I32, [_VP, _VP, _VP, _P, _P, _I64, _VP, _VP, _P]),
    "cs_slot_gather": (_I32, [_VP, _VP, _VP, _P, _P, _I64, _VP, _VP, _P]),
    "cs_slot_copy": (_I32, [_VP, _P, _P, _I64, _P]),
    "cs_page_copy": (_I32, [_VP, _P, _P, _I64, _P]),
    "cs_mapping_scatter": (_I32, [_P, _I64, _P, _P, _I64, _P]),
    "cs_mapping_gather": (_I32, [_P, _I64, _P, _P, _I64, _P]),
    "cs_freelist_release": (_I32, [_P, _I64, _P, _I64, _P]),
    "cs_wca_same_rows": (_I32, [_P, _P, _I64, _I32, _P, _P]),
    "cs_rows_remap": (_I32, [_VP, _VP, _VP, _VP, _VP, _VP, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P]),
    "cs_rows_missing": (_I32, [_P, _I64, _P, _I64, _P, _P]),
    "cs_rows_scatter": (_I32, [_VP, _P, _I64, _VP, _P, _P]),
    "cs_rows_gather": (_I32, [_VP, _P, _I64, _VP, _P, _P]),
    "cs_copy_async": (_I32, [_P, _P, _I64, _I32, _P]),
    "cs_wca_update": (_I32, [ctypes.POINTER(CsWcaUpdateArgs), _P]),
    "cs_wca_initialize": (_I32, [ctypes.POINTER(CsWcaInitializeArgs), _P]),
    "cs_snapshot_convert": (_I32, [_VP, _VP, _I32, _P, _P]),
    "cs_freelist_acquire": (_I32, [_P, _I64, _I64, _P, _P, _P]),
    "cs_wca_score": (_I32, [_VP, _P, _VP, _P, _P, _P, _P]),
    "cs_wca_alpha": (_I32, [_P, _P, _I64, ctypes.c_double, _I32, _P, _P, _P]),
    "cs_wca_promote": (_I32, [_P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I32, _P]),
    "cs_mask_nonzero": (_I32, [_P, _P, _I64, _P, _P, _P]),
    "cs_wca_blend": (_I32, [_VP, _VP, _P, _VP, _VP, _P, _P, _VP, _VP, _P, _P]),
    "cs_wca_head_cosine": (_I32, [_VP, _VP, _P, ctypes.c_double, _P, _P]),
    "cs_wca_init_masks": (_I32, [_P, _P, _P, _I64, _P, _P, _P, _P]),
    "cs_wca_used_alpha": (_I32, [_P, _P, _P, _P, _I64, _I32, _P, _P]),
    "cs_wca_gate": (_I32, [_P, _P, _P, _I64, _I32, ctypes.c_double, _P, _P, _P]),
    "cs_wca_commit": (_I32, [_P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I32, _P]),
}

_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise RuntimeError(
            f"{_LIB_PATH} is missing: build it with `make -C cacheslide_amd/csrc` "
            "(or __graft_entry__.build()); cacheslide_amd has no CPU fallback"
        )
    lib = ctypes.CDLL(os.fspath(_LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


class HipError(RuntimeError):
    """A library call returned a launch/runtime failure."""


def check(status: int, what: str) -> None:
    if status == CS_OK:
        return
    message = load().cs_last_error().decode(errors="replace")
    if status in (CS_EINVAL, CS_EUNSUPPORTED):
        raise ValueError(f"{what}: {message}")
    raise HipError(f"{what}: {message} (status {status})")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All compute runs on the HIP device; CPU tensors are rejected."""
    device = None
    for tensor in tensors:
        if tensor is None:
            continue
        if tensor.device.type != "cuda":
            raise ValueError(
                "cacheslide_amd computes on the HIP device only; got a tensor on "
                f"{tensor.device}"
            )
        if device is None:
            device = tensor.device
        elif tensor.device != device:
            raise ValueError("all tensors must be on the same HIP device")
    if device is None:
        raise ValueError("no device tensor given")
    if device.index not in _PREPARED:
        _prepare(device)
    return device


# Devices whose helper stream exists (cs_prepare_device): made at the first
# use of a device, before the caller's process has created many streams, so
# that the HIP runtime gives it a hardware queue other than the caller's.
_PREPARED: set = set()


def _prepare(device: torch.device) -> None:
    with torch.cuda.device(device):
        call("cs_prepare_device")
    _PREPARED.add(device.index)


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as error:
        raise ValueError(f"unsupported dtype {dtype}") from error


def view(tensor: torch.Tensor | None) -> CsView:
    """A CsView of a device tensor (absent view for None)."""
    v = CsView()
    if tensor is None:
        return v
    if tensor.ndim > 6:
        raise ValueError("views have at most 6 dimensions")
    nd = tensor.ndim
    # an empty tensor keeps its shape for validation with its data absent
    v.data = tensor.data_ptr() if tensor.numel() else None
    v.dtype = dtype_code(tensor.dtype)
    v.ndim = nd
    v.shape[:nd] = tensor.shape
    v.stride[:nd] = tensor.stride()
    return v


# CsView as bytes: data, dtype, ndim, shape[6], stride[6]
_VIEW = struct.Struct("<qii6q6q")
assert _VIEW.size == ctypes.sizeof(CsView)


def pack_view3(target, offset: int, tensor: torch.Tensor) -> None:
    """Write view(tensor) of a 3-d tensor into the CsView field of a ctypes
    structure at byte ``offset`` (one pack, for per-call argument blocks)."""
    s0, s1, s2 = tensor.shape
    r0, r1, r2 = tensor.stride()
    _VIEW.pack_into(target, offset, tensor.data_ptr() if s0 * s1 * s2 else 0, dtype_code(tensor.dtype), 3,
                    s0, s1, s2, 0, 0, 0, r0, r1, r2, 0, 0, 0)


def vref(tensor: torch.Tensor | None):
    return ctypes.byref(view(tensor))


def ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p:
    if tensor is None:
        return ctypes.c_void_p(None)
    return ctypes.c_void_p(tensor.data_ptr() if tensor.numel() else None)


def new_flags(device: torch.device, n: int = 1) -> torch.Tensor:
    # torch.zeros launches a fill kernel (no memset node under graph capture)
    return torch.zeros(n, dtype=torch.int32, device=device)


def read_flags(flags: torch.Tensor) -> list[int]:
    """Synchronising readback of a flag tensor."""
    return [int(x) for x in flags.cpu().tolist()]


def index_tensor(values, device: torch.device, name: str) -> torch.Tensor:
    """Host int list or int tensor -> contiguous int64 device tensor."""
    if isinstance(values, torch.Tensor):
        return values.to(device=device, dtype=torch.long).contiguous()
    return torch.tensor(list(values), dtype=torch.long, device=device)
