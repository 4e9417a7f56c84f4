"""The C-ABI library loads on the CPU and exports every declared entry point.

No kernels are launched here (no GPU is needed to dlopen the library).
"""

import ctypes
import re
from pathlib import Path

import torch

from cacheslide_amd import _hip

HEADER = Path(__file__).resolve().parents[1] / "include" / "cacheslide_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(cs_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"cs_ccpe_attention", "cs_ccpe_prefill_bf16", "cs_ccpe_decode_bf16",
            "cs_slot_scatter", "cs_slot_gather", "cs_wca_promote"} <= names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    lib = _hip.load()
    for name in sorted(declared_symbols()):
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_binding_covers_every_declared_symbol():
    assert declared_symbols() == set(_hip.SIGNATURES)


def test_version_and_error_strings():
    lib = _hip.load()
    assert lib.cs_version().startswith(b"cacheslide_hip")
    assert isinstance(lib.cs_last_error(), bytes)


def test_argument_errors_need_no_device():
    # null arguments are rejected before any HIP call
    lib = _hip.load()
    status = lib.cs_ccpe_attention(None, None)
    assert status == _hip.CS_EINVAL
    assert b"null" in lib.cs_last_error()
    # per split: gate total and carry (f64), accumulator (128 f32), max, sum,
    # fixup-queue entry; plus the queue counter
    assert lib.cs_ccpe_decode_workspace_bytes(2, 4, 1000, 256) == 2 * 4 * 4 * (8 + 8 + 4 * 128 + 4 + 4)


def test_snapshot_entry_points_check_arguments_without_a_device():
    lib = _hip.load()
    buf = ctypes.create_string_buffer(16)
    assert lib.cs_copy_async(None, None, 0, _hip.COPY_H2D, None) == _hip.CS_OK   # nothing to move
    assert lib.cs_copy_async(buf, buf, -1, _hip.COPY_H2D, None) == _hip.CS_EINVAL
    assert lib.cs_copy_async(None, buf, 16, _hip.COPY_H2D, None) == _hip.CS_EINVAL
    assert lib.cs_copy_async(buf, buf, 16, 7, None) == _hip.CS_EINVAL
    assert b"copy kind" in lib.cs_last_error()
    flags = ctypes.c_int32(0)
    assert lib.cs_snapshot_convert(None, None, 1, ctypes.byref(flags), None) == _hip.CS_EINVAL
    ints = _hip.CsView()
    ints.data, ints.dtype, ints.ndim = ctypes.addressof(buf), _hip.CS_I32, 1
    ints.shape[0], ints.stride[0] = 4, 1
    assert lib.cs_snapshot_convert(ctypes.byref(ints), None, 1, ctypes.byref(flags), None) == _hip.CS_EINVAL
    assert b"floating point" in lib.cs_last_error()
    strided = _hip.CsView()
    strided.data, strided.dtype, strided.ndim = ctypes.addressof(buf), _hip.CS_BF16, 1
    strided.shape[0], strided.stride[0] = 4, 2
    assert lib.cs_snapshot_convert(ctypes.byref(strided), None, 1, ctypes.byref(flags), None) == _hip.CS_EINVAL
    assert b"contiguous" in lib.cs_last_error()


def test_wca_update_checks_arguments_without_a_device():
    lib = _hip.load()
    assert lib.cs_wca_update(None, None) == _hip.CS_EINVAL
    assert b"null" in lib.cs_last_error()
    args = _hip.CsWcaUpdateArgs()          # no status block
    assert lib.cs_wca_update(ctypes.byref(args), None) == _hip.CS_EINVAL
    assert ctypes.sizeof(_hip.CsWcaUpdateArgs) == 896   # the C struct's size on x86-64
    # clearing the status at the end (bit 1) needs a report word; refused
    # before any launch (host buffers stand in for the status block)
    block = (ctypes.c_int64 * 4)()
    args.flags, args.counts = ctypes.addressof(block), ctypes.addressof(block) + 8
    args.clear_status = 2
    assert lib.cs_wca_update(ctypes.byref(args), None) == _hip.CS_EINVAL
    assert b"report" in lib.cs_last_error()


def test_wca_update_argument_packs_match_the_ctypes_fields():
    """The update's per-call argument block is written by two struct packs;
    they must land exactly where the ctypes fields (the C layout) are."""
    t = torch.empty((5, 3, 16), dtype=torch.bfloat16)[:, 1:, :]  # strided view
    packed = _hip.CsWcaUpdateArgs()
    _hip.pack_view3(packed, _hip.CsWcaUpdateArgs.recomputed_v.offset, t)
    ref = _hip.view(t)
    got = packed.recomputed_v
    assert (got.data, got.dtype, got.ndim) == (ref.data, ref.dtype, ref.ndim)
    assert list(got.shape) == list(ref.shape) and list(got.stride) == list(ref.stride)
    empty = torch.empty((0, 2, 16), dtype=torch.float32)
    _hip.pack_view3(packed, _hip.CsWcaUpdateArgs.fused_k.offset, empty)
    assert packed.fused_k.data is None and list(packed.fused_k.shape[:3]) == [0, 2, 16]
    names = [name for name, _ in _hip.CsWcaUpdateArgs._fields_]
    tail = names[names.index("rows"):]
    values = list(range(1, len(tail) + 1))
    values[tail.index("epsilon")] = 0.25
    values[tail.index("threshold")] = 0.5
    _hip.WCA_UPDATE_TAIL.pack_into(packed, _hip.CsWcaUpdateArgs.rows.offset, *values)
    for name, value in zip(tail, values):
        assert getattr(packed, name) == value, name


def test_decode_refuses_a_small_workspace_without_a_device():
    """cs_ccpe_decode_bf16 checks workspace_bytes against the size its
    max_nk / split / batch / heads need before any launch (host pointers stand
    in for device buffers: nothing is dereferenced)."""
    lib = _hip.load()
    buf = ctypes.create_string_buffer(4096 + 16)
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    src = _hip.CsKvSource()
    src.cache, src.block_table = base, base
    src.s_block, src.s_head, src.s_offset, src.block_size = 4096, 4096, 256, 16
    src.num_blocks, src.bt_stride, src.bt_cols = 1, 1, 1
    need = lib.cs_ccpe_decode_workspace_bytes(2, 4, 1000, 256)
    args = [base, 512, 128, 2, 4, 1, base, 1000, ctypes.byref(src), base, 64, 256, base]
    tail = [base, base, None]
    assert lib.cs_ccpe_decode_bf16(*args, need - 1, *tail) == _hip.CS_EINVAL
    assert b"workspace holds" in lib.cs_last_error()
    # the slot form checks its sidecar alignment before any launch
    slot_src = _hip.CsKvSource()
    slot_src.cache, slot_src.slots = base, base
    slot_src.s_block, slot_src.s_head, slot_src.s_offset, slot_src.block_size = 4096, 4096, 256, 16
    slot_src.num_blocks, slot_src.side_rows = 1, 4
    slot_src.side_k, slot_src.side_v, slot_src.side_s_row, slot_src.side_s_head = base + 2, base, 128, 128
    args[8] = ctypes.byref(slot_src)
    # a slot map must state its width
    assert lib.cs_ccpe_decode_bf16(*args, need, *tail) == _hip.CS_EINVAL
    assert b"slot map needs at least one column" in lib.cs_last_error()
    slot_src.slots_cols = 1000
    assert lib.cs_ccpe_decode_bf16(*args, need, *tail) == _hip.CS_EINVAL
    assert b"sidecar rows must be 16-byte aligned" in lib.cs_last_error()


def test_prepare_device_reports_a_missing_device():
    """Without a HIP device the call returns an error status and names the
    failing runtime call instead of crashing (on a GPU host it succeeds)."""
    if torch.cuda.is_available():
        return
    lib = _hip.load()
    assert lib.cs_prepare_device() != _hip.CS_OK
    assert lib.cs_last_error()
