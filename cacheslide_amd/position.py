"""CoPE contextual positions and CCPE attention on the MI355X kernels.

Drop-in for src/cacheslide_vllm/position.py: the same names, signatures,
argument meaning and exception types/messages.  Every computation runs in
libcacheslide_hip.so; tensors must live on the HIP device.

Value checks that the reference performs with host-side ``.all()`` reductions
(nonfinite inputs, duplicate positions, invalid contextual paths) are computed
by kernels into a flag word; the host reads the word once per call and raises
the exception of the first failing check in the reference's order.
"""

from __future__ import annotations

import ctypes

import math
import re
from collections import Counter
from collections.abc import Callable, Sequence
from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor, nn

from . import _hip
from ._hip import call, ptr, vref

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


class CCPEPositionError(ValueError):
    """A canonical substitution does not define a valid contextual path."""


# --------------------------------------------------------------------------
# reference-ordered checks
# --------------------------------------------------------------------------
class _Checks:
    """Host checks raise in order, after any earlier device check that failed."""

    def __init__(self, device: torch.device):
        self.device = device
        self.flags = _hip.new_flags(device)
        self.steps: list[tuple[int, type, str]] = []

    def device_step(self, bits: int, exc: type, message: str) -> None:
        self.steps.append((bits, exc, message))

    def finish(self, pending: BaseException | None = None, value: int | None = None) -> None:
        """Raise the first registered device check that fired, then ``pending``;
        ``value``: the flags word already read after the last launch."""
        if value is None:
            value = _hip.read_flags(self.flags)[0] if self.steps else 0
        for bits, exc, message in self.steps:
            if value & bits:
                raise exc(message)
        if pending is not None:
            raise pending

    def fail(self, error: BaseException) -> None:
        self.finish(error)

    @property
    def flags_ptr(self):
        return ptr(self.flags)

    @property
    def stream(self):
        return _hip.stream_of(self.device)


def _device_of(tensor: Tensor) -> torch.device:
    if not isinstance(tensor, Tensor):
        raise ValueError("expected a tensor")
    return _hip.require_device(tensor)


def _finite_scan(ck: _Checks, tensor: Tensor, bit: int) -> None:
    call("cs_check_finite", vref(tensor), bit, ck.flags_ptr, ck.stream)


def _rows(name: str, tensor: Tensor, ck: _Checks, bit: int) -> None:
    """position.py:117-124: finite floating [token, head, dimension]."""
    message = f"{name} must be finite floating [token, head, dimension]"
    if (
        not isinstance(tensor, Tensor)
        or tensor.ndim != 3
        or not tensor.is_floating_point()
        or min(tensor.shape[1:]) < 1
    ):
        ck.fail(ValueError(message))
    if tensor.device != ck.device:
        return  # the caller's device-match check reports it
    _finite_scan(ck, tensor, bit)
    ck.device_step(bit, ValueError, message)


def _positions(
    name: str, tensor: Tensor, n: int, device: torch.device, ck: _Checks, is_key: bool,
    exc: type = ValueError,
) -> None:
    """position.py:127-137: nonnegative distinct int64 [n] on the device."""
    if (
        not isinstance(tensor, Tensor)
        or tensor.ndim != 1
        or tensor.shape[0] != n
        or tensor.dtype != torch.long
        or tensor.device != device
    ):
        ck.fail(exc(f"{name} must be nonnegative int64 [{n}] on {device}"))
    call("cs_check_positions", ptr(tensor), n, 1 if is_key else 0, ck.flags_ptr, ck.stream)
    neg = _hip.FLAG_KPOS_NEGATIVE if is_key else _hip.FLAG_QPOS_NEGATIVE
    dup = _hip.FLAG_KPOS_DUPLICATE if is_key else _hip.FLAG_QPOS_DUPLICATE
    ck.device_step(neg, exc, f"{name} must be nonnegative int64 [{n}] on {device}")
    ck.device_step(dup, exc, f"{name} must identify distinct token positions")


def _qk_layout(query: Tensor, key: Tensor, ck: _Checks) -> None:
    """position.py:140-150."""
    _rows("query", query, ck, _hip.FLAG_Q_NONFINITE)
    _rows("key", key, ck, _hip.FLAG_K_NONFINITE)
    if query.device != key.device or query.dtype != key.dtype:
        ck.fail(ValueError("Q/K dtype and device must match"))
    if query.shape[-1] != key.shape[-1]:
        ck.fail(ValueError("Q/K head dimensions must match"))
    if query.shape[1] % key.shape[1]:
        ck.fail(ValueError("query heads must be a multiple of KV heads for GQA"))
    if key.shape[0] == 0:
        ck.fail(ValueError("attention requires at least one key"))


def _accumulation_dtype(tensor: Tensor) -> torch.dtype:
    return torch.float64 if tensor.dtype == torch.float64 else torch.float32


def _mask_view(mask: Tensor | None, nq: int, nk: int) -> Tensor | None:
    """[q,k] / [1,q,k] / [H,q,k] bool -> a 3-d view (no copy)."""
    if mask is None:
        return None
    if mask.ndim == 2:
        return mask.unsqueeze(0)
    return mask


# --------------------------------------------------------------------------
# validate_contextual_path
# --------------------------------------------------------------------------
def validate_contextual_path(
    positions: Tensor,
    query_positions: Tensor,
    key_positions: Tensor,
    *,
    attention_mask: Tensor | None = None,
    atol: float = 1e-6,
) -> None:
    """Structural checks of a causal CoPE path (position.py:28-114).

    Valid cells are causal (key <= query coordinate) and enabled by the mask.
    With rounding = eps(dtype) * |p|: p >= -(atol + rounding); p <= (q - k + 1)
    + atol + rounding; adjacent valid pairs are nonincreasing within
    atol + both roundings and drop by at most the key gap plus that tolerance.
    """
    message = "positions must be finite floating [head,query,key]"
    if (
        not isinstance(positions, Tensor)
        or positions.ndim != 3
        or not positions.is_floating_point()
        or positions.shape[0] < 1
        or positions.shape[2] < 1
    ):
        raise CCPEPositionError(message)
    device = _device_of(positions)
    ck = _Checks(device)
    _finite_scan(ck, positions, _hip.FLAG_POS_NONFINITE)
    ck.device_step(_hip.FLAG_POS_NONFINITE, CCPEPositionError, message)
    if isinstance(atol, bool) or not isinstance(atol, (int, float)) or not math.isfinite(atol) or atol < 0:
        ck.fail(CCPEPositionError("atol must be finite and nonnegative"))
    for name, coordinates, size, is_key in (
        ("query_positions", query_positions, positions.shape[1], False),
        ("key_positions", key_positions, positions.shape[2], True),
    ):
        if not isinstance(coordinates, Tensor):
            ck.fail(CCPEPositionError(f"{name} must be an int64 tensor"))
        _positions(name, coordinates, size, device, ck, is_key, exc=CCPEPositionError)
    ck.device_step(_hip.FLAG_KPOS_UNSORTED, CCPEPositionError, "key_positions must be strictly increasing")
    if attention_mask is not None:
        if (
            not isinstance(attention_mask, Tensor)
            or attention_mask.dtype != torch.bool
            or attention_mask.device != device
            or attention_mask.shape
            not in (positions.shape[1:], (1, *positions.shape[1:]), positions.shape)
        ):
            ck.fail(CCPEPositionError("attention_mask must be bool [query,key] or [head,query,key]"))
    mask = _mask_view(attention_mask, positions.shape[1], positions.shape[2])
    call(
        "cs_validate_contextual_path", vref(positions), ptr(query_positions), ptr(key_positions),
        vref(mask), float(atol), ck.flags_ptr, ck.stream,
    )
    for bit, text in _PATH_MESSAGES:
        ck.device_step(bit, CCPEPositionError, text)
    ck.finish()


_PATH_MESSAGES = (
    (_hip.FLAG_PATH_NEGATIVE, "causal contextual positions must be nonnegative"),
    (_hip.FLAG_PATH_AVAILABLE, "causal contextual count exceeds available gates"),
    (_hip.FLAG_PATH_INCREASING, "causal contextual path must be nonincreasing"),
    (_hip.FLAG_PATH_GAP, "causal contextual path exceeds one gate per token"),
)


# --------------------------------------------------------------------------
# traces
# --------------------------------------------------------------------------
@dataclass(frozen=True)
class CoPEPositionTrace:
    """Detached positions from CoPE gates, with layout/checkpoint metadata.

    Built by ``CoPE.position_trace`` (position.py:196-272); tensors are copied
    to the host as in the reference, since traces feed offline calibration.
    """

    positions: Tensor
    masked_logits: Tensor
    allowed_mask: Tensor
    query_positions: Tensor
    key_positions: Tensor
    max_positions: int
    checkpoint_id: str
    source_query_indices: Tensor | None = None
    source_key_indices: Tensor | None = None

    def project(
        self,
        query_indices: Tensor,
        key_indices: Tensor,
        *,
        canonical_positions: bool = True,
    ) -> "CoPEPositionTrace":
        """Fixed-query x fixed-key sub-trace; canonical mode renumbers keys 0..F-1."""
        for name, indices, size in (
            ("query_indices", query_indices, self.positions.shape[1]),
            ("key_indices", key_indices, self.positions.shape[2]),
        ):
            values = indices.tolist() if isinstance(indices, Tensor) else None
            if (
                values is None
                or indices.ndim != 1
                or indices.dtype != torch.long
                or indices.device.type != "cpu"
                or any(v < 0 or v >= size for v in values)
                or len(set(values)) != len(values)
            ):
                raise ValueError(f"{name} must contain distinct valid CPU int64 indices")
        qsel = query_indices.tolist()
        ksel = key_indices.tolist()
        all_q = self.query_positions.tolist()
        all_k = self.key_positions.tolist()
        query_pos = [all_q[i] for i in qsel]
        key_pos = [all_k[i] for i in ksel]
        if any(b <= a for a, b in zip(key_pos, key_pos[1:])):
            raise ValueError("projected keys must retain causal token order")
        if canonical_positions:
            ordinal = {pos: index for index, pos in enumerate(key_pos)}
            if any(pos not in ordinal for pos in query_pos):
                raise ValueError("canonical query positions must belong to projected keys")
            query_pos = [ordinal[pos] for pos in query_pos]
            key_pos = list(range(len(ksel)))
        src_q = (
            self.source_query_indices.tolist()
            if self.source_query_indices is not None
            else list(range(self.positions.shape[1]))
        )
        src_k = (
            self.source_key_indices.tolist()
            if self.source_key_indices is not None
            else list(range(self.positions.shape[2]))
        )
        return CoPEPositionTrace(
            positions=self.positions[:, query_indices][:, :, key_indices].clone(),
            masked_logits=self.masked_logits,
            allowed_mask=self.allowed_mask,
            query_positions=torch.tensor(query_pos, dtype=torch.long),
            key_positions=torch.tensor(key_pos, dtype=torch.long),
            max_positions=self.max_positions,
            checkpoint_id=self.checkpoint_id,
            source_query_indices=torch.tensor([src_q[i] for i in qsel], dtype=torch.long),
            source_key_indices=torch.tensor([src_k[i] for i in ksel], dtype=torch.long),
        )


# --------------------------------------------------------------------------
# CoPE module
# --------------------------------------------------------------------------
class CoPE(nn.Module):
    """Learned contextual bias shared across heads; embeddings [dim, maxpos]."""

    def __init__(
        self,
        head_dim: int,
        max_positions: int,
        *,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> None:
        super().__init__()
        if head_dim < 1 or max_positions < 2:
            raise ValueError("head_dim must be positive and max_positions at least two")
        self.head_dim = head_dim
        self.max_positions = max_positions
        self.position_embeddings = nn.Parameter(
            torch.zeros(head_dim, max_positions, device=device, dtype=dtype)
        )

    def contextual_positions(self, logits: Tensor, allowed_mask: Tensor) -> Tensor:
        """Mask before sigmoid, reverse-cumsum over keys, clamp (position.py:295-307)."""
        if not isinstance(logits, Tensor) or logits.ndim != 3 or not logits.is_floating_point():
            raise ValueError("logits must be floating [head,query,key]")
        if allowed_mask.shape != logits.shape or allowed_mask.dtype != torch.bool:
            raise ValueError("allowed_mask must be bool with the logits shape")
        if allowed_mask.device != logits.device:
            raise ValueError("allowed_mask and logits must share a device")
        device = _device_of(logits)
        ck = _Checks(device)
        out = torch.empty(logits.shape, dtype=logits.dtype, device=device)
        call(
            "cs_contextual_positions", vref(logits), vref(allowed_mask), self.max_positions,
            vref(out), ck.flags_ptr, ck.stream,
        )
        ck.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError, "unmasked logits must be finite")
        ck.finish()
        return out

    def positional_bias(self, query: Tensor, positions: Tensor) -> Tensor:
        """Interpolate between floor(p) and its clamped right neighbour (position.py:309-344).

        bias = QE[floor p] + (p - floor p) * (QE[min(floor p + 1, P-1)] - QE[floor p])
        with QE = query . E in the accumulation dtype (unscaled query).
        """
        device = _device_of(query)
        ck = _Checks(device)
        _rows("query", query, ck, _hip.FLAG_Q_NONFINITE)
        if query.shape[-1] != self.head_dim:
            ck.fail(ValueError("query dimension does not match the learned embeddings"))
        if query.device != self.position_embeddings.device:
            ck.fail(ValueError("query and learned embeddings must share a device"))
        message = "positions must be bounded query-dependent [head,query,key]"
        if (
            not isinstance(positions, Tensor)
            or positions.ndim != 3
            or positions.shape[:2] != (query.shape[1], query.shape[0])
            or not positions.is_floating_point()
            or positions.device != query.device
        ):
            ck.fail(ValueError(message))
        call("cs_check_bias_positions", vref(positions), self.max_positions, ck.flags_ptr, ck.stream)
        ck.device_step(_hip.FLAG_POS_INVALID, ValueError, message)
        out = torch.empty(positions.shape, dtype=_accumulation_dtype(query), device=device)
        call(
            "cs_cope_positional_bias", vref(query), vref(self.position_embeddings.detach()),
            vref(positions), vref(out), ck.flags_ptr, ck.stream,
        )
        ck.finish()
        return out

    def forward(
        self,
        query: Tensor,
        key: Tensor,
        query_positions: Tensor,
        key_positions: Tensor | None = None,
        *,
        attention_mask: Tensor | None = None,
        fixed_positions: Tensor | None = None,
    ) -> Tensor:
        """Bias for every (head, query, key) cell (position.py:346-367)."""
        positions = (
            self._contextual(query, key, query_positions, key_positions, attention_mask)
            if fixed_positions is None
            else fixed_positions
        )
        if positions.shape != (query.shape[1], query.shape[0], key.shape[0]):
            raise ValueError("fixed_positions must exactly match [head,query,key]")
        return self.positional_bias(query, positions)

    def _contextual(self, query, key, query_positions, key_positions, attention_mask) -> Tensor:
        device = _device_of(query)
        ck = _Checks(device)
        _qk_layout(query, key, ck)
        _positions("query_positions", query_positions, query.shape[0], device, ck, False)
        if key_positions is None:
            key_positions = torch.arange(key.shape[0], device=device)
        _positions("key_positions", key_positions, key.shape[0], device, ck, True)
        ck.device_step(_hip.FLAG_KPOS_UNSORTED, ValueError,
                       "key_positions must be strictly increasing for reverse cumsum")
        mask = _checked_mask(attention_mask, query, key, ck)
        positions = torch.empty(
            (query.shape[1], query.shape[0], key.shape[0]), dtype=_accumulation_dtype(query),
            device=device,
        )
        args = _ccpe_args(query, key, key[:, :, :1], self.position_embeddings.detach(),
                          query_positions, key_positions, ck)
        args.attn_mask = _hip.view(mask)
        args.pos_out = _hip.view(positions)
        call("cs_ccpe_attention", args, ck.stream)
        ck.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError,
                       "attention logits overflowed the accumulation dtype")
        ck.finish()
        return positions

    def position_trace(
        self,
        query: Tensor,
        key: Tensor,
        query_positions: Tensor,
        key_positions: Tensor | None = None,
        *,
        checkpoint_id: str,
        attention_mask: Tensor | None = None,
        max_elements: int = 1_000_000,
    ) -> CoPEPositionTrace:
        """Explicitly bounded calibration trace (position.py:369-401)."""
        device = _device_of(query)
        ck = _Checks(device)
        _qk_layout(query, key, ck)
        ck.finish()
        if not checkpoint_id.strip():
            raise ValueError("a trained CoPE checkpoint identifier is required")
        if query.shape[1] * query.shape[0] * key.shape[0] > max_elements:
            raise ValueError("CoPE trace exceeds max_elements; use a smaller calibration")
        if key_positions is None:
            key_positions = torch.arange(key.shape[0], device=device)
        positions = self._contextual(query, key, query_positions, key_positions, attention_mask)
        ck = _Checks(device)
        logits = torch.empty(positions.shape, dtype=positions.dtype, device=device)
        call("cs_ccpe_logits", vref(query), vref(key), vref(logits), ck.flags_ptr, ck.stream)
        ck.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError,
                       "attention logits overflowed the accumulation dtype")
        ck.finish()
        allowed = _allowed_mask(query_positions, key_positions, attention_mask, query.shape[1])
        masked = logits.masked_fill(~allowed, -torch.inf)
        return CoPEPositionTrace(
            positions=positions.detach().cpu().clone(),
            masked_logits=masked.detach().cpu(),
            allowed_mask=allowed.detach().cpu().clone(),
            query_positions=query_positions.detach().cpu().clone(),
            key_positions=key_positions.detach().cpu().clone(),
            max_positions=self.max_positions,
            checkpoint_id=checkpoint_id,
        )


def _allowed_mask(query_positions, key_positions, attention_mask, heads) -> Tensor:
    """Causal & mask as a [H, q, k] bool tensor (position.py:180-192)."""
    causal = key_positions[None, :] <= query_positions[:, None]
    mask = causal.unsqueeze(0).expand(heads, -1, -1)
    if attention_mask is not None:
        mask = mask & _mask_view(attention_mask, 0, 0)
    return mask


def _checked_mask(attention_mask, query, key, ck: _Checks) -> Tensor | None:
    """The per-chunk mask checks of _allowed (position.py:182-192)."""
    if attention_mask is None:
        return None
    if attention_mask.dtype != torch.bool or attention_mask.device != query.device:
        ck.fail(ValueError("attention_mask must be bool on the query device"))
    mask = attention_mask
    if mask.shape == (query.shape[0], key.shape[0]):
        mask = mask.unsqueeze(0)
    if mask.shape not in ((1, query.shape[0], key.shape[0]), (query.shape[1], query.shape[0], key.shape[0])):
        ck.fail(ValueError("attention_mask must be [query,key] or [head,query,key]"))
    return mask


def _ccpe_args(query, key, value, e, query_positions, key_positions, ck: _Checks) -> _hip.CsCcpeArgs:
    args = _hip.CsCcpeArgs()
    args.q = _hip.view(query)
    args.k = _hip.view(key)
    args.v = _hip.view(value)
    args.e = _hip.view(e)
    args.qpos = ptr(query_positions)
    args.kpos = ptr(key_positions)
    args.flags = ck.flags_ptr
    args.chunk_rows = 1
    return args


# --------------------------------------------------------------------------
# cope_attention
# --------------------------------------------------------------------------
def cope_attention(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    cope: CoPE,
    query_positions: Tensor,
    key_positions: Tensor | None = None,
    *,
    attention_mask: Tensor | None = None,
    visibility_mask: Tensor | None = None,
    fixed_positions: Tensor | None = None,
    positions_transform: Callable[[Tensor, Tensor, Tensor], Tensor] | None = None,
    visibility_transform: Callable[[Tensor, Tensor], Tensor] | None = None,
    query_chunk_size: int = 128,
    return_positions: bool = False,
) -> Tensor | tuple[Tensor, Tensor]:
    """Causal/GQA CoPE attention (position.py:404-560) on the HIP kernels.

    Order per query row: causal gates -> positions (or fixed / transformed
    positions) -> learned bias -> visibility -> masked softmax -> P.V; rows
    with no visible key are zero.  ``CanonicalPositionPolicy`` and
    ``SelectedAssociationPolicy`` transforms are lowered to kernel data and run
    fused over all rows; any other callable is evaluated per query chunk on
    kernel-produced positions, as in the reference.
    """
    from .attention import CanonicalPositionPolicy, SelectedAssociationPolicy

    device = _device_of(query)
    ck = _Checks(device)
    _qk_layout(query, key, ck)
    _rows("value", value, ck, _hip.FLAG_V_NONFINITE)
    if value.shape[:2] != key.shape[:2] or value.device != key.device or value.dtype != key.dtype:
        ck.fail(ValueError("K/V token count, heads, dtype and device must match"))
    if not isinstance(query_chunk_size, int) or isinstance(query_chunk_size, bool) or query_chunk_size < 1:
        ck.fail(ValueError("query_chunk_size must be a positive integer"))
    if positions_transform is not None:
        if not callable(positions_transform):
            ck.fail(CCPEPositionError("positions_transform must be callable"))
        if fixed_positions is not None:
            ck.fail(CCPEPositionError("positions_transform and fixed_positions are mutually exclusive"))
    if visibility_transform is not None:
        if not callable(visibility_transform):
            ck.fail(ValueError("visibility_transform must be callable"))
        if visibility_mask is not None:
            ck.fail(ValueError("visibility_transform and visibility_mask are mutually exclusive"))
    nq, hq, nk = query.shape[0], query.shape[1], key.shape[0]
    _positions("query_positions", query_positions, nq, device, ck, False)
    default_keys = key_positions is None
    if default_keys:
        key_positions = torch.arange(nk, device=device)
    _positions("key_positions", key_positions, nk, device, ck, True)
    for name, mask in (("attention_mask", attention_mask), ("visibility_mask", visibility_mask)):
        if mask is not None and mask.shape not in ((nq, nk), (1, nq, nk), (hq, nq, nk)):
            ck.fail(ValueError(f"{name} has an incompatible full-query shape"))
    if fixed_positions is not None and fixed_positions.shape != (hq, nq, nk):
        ck.fail(ValueError("fixed_positions must be full query-dependent [head,query,key]"))
    # per-chunk checks of the reference, global here
    ck.device_step(_hip.FLAG_KPOS_UNSORTED, ValueError,
                   "key_positions must be strictly increasing for reverse cumsum")
    amask = _checked_mask(attention_mask, query, key, ck)
    e = cope.position_embeddings.detach()
    if e.device != device:
        ck.fail(ValueError("query and learned embeddings must share a device"))
    if nq == 0:
        ck.finish()
        output = torch.empty((0, hq, value.shape[2]), dtype=value.dtype, device=device)
        if return_positions:
            return output, torch.empty((hq, 0, nk), dtype=_accumulation_dtype(query), device=device)
        return output

    canonical = positions_transform if isinstance(positions_transform, CanonicalPositionPolicy) else None
    selected = visibility_transform if isinstance(visibility_transform, SelectedAssociationPolicy) else None
    generic_positions = positions_transform is not None and canonical is None
    generic_visibility = visibility_transform is not None and selected is None
    if generic_positions or generic_visibility:
        return _chunked_attention(
            query, key, value, cope, query_positions, key_positions, amask, visibility_mask,
            fixed_positions, positions_transform, visibility_transform, query_chunk_size,
            return_positions, ck,
        )

    if default_keys and _fast_path_ok(query, key, value, e, cope, amask, visibility_mask,
                                      fixed_positions, canonical, selected, return_positions):
        from .ccpe import _prefill_dense

        output = _prefill_dense(query, key, value, e, query_positions, ck)
        ck.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError,
                       "attention logits overflowed the accumulation dtype")
        ck.device_step(_hip.FLAG_SCORE_NONFINITE, ValueError, "contextual attention logits are not finite")
        ck.finish()
        return output

    if fixed_positions is not None:
        call("cs_check_bias_positions", vref(fixed_positions), cope.max_positions, ck.flags_ptr, ck.stream)

    output = torch.empty((nq, hq, value.shape[2]), dtype=value.dtype, device=device)
    trace = None
    if return_positions:
        trace_dtype = fixed_positions.dtype if fixed_positions is not None else _accumulation_dtype(query)
        trace = torch.empty((hq, nq, nk), dtype=trace_dtype, device=device)
    args = _ccpe_args(query, key, value, e, query_positions, key_positions, ck)
    args.attn_mask = _hip.view(amask)
    args.vis_mask = _hip.view(_mask_view(visibility_mask, nq, nk))
    args.fixed_pos = _hip.view(fixed_positions)
    args.out = _hip.view(output)
    args.pos_out = _hip.view(trace)
    keep = []
    chunk_flags = None
    lowered = None
    if canonical is not None:
        lowered = canonical._lower(device, query_positions, key_positions)
        if lowered.reason or not lowered.fits(hq):
            # A profile that does not match the plan is only an error when some
            # query row is fixed; it is never handed to the kernel.
            if lowered.any_fixed_row():
                ck.finish()
                lowered.raise_lookup_error()
                raise ValueError("CCPE profile shape does not match the fixed tokens and heads")
            canonical = None
    if canonical is not None:
        keep.append(lowered)
        args.canonical = _hip.view(lowered.canonical)
        args.q_ord = ptr(lowered.q_rows)
        args.k_ord = ptr(lowered.k_ord)
        args.strict = 1 if canonical.mode == "strict_contextual" else 0
        n_chunks = (nq + query_chunk_size - 1) // query_chunk_size
        # one word more: on the MFMA path the flags word is copied behind the
        # chunk flags, so one readback returns both
        chunk_buf = _hip.new_flags(device, n_chunks + 1)
        chunk_flags = chunk_buf[:n_chunks]
        args.chunk_rows = query_chunk_size
        args.chunk_flags = ptr(chunk_flags)
    if selected is not None:
        sel_rows, fixed_keys = selected._lower(device, query_positions, key_positions)
        keep += [sel_rows, fixed_keys]
        args.sel_rows = ptr(sel_rows)
        args.fixed_keys = ptr(fixed_keys)
    # The MFMA reuse-call path (a SelectedAssociationPolicy, a canonical
    # profile or both); the flags word it leaves (with the chunk flags, when
    # there are any) is read once here and serves every check below (one wait
    # for the device per call).
    flags_value = None
    chunk_values = None
    if ((selected is not None or canonical is not None) and default_keys
            and _policy_fast_ok(query, key, value, e, cope, amask, visibility_mask, fixed_positions,
                                return_positions, lowered if canonical is not None else None)
            and _policy_prefill(args, query, key, ck)):
        if chunk_flags is not None:
            chunk_buf[n_chunks:].copy_(ck.flags)
            values = _hip.read_flags(chunk_buf)
            flags_value, chunk_values = values[-1], values[:-1]
        else:
            flags_value = _hip.read_flags(ck.flags)[0]
        if flags_value & _hip.FLAG_POLICY_GENERIC:
            # more fixed/dynamic boundary keys than the path checker holds: the
            # generic kernel runs the call
            ck.flags.bitwise_and_(~_hip.FLAG_POLICY_GENERIC)
            if chunk_flags is not None:
                chunk_flags.zero_()
            flags_value = None
            chunk_values = None
            call("cs_ccpe_attention", args, ck.stream)
    else:
        call("cs_ccpe_attention", args, ck.stream)
    ck.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError, "attention logits overflowed the accumulation dtype")
    ck.device_step(_hip.FLAG_POS_INVALID, ValueError, "positions must be bounded query-dependent [head,query,key]")
    ck.device_step(_hip.FLAG_SCORE_NONFINITE, ValueError, "contextual attention logits are not finite")
    if chunk_flags is not None:
        _raise_policy_errors(ck, chunk_flags, lowered, flags_value, chunk_values)
    ck.finish(value=flags_value)
    if return_positions:
        return output, trace
    return output


_TRANSFORM_BOUNDS_MESSAGE = ("positions_transform must return bounded finite positions "
                             "with the contextual shape, dtype and device")


def _raise_policy_errors(ck: _Checks, chunk_flags: Tensor, lowered, flags_value: int | None = None,
                         values: list[int] | None = None) -> None:
    """In chunk order, the first chunk holding a fixed query row that fails:
    profile lookup, then the strict path checks, then the bounds of the
    substituted positions (position.py:485-516 with attention.py:32-57).
    ``values``: the chunk flags already read with the flags word."""
    from .attention import CHUNK_CANON_OUT_OF_RANGE, CHUNK_HAS_FIXED_ROW

    ck.finish(value=flags_value)
    if values is None:
        values = _hip.read_flags(chunk_flags)
    for value in values:
        if not value & CHUNK_HAS_FIXED_ROW:
            continue
        lowered.raise_lookup_error(value)
        for bit, text in _PATH_MESSAGES:      # strict validation inside the transform
            if value & bit:
                raise CCPEPositionError(text)
        if value & CHUNK_CANON_OUT_OF_RANGE:  # then the bounds check of its result
            raise CCPEPositionError(_TRANSFORM_BOUNDS_MESSAGE)


def _policy_fast_ok(query, key, value, e, cope, amask, visibility_mask, fixed_positions, return_positions,
                    lowered) -> bool:
    """The reuse call of runtime.py:576-609 on MFMA: the dense fast path's
    conditions with a SelectedAssociationPolicy, an fp32 profile or both."""
    if not _fast_path_ok(query, key, value, e, cope, amask, visibility_mask, fixed_positions, None, None,
                         return_positions):
        return False
    return lowered is None or lowered.canonical.dtype == torch.float32


def _policy_prefill(args, query: Tensor, key: Tensor, ck: _Checks) -> bool:
    """Launch cs_ccpe_prefill_policy_bf16 into args.out; False (nothing
    launched) for a layout it does not take.  A plan with more fixed/dynamic
    boundary keys than the path checker holds sets FLAG_POLICY_GENERIC: the
    caller then runs the generic kernel."""
    device = ck.device
    lib = _hip.load()
    nq, hq, nk = query.shape[0], query.shape[1], key.shape[0]
    need = int(lib.cs_ccpe_prefill_policy_workspace_bytes(nq, hq, nk))
    workspace = torch.empty(need + 256, dtype=torch.uint8, device=device)
    start = (-workspace.data_ptr()) % 256
    kpos = args.kpos
    args.kpos = None  # keys at their default coordinates 0..nk-1
    try:
        status = lib.cs_ccpe_prefill_policy_bf16(ctypes.byref(args), workspace.data_ptr() + start, need, ck.stream)
    finally:
        args.kpos = kpos
    if status == _hip.CS_EUNSUPPORTED:
        return False
    _hip.check(status, "cs_ccpe_prefill_policy_bf16")
    return True


def _fast_path_ok(query, key, value, e, cope, amask, visibility_mask, fixed_positions, canonical,
                  selected, return_positions) -> bool:
    """bf16, D = Dv = 128, default key coordinates, no masks/policies/traces."""
    if query.dtype != torch.bfloat16 or query.shape[2] != 128 or value.shape[2] != 128:
        return False
    if amask is not None or visibility_mask is not None or fixed_positions is not None:
        return False
    if canonical is not None or selected is not None or return_positions:
        return False
    if e.dtype != torch.float32 or not e.is_contiguous() or cope.max_positions > 128:
        return False
    for t in (query, key, value):
        if t.stride(2) != 1 or t.data_ptr() % 16 or t.stride(0) % 8 or t.stride(1) % 8:
            return False
    group = query.shape[1] // key.shape[1]
    return group in (1, 2, 4, 8, 16, 32)


def _chunked_attention(query, key, value, cope, query_positions, key_positions, amask,
                       visibility_mask, fixed_positions, positions_transform,
                       visibility_transform, chunk, return_positions, ck: _Checks):
    """Per-chunk evaluation with user callables (position.py:485-548)."""
    device = ck.device
    nq, hq, nk = query.shape[0], query.shape[1], key.shape[0]
    acc = _accumulation_dtype(query)
    e = cope.position_embeddings.detach()
    ck.finish()  # all pre-loop checks raise before any callable runs
    output = torch.empty((nq, hq, value.shape[2]), dtype=value.dtype, device=device)
    trace = None
    if return_positions:
        trace_dtype = fixed_positions.dtype if fixed_positions is not None else acc
        trace = torch.empty((hq, nq, nk), dtype=trace_dtype, device=device)
    if fixed_positions is not None:
        cc = _Checks(device)
        call("cs_check_bias_positions", vref(fixed_positions), cope.max_positions, cc.flags_ptr, cc.stream)
        fixed_flags = cc
    else:
        fixed_flags = None
    for start in range(0, nq, chunk):
        end = min(start + chunk, nq)
        q = query[start:end]
        qpos = query_positions[start:end]
        cmask = amask[:, start:end] if amask is not None else None
        cc = _Checks(device)
        positions = None
        if positions_transform is not None:
            contextual = torch.empty((hq, end - start, nk), dtype=acc, device=device)
            args = _ccpe_args(q, key, value, e, qpos, key_positions, cc)
            args.attn_mask = _hip.view(cmask)
            args.pos_out = _hip.view(contextual)
            call("cs_ccpe_attention", args, cc.stream)
            cc.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError,
                           "attention logits overflowed the accumulation dtype")
            cc.finish()
            transformed = positions_transform(contextual, qpos, key_positions)
            message = _TRANSFORM_BOUNDS_MESSAGE
            if (
                not isinstance(transformed, Tensor)
                or transformed.shape != contextual.shape
                or transformed.dtype != contextual.dtype
                or transformed.device != contextual.device
            ):
                raise CCPEPositionError(message)
            cc = _Checks(device)
            call("cs_check_bias_positions", vref(transformed), cope.max_positions, cc.flags_ptr, cc.stream)
            cc.device_step(_hip.FLAG_POS_INVALID, CCPEPositionError, message)
            cc.finish()
            positions = transformed
            cc = _Checks(device)
        elif fixed_positions is not None:
            positions = fixed_positions[:, start:end]
        vis = None
        if visibility_mask is not None:
            vis = _mask_view(visibility_mask, 0, 0)[:, start:end]
        elif visibility_transform is not None:
            vis = visibility_transform(qpos, key_positions)
            if not isinstance(vis, Tensor):
                raise ValueError("visibility_transform must return a bool tensor")
            vis = _checked_mask(vis, q, key, cc)
        args = _ccpe_args(q, key, value, e, qpos, key_positions, cc)
        args.attn_mask = _hip.view(cmask)
        args.vis_mask = _hip.view(vis)
        args.fixed_pos = _hip.view(positions)
        args.out = _hip.view(output[start:end])
        args.pos_out = _hip.view(trace[:, start:end] if trace is not None else None)
        call("cs_ccpe_attention", args, cc.stream)
        cc.device_step(_hip.FLAG_LOGIT_NONFINITE, ValueError, "attention logits overflowed the accumulation dtype")
        if fixed_flags is not None:
            fixed_flags.device_step(_hip.FLAG_POS_INVALID, ValueError,
                                    "positions must be bounded query-dependent [head,query,key]")
            fixed_flags.finish()
            fixed_flags = None
        cc.device_step(_hip.FLAG_POS_INVALID, ValueError, "positions must be bounded query-dependent [head,query,key]")
        cc.device_step(_hip.FLAG_SCORE_NONFINITE, ValueError, "contextual attention logits are not finite")
        cc.finish()
    if return_positions:
        return output, trace
    return output


# --------------------------------------------------------------------------
# CCPE profiles (position.py:563-748)
# --------------------------------------------------------------------------
@dataclass(frozen=True)
class ChunkIdentity:
    role: str
    content_hash: str
    length: int

    def __post_init__(self) -> None:
        if not self.role.strip() or not re.fullmatch(r"[0-9a-f]{64}", self.content_hash):
            raise ValueError("chunk needs a nonempty role and lowercase SHA-256 hash")
        if not isinstance(self.length, int) or isinstance(self.length, bool):
            raise ValueError("chunk length must be a positive integer")
        if self.length <= 0:
            raise ValueError("chunk length must be a positive integer")


@dataclass(frozen=True)
class CCPEProfile:
    """A bounded task profile tied to ordered chunks and a trained checkpoint."""

    trained_profile_version: str
    checkpoint_id: str
    chunks: tuple[ChunkIdentity, ...]
    query_positions: Tensor
    key_positions: Tensor
    canonical_positions: Tensor
    max_positions: int
    histogram_bin_width: float
    sample_count: int

    @classmethod
    def calibrate(
        cls,
        traces: Sequence[CoPEPositionTrace],
        chunks: Sequence[ChunkIdentity],
        *,
        trained_profile_version: str,
        histogram_bin_width: float = 0.25,
        max_elements: int = 1_000_000,
    ) -> "CCPEProfile":
        """The modal calibration sample (position.py:594-699).

        Every trace's positions are recomputed on the device from its masked
        logits and must agree within 1e-6; the samples are quantised to
        ``histogram_bin_width`` as whole joint patterns, and the first sample of
        the most frequent pattern (ties: the lexicographically smallest pattern)
        becomes the canonical table.  No pattern is assembled from per-cell modes.
        """
        first = _calibration_layout(traces, chunks, trained_profile_version, histogram_bin_width,
                                    max_elements)
        device = torch.device("cuda", torch.cuda.current_device())
        samples = [_verified_positions(trace, first, device) for trace in traces]
        return cls(
            trained_profile_version=trained_profile_version,
            checkpoint_id=first.checkpoint_id,
            chunks=tuple(chunks),
            query_positions=first.query_positions.detach().cpu().clone(),
            key_positions=first.key_positions.detach().cpu().clone(),
            canonical_positions=_modal_sample(samples, histogram_bin_width).clone(),
            max_positions=first.max_positions,
            histogram_bin_width=histogram_bin_width,
            sample_count=len(traces),
        )

    def lookup_reason(
        self,
        chunks: Sequence[ChunkIdentity],
        query_ordinals: Sequence[int] | None,
        key_positions: Tensor | None,
        checkpoint_id: str,
        trained_profile_version: str,
    ) -> str | None:
        """Why lookup would fail (position.py:718-737), or None; host metadata only."""
        if key_positions is None:
            expected_keys = list(range(sum(chunk.length for chunk in chunks)))
        else:
            expected_keys = key_positions.cpu().tolist()
        if tuple(chunks) != self.chunks:
            return "ordered chunk identities/lengths do not match CCPE profile"
        if checkpoint_id != self.checkpoint_id or trained_profile_version != self.trained_profile_version:
            return "trained checkpoint/profile version does not match"
        if expected_keys != self.key_positions.tolist():
            return "key positions do not match CCPE profile"
        if query_ordinals is not None:
            known = set(self.query_positions.tolist())
            if any(int(o) not in known for o in query_ordinals):
                return "CCPE profile has no contextual trace for these query positions"
        return None

    def lookup(
        self,
        chunks: Sequence[ChunkIdentity],
        query_positions: Tensor,
        key_positions: Tensor | None = None,
        *,
        checkpoint_id: str,
        trained_profile_version: str,
        strict: bool = True,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> Tensor | None:
        """Selected query rows [H, rows, F] of the canonical positions, or fail."""
        reason = self.lookup_reason(chunks, None, key_positions, checkpoint_id, trained_profile_version)
        if reason is None and (query_positions.ndim != 1 or query_positions.dtype != torch.long):
            reason = "query positions must be an int64 vector"
        if reason is None:
            reason = self.lookup_reason(chunks, query_positions.tolist(), key_positions,
                                        checkpoint_id, trained_profile_version)
        if reason:
            if strict:
                raise ValueError(reason)
            return None
        known = {pos: index for index, pos in enumerate(self.query_positions.tolist())}
        rows = [known[int(pos)] for pos in query_positions.tolist()]
        return self.canonical_positions[:, rows].to(
            device=device or query_positions.device,
            dtype=dtype or self.canonical_positions.dtype,
        )


def _calibration_layout(traces, chunks, version, bin_width, max_elements) -> CoPEPositionTrace:
    """Checks on the calibration set as a whole, in the reference's order; returns
    the first trace, whose layout every other trace must share."""
    if not traces or not version.strip():
        raise ValueError("calibration needs traces and a trained profile version")
    if not math.isfinite(bin_width) or bin_width <= 0:
        raise ValueError("histogram_bin_width must be finite and positive")
    first = traces[0]
    if not isinstance(first, CoPEPositionTrace):
        raise ValueError("calibration requires genuine CoPEPositionTrace inputs")
    if not chunks or sum(c.length for c in chunks) != first.key_positions.numel():
        raise ValueError("ordered chunk lengths must exactly match trace keys")
    elements = sum(t.positions.numel() + t.masked_logits.numel()
                   for t in traces if isinstance(t, CoPEPositionTrace))
    if elements > max_elements:
        raise ValueError("CCPE calibration exceeds max_elements")
    if first.positions.ndim != 3 or first.max_positions < 2:
        raise ValueError("invalid contextual trace dimensions")
    if not first.checkpoint_id.strip():
        raise ValueError("trace must identify a trained CoPE checkpoint")
    return first


def _verified_positions(trace, first: CoPEPositionTrace, device: torch.device) -> Tensor:
    """A trace's positions (host copy) once its layout matches ``first`` and the
    positions are what the CoPE gates give for its masked logits."""
    if not isinstance(trace, CoPEPositionTrace):
        raise ValueError("calibration requires genuine CoPEPositionTrace inputs")
    same_layout = (
        trace.positions.shape == first.positions.shape
        and trace.max_positions == first.max_positions
        and trace.checkpoint_id == first.checkpoint_id
        and torch.equal(trace.query_positions, first.query_positions)
        and torch.equal(trace.key_positions, first.key_positions)
    )
    if not same_layout:
        raise ValueError("calibration trace layout/checkpoint mismatch")
    logits, allowed = trace.masked_logits, trace.allowed_mask
    if (logits.ndim != 3 or logits.shape[0] != trace.positions.shape[0]
            or allowed.shape != logits.shape or allowed.dtype != torch.bool):
        raise ValueError("invalid masked contextual trace")
    expected = _trace_positions(trace, device)
    if expected is None:
        raise ValueError("invalid masked contextual trace")
    if trace.source_query_indices is not None:
        expected = expected[:, trace.source_query_indices.tolist()]
    if trace.source_key_indices is not None:
        expected = expected[:, :, trace.source_key_indices.tolist()]
    if expected.shape != trace.positions.shape:
        raise ValueError("projected trace source mapping has an invalid shape")
    if not _close(trace.positions, expected, device):
        raise ValueError("trace positions were not produced by CoPE gates")
    return trace.positions.detach().cpu()


def _modal_sample(samples: list[Tensor], bin_width: float) -> Tensor:
    """First sample of the most frequent quantised joint pattern; among equally
    frequent patterns the lexicographically smallest wins (position.py:676-688)."""
    counts: Counter[tuple[int, ...]] = Counter()
    first_seen: dict[tuple[int, ...], int] = {}
    for index, sample in enumerate(samples):
        pattern = _quantise(sample, bin_width)
        counts[pattern] += 1
        first_seen.setdefault(pattern, index)
    top = max(counts.values())
    winner = min(pattern for pattern, n in counts.items() if n == top)
    return samples[first_seen[winner]]


def _quantise(sample: Tensor, width: float) -> tuple[int, ...]:
    """The joint histogram key of a sample: each position divided by the bin
    width in the sample's own dtype (position.py:680-681 divides the fp32 or
    fp64 positions tensor by the Python width, so the quotient is rounded to
    that dtype), then rounded half to even."""
    flat = sample.detach().cpu().flatten()
    if flat.dtype in (torch.float32, torch.float64):
        values = flat.numpy()
        quotient = values / values.dtype.type(width)
    else:
        # reduced-precision positions: the quotient is formed in fp32 and
        # rounded back to the positions' dtype before the bin is taken
        quotient = (flat.float() / torch.tensor(width, dtype=torch.float32)).to(flat.dtype).float().numpy()
    return tuple(np.rint(quotient).astype(np.int64).tolist())


def _trace_positions(trace: CoPEPositionTrace, device: torch.device) -> Tensor | None:
    """Recompute a trace's positions from its masked logits on the device."""
    logits = trace.masked_logits.to(device)
    allowed = trace.allowed_mask.to(device)
    ck = _Checks(device)
    call("cs_check_finite", vref(trace.positions.to(device)), _hip.FLAG_POS_NONFINITE, ck.flags_ptr, ck.stream)
    clean = logits.masked_fill(~allowed, 0.0)
    call("cs_check_finite", vref(clean), _hip.FLAG_LOGIT_NONFINITE, ck.flags_ptr, ck.stream)
    out = torch.empty(logits.shape, dtype=logits.dtype, device=device)
    call("cs_contextual_positions", vref(logits), vref(allowed), trace.max_positions, vref(out),
         ck.flags_ptr, ck.stream)
    flags = _hip.read_flags(ck.flags)[0]
    if flags & (_hip.FLAG_POS_NONFINITE | _hip.FLAG_LOGIT_NONFINITE):
        return None
    # masked entries must be exactly -inf
    neg = logits.masked_fill(allowed, -torch.inf)
    if not bool(torch.isneginf(neg).all()):
        return None
    return out.cpu()


def _close(a: Tensor, b: Tensor, device: torch.device) -> bool:
    """|a - b| <= 1e-6 + 1e-6 |b| elementwise (torch.allclose atol = rtol = 1e-6)."""
    a_list = a.flatten().tolist()
    b_list = b.flatten().tolist()
    return all(abs(x - y) <= 1e-6 + 1e-6 * abs(y) for x, y in zip(a_list, b_list))
