"""CCPE coordinate and WCA visibility policies (src/cacheslide_vllm/attention.py:18-72).

Both policies keep the reference's callable interface, evaluated by kernels.
``cope_attention`` recognises them and lowers them to kernel data instead of
calling them per query chunk:

* CanonicalPositionPolicy -> per-row profile row index, per-key fixed ordinal,
  the profile's canonical [H, F, F] tensor and the strict-validation switch;
* SelectedAssociationPolicy -> per-row "selected" and per-key "fixed" flags.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import Tensor

from . import _hip
from ._hip import call, ptr, vref
from .contracts import RequestPlan
from .position import ChunkIdentity, validate_contextual_path


CHUNK_HAS_FIXED_ROW = 1 << 30   # kernel chunk flag: the chunk holds a fixed query row
CHUNK_UNKNOWN_ROW = 1 << 29     # ... one whose ordinal the profile has no trace for
CHUNK_CANON_OUT_OF_RANGE = 1 << 28  # a substituted canonical cell outside [0, P-1]


_FIXED_CACHE: dict[int, tuple] = {}


def _fixed_positions(fixed: tuple[int, ...]) -> Tensor:
    """The plan's fixed positions as a CPU int64 tensor (ascending, as the plan
    lists them), cached per tuple: the runtime reuses one plan for every layer."""
    hit = _FIXED_CACHE.get(id(fixed))
    if hit is not None and hit[0] is fixed:
        return hit[1]
    tensor = torch.tensor(fixed, dtype=torch.long)
    if len(_FIXED_CACHE) >= 8:
        _FIXED_CACHE.clear()
    _FIXED_CACHE[id(fixed)] = (fixed, tensor)
    return tensor


_FIXED_DEVICE: dict[tuple, tuple] = {}


def _fixed_on(fixed: tuple[int, ...], device) -> Tensor:
    """The plan's fixed positions sorted on ``device`` (read only), cached per
    tuple and device like ``_fixed_positions``: one host-to-device copy and
    sort per plan, not per call."""
    key = (id(fixed), str(device))
    hit = _FIXED_DEVICE.get(key)
    if hit is not None and hit[0] is fixed:
        return hit[1]
    tensor = torch.sort(_fixed_positions(fixed).to(device)).values
    if len(_FIXED_DEVICE) >= 8:
        _FIXED_DEVICE.clear()
    _FIXED_DEVICE[key] = (fixed, tensor)
    return tensor


def _memo_of(profile, fallback: dict) -> dict:
    """A memo dict kept on the profile object (immutable calibration data),
    or ``fallback`` for a profile that takes no attributes."""
    memo = getattr(profile, "__dict__", {}).get("_lowering_memo")
    if memo is None:
        memo = {}
        try:
            object.__setattr__(profile, "_lowering_memo", memo)
        except (AttributeError, TypeError):
            return fallback
    return memo


def _policy_tables(policy: "CanonicalPositionPolicy", device) -> tuple:
    """Position -> profile row and position -> fixed ordinal tables on the
    device (-1 where the position is not fixed; a fixed ordinal the profile
    never traced maps to -2, a repeated one to its last row), with the
    untraced flag, the profile's row count, the fixed count and the reason
    profile.lookup would refuse the plan (None when it accepts it)."""
    fixed = _fixed_positions(policy.plan.fixed_indices)
    count = fixed.numel()
    profile = policy.profile
    traced = profile.query_positions.detach().to("cpu", torch.long).reshape(-1)
    size = int(fixed.max()) + 1 if count else 1
    rows_of = torch.full((count,), -2, dtype=torch.long)
    inside = (traced >= 0) & (traced < count)
    if count and bool(inside.any()):
        rows_of.scatter_reduce_(0, traced[inside], torch.arange(traced.numel())[inside], reduce="amax",
                                include_self=False)
    q_table = torch.full((size,), -1, dtype=torch.long)
    k_table = torch.full((size,), -1, dtype=torch.long)
    if count:
        q_table[fixed] = rows_of
        k_table[fixed] = torch.arange(count)
    chunks = tuple(ChunkIdentity(*entry) for entry in policy.plan.fixed_layout)
    reason = profile.lookup_reason(chunks, None, None, policy.checkpoint_id, profile.trained_profile_version)
    return (q_table.to(device), k_table.to(device), size, bool((rows_of == -2).any()),
            int(torch.unique(traced).numel()), count, reason)


class _LoweredCanonical:
    """Kernel inputs for one CanonicalPositionPolicy over one call's coordinates."""

    def __init__(self, policy: "CanonicalPositionPolicy", device, query_positions, key_positions):
        # the call-independent part (position -> profile row / fixed ordinal
        # tables, the profile lookup's decision) once per profile, plan and
        # device: the runtime builds a new policy per call around the same
        # profile and plan
        fixed = policy.plan.fixed_indices
        cache = _memo_of(policy.profile, policy._device_cache)
        key = ("tables", id(fixed), policy.checkpoint_id, str(device))
        hit = cache.get(key)
        if hit is None or hit[0] is not fixed:
            hit = cache[key] = (fixed, _policy_tables(policy, device))
        q_dev, k_dev, size, self.unknown, self.profile_rows, self.fixed_count, self.reason = hit[1]
        self.q_rows = torch.empty(query_positions.shape[0], dtype=torch.long, device=device)
        self.k_ord = torch.empty(key_positions.shape[0], dtype=torch.long, device=device)
        stream = _hip.stream_of(device)
        call("cs_mapping_gather", ptr(q_dev), size, ptr(query_positions), ptr(self.q_rows),
             query_positions.shape[0], stream)
        call("cs_mapping_gather", ptr(k_dev), size, ptr(key_positions), ptr(self.k_ord),
             key_positions.shape[0], stream)
        self._tables = (q_dev, k_dev)
        self.canonical = policy._canonical_on(device)

    def fits(self, heads: int) -> bool:
        """The canonical tensor covers every (head, profile row, fixed ordinal) the kernel reads."""
        c = self.canonical
        return (
            c.ndim == 3
            and c.shape[0] == heads
            and c.shape[1] == self.profile_rows
            and c.shape[2] >= self.fixed_count
        )

    def any_fixed_row(self) -> bool:
        return bool((self.q_rows != -1).any().item())

    def raise_lookup_error(self, chunk_bits: int | None = None) -> None:
        """The ValueError profile.lookup raises for a chunk with fixed rows
        (position.py:718-738): a plan/profile mismatch for any such chunk, an
        untraced query ordinal only for a chunk that holds one (kernel chunk
        bit 29; without chunk bits, any row of the call)."""
        if self.reason:
            raise ValueError(self.reason)
        if chunk_bits is None:
            untraced = self.unknown and -2 in self.q_rows.cpu().tolist()
        else:
            untraced = bool(chunk_bits & CHUNK_UNKNOWN_ROW)
        if untraced:
            raise ValueError("CCPE profile has no contextual trace for these query positions")


@dataclass(frozen=True)
class CanonicalPositionPolicy:
    """Replace fixed-query x fixed-key positions with calibrated profile values.

    ``strict_contextual`` validates the hybrid path (validate_contextual_path)
    and raises CCPEPositionError; ``mixed_bias_override`` does not check.
    """

    plan: RequestPlan
    profile: object
    checkpoint_id: str
    mode: str = "strict_contextual"
    _device_cache: dict = field(default_factory=dict, compare=False, repr=False)

    def __post_init__(self):
        if not isinstance(self.mode, str) or self.mode not in {
            "strict_contextual",
            "mixed_bias_override",
        }:
            raise ValueError("unknown CCPE position policy")

    def _canonical_on(self, device) -> Tensor:
        cache = _memo_of(self.profile, self._device_cache)
        key = ("canonical", str(device))
        if key not in cache:
            cache[key] = self.profile.canonical_positions.to(device)
        return cache[key]

    def _lower(self, device, query_positions: Tensor, key_positions: Tensor) -> _LoweredCanonical:
        return _LoweredCanonical(self, device, query_positions, key_positions)

    def __call__(self, contextual: Tensor, queries: Tensor, keys: Tensor) -> Tensor:
        """attention.py:32-57: substitute, then validate in strict mode."""
        ordinal = {position: i for i, position in enumerate(self.plan.fixed_indices)}
        query_list = queries.tolist()
        rows = [i for i, p in enumerate(query_list) if p in ordinal]
        if not rows:
            return contextual
        chunks = tuple(ChunkIdentity(*entry) for entry in self.plan.fixed_layout)
        canonical = self.profile.lookup(
            chunks,
            torch.tensor([ordinal[query_list[i]] for i in rows]),
            checkpoint_id=self.checkpoint_id,
            trained_profile_version=self.profile.trained_profile_version,
            device=contextual.device,
            dtype=contextual.dtype,
        )
        key_list = keys.tolist()
        columns = [i for i, p in enumerate(key_list) if p in ordinal]
        device = _hip.require_device(contextual)
        result = contextual.clone()
        if columns:
            row_idx = torch.tensor(rows, dtype=torch.long, device=device)
            row_ord = torch.arange(len(rows), dtype=torch.long, device=device)
            col_idx = torch.tensor(columns, dtype=torch.long, device=device)
            col_ord = torch.tensor([ordinal[key_list[i]] for i in columns], dtype=torch.long,
                                   device=device)
            call("cs_canonical_substitute", vref(result), vref(canonical), ptr(row_idx),
                 ptr(row_ord), len(rows), ptr(col_idx), ptr(col_ord), len(columns),
                 _hip.stream_of(device))
        if self.mode == "strict_contextual":
            validate_contextual_path(result, queries, keys)
        elif self.mode != "mixed_bias_override":
            raise ValueError("unknown CCPE position policy")
        return result


@dataclass(frozen=True)
class SelectedAssociationPolicy:
    """visible(q, k) = not selected(q) or not fixed(k) or q == k (attention.py:60-72)."""

    fixed_indices: tuple[int, ...]
    selected_indices: Tensor

    def _sets(self, device) -> tuple[Tensor, Tensor]:
        """Fixed and selected positions on the device, each sorted ascending
        (the kernels test membership by binary search)."""
        fixed_indices = self.fixed_indices
        if not isinstance(fixed_indices, tuple):
            fixed_indices = tuple(fixed_indices)
        fixed = _fixed_on(fixed_indices, device)
        selected = self.selected_indices.to(device=device, dtype=torch.long).reshape(-1)
        return fixed, torch.sort(selected).values

    def _lower(self, device, query_positions: Tensor, key_positions: Tensor) -> tuple[Tensor, Tensor]:
        fixed, selected = self._sets(device)
        sel_rows = torch.empty(query_positions.shape[0], dtype=torch.uint8, device=device)
        fixed_keys = torch.empty(key_positions.shape[0], dtype=torch.uint8, device=device)
        stream = _hip.stream_of(device)
        call("cs_isin", ptr(query_positions), query_positions.shape[0], ptr(selected),
             selected.numel(), ptr(sel_rows), stream)
        call("cs_isin", ptr(key_positions), key_positions.shape[0], ptr(fixed), fixed.numel(),
             ptr(fixed_keys), stream)
        return sel_rows, fixed_keys

    def __call__(self, queries: Tensor, keys: Tensor) -> Tensor:
        device = _hip.require_device(queries, keys)
        fixed, selected = self._sets(device)
        nq, nk = queries.shape[0], keys.shape[0]
        buffer = torch.empty(nq * nk + nq + nk, dtype=torch.uint8, device=device)
        q = queries.to(torch.long).contiguous()
        k = keys.to(torch.long).contiguous()
        call("cs_selected_visibility", ptr(q), nq, ptr(k), nk, ptr(fixed), fixed.numel(),
             ptr(selected), selected.numel(), ptr(buffer), _hip.stream_of(device))
        return buffer[: nq * nk].view(torch.bool).view(nq, nk)
