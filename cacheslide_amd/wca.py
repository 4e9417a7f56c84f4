"""Request-local weighted cache adaptation (src/cacheslide_vllm/wca.py) on the HIP kernels.

Tokens are indexed in assembled-prompt order; K/V tensors are [token, head,
dimension] on the HIP device; layer numbers are one based.  All arithmetic
is fp64 in the kernels: per-token squared deviations and norms are exact
(correctly rounded) sums, and the blend ``w * new + (1 - w) * old`` rounds
exactly where the reference's separate tensor operations round.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _hip
from ._hip import call, ptr, vref
from .policy import WCAConfig, _finite_number


class WCANumericalError(ValueError):
    """Nonfinite WCA data or arithmetic; the caller may fall back to full prefill.

    Shape, policy and call-order violations remain plain ValueError.
    """


class _Flags:
    def __init__(self, device):
        self.device = device
        self.tensor = _hip.new_flags(device)
        self.steps: list[tuple[int, type, str]] = []

    @property
    def ptr(self):
        return ptr(self.tensor)

    @property
    def stream(self):
        return _hip.stream_of(self.device)

    def step(self, bits: int, exc: type, message: str) -> None:
        self.steps.append((bits, exc, message))

    def finish(self, pending: BaseException | None = None) -> None:
        value = _hip.read_flags(self.tensor)[0] if self.steps else 0
        for bits, exc, message in self.steps:
            if value & bits:
                raise exc(message)
        if pending is not None:
            raise pending


_NONFINITE_BIT = {"cached_k": 1 << 20, "recomputed_k": 1 << 21, "cached_v": 1 << 22,
                  "recomputed_v": 1 << 23, "a": 1 << 20, "b": 1 << 21}


def _kv(name: str, tensor: Tensor, fl: _Flags) -> None:
    """wca.py:31-37."""
    if not isinstance(tensor, Tensor) or tensor.ndim != 3 or not tensor.is_floating_point():
        fl.finish(ValueError(f"{name} must be floating [token, head, dimension]"))
    if min(tensor.shape[1:]) < 1:
        fl.finish(ValueError(f"{name} must have nonempty heads/dimension"))
    bit = _NONFINITE_BIT[name]
    call("cs_check_finite", vref(tensor), bit, fl.ptr, fl.stream)
    fl.step(bit, WCANumericalError, f"{name} must have finite values")


def _matching(name: str, tensor: Tensor, reference_shape, reference: Tensor, fl: _Flags) -> None:
    """wca.py:40-47: same shape, dtype and device as the reference rows."""
    if not isinstance(tensor, Tensor) or (tensor.shape, tensor.dtype, tensor.device) != (
        reference_shape,
        reference.dtype,
        reference.device,
    ):
        fl.finish(ValueError(f"{name} shape, dtype and device must match its reference"))
    _kv(name, tensor, fl)


def _mask(name: str, tensor: Tensor, n: int, device) -> None:
    if tensor.shape != (n,) or tensor.dtype != torch.bool or tensor.device != device:
        raise ValueError(f"{name} must be a bool [{n}] tensor on {device}")


def _score(old: Tensor, fresh: Tensor, rows: Tensor | None, fl: _Flags) -> tuple[Tensor, Tensor]:
    n = fresh.shape[0]
    err = torch.empty(n, dtype=torch.float64, device=fresh.device)
    norm = torch.empty(n, dtype=torch.float64, device=fresh.device)
    call("cs_wca_score", vref(old), ptr(rows), vref(fresh), ptr(err), ptr(norm), fl.ptr, fl.stream)
    return err, norm


def _epsilon(epsilon) -> None:
    _finite_number("epsilon", epsilon)
    if epsilon <= 0:
        raise ValueError("epsilon must be finite and positive")


def squared_deviation(cached_k: Tensor, recomputed_k: Tensor) -> Tensor:
    """err[t] = sum over heads and dims of (recomputed - cached)^2, fp64 (wca.py:55-62)."""
    fl = _Flags(_hip.require_device(cached_k))
    _kv("cached_k", cached_k, fl)
    _matching("recomputed_k", recomputed_k, cached_k.shape, cached_k, fl)
    err, _ = _score(cached_k, recomputed_k, None, fl)
    fl.step(2, WCANumericalError, "squared deviation overflowed float64")
    fl.finish()
    return err


def _alpha(err, norm, epsilon, clamp, fl: _Flags) -> Tensor:
    alpha = torch.empty_like(err)
    call("cs_wca_alpha", ptr(err), ptr(norm), err.numel(), float(epsilon), 1 if clamp else 0,
         ptr(alpha), fl.ptr, fl.stream)
    fl.step(2 | 16, WCANumericalError, "adaptation weight overflowed float64")
    fl.step(4, WCANumericalError, "adaptation weight overflowed; inspect the K magnitudes")
    return alpha


def adaptation_weight(
    cached_k: Tensor,
    recomputed_k: Tensor,
    *,
    epsilon: float = 1e-8,
    clamp: bool = False,
) -> Tensor:
    """alpha = ||K_new - K_cache||^2 / (||K_cache||^2 + epsilon) per token (wca.py:65-93)."""
    fl = _Flags(_hip.require_device(cached_k))
    _kv("cached_k", cached_k, fl)
    _matching("recomputed_k", recomputed_k, cached_k.shape, cached_k, fl)
    try:
        _epsilon(epsilon)
        if type(clamp) is not bool:
            raise ValueError("clamp must be a boolean")
    except ValueError as error:
        fl.finish(error)
    err, norm = _score(cached_k, recomputed_k, None, fl)
    alpha = _alpha(err, norm, epsilon, clamp, fl)
    fl.finish()
    return alpha


def mean_head_cosine(a: Tensor, b: Tensor, *, epsilon: float = 1e-8) -> Tensor:
    """Mean over heads of the clamped cosine of amax-scaled rows (wca.py:96-112)."""
    fl = _Flags(_hip.require_device(a))
    _kv("a", a, fl)
    _matching("b", b, a.shape, a, fl)
    try:
        _epsilon(epsilon)
    except ValueError as error:
        fl.finish(error)
    fl.finish()
    out = torch.empty(a.shape[0], dtype=torch.float64, device=a.device)
    call("cs_wca_head_cosine", vref(a), vref(b), ptr(None), float(epsilon), ptr(out), fl.stream)
    return out


@dataclass(frozen=True)
class WCAUpdate:
    """Corrected current-layer rows and selection changes for the next layer."""

    indices: Tensor
    fused_k: Tensor
    fused_v: Tensor
    alpha: Tensor
    removed_indices: Tensor
    promoted_indices: Tensor
    next_indices: Tensor


def _nonzero(a: Tensor, b: Tensor | None) -> Tensor:
    """Ascending indices of a | b on the device (one readback for the count)."""
    n = a.numel()
    out = torch.empty(max(n, 1), dtype=torch.long, device=a.device)
    count = torch.zeros(1, dtype=torch.long, device=a.device)
    call("cs_mask_nonzero", ptr(a), ptr(b), n, ptr(out), ptr(count), _hip.stream_of(a.device))
    return out[: int(count.item())]


@dataclass
class WCAState:
    """Per-request WCA state (wca.py:128-304); masks are device bool tensors."""

    config: WCAConfig
    reused_mask: Tensor
    mandatory_mask: Tensor
    initial_deviation: Tensor
    candidate_mask: Tensor
    selected_mask: Tensor
    removed_mask: Tensor
    alpha: Tensor
    budget: int
    last_layer: int = 1

    @classmethod
    def initialize(
        cls,
        cached_k: Tensor,
        recomputed_k: Tensor,
        reused_mask: Tensor,
        mandatory_mask: Tensor,
        config: WCAConfig | None = None,
    ) -> "WCAState":
        config = config or WCAConfig()
        device = _hip.require_device(cached_k)
        fl = _Flags(device)
        _kv("cached_k", cached_k, fl)
        _matching("recomputed_k", recomputed_k, cached_k.shape, cached_k, fl)
        err, norm = _score(cached_k, recomputed_k, None, fl)
        fl.step(2, WCANumericalError, "squared deviation overflowed float64")
        n = cached_k.shape[0]
        try:
            _mask("reused_mask", reused_mask, n, device)
            _mask("mandatory_mask", mandatory_mask, n, device)
        except ValueError as error:
            fl.finish(error)
        candidate = torch.empty(n, dtype=torch.bool, device=device)
        counts = torch.zeros(2, dtype=torch.long, device=device)
        call("cs_wca_init_masks", ptr(err), ptr(reused_mask), ptr(mandatory_mask), n,
             ptr(candidate), ptr(counts), fl.ptr, fl.stream)
        fl.step(32, ValueError, "every dynamic/non-reused token must be mandatory")
        alpha = _alpha(err, norm, config.epsilon, config.clamp_alpha, fl)
        fl.finish()
        n_reused, n_candidates = (int(x) for x in counts.cpu().tolist())
        budget = min(math.ceil(config.correction_fraction * n_reused), n_candidates)
        state = cls(
            config=config,
            reused_mask=reused_mask.clone(),
            mandatory_mask=mandatory_mask.clone(),
            initial_deviation=err,
            candidate_mask=candidate,
            selected_mask=torch.zeros(n, dtype=torch.bool, device=device),
            removed_mask=torch.zeros(n, dtype=torch.bool, device=device),
            alpha=alpha,
            budget=budget,
        )
        state._promote()
        return state

    @property
    def active_indices(self) -> Tensor:
        """Sorted global token indices to compute at the next layer."""
        return _nonzero(self.selected_mask, self.mandatory_mask)

    @property
    def selected_indices(self) -> Tensor:
        return _nonzero(self.selected_mask, None)

    def _promote(self) -> Tensor:
        """Fill the budget with the largest initial deviations, ties to lower index."""
        n = self.selected_mask.numel()
        device = self.selected_mask.device
        scratch = torch.empty(max(n, 1), dtype=torch.long, device=device)
        promoted = torch.empty(max(n, 1), dtype=torch.long, device=device)
        count = torch.zeros(1, dtype=torch.long, device=device)
        call("cs_wca_promote", ptr(self.initial_deviation), ptr(self.candidate_mask),
             ptr(self.removed_mask), ptr(self.selected_mask), n, self.budget, ptr(scratch),
             ptr(promoted), ptr(count), _hip.stream_of(device))
        return promoted[: int(count.item())]

    def update(
        self,
        layer_index: int,
        cached_k: Tensor,
        cached_v: Tensor,
        recomputed_k: Tensor,
        recomputed_v: Tensor,
        computed_indices: Tensor | None = None,
    ) -> WCAUpdate:
        """Fuse sparse recomputed rows against the full current-layer cache (wca.py:217-304)."""
        if layer_index != self.last_layer + 1:
            raise ValueError("layers must update consecutively after full layer one")
        device = _hip.require_device(cached_k)
        fl = _Flags(device)
        _kv("cached_k", cached_k, fl)
        _matching("cached_v", cached_v, cached_k.shape, cached_k, fl)
        if cached_k.shape[0] != self.reused_mask.numel():
            fl.finish(ValueError("cache token count differs from the request"))
        if cached_k.device != self.reused_mask.device:
            fl.finish(ValueError("cache device differs from the request"))
        indices = self.active_indices
        if computed_indices is not None:
            if (
                computed_indices.dtype != torch.long
                or computed_indices.device != indices.device
                or computed_indices.cpu().tolist() != indices.cpu().tolist()
            ):
                fl.finish(ValueError("computed_indices must equal sorted active_indices"))
        a = indices.numel()
        rows_shape = (a, *cached_k.shape[1:])
        _matching("recomputed_k", recomputed_k, rows_shape, cached_k, fl)
        _matching("recomputed_v", recomputed_v, rows_shape, cached_v, fl)
        err, norm = _score(cached_k, recomputed_k, indices, fl)
        next_alpha = _alpha(err, norm, self.config.epsilon, self.config.clamp_alpha, fl)
        used = torch.empty(a, dtype=torch.float64, device=device)
        call("cs_wca_used_alpha", ptr(self.alpha), ptr(next_alpha), ptr(indices),
             ptr(self.mandatory_mask), a, 1 if self.config.weight_update == "previous_layer" else 0,
             ptr(used), fl.stream)
        fused_k = torch.empty(rows_shape, dtype=cached_k.dtype, device=device)
        fused_v = torch.empty(rows_shape, dtype=cached_v.dtype, device=device)
        call("cs_wca_blend", vref(cached_k), vref(cached_v), ptr(indices), vref(recomputed_k),
             vref(recomputed_v), ptr(used), ptr(None), vref(fused_k), vref(fused_v), fl.ptr,
             fl.stream)
        fl.step(8, WCANumericalError, "weighted K/V overflowed the cache dtype")

        removed = indices[:0]
        if layer_index % self.config.gate_interval == 0 and a:
            cosine = torch.empty(a, dtype=torch.float64, device=device)
            call("cs_wca_head_cosine", vref(recomputed_k), vref(cached_k), ptr(indices),
                 float(self.config.epsilon), ptr(cosine), fl.stream)
            removed_buf = torch.empty(a, dtype=torch.long, device=device)
            count = torch.zeros(1, dtype=torch.long, device=device)
            call("cs_wca_gate", ptr(cosine), ptr(indices), ptr(self.selected_mask), a,
                 1 if self.config.convergence_mode == "distance_lt" else 0,
                 float(self.config.convergence_threshold), ptr(removed_buf), ptr(count), fl.stream)
            fl.finish()  # nothing is committed before the numeric checks pass
            removed = removed_buf[: int(count.item())]
        else:
            fl.finish()
        call("cs_wca_commit", ptr(self.alpha), ptr(next_alpha), ptr(indices), a, ptr(removed),
             removed.numel(), ptr(self.selected_mask), ptr(self.candidate_mask),
             ptr(self.removed_mask), fl.stream)
        promoted = self._promote()
        self.last_layer = layer_index
        return WCAUpdate(
            indices=indices,
            fused_k=fused_k,
            fused_v=fused_v,
            alpha=used,
            removed_indices=removed,
            promoted_indices=promoted,
            next_indices=self.active_indices,
        )
