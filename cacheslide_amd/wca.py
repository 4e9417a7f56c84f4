"""Request-local weighted cache adaptation (src/cacheslide_vllm/wca.py) on the HIP kernels.

Tokens are indexed in assembled-prompt order; K/V tensors are [token, head,
dimension] on the HIP device; layer numbers are one based.  All arithmetic
is fp64 in the kernels: per-token squared deviations and norms are exact
(correctly rounded) sums, and the blend ``w * new + (1 - w) * old`` rounds
exactly where the reference's separate tensor operations round.
"""

from __future__ import annotations

import ctypes
import math
import struct
import threading
from dataclasses import dataclass, field

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
    """Device status block: int32 check flags in word 0, then int64 counters.

    Kernels OR check bits into the flags and write counts into the counters;
    ``finish`` reads the whole block back with one synchronising copy and
    raises the first registered check that fired (registration order is the
    reference's order of checks).
    """

    def __init__(self, device, counters: int = 0):
        self.device = device
        # torch.zeros launches a fill kernel (no memset node under graph capture)
        self.block = torch.zeros(1 + counters, dtype=torch.int64, device=device)
        self.steps: list[tuple[int, type, str]] = []
        self.counts: list[int] = []
        self.stream = _hip.stream_of(device)  # the launch stream of every call of this block

    @property
    def ptr(self):
        return ctypes.c_void_p(self.block.data_ptr())

    def counter(self, i: int):
        return ctypes.c_void_p(self.block.data_ptr() + 8 * (1 + i))

    @property
    def abort_mask(self) -> int:
        """Every registered check bit: device commits skip when one is set."""
        mask = 0
        for bits, _, _ in self.steps:
            mask |= bits
        return mask

    def step(self, bits: int, exc: type, message: str) -> None:
        self.steps.append((bits, exc, message))

    def finish(self, pending: BaseException | None = None, *, read: bool = False) -> None:
        value = 0
        if self.steps or read:
            words = [int(x) for x in self.block.cpu().tolist()]
            value, self.counts = words[0] & 0xFFFFFFFF, words[1:]
        for bits, exc, message in self.steps:
            if value & bits:
                raise exc(message)
        if pending is not None:
            raise pending


_NONFINITE_BIT = {"cached_k": 1 << 20, "recomputed_k": 1 << 21, "cached_v": 1 << 22,
                  "recomputed_v": 1 << 23, "a": 1 << 20, "b": 1 << 21}


def _kv(name: str, tensor: Tensor, fl: _Flags, view=None) -> None:
    """wca.py:31-37."""
    if not isinstance(tensor, Tensor) or tensor.ndim != 3 or not tensor.is_floating_point():
        fl.finish(ValueError(f"{name} must be floating [token, head, dimension]"))
    if min(tensor.shape[1:]) < 1:
        fl.finish(ValueError(f"{name} must have nonempty heads/dimension"))
    bit = _NONFINITE_BIT[name]
    call("cs_check_finite", view if view is not None else vref(tensor), bit, fl.ptr, fl.stream)
    _finite_step(name, fl)


def _finite_step(name: str, fl: _Flags) -> None:
    fl.step(_NONFINITE_BIT[name], WCANumericalError, f"{name} must have finite values")


def _alpha_steps(fl: _Flags) -> None:
    fl.step(2 | 16, WCANumericalError, "adaptation weight overflowed float64")
    fl.step(4, WCANumericalError, "adaptation weight overflowed; inspect the K magnitudes")


_COMPUTED_MESSAGE = "computed_indices must equal sorted active_indices"
_BLEND_MESSAGE = "weighted K/V overflowed the cache dtype"
_UPDATE_STEPS: dict = {}


def _update_steps(computed: bool) -> tuple[list, int]:
    """The one-call update's checks in the order its launches make them (the
    reference's order of checks in WCAState.update), and their bits together
    (the device commits nothing when one of them is set)."""
    if computed not in _UPDATE_STEPS:
        names = ["cached_k", "cached_v", None, "recomputed_k", "recomputed_v"]
        steps = []
        for name in names:
            if name is None:
                if computed:
                    steps.append((64, ValueError, _COMPUTED_MESSAGE))
                continue
            steps.append((_NONFINITE_BIT[name], WCANumericalError, f"{name} must have finite values"))
        steps.append((2 | 16, WCANumericalError, "adaptation weight overflowed float64"))
        steps.append((4, WCANumericalError, "adaptation weight overflowed; inspect the K magnitudes"))
        steps.append((8, WCANumericalError, _BLEND_MESSAGE))
        mask = 0
        for bits, _, _ in steps:
            mask |= bits
        _UPDATE_STEPS[computed] = (steps, mask)
    return _UPDATE_STEPS[computed]


# the one-call initialize's checks in the order the checked path registers them
_INIT_STEPS = (
    (1 << 20, WCANumericalError, "cached_k must have finite values"),
    (1 << 21, WCANumericalError, "recomputed_k must have finite values"),
    (2, WCANumericalError, "squared deviation overflowed float64"),
    (32, ValueError, "every dynamic/non-reused token must be mandatory"),
    (2 | 16, WCANumericalError, "adaptation weight overflowed float64"),
    (4, WCANumericalError, "adaptation weight overflowed; inspect the K magnitudes"),
)
_INIT_CK = _hip.CsWcaInitializeArgs.cached_k.offset
_INIT_RK = _hip.CsWcaInitializeArgs.recomputed_k.offset


_INIT_STATUS = threading.local()


def _init_status(device) -> list:
    """This thread's status block for one-call initializes on ``device``:
    [device int64[6] block, pinned host int64[6] report, dirty].  The call's
    last kernel zeroes the block, so only a new block or one left by a call
    that returned an error is cleared by the next call."""
    table = getattr(_INIT_STATUS, "table", None)
    if table is None:
        table = _INIT_STATUS.table = {}
    status = table.get(device)
    if status is None:
        status = table[device] = [torch.empty(6, dtype=torch.int64, device=device),
                                  torch.empty(6, dtype=torch.int64, pin_memory=True), True]
    return status


def _initialize_inputs_pass(cached_k, recomputed_k, reused_mask, mandatory_mask) -> bool:
    """True when none of initialize's host-side checks (_kv, _matching, _mask) would raise,
    for a request of 1 .. 2^24 tokens."""
    if not all(isinstance(t, Tensor) for t in (cached_k, recomputed_k, reused_mask, mandatory_mask)):
        return False
    if cached_k.ndim != 3 or not cached_k.is_floating_point() or min(cached_k.shape[1:]) < 1:
        return False
    n = cached_k.shape[0]
    if not 0 < n <= 1 << 24:
        return False
    if (recomputed_k.shape, recomputed_k.dtype, recomputed_k.device) != (cached_k.shape, cached_k.dtype,
                                                                       cached_k.device):
        return False
    return all(m.shape == (n,) and m.dtype == torch.bool and m.device == cached_k.device and m.is_contiguous()
               for m in (reused_mask, mandatory_mask))


# byte offsets of the per-call fields of cs_wca_update_args
_CK, _CV, _RK, _RV, _FK, _FV = (getattr(_hip.CsWcaUpdateArgs, f).offset for f in (
    "cached_k", "cached_v", "recomputed_k", "recomputed_v", "fused_k", "fused_v"))
_TAIL = _hip.CsWcaUpdateArgs.rows.offset
# the whole cs_wca_update_args block in one pack: six 3-d views, then the tail
_VIEW3 = "qii3q3x3q3x".replace("3x", "24x")
_UPDATE_ALL = struct.Struct("<" + _VIEW3 * 6 + _hip.WCA_UPDATE_TAIL.format.lstrip("<"))
assert (_CK, _CV, _RK, _RV, _FK, _FV) == tuple(i * _hip._VIEW.size for i in range(6))
assert _TAIL == 6 * _hip._VIEW.size
assert _UPDATE_ALL.size == ctypes.sizeof(_hip.CsWcaUpdateArgs)


def _matching(name: str, tensor: Tensor, reference_shape, reference: Tensor, fl: _Flags,
              view=None) -> None:
    """wca.py:40-47: same shape, dtype and device as the reference rows."""
    if not isinstance(tensor, Tensor) or (tensor.shape, tensor.dtype, tensor.device) != (
        reference_shape,
        reference.dtype,
        reference.device,
    ):
        fl.finish(ValueError(f"{name} shape, dtype and device must match its reference"))
    _kv(name, tensor, fl, view)


def _mask(name: str, tensor: Tensor, n: int, device) -> None:
    if tensor.shape != (n,) or tensor.dtype != torch.bool or tensor.device != device:
        raise ValueError(f"{name} must be a bool [{n}] tensor on {device}")


def _score(old: Tensor, fresh: Tensor, rows: Tensor | None, fl: _Flags, out=None,
           views=None) -> tuple[Tensor, Tensor]:
    n = fresh.shape[0]
    if out is None:
        out = (torch.empty(n, dtype=torch.float64, device=fresh.device),
               torch.empty(n, dtype=torch.float64, device=fresh.device))
    err, norm = out
    old_view, fresh_view = views if views is not None else (vref(old), vref(fresh))
    call("cs_wca_score", old_view, ptr(rows), fresh_view, ptr(err), ptr(norm), fl.ptr, fl.stream)
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


def _alpha(err, norm, epsilon, clamp, fl: _Flags, out: Tensor | None = None) -> Tensor:
    alpha = torch.empty_like(err) if out is None else out
    call("cs_wca_alpha", ptr(err), ptr(norm), err.numel(), float(epsilon), 1 if clamp else 0,
         ptr(alpha), fl.ptr, fl.stream)
    _alpha_steps(fl)
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


def _nonzero_launch(a: Tensor, b: Tensor | None, count) -> Tensor:
    """Ascending indices of a | b into a device buffer; the count goes to ``count``."""
    n = a.numel()
    out = torch.empty(max(n, 1), dtype=torch.long, device=a.device)
    call("cs_mask_nonzero", ptr(a), ptr(b), n, ptr(out), count, _hip.stream_of(a.device))
    return out


def _nonzero(a: Tensor, b: Tensor | None) -> Tensor:
    """Ascending indices of a | b on the device (one readback for the count)."""
    fl = _Flags(a.device, 1)
    out = _nonzero_launch(a, b, fl.counter(0))
    fl.finish(read=True)
    return out[: fl.counts[0]]


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
    # active_indices of the current masks, kept with the tensor versions it
    # was computed from: kernels here update the masks in place, and refresh
    # it themselves; any other in-place change to a mask (or to the cached
    # index tensor) bumps a version and forces a recount.
    _active: Tensor | None = field(default=None, repr=False, compare=False)
    _active_key: tuple = field(default=(), repr=False, compare=False)
    # device work space of the updates, reused from call to call (launches of
    # one state are ordered on its stream): fp64 deviation, norm, next weight
    # and cosine rows; the int64 promotion scratch
    _work_f64: Tensor | None = field(default=None, repr=False, compare=False)
    _work_i64: Tensor | None = field(default=None, repr=False, compare=False)
    _update_args: object = field(default=None, repr=False, compare=False)
    _status_block: object = field(default=None, repr=False, compare=False)
    _status_dirty: bool = field(default=True, repr=False, compare=False)

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
        if _initialize_inputs_pass(cached_k, recomputed_k, reused_mask, mandatory_mask):
            return cls._initialize_device(cached_k, recomputed_k, reused_mask, mandatory_mask, config, device)
        fl = _Flags(device, 2)
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
        # the kernels read the masks as contiguous bytes
        call("cs_wca_init_masks", ptr(err), ptr(reused_mask.contiguous()), ptr(mandatory_mask.contiguous()),
             n, ptr(candidate), fl.counter(0), fl.ptr, fl.stream)
        fl.step(32, ValueError, "every dynamic/non-reused token must be mandatory")
        alpha = _alpha(err, norm, config.epsilon, config.clamp_alpha, fl)
        fl.finish(read=True)
        n_reused, n_candidates = fl.counts
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

    @classmethod
    def _initialize_device(cls, cached_k, recomputed_k, reused_mask, mandatory_mask, config,
                           device) -> "WCAState":
        """The launches of the checked initialize and _promote in one
        cs_wca_initialize call (the budget taken on the device), one readback."""
        n = cached_k.shape[0]
        err = torch.empty(n, dtype=torch.float64, device=device)
        norm = torch.empty(n, dtype=torch.float64, device=device)
        alpha = torch.empty(n, dtype=torch.float64, device=device)
        candidate = torch.empty(n, dtype=torch.bool, device=device)
        zeroed = torch.zeros(2 * n, dtype=torch.bool, device=device)  # selected, removed
        selected, removed = zeroed[:n], zeroed[n:]
        ibuf = torch.empty(4 * n, dtype=torch.long, device=device)  # scratch 2n, promoted, active
        status = _init_status(device)
        block, host = status[0], status[1]
        a = _hip.CsWcaInitializeArgs()
        _hip.pack_view3(a, _INIT_CK, cached_k)
        _hip.pack_view3(a, _INIT_RK, recomputed_k)
        ib, sp = ibuf.data_ptr(), block.data_ptr()
        a.reused, a.mandatory, a.n = reused_mask.data_ptr(), mandatory_mask.data_ptr(), n
        a.epsilon, a.fraction = float(config.epsilon), float(config.correction_fraction)
        a.clamp = 1 if config.clamp_alpha else 0
        a.err, a.norm, a.alpha = err.data_ptr(), norm.data_ptr(), alpha.data_ptr()
        a.candidate, a.selected, a.removed = candidate.data_ptr(), selected.data_ptr(), removed.data_ptr()
        a.scratch, a.promoted, a.active = ib, ib + 16 * n, ib + 24 * n
        a.flags, a.counts, a.report = sp, sp + 8, host.data_ptr()
        a.clear_status = 1 if status[2] else 0
        status[2] = True
        call("cs_wca_initialize", ctypes.byref(a), _hip.stream_of(device))
        status[2] = False  # the call's last kernel leaves the block zeroed
        # the state's own mask copies, queued while the device works
        reused_copy, mandatory_copy = reused_mask.clone(), mandatory_mask.clone()
        torch.cuda.current_stream(device).synchronize()
        words = host.tolist()
        value = words[0] & 0xFFFFFFFF
        for bits, exc, message in _INIT_STEPS:
            if value & bits:
                raise exc(message)
        budget, n_active = words[3], words[5]
        state = cls(
            config=config,
            reused_mask=reused_copy,
            mandatory_mask=mandatory_copy,
            initial_deviation=err,
            candidate_mask=candidate,
            selected_mask=selected,
            removed_mask=removed,
            alpha=alpha,
            budget=budget,
        )
        state._cache_active(ibuf[3 * n:3 * n + n_active], n_active)
        return state

    def _mask_key(self) -> tuple:
        sel, mand = self.selected_mask, self.mandatory_mask
        return (id(sel), sel._version, id(mand), mand._version)

    def _cache_active(self, buffer: Tensor, count: int) -> Tensor:
        self._active = buffer[:count]
        self._active_key = self._mask_key() + (self._active._version,)
        return self._active

    @property
    def active_indices(self) -> Tensor:
        """Sorted global token indices to compute at the next layer."""
        active = self._active
        if active is not None and self._active_key == self._mask_key() + (active._version,):
            return active
        fl = _Flags(self.selected_mask.device, 1)
        buffer = _nonzero_launch(self.selected_mask, self.mandatory_mask, fl.counter(0))
        fl.finish(read=True)
        return self._cache_active(buffer, fl.counts[0])

    @property
    def selected_indices(self) -> Tensor:
        return _nonzero(self.selected_mask, None)

    def _workspace(self) -> tuple[Tensor, Tensor]:
        n = self.selected_mask.numel()
        if self._work_f64 is None:
            device = self.selected_mask.device
            self._work_f64 = torch.empty(max(4 * n, 1), dtype=torch.float64, device=device)
            self._work_i64 = torch.empty(max(2 * n, 1), dtype=torch.long, device=device)
        return self._work_f64, self._work_i64

    def _promote_launch(self, fl: _Flags, counter: int, abort_mask: int = 0) -> Tensor:
        """Launch the promotion; its count goes to counter ``counter`` of ``fl``.
        With ``abort_mask`` it promotes nothing when fl's flags hold one of those bits."""
        n = self.selected_mask.numel()
        scratch = self._workspace()[1]
        promoted = torch.empty(max(n, 1), dtype=torch.long, device=self.selected_mask.device)
        call("cs_wca_promote", ptr(self.initial_deviation), ptr(self.candidate_mask),
             ptr(self.removed_mask), ptr(self.selected_mask), n, self.budget, ptr(scratch),
             ptr(promoted), fl.counter(counter), fl.ptr if abort_mask else ctypes.c_void_p(None),
             abort_mask, fl.stream)
        return promoted

    def _promote(self) -> Tensor:
        """Fill the budget with the largest initial deviations, ties to lower index."""
        fl = _Flags(self.selected_mask.device, 2)
        promoted = self._promote_launch(fl, 0)
        active = _nonzero_launch(self.selected_mask, self.mandatory_mask, fl.counter(1))
        fl.finish(read=True)
        self._cache_active(active, fl.counts[1])
        return promoted[: fl.counts[0]]

    def update(
        self,
        layer_index: int,
        cached_k: Tensor,
        cached_v: Tensor,
        recomputed_k: Tensor,
        recomputed_v: Tensor,
        computed_indices: Tensor | None = None,
    ) -> WCAUpdate:
        """Fuse sparse recomputed rows against the full current-layer cache (wca.py:217-304).

        When every host-side check passes, the device work is one library call
        (``cs_wca_update``); otherwise the checked path below raises in the
        reference's order of checks.
        """
        if layer_index != self.last_layer + 1:
            raise ValueError("layers must update consecutively after full layer one")
        device = _hip.require_device(cached_k)
        if self._inputs_pass(cached_k, cached_v, recomputed_k, recomputed_v, computed_indices):
            return self._update_device(layer_index, device, cached_k, cached_v, recomputed_k,
                                       recomputed_v, computed_indices)
        return self._update_checked(layer_index, device, cached_k, cached_v, recomputed_k,
                                    recomputed_v, computed_indices)

    def _inputs_pass(self, cached_k, cached_v, recomputed_k, recomputed_v, computed) -> bool:
        """True when none of update's host-side checks (_kv, _matching, counts) would raise."""
        if not all(isinstance(t, Tensor) for t in (cached_k, cached_v, recomputed_k, recomputed_v)):
            return False
        if cached_k.ndim != 3 or not cached_k.is_floating_point() or min(cached_k.shape[1:]) < 1:
            return False
        if (cached_v.shape, cached_v.dtype, cached_v.device) != (cached_k.shape, cached_k.dtype,
                                                                 cached_k.device):
            return False
        if cached_k.shape[0] != self.reused_mask.numel() or cached_k.device != self.reused_mask.device:
            return False
        indices = self.active_indices
        if computed is not None and (
            not isinstance(computed, Tensor)
            or computed.dtype != torch.long
            or computed.device != indices.device
            or computed.shape != indices.shape
        ):
            return False
        rows_shape = (indices.numel(), *cached_k.shape[1:])
        return all((t.shape, t.dtype, t.device) == (rows_shape, ref.dtype, ref.device)
                   for t, ref in ((recomputed_k, cached_k), (recomputed_v, cached_v)))

    def _status(self, device) -> tuple:
        """The one-call update's status: a device int64[4] block (flags word,
        three counts) that cs_wca_update zeroes again after its last kernel
        has copied it into the pinned host mirror, and the launch stream: the
        caller's current stream at this call (kept while it stays current)."""
        raw = torch._C._cuda_getCurrentRawStream(device.index)
        status = self._status_block
        if status is None or status[0].device != device:
            block = torch.zeros(4, dtype=torch.int64, device=device)
            host = torch.zeros(4, dtype=torch.int64, pin_memory=True)
            status = self._status_block = (block, host, _hip.stream_of(device),
                                           torch.cuda.current_stream(device), raw)
            self._status_dirty = True
        elif status[4] != raw:
            # the block was left zeroed by the last call, which was waited for
            status = self._status_block = (status[0], status[1], _hip.stream_of(device),
                                           torch.cuda.current_stream(device), raw)
        return status

    def _update_device(self, layer_index, device, cached_k, cached_v, recomputed_k, recomputed_v,
                       computed_indices) -> WCAUpdate:
        """The launches of _update_checked in one cs_wca_update call, with its checks registered."""
        indices = self.active_indices
        a, n = indices.numel(), self.selected_mask.numel()
        block, host, stream, torch_stream, _ = self._status(device)
        work, scratch = self._workspace()
        gate = layer_index % self.config.gate_interval == 0 and a > 0
        # fresh outputs in two allocations: fused K and V; the index lists and the weights used
        m = max(n, 1)
        fused = torch.empty((2, a, *cached_k.shape[1:]), dtype=cached_k.dtype, device=device)
        fused_k, fused_v = fused[0], fused[1]
        # int64 [used (fp64 bits) a | promoted m | active m | removed a]
        ibuf = torch.empty(2 * m + 2 * a, dtype=torch.long, device=device)
        ib = ibuf.data_ptr()
        computed = computed_indices.contiguous() if computed_indices is not None else None
        steps, abort_mask = _update_steps(computed is not None)
        u = self._update_args
        if u is None:
            u = self._update_args = _hip.CsWcaUpdateArgs()
        # the six views and every field from rows to report in one pack; the
        # fused outputs are the two halves of the contiguous [2, a, H, D] block
        config = self.config
        code = _hip.dtype_code(cached_k.dtype)
        _, hh, dd = cached_k.shape
        views = []
        for tensor in (cached_k, cached_v, recomputed_k, recomputed_v):
            s0, s1, s2 = tensor.shape
            views += (tensor.data_ptr() if s0 * s1 * s2 else 0, code, 3, s0, s1, s2, *tensor.stride())
        fk = fused.data_ptr() if a * hh * dd else 0
        fv = fk + a * hh * dd * fused.element_size() if fk else 0
        views += (fk, code, 3, a, hh, dd, hh * dd, dd, 1, fv, code, 3, a, hh, dd, hh * dd, dd, 1)
        base = work.data_ptr()
        flags = block.data_ptr()
        # the per-token state (NULL for a request without tokens)
        state = (self.alpha.data_ptr(), self.initial_deviation.data_ptr(), self.selected_mask.data_ptr(),
                 self.candidate_mask.data_ptr(), self.removed_mask.data_ptr(),
                 self.mandatory_mask.data_ptr(), scratch.data_ptr()) if n else (0,) * 7
        # clear_status bit 1: the call leaves the block zeroed; bit 0 also zeroes it first
        _UPDATE_ALL.pack_into(
            u, 0, *views, indices.data_ptr() if a else 0, computed.data_ptr() if computed is not None and a else 0,
            a, n, self.budget, *state[:6], base, base + 8 * n, base + 16 * n, base + 24 * n,
            ib, ib + 8 * (a + 2 * m) if gate else 0, ib + 8 * a, state[6], ib + 8 * (a + m),
            flags, flags + 8, float(config.epsilon), float(config.convergence_threshold),
            1 if config.clamp_alpha else 0, 1 if config.weight_update == "previous_layer" else 0,
            1 if gate else 0, 1 if config.convergence_mode == "distance_lt" else 0, abort_mask,
            3 if self._status_dirty else 2, host.data_ptr())
        self._status_dirty = True
        call("cs_wca_update", ctypes.byref(u), stream)
        self._status_dirty = False
        used = ibuf[:a].view(torch.float64)  # while the device works
        torch_stream.synchronize()
        words = host.tolist()
        value = words[0] & 0xFFFFFFFF
        for bits, exc, message in steps:
            if value & bits:
                raise exc(message)
        n_removed, n_promoted, n_active = words[1:4]
        promoted = ibuf[a:a + n_promoted]
        active = ibuf[a + m:a + m + n_active]
        removed = ibuf[a + 2 * m:a + 2 * m + n_removed] if gate else indices[:0]
        return self._finish_update(layer_index, indices, fused_k, fused_v, used, removed, promoted,
                                   active)

    def _finish_update(self, layer_index, indices, fused_k, fused_v, used, removed, promoted,
                       next_indices) -> WCAUpdate:
        self._active = next_indices
        self._active_key = self._mask_key() + (next_indices._version,)
        self.last_layer = layer_index
        return WCAUpdate(
            indices=indices,
            fused_k=fused_k,
            fused_v=fused_v,
            alpha=used,
            removed_indices=removed,
            promoted_indices=promoted,
            next_indices=next_indices,
        )

    def _update_checked(self, layer_index, device, cached_k, cached_v, recomputed_k, recomputed_v,
                        computed_indices) -> WCAUpdate:
        """One library call per step, each host check in the reference's place (wca.py:217-304)."""
        # counters: removed, promoted, next active
        fl = _Flags(device, 3)
        # each tensor's view is built once for all the calls below
        ck, cv = ctypes.byref(_hip.view(cached_k)), ctypes.byref(_hip.view(cached_v))
        _kv("cached_k", cached_k, fl, ck)
        _matching("cached_v", cached_v, cached_k.shape, cached_k, fl, cv)
        if cached_k.shape[0] != self.reused_mask.numel():
            fl.finish(ValueError("cache token count differs from the request"))
        if cached_k.device != self.reused_mask.device:
            fl.finish(ValueError("cache device differs from the request"))
        indices = self.active_indices
        a = indices.numel()
        if computed_indices is not None:
            if (
                not isinstance(computed_indices, Tensor)
                or computed_indices.dtype != torch.long
                or computed_indices.device != indices.device
                or computed_indices.shape != indices.shape
            ):
                fl.finish(ValueError(_COMPUTED_MESSAGE))
            # element equality on the device, raised in this place of the check order
            call("cs_wca_same_rows", ptr(computed_indices.contiguous()), ptr(indices), a, 64, fl.ptr,
                 fl.stream)
            fl.step(64, ValueError, _COMPUTED_MESSAGE)
        rows_shape = (a, *cached_k.shape[1:])
        rk = ctypes.byref(_hip.view(recomputed_k)) if isinstance(recomputed_k, Tensor) else None
        rv = ctypes.byref(_hip.view(recomputed_v)) if isinstance(recomputed_v, Tensor) else None
        _matching("recomputed_k", recomputed_k, rows_shape, cached_k, fl, rk)
        _matching("recomputed_v", recomputed_v, rows_shape, cached_v, fl, rv)
        work = self._workspace()[0]
        n = self.selected_mask.numel()
        err, norm = _score(cached_k, recomputed_k, indices, fl, out=(work[:a], work[n:n + a]),
                           views=(ck, rk))
        next_alpha = _alpha(err, norm, self.config.epsilon, self.config.clamp_alpha, fl,
                            out=work[2 * n:2 * n + a])
        used = torch.empty(a, dtype=torch.float64, device=device)
        call("cs_wca_used_alpha", ptr(self.alpha), ptr(next_alpha), ptr(indices),
             ptr(self.mandatory_mask), a, 1 if self.config.weight_update == "previous_layer" else 0,
             ptr(used), fl.stream)
        fused_k = torch.empty(rows_shape, dtype=cached_k.dtype, device=device)
        fused_v = torch.empty(rows_shape, dtype=cached_v.dtype, device=device)
        call("cs_wca_blend", ck, cv, ptr(indices), rk, rv, ptr(used), ptr(None), vref(fused_k),
             vref(fused_v), fl.ptr, fl.stream)
        fl.step(8, WCANumericalError, _BLEND_MESSAGE)

        gate = layer_index % self.config.gate_interval == 0 and a > 0
        removed_buf = None
        if gate:
            cosine = work[3 * n:3 * n + a]
            call("cs_wca_head_cosine", rk, ck, ptr(indices), float(self.config.epsilon), ptr(cosine),
                 fl.stream)
            removed_buf = torch.empty(a, dtype=torch.long, device=device)
            call("cs_wca_gate", ptr(cosine), ptr(indices), ptr(self.selected_mask), a,
                 1 if self.config.convergence_mode == "distance_lt" else 0,
                 float(self.config.convergence_threshold), ptr(removed_buf), fl.counter(0),
                 fl.stream)
        # Commit and promotion run on the device only when no check fired
        # (wca.py:289-295 commits after its checks); one readback follows.
        abort = fl.abort_mask
        call("cs_wca_commit", ptr(self.alpha), ptr(next_alpha), ptr(indices), a, ptr(removed_buf),
             fl.counter(0) if gate else ctypes.c_void_p(None), ptr(self.selected_mask),
             ptr(self.candidate_mask), ptr(self.removed_mask), fl.ptr, abort, fl.stream)
        promoted_buf = self._promote_launch(fl, 1, abort)
        active_buf = torch.empty(max(n, 1), dtype=torch.long, device=device)
        call("cs_mask_nonzero", ptr(self.selected_mask), ptr(self.mandatory_mask), n, ptr(active_buf),
             fl.counter(2), fl.stream)
        fl.finish(read=True)
        n_removed, n_promoted, n_active = fl.counts
        removed = removed_buf[:n_removed] if gate else indices[:0]
        return self._finish_update(layer_index, indices, fused_k, fused_v, used, removed,
                                   promoted_buf[:n_promoted], active_buf[:n_active])
