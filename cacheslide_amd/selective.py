"""The selective prefill / decode loop of one CacheSlide request, on this package.

Counterpart of ``CacheSlideRuntime`` (src/cacheslide_vllm/runtime.py:57-609):
the caller's model runs its layers; each attention layer calls
``SelectiveRuntime.attention`` (the engine's attention handler), and the
runtime decides, per request and layer, what is computed and what is reused:

* preflight (runtime.py:110-131): calibrated CCPE profiles for every layer,
  reusable tokens, and a committed population of layer pages in the store;
* prefill (runtime.py:397-456): the layer loop over the rows WCA keeps
  active, carrying continuing rows and restoring newly selected fixed rows
  from the layer's input snapshot (``runtime_rows``), persisting snapshots
  when populating, and scattering the last layer's rows into the output;
* attention (runtime.py:474-573): cached fixed-token K/V from the layer's
  snapshot (with a one-layer prefetch), WCA initialisation at the calibration
  layer and WCA updates after it, the SLIDE arena writes (promotion while the
  page load is in flight, baseline write, fused-row update with the canonical
  mirror, decode with hole reuse), then CCPE attention with the canonical
  position policy and the selected-row association (runtime.py:576-609);
* full-prefill fallback (runtime.py:345-383) on a reuse failure, a capacity or
  integrity error, a strict-CCPE rejection or a WCA numerical error, before
  any token is sampled.

The decode step reads the arena in place through its slot map with the fused
decode kernel when the layout allows it (bf16, head dim 128), which equals
``gather`` + ``cope_attention`` (runtime.py:489-508); otherwise it gathers.

What differs from the reference: the model, adapters and vLLM step context
are the caller's; a request is named by ``request_id`` and its
``RequestPlan``; pages go through ``LayerSnapshots`` (pinned staging and a
device-side check) instead of safetensors on the compute thread.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable

import torch
from torch import Tensor

from . import _hip
from .attention import CanonicalPositionPolicy, SelectedAssociationPolicy
from .ccpe import ccpe_decode_arena
from .contracts import RequestPlan
from .errors import CacheCapacityError, CacheIntegrityError
from .policy import WCAConfig
from .position import CCPEPositionError, cope_attention
from .runtime_rows import ReuseFailure, gather_rows, next_layer_rows, scatter_rows
from .snapshot import LayerSnapshots
from .wca import WCANumericalError, WCAState

# Failures that allow a full-prefill retry before any token is sampled (runtime.py:347-353)
_RETRYABLE = (ReuseFailure, CacheCapacityError, CacheIntegrityError, CCPEPositionError, WCANumericalError)
_COMMITTED = b"cacheslide-runtime-v1"


@dataclass(frozen=True)
class RuntimeOptions:
    """The engine settings the selective loop reads (config.py:11-28)."""

    query_chunk_size: int = 64
    calibration_layer: int = 0
    wca: WCAConfig = field(default_factory=WCAConfig)
    selected_attention: str = "updated_and_self"
    ccpe_position_policy: str = "strict_contextual"
    max_prompt_tokens: int = 32768

    def __post_init__(self) -> None:
        if type(self.query_chunk_size) is not int or self.query_chunk_size < 1:
            raise ValueError("query_chunk_size must be a positive integer")
        if type(self.calibration_layer) is not int or self.calibration_layer < 0:
            raise ValueError("calibration_layer must be a nonnegative layer index")
        if self.selected_attention not in ("updated_and_self", "all"):
            raise ValueError("unknown selected_attention policy")
        if self.ccpe_position_policy not in ("strict_contextual", "mixed_bias_override"):
            raise ValueError("unknown CCPE position policy")


@dataclass
class _Request:
    plan: RequestPlan
    reuse: bool
    profiles: dict[int, Any]
    reason: str
    prefill_tokens: int
    snaps: LayerSnapshots | None = None
    wca: WCAState | None = None
    dense_kv: dict[int, tuple[Tensor, Tensor]] = field(default_factory=dict)
    arenas: dict[int, Any] = field(default_factory=dict)
    write_cache: bool = False
    selected_at_layer: Tensor | None = None
    metrics: dict[str, Any] = field(default_factory=dict)


def _finite(x: Tensor | None) -> bool:
    """All values finite (cs_check_finite, one readback)."""
    if x is None or x.numel() == 0:
        return True
    flags = _hip.new_flags(x.device)
    _hip.call("cs_check_finite", _hip.vref(x), 1, _hip.ptr(flags), _hip.stream_of(x.device))
    return _hip.read_flags(flags)[0] == 0


class SelectiveRuntime:
    """One request at a time over a page store, calibrated profiles and
    (optionally) SLIDE arenas from ``arena_factory(layer, prompt_length,
    max_selected, existing=None)``."""

    def __init__(self, *, layers: int, kv_heads: int, head_dim: int, hidden_size: int, store,
                 profiles, identity: str, checkpoint_id: str, options: RuntimeOptions | None = None,
                 arena_factory: Callable | None = None):
        options = options or RuntimeOptions()
        if options.calibration_layer >= layers:
            raise ValueError("calibration_layer is outside the model")
        self.layers, self.kv_heads, self.head_dim, self.hidden_size = layers, kv_heads, head_dim, hidden_size
        self.store, self.profiles, self.identity = store, profiles, identity
        self.checkpoint_id, self.options, self.arena_factory = checkpoint_id, options, arena_factory
        self.requests: dict[str, _Request] = {}
        self.active: _Request | None = None
        self.last_metrics: dict = {}

    # -- preflight, pages ---------------------------------------------------------
    def _commit_key(self, plan: RequestPlan) -> str:
        return plan.cache_key(self.identity, 0) + "/committed"

    def _preflight(self, plan: RequestPlan) -> tuple[bool, dict, str]:
        """runtime.py:110-131."""
        if self.profiles is None:
            return False, {}, "no calibrated CCPE profiles"
        profiles = {}
        for layer in range(self.layers):
            profile = self.profiles.get(plan, layer)
            if profile is None:
                return False, {}, "CCPE profile miss"
            profiles[layer] = profile
        if not plan.fixed_indices:
            return False, profiles, "no reusable tokens"
        keys = [self._commit_key(plan)] + [
            plan.cache_key(self.identity, layer) + "/" + kind
            for layer in range(self.layers) for kind in ("kv", "state")
        ]
        if not all(self.store.contains(key) for key in keys):
            return False, profiles, "immutable cache miss"
        return True, profiles, "hit"

    def _discard_uncommitted(self, state: _Request) -> None:
        if state.snaps is None:
            return
        for key in reversed(state.snaps.created_keys):
            if self.store.contains(key):
                self.store.delete(key)
        state.snaps.created_keys.clear()

    def _snapshots(self, state: _Request, device) -> LayerSnapshots:
        if state.snaps is None:
            state.snaps = LayerSnapshots(
                self.store, state.plan, self.identity, device, layers=self.layers,
                kv_heads=self.kv_heads, head_dim=self.head_dim, hidden_size=self.hidden_size,
                reuse=state.reuse, write_cache=state.write_cache)
        state.snaps.reuse, state.snaps.write_cache = state.reuse, state.write_cache
        return state.snaps

    def release(self, request_id: str) -> None:
        """runtime.py:151-171: drain loads, retire arenas, drop uncommitted pages."""
        state = self.requests.pop(request_id, None)
        if state is None:
            return
        if state.snaps is not None:
            state.snaps.release()
        self._record_metrics(state)
        for arena in state.arenas.values():
            arena.invalidate()
        self._discard_uncommitted(state)
        if state.snaps is not None:
            state.snaps.close()
        self.last_metrics = dict(state.metrics)

    def _record_metrics(self, state: _Request) -> None:
        state.metrics["paged_layers"] = {str(layer): arena.stats() for layer, arena in state.arenas.items()}
        self.last_metrics = dict(state.metrics)

    def close(self) -> None:
        for request_id in tuple(self.requests):
            self.release(request_id)

    # -- one forward ----------------------------------------------------------------
    def run(self, model, hidden: Tensor, positions: Tensor, request_id: str, plan: RequestPlan) -> Tensor:
        """runtime.py:274-395: prefill (positions 0..n-1) with fallback, or one decode token."""
        if self.active is not None:
            raise RuntimeError("CacheSlide does not allow concurrent model forwards")
        n = len(plan.token_ids)
        if n > self.options.max_prompt_tokens:
            raise ValueError("prompt exceeds the configured CacheSlide token budget")
        pos = positions.tolist()
        prefill = pos == list(range(n))
        if prefill:
            self.release(request_id)
            if plan.operation == "calibrate":
                raise ValueError("use the offline calibrate command, not generation")
            hit, profiles, reason = self._preflight(plan)
            state = _Request(plan, plan.operation == "reuse" and hit, profiles, reason, n)
            state.write_cache = plan.operation == "populate" and not hit and bool(profiles)
            state.metrics = {
                "request_id": request_id, "operation": plan.operation, "cache_hit": state.reuse,
                "reason": reason, "prompt_tokens": n, "layer_rows": [], "snapshot_bytes_written": 0,
                "fallback": False, "position_policy_fallback": False,
                "ccpe_position_policy": self.options.ccpe_position_policy, "decode_tokens": 0,
                "restored_rows": 0,
            }
            self.requests[request_id] = state
        else:
            state = self.requests.get(request_id)
            if state is None or state.plan != plan:
                raise ValueError("decode requires the unchanged populated request state")
            if pos != [n + state.metrics["decode_tokens"]]:
                raise ValueError("decode tokens must arrive once in consecutive order")
        self.active = state
        try:
            if prefill:
                try:
                    output = self._prefill(model, hidden, positions, state)
                except _RETRYABLE as exc:
                    self._fall_back(state, exc)
                    output = self._prefill(model, hidden, positions, state)
                self.last_metrics = dict(state.metrics)
                return output
            residual = None
            for layer in model.layers:
                hidden, residual = layer(positions, hidden, residual)
            hidden, _ = model.norm(hidden, residual)
            state.metrics["decode_tokens"] += 1
            self._record_metrics(state)
            return hidden
        finally:
            self.active = None

    def _fall_back(self, state: _Request, exc: BaseException) -> None:
        """runtime.py:354-383: no token has been sampled; recompute every layer."""
        if state.snaps is not None:
            state.snaps.release()
        for arena in state.arenas.values():
            arena.invalidate()
        state.arenas.clear()
        state.dense_kv.clear()
        self._discard_uncommitted(state)
        state.reuse = state.write_cache = False
        if isinstance(exc, CCPEPositionError):
            state.profiles.clear()
            state.metrics["position_policy_fallback"] = True
            state.metrics["ccpe_position_policy"] = "plain_cope_fallback"
        state.wca = None
        state.selected_at_layer = None
        state.metrics.update(cache_hit=False, fallback=True, reason=str(exc), layer_rows=[],
                             restored_rows=0, snapshot_bytes_written=0)

    def _prefill(self, model, hidden: Tensor, positions: Tensor, state: _Request) -> Tensor:
        """runtime.py:397-456."""
        hidden = hidden.clone()
        device = hidden.device
        n = len(positions)
        snaps = self._snapshots(state, device)
        if state.write_cache and self.store.contains(self._commit_key(state.plan)):
            raise ReuseFailure("incomplete committed population requires cache repair")
        if state.write_cache:      # runtime.py:141-149: drop orphan pages of this identity
            for layer in range(self.layers):
                for kind in ("state", "kv"):
                    key = snaps.key(layer, kind)
                    if self.store.contains(key):
                        self.store.delete(key)
        residual = None
        previous = torch.arange(n, device=device)
        fixed = torch.tensor(state.plan.fixed_indices, dtype=torch.long, device=device)
        snaps.prefetch(0, hidden.dtype)
        for index, layer in enumerate(model.layers):
            active = state.wca.active_indices if state.wca is not None else previous
            if state.wca is not None:
                rows = next_layer_rows(hidden, residual, previous, active, fixed,
                                       read_snapshot=lambda i=index: snaps.read(i, "state", hidden.dtype),
                                       check=False)
                state.metrics["restored_rows"] += rows.check()
                hidden, residual = rows.hidden, rows.residual
            if state.write_cache:
                snaps.put(index, "state", {
                    "hidden": gather_rows(hidden, fixed),
                    "residual": gather_rows(residual, fixed) if residual is not None else hidden.new_empty((0,)),
                })
            state.metrics["layer_rows"].append(len(active))
            state.selected_at_layer = None
            if state.wca is not None:
                selected = state.wca.selected_indices
                state.selected_at_layer = selected[~state.wca.mandatory_mask[selected]]
            hidden, residual = layer(positions[active], hidden, residual)
            if not (_finite(hidden) and _finite(residual)):
                if state.reuse:
                    raise ReuseFailure("WCA produced nonfinite layer output")
                raise ValueError("full CoPE recomputation produced nonfinite output")
            previous = active
        hidden, _ = model.norm(hidden, residual)
        output = scatter_rows(hidden, previous, n)
        if state.write_cache:
            self.store.put(self._commit_key(state.plan), _COMMITTED, selected_count=0)
            self.store.submit_spill(self._commit_key(state.plan)).result()
            snaps.created_keys.clear()
            state.write_cache = False
        state.metrics["snapshot_bytes_written"] = snaps.metrics["snapshot_bytes_written"]
        state.metrics["computed_token_layers"] = sum(state.metrics["layer_rows"])
        state.metrics["dense_token_layers"] = n * self.layers
        self._record_metrics(state)
        return output

    # -- the attention handler -------------------------------------------------------
    def attention(self, layer: int, positions: Tensor, q: Tensor, k: Tensor, v: Tensor, cope) -> Tensor:
        """runtime.py:474-573."""
        state = self.active
        chunk = self.options.query_chunk_size
        if state is None:    # profiling call without a request
            return cope_attention(q, k, v, cope, positions, key_positions=positions, query_chunk_size=chunk)
        n = state.prefill_tokens
        first = int(positions[0])
        if first >= n:
            return self._decode_attention(state, layer, first, q, k, v, positions, cope)
        device = k.device
        plan = state.plan
        fixed = torch.tensor(plan.fixed_indices, dtype=torch.long, device=device)
        sparse = state.reuse and state.wca is not None
        fixed_rows = torch.isin(positions, fixed) if sparse else None
        selected = positions[fixed_rows] if sparse else positions[:0]
        arena, relocated = None, False
        snaps = state.snaps
        if self.arena_factory is not None:
            arena = self.arena_factory(layer, n, len(selected))
            state.arenas[layer] = arena
            pending = snaps.kv_future if snaps is not None else None
            if sparse and len(selected) and pending is not None and not pending.done():
                # stage the fresh selected rows while the page read is in flight
                arena.promote_selected(selected, k[fixed_rows], v[fixed_rows], load_future=pending).result()
                relocated = True
        kv_shape = (n, *k.shape[1:])
        if state.reuse:
            cache = snaps.read(layer, "kv", k.dtype)
            width = k.shape[1] * k.shape[2]
            cached_k = scatter_rows(cache["k"].reshape(len(fixed), width), fixed, n).view(kv_shape)
            cached_v = scatter_rows(cache["v"].reshape(len(fixed), width), fixed, n).view(kv_shape)
            snaps.prefetch(layer + 1, k.dtype)
        else:
            cached_k, cached_v = k.new_zeros(kv_shape), v.new_zeros(kv_shape)
        if sparse:
            update = state.wca.update(layer + 1, cached_k, cached_v, k, v, computed_indices=positions)
            full_k = cached_k.clone().index_copy_(0, positions, update.fused_k)
            full_v = cached_v.clone().index_copy_(0, positions, update.fused_v)
            if arena is not None:
                arena.write_prefill(cached_k, cached_v)
                if len(selected) and not relocated:
                    arena.write_selected_ready(selected, update.fused_k[fixed_rows], update.fused_v[fixed_rows])
                arena.update_selected(positions, update.fused_k, update.fused_v)
        else:
            full_k, full_v = k, v
            if state.reuse and layer == self.options.calibration_layer:
                reused = torch.zeros(n, dtype=torch.bool, device=device)
                reused[fixed] = True
                mandatory = torch.zeros_like(reused)
                mandatory[list(plan.mandatory_indices)] = True
                # dynamic rows compare to themselves: only fixed-token error selects work
                cached_k = torch.where(reused[:, None, None], cached_k, k)
                state.wca = WCAState.initialize(cached_k, k, reused, mandatory, self.options.wca)
                state.wca.last_layer = layer + 1
            if arena is not None:
                arena.write_prefill(full_k, full_v)
        if state.write_cache:
            snaps.put(layer, "kv", {"k": full_k.index_select(0, fixed), "v": full_v.index_select(0, fixed)})
        if arena is None:
            state.dense_kv[layer] = (full_k, full_v)
        else:
            full_k, full_v = arena.gather(range(n))
        return self._attend(state, layer, q, full_k, full_v, positions, cope)

    def _decode_attention(self, state: _Request, layer: int, position: int, q, k, v, positions, cope) -> Tensor:
        """runtime.py:489-508: append the token, then attend over every logical token."""
        n = state.prefill_tokens
        if self.arena_factory is None:
            old_k, old_v = state.dense_kv[layer]
            full_k, full_v = torch.cat((old_k, k)), torch.cat((old_v, v))
            state.dense_kv[layer] = (full_k, full_v)
            return self._attend(state, layer, q, full_k, full_v, positions, cope)
        arena = state.arenas[layer]
        self.arena_factory(layer, n, 0, existing=arena)
        arena.decode(position, k[0], v[0], arena.canonical_slot(position))
        if q.dtype == torch.bfloat16 and q.shape[-1] == 128 and cope.position_embeddings.dtype == torch.float32:
            # the decode query is never a fixed or selected row: both policies
            # leave it plain CoPE, which the fused slot-map kernel computes
            return ccpe_decode_arena(q, arena, cope)[0].unsqueeze(0)
        full_k, full_v = arena.gather(range(position + 1))
        return self._attend(state, layer, q, full_k, full_v, positions, cope)

    def _attend(self, state: _Request, layer: int, q, k, v, positions, cope) -> Tensor:
        """runtime.py:576-609: canonical positions for fixed x fixed cells, and
        the selected rows' association applied after the gates."""
        profile = state.profiles.get(layer)
        positional = (CanonicalPositionPolicy(state.plan, profile, self.checkpoint_id,
                                              self.options.ccpe_position_policy)
                      if profile is not None else None)
        visibility = (SelectedAssociationPolicy(state.plan.fixed_indices, state.selected_at_layer)
                      if state.selected_at_layer is not None
                      and self.options.selected_attention == "updated_and_self" else None)
        return cope_attention(q, k, v, cope, positions, positions_transform=positional,
                              visibility_transform=visibility, query_chunk_size=self.options.query_chunk_size)
