"""CPU restatement of the CacheSlide runtime's call order -- TEST INFRASTRUCTURE.

Follows src/cacheslide_vllm/runtime.py with dense K/V (its ``arena_factory =
None`` branch) over this package's numpy oracle: preflight (:110-131), prefill
with the full-prefill fallback (:274-395), the selective layer loop with row
carry-over and snapshot restore (:397-456), the attention handler (:474-573)
and ``_attend`` with the two policies (:576-609).  Profiles are calibrated
in memory from a full forward of the calibration request, as
``CCPEProfile.calibrate`` does with one sample (position.py:594-699: the
canonical table is that sample's fixed x fixed positions).  Pages are numpy
arrays in a dict keyed like the runtime's store.

The model is the caller's (a torch module on the CPU); its attention layers
call ``OracleRuntime.attention`` with torch tensors, which are handed to the
numpy oracle as float32 arrays.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import ccpe as orc
from . import wca as owca


class ReuseFailure(RuntimeError):
    pass


class PositionError(ValueError):
    """The runtime's CCPEPositionError: a strict path or transform rejection."""


@dataclass
class _State:
    plan: object
    reuse: bool
    profiles: dict
    reason: str
    prefill_tokens: int
    wca: owca.State | None = None
    dense_kv: dict = field(default_factory=dict)
    write_cache: bool = False
    selected_at_layer: np.ndarray | None = None
    metrics: dict = field(default_factory=dict)
    pending: dict = field(default_factory=dict)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


class OracleRuntime:
    def __init__(self, *, layers: int, identity: str, options, fraction: float, gate_interval: int = 4,
                 threshold: float = 0.12, mode: str = "paper_cosine_lt"):
        self.layers, self.identity, self.options = layers, identity, options
        self.fraction, self.gate_interval, self.threshold = fraction, gate_interval, threshold
        self.mode = mode
        self.store: dict[str, dict[str, np.ndarray]] = {}
        self.profiles: dict[str, np.ndarray] = {}
        self.requests: dict[str, _State] = {}
        self.active: _State | None = None
        self.last_metrics: dict = {}
        self._trace: dict | None = None

    # -- calibration ---------------------------------------------------------------
    def calibrate(self, model, plan) -> None:
        """Canonical fixed x fixed positions of every layer from a full forward."""
        self._trace = {"plan": plan}
        try:
            model.forward(torch.tensor(plan.token_ids))
        finally:
            trace, self._trace = self._trace, None
        for layer in range(self.layers):
            self.profiles[plan.profile_key(self.identity, layer)] = trace[layer]

    def _key(self, plan, layer: int, kind: str) -> str:
        return plan.cache_key(self.identity, layer) + "/" + kind

    def _preflight(self, plan):
        profiles = {}
        for layer in range(self.layers):
            table = self.profiles.get(plan.profile_key(self.identity, layer))
            if table is None:
                return False, {}, "CCPE profile miss"
            profiles[layer] = table
        if not plan.fixed_indices:
            return False, profiles, "no reusable tokens"
        keys = [self._key(plan, 0, "committed")] + [
            self._key(plan, layer, kind) for layer in range(self.layers) for kind in ("kv", "state")]
        if not all(key in self.store for key in keys):
            return False, profiles, "immutable cache miss"
        return True, profiles, "hit"

    # -- one forward ------------------------------------------------------------------
    def run(self, model, hidden: torch.Tensor, positions: torch.Tensor, request_id: str, plan) -> torch.Tensor:
        n = len(plan.token_ids)
        pos = positions.tolist()
        prefill = pos == list(range(n))
        if prefill:
            self.requests.pop(request_id, None)
            hit, profiles, reason = self._preflight(plan)
            state = _State(plan, plan.operation == "reuse" and hit, profiles, reason, n)
            state.write_cache = plan.operation == "populate" and not hit and bool(profiles)
            state.metrics = {"cache_hit": state.reuse, "reason": reason, "layer_rows": [], "fallback": False,
                             "position_policy_fallback": False, "decode_tokens": 0, "restored_rows": 0}
            self.requests[request_id] = state
        else:
            state = self.requests[request_id]
            assert pos == [n + state.metrics["decode_tokens"]]
        self.active = state
        try:
            if prefill:
                try:
                    out = self._prefill(model, hidden, positions, state)
                except (ReuseFailure, PositionError, owca.NumericalError) as exc:
                    state.dense_kv.clear()
                    state.pending.clear()
                    state.reuse = state.write_cache = False
                    if isinstance(exc, PositionError):
                        state.profiles.clear()
                        state.metrics["position_policy_fallback"] = True
                    state.wca, state.selected_at_layer = None, None
                    state.metrics.update(cache_hit=False, fallback=True, reason=str(exc), layer_rows=[],
                                         restored_rows=0)
                    out = self._prefill(model, hidden, positions, state)
                self.last_metrics = dict(state.metrics)
                return out
            residual = None
            for layer in model.layers:
                hidden, residual = layer(positions, hidden, residual)
            hidden, _ = model.norm(hidden, residual)
            state.metrics["decode_tokens"] += 1
            self.last_metrics = dict(state.metrics)
            return hidden
        finally:
            self.active = None

    def _prefill(self, model, hidden, positions, state: _State) -> torch.Tensor:
        """runtime.py:397-456 with the reference's lookup tables."""
        hidden = hidden.clone()
        n = len(positions)
        residual = None
        previous = np.arange(n)
        fixed = np.array(state.plan.fixed_indices, dtype=np.int64)
        for index, layer in enumerate(model.layers):
            active = state.wca.active if state.wca is not None else previous
            if state.wca is not None:
                lookup = np.full(n, -1)
                lookup[previous] = np.arange(len(previous))
                rows = lookup[active]
                continuing = rows >= 0
                h, r = _np(hidden), _np(residual)
                nh = np.empty((len(active), h.shape[1]), np.float32)
                nr = np.empty_like(nh)
                nh[continuing], nr[continuing] = h[rows[continuing]], r[rows[continuing]]
                if not continuing.all():
                    snap = self.store[self._key(state.plan, index, "state")]
                    ordinal = np.full(n, -1)
                    ordinal[fixed] = np.arange(len(fixed))
                    restored = ordinal[active[~continuing]]
                    if (restored < 0).any():
                        raise ReuseFailure("a mandatory dynamic row was lost")
                    nh[~continuing] = snap["hidden"][restored]
                    nr[~continuing] = snap["residual"][restored]
                    state.metrics["restored_rows"] += int((~continuing).sum())
                hidden, residual = torch.from_numpy(nh), torch.from_numpy(nr)
            if state.write_cache:
                self.store[self._key(state.plan, index, "state")] = {
                    "hidden": _np(hidden)[fixed],
                    "residual": _np(residual)[fixed] if residual is not None else np.zeros((0,), np.float32)}
            state.metrics["layer_rows"].append(len(active))
            state.selected_at_layer = None
            if state.wca is not None:
                sel = np.flatnonzero(state.wca.selected)
                state.selected_at_layer = sel[~state.wca.mandatory[sel]]
            hidden, residual = layer(torch.from_numpy(np.asarray(active)), hidden, residual)
            if not (torch.isfinite(hidden).all() and torch.isfinite(residual).all()):
                raise ReuseFailure("WCA produced nonfinite layer output") if state.reuse else ValueError(
                    "full CoPE recomputation produced nonfinite output")
            previous = np.asarray(active)
        hidden, _ = model.norm(hidden, residual)
        out = torch.zeros((n, hidden.shape[1]))
        out[torch.from_numpy(previous)] = hidden
        if state.write_cache:
            self.store[self._key(state.plan, 0, "committed")] = {}
            state.write_cache = False
        state.metrics["computed_token_layers"] = sum(state.metrics["layer_rows"])
        state.metrics["dense_token_layers"] = n * self.layers
        return out

    # -- the attention handler ------------------------------------------------------------
    def attention(self, layer, positions, q, k, v, cope) -> torch.Tensor:
        e = _np(cope.position_embeddings)
        qn, kn, vn, pos = _np(q), _np(k), _np(v), positions.cpu().numpy().astype(np.int64)
        chunk = self.options.query_chunk_size
        if self._trace is not None:            # calibration: full contexts, record fixed x fixed
            plan = self._trace["plan"]
            fixed = np.array(plan.fixed_indices)
            out, trace = orc.cope_attention(qn, kn, vn, e, pos, query_chunk_size=chunk, return_positions=True)
            self._trace[layer] = trace[:, fixed][:, :, fixed].astype(np.float32)
            return torch.from_numpy(out)
        state = self.active
        if state is None:                      # a forward outside any request: plain CoPE
            return torch.from_numpy(orc.cope_attention(qn, kn, vn, e, pos, pos, query_chunk_size=chunk))
        n = state.prefill_tokens
        if int(pos[0]) >= n:
            old_k, old_v = state.dense_kv[layer]
            full_k, full_v = np.concatenate([old_k, kn]), np.concatenate([old_v, vn])
            state.dense_kv[layer] = (full_k, full_v)
            return self._attend(state, layer, qn, full_k, full_v, pos, e)
        plan = state.plan
        fixed = np.array(plan.fixed_indices, dtype=np.int64)
        sparse = state.reuse and state.wca is not None
        cached_k = np.zeros((n, *kn.shape[1:]), np.float32)
        cached_v = np.zeros_like(cached_k)
        if state.reuse:
            page = self.store[self._key(plan, layer, "kv")]
            cached_k[fixed], cached_v[fixed] = page["k"], page["v"]
        if sparse:
            idx, fk, fv, used, removed, promoted, nxt = state.wca.update(
                layer + 1, cached_k.astype(np.float64), cached_v.astype(np.float64),
                kn.astype(np.float64), vn.astype(np.float64))
            assert np.array_equal(idx, pos)
            full_k, full_v = cached_k.copy(), cached_v.copy()
            full_k[pos], full_v[pos] = fk.astype(np.float32), fv.astype(np.float32)
        else:
            full_k, full_v = kn, vn
            if state.reuse and layer == self.options.calibration_layer:
                reused = np.zeros(n, bool)
                reused[fixed] = True
                mandatory = np.zeros(n, bool)
                mandatory[list(plan.mandatory_indices)] = True
                ck = np.where(reused[:, None, None], cached_k, kn)
                state.wca = owca.State(ck.astype(np.float64), kn.astype(np.float64), reused, mandatory,
                                       fraction=self.fraction, gate_interval=self.gate_interval,
                                       threshold=self.threshold, mode=self.mode, dtype="float32")
                state.wca.last_layer = layer + 1
        if state.write_cache:
            self.store[self._key(plan, layer, "kv")] = {"k": full_k[fixed], "v": full_v[fixed]}
        state.dense_kv[layer] = (full_k, full_v)
        return self._attend(state, layer, qn, full_k, full_v, pos, e)

    def _attend(self, state, layer, q, k, v, pos, e) -> torch.Tensor:
        fixed = list(state.plan.fixed_indices)
        table = state.profiles.get(layer)
        strict = self.options.ccpe_position_policy == "strict_contextual"
        positional = None
        if table is not None:
            def positional(p, qpos, kpos):
                return orc.canonical_policy(p, qpos, kpos, fixed, table, list(range(len(fixed))), strict)
        visibility = None
        if state.selected_at_layer is not None and self.options.selected_attention == "updated_and_self":
            selected = state.selected_at_layer

            def visibility(qpos, kpos):
                return orc.selected_visibility(qpos, kpos, fixed, selected)
        try:
            out = orc.cope_attention(q, k, v, e, pos, positions_transform=positional,
                                     visibility_transform=visibility,
                                     query_chunk_size=self.options.query_chunk_size)
        except orc.PathError as err:
            raise PositionError(orc.PATH_MESSAGES[err.kind]) from err
        return torch.from_numpy(np.ascontiguousarray(out, dtype=np.float32))
