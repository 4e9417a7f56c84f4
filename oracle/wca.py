"""CPU oracle for WCA (test infrastructure only).

Follows src/cacheslide_vllm/wca.py in float64.  Per-token sums use
``math.fsum`` (the correctly rounded sum of the rounded fp64 squares), which
is order independent; torch's own reduction can differ from it in the last
ulps, which is why the kernels use the same exact summation.
"""

from __future__ import annotations

import math

import numpy as np

from .ccpe import bf16_round


class NumericalError(ValueError):
    pass


def _rows64(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).reshape(x.shape[0], -1)


def squared_deviation(cached: np.ndarray, fresh: np.ndarray) -> np.ndarray:
    """sum over heads/dims of (fresh - cached)^2 in fp64 (wca.py:55-62)."""
    d = _rows64(fresh) - _rows64(cached)
    sq = d * d
    out = np.array([math.fsum(row) for row in sq], dtype=np.float64)
    if not np.isfinite(out).all():
        raise NumericalError("squared deviation overflowed float64")
    return out


def adaptation_weight(cached, fresh, *, epsilon=1e-8, clamp=False) -> np.ndarray:
    """err / (sum cached^2 + epsilon) (wca.py:65-93)."""
    d = _rows64(fresh) - _rows64(cached)
    num = np.array([math.fsum(row) for row in d * d], dtype=np.float64)
    c = _rows64(cached)
    den = np.array([math.fsum(row) for row in c * c], dtype=np.float64) + epsilon
    if not np.isfinite(num).all() or not np.isfinite(den).all():
        raise NumericalError("adaptation weight overflowed float64")
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        out = num / den
    if not np.isfinite(out).all():
        raise NumericalError("adaptation weight overflowed; inspect the K magnitudes")
    return np.clip(out, 0, 1) if clamp else out


def mean_head_cosine(a, b, *, epsilon=1e-8) -> np.ndarray:
    """Mean over heads of clamped cosine of amax-scaled rows (wca.py:96-112)."""
    a64, b64 = np.asarray(a, np.float64), np.asarray(b, np.float64)
    sa = np.maximum(np.abs(a64).max(-1, keepdims=True), epsilon)
    sb = np.maximum(np.abs(b64).max(-1, keepdims=True), epsilon)
    xa, xb = a64 / sa, b64 / sb
    na = np.sqrt((xa * xa).sum(-1, keepdims=True))
    nb = np.sqrt((xb * xb).sum(-1, keepdims=True))
    tiny = np.finfo(np.float64).tiny
    ua, ub = xa / np.maximum(na, tiny), xb / np.maximum(nb, tiny)
    return np.clip((ua * ub).sum(-1), -1, 1).mean(-1)


def to_dtype(x64: np.ndarray, dtype: str) -> np.ndarray:
    """fp64 -> cache dtype as torch converts (through float32 for 16-bit types);
    returned as float64 values of the rounded numbers."""
    f32 = x64.astype(np.float32)
    if dtype == "float64":
        return x64
    if dtype == "float32":
        return f32.astype(np.float64)
    if dtype == "bfloat16":
        return bf16_round(f32).astype(np.float64)
    if dtype == "float16":
        return f32.astype(np.float16).astype(np.float64)
    raise ValueError(dtype)


def blend(weight: np.ndarray, fresh: np.ndarray, old: np.ndarray, dtype: str) -> np.ndarray:
    """w * new + (1 - w) * old in fp64, each product and the sum rounded (wca.py:266-272)."""
    w = np.asarray(weight, np.float64)[:, None, None]
    fused = w * np.asarray(fresh, np.float64) + (1 - w) * np.asarray(old, np.float64)
    return to_dtype(fused, dtype)


class State:
    """WCAState (wca.py:128-304) over numpy bool masks."""

    def __init__(self, cached, fresh, reused, mandatory, *, fraction=0.26, epsilon=1e-8,
                 gate_interval=4, threshold=0.12, mode="paper_cosine_lt",
                 weight_update="previous_layer", clamp=False, dtype="float32"):
        self.eps, self.gate, self.threshold = epsilon, gate_interval, threshold
        self.mode, self.weight_update, self.clamp, self.dtype = mode, weight_update, clamp, dtype
        err = squared_deviation(cached, fresh)
        if ((~reused) & (~mandatory)).any():
            raise ValueError("every dynamic/non-reused token must be mandatory")
        self.reused, self.mandatory = reused.copy(), mandatory.copy()
        self.initial = err
        self.candidate = reused & (err > 0)
        self.budget = min(math.ceil(fraction * int(reused.sum())), int(self.candidate.sum()))
        self.selected = np.zeros_like(self.candidate)
        self.removed = np.zeros_like(self.candidate)
        self.alpha = adaptation_weight(cached, fresh, epsilon=epsilon, clamp=clamp)
        self.last_layer = 1
        self.promote()

    @property
    def active(self) -> np.ndarray:
        return np.flatnonzero(self.selected | self.mandatory)

    def promote(self) -> np.ndarray:
        """Stable descending order of initial error; ties to the lower index (wca.py:202-215)."""
        available = np.flatnonzero(self.candidate & ~self.selected & ~self.removed)
        slots = max(0, self.budget - int(self.selected.sum()))
        order = np.argsort(-self.initial[available], kind="stable")
        promoted = available[order[:slots]]
        self.selected[promoted] = True
        return promoted

    def update(self, layer, cached_k, cached_v, fresh_k, fresh_v):
        """wca.py:217-304: returns (indices, fused_k, fused_v, used_alpha, removed, promoted, next)."""
        if layer != self.last_layer + 1:
            raise ValueError("layers must update consecutively after full layer one")
        idx = self.active
        old_k, old_v = cached_k[idx], cached_v[idx]
        nxt = adaptation_weight(old_k, fresh_k, epsilon=self.eps, clamp=self.clamp)
        used = self.alpha[idx] if self.weight_update == "previous_layer" else nxt
        used = np.where(self.mandatory[idx], 1.0, used)
        fk = blend(used, fresh_k, old_k, self.dtype)
        fv = blend(used, fresh_v, old_v, self.dtype)
        if not np.isfinite(fk).all() or not np.isfinite(fv).all():
            raise NumericalError("weighted K/V overflowed the cache dtype")
        removed = idx[:0]
        if layer % self.gate == 0:
            cos = mean_head_cosine(fresh_k, old_k, epsilon=self.eps)
            metric = cos if self.mode == "paper_cosine_lt" else 1 - cos
            removed = idx[self.selected[idx] & (metric < self.threshold)]
        self.alpha[idx] = nxt
        self.selected[removed] = False
        self.candidate[removed] = False
        self.removed[removed] = True
        promoted = self.promote()
        self.last_layer = layer
        return idx, fk, fv, used, removed, promoted, self.active
