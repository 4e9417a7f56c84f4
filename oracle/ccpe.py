"""CPU oracle for CoPE / CCPE attention (test infrastructure only).

Follows src/cacheslide_vllm/position.py and attention.py operation by
operation, in numpy.  Inputs are numpy arrays already in the accumulation
dtype (float32 for bf16/f16/f32 tensors, float64 for f64), exactly as the
reference's ``.to(dtype)`` produces them; ``bf16_round`` reproduces the final
cast of bf16 outputs.
"""

from __future__ import annotations

import math

import numpy as np


class PathError(ValueError):
    """validate_contextual_path failure; ``kind`` names the failing check."""

    def __init__(self, kind: str):
        super().__init__(kind)
        self.kind = kind


PATH_MESSAGES = {
    "nonnegative": "causal contextual positions must be nonnegative",
    "available": "causal contextual count exceeds available gates",
    "nonincreasing": "causal contextual path must be nonincreasing",
    "gap": "causal contextual path exceeds one gate per token",
    # the bounds check of a positions_transform result (position.py:504-516)
    "transform": "positions_transform must return bounded finite positions "
                 "with the contextual shape, dtype and device",
}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out)


def acc_dtype(dtype) -> type:
    return np.float64 if np.dtype(dtype) == np.float64 else np.float32


def logits(q: np.ndarray, k: np.ndarray) -> np.ndarray:
    """(q . k) / sqrt(D) over all (head, query, key), KV heads repeated (position.py:157-164)."""
    acc = q.dtype.type
    group = q.shape[1] // k.shape[1]
    kk = np.repeat(k, group, axis=1)
    dots = np.einsum("qhd,khd->hqk", q, kk, dtype=acc)
    return (dots / acc(math.sqrt(q.shape[-1]))).astype(acc)


def allowed_mask(qpos: np.ndarray, kpos: np.ndarray, heads: int, attention_mask=None) -> np.ndarray:
    """causal key_pos <= query_pos AND attention_mask (position.py:180-192)."""
    mask = kpos[None, :] <= qpos[:, None]
    mask = np.broadcast_to(mask[None], (heads, *mask.shape))
    if attention_mask is not None:
        am = attention_mask if attention_mask.ndim == 3 else attention_mask[None]
        mask = mask & am
    return np.array(mask)


def sigmoid(x: np.ndarray) -> np.ndarray:
    acc = x.dtype.type
    with np.errstate(over="ignore"):
        return (acc(1) / (acc(1) + np.exp(-x))).astype(acc)


def contextual_positions(logits_: np.ndarray, allowed: np.ndarray, max_positions: int) -> np.ndarray:
    """sigmoid(masked logits), reverse cumsum accumulated in float64 and rounded
    once, clamp(0, P-1) (position.py:295-307; torch's CPU cumsum of float32
    accumulates in float64)."""
    acc = logits_.dtype.type
    gates = np.where(allowed, sigmoid(logits_), acc(0)).astype(acc)
    suffix = np.flip(np.cumsum(np.flip(gates.astype(np.float64), -1), axis=-1), -1)
    return np.clip(suffix.astype(acc), acc(0), acc(max_positions - 1))


def qe_table(q: np.ndarray, e: np.ndarray) -> np.ndarray:
    """QE[h, q, p] = q[q, h, :] . E[:, p] with unscaled q (position.py:335-338)."""
    acc = q.dtype.type
    return np.einsum("qhd,dp->hqp", q, e.astype(acc), dtype=acc)


def positional_bias(q: np.ndarray, e: np.ndarray, positions: np.ndarray) -> np.ndarray:
    """low + frac * (high - low) at floor(p) and min(floor(p) + 1, P-1) (position.py:339-344)."""
    acc = q.dtype.type
    npos = e.shape[1]
    table = qe_table(q, e)
    lower = np.floor(positions).astype(np.int64)
    upper = np.minimum(lower + 1, npos - 1)
    frac = (positions - lower).astype(acc)
    low = np.take_along_axis(table, lower, axis=-1)
    high = np.take_along_axis(table, upper, axis=-1)
    return (low + frac * (high - low)).astype(acc)


def cope_attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    e: np.ndarray,
    qpos: np.ndarray,
    kpos: np.ndarray | None = None,
    *,
    attention_mask=None,
    visibility_mask=None,
    fixed_positions=None,
    positions_transform=None,
    visibility_transform=None,
    query_chunk_size: int = 128,
    return_positions: bool = False,
):
    """cope_attention (position.py:404-560): per query chunk, gates -> positions
    (or fixed / transformed) -> bias -> visibility -> masked softmax -> P.V;
    rows without an allowed key give zero.  Returns float arrays in the
    accumulation dtype (the caller applies the output dtype's rounding)."""
    acc = q.dtype.type
    nq, hq = q.shape[0], q.shape[1]
    nk = k.shape[0]
    if kpos is None:
        kpos = np.arange(nk, dtype=np.int64)
    group = hq // k.shape[1]
    vv = np.repeat(v, group, axis=1).astype(acc)
    outputs, traces = [], []
    npos = e.shape[1]
    for start in range(0, nq, query_chunk_size):
        end = min(start + query_chunk_size, nq)
        qc = q[start:end]
        cmask = None if attention_mask is None else attention_mask[..., start:end, :]
        allowed = allowed_mask(qpos[start:end], kpos, hq, cmask)
        lg = logits(qc, k)
        if fixed_positions is None:
            positions = contextual_positions(lg, allowed, npos)
        else:
            positions = fixed_positions[:, start:end]
        if positions_transform is not None:
            positions = positions_transform(positions, qpos[start:end], kpos)
            # position.py:504-516: a transform's result must be finite and in [0, P-1]
            if not np.isfinite(positions).all() or (positions < 0).any() or (positions > npos - 1).any():
                raise PathError("transform")
        lg = (lg + positional_bias(qc, e, positions)).astype(acc)
        vis = None
        if visibility_mask is not None:
            vis = visibility_mask[..., start:end, :]
        elif visibility_transform is not None:
            vis = visibility_transform(qpos[start:end], kpos)
        if vis is not None:
            allowed = allowed & allowed_mask(qpos[start:end], kpos, hq, vis)
        any_allowed = allowed.any(-1, keepdims=True)
        masked = np.where(allowed, lg, -np.inf)
        masked = np.where(any_allowed, masked, acc(0))
        peak = masked.max(-1, keepdims=True)
        ex = np.exp(masked - peak).astype(acc)
        probs = (ex / ex.sum(-1, keepdims=True)).astype(acc)
        probs = np.where(allowed, probs, acc(0))
        outputs.append(np.einsum("hqk,khd->qhd", probs, vv, dtype=acc))
        traces.append(positions)
    out = np.concatenate(outputs, axis=0) if outputs else np.zeros((0, hq, v.shape[2]), acc)
    if return_positions:
        return out, np.concatenate(traces, axis=1)
    return out


def dense_reference(q, k, v, e, qpos, kpos, max_positions):
    """Per-query, per-head textbook loop with the ceil convention (the independent
    check of tests/test_position.py:80-96); forward values equal floor+1."""
    out = np.zeros((q.shape[0], q.shape[1], v.shape[2]), dtype=np.float64)
    group = q.shape[1] // k.shape[1]
    for qi, pos in enumerate(qpos):
        for hi in range(q.shape[1]):
            kv = hi // group
            lg = (k[:, kv].astype(np.float64) @ q[qi, hi].astype(np.float64)) / math.sqrt(q.shape[-1])
            mask = kpos <= pos
            gates = np.where(mask, 1.0 / (1.0 + np.exp(-lg)), 0.0)
            p = np.clip(np.flip(np.cumsum(np.flip(gates))), 0, max_positions - 1)
            table = q[qi, hi].astype(np.float64) @ e.astype(np.float64)
            fl, ce = np.floor(p).astype(int), np.ceil(p).astype(int)
            bias = table[fl] + (p - fl) * (table[ce] - table[fl])
            s = np.where(mask, lg + bias, -np.inf)
            w = np.exp(s - s.max())
            w /= w.sum()
            out[qi, hi] = w @ v[:, kv].astype(np.float64)
    return out


def validate_contextual_path(positions, qpos, kpos, *, attention_mask=None, atol=1e-6) -> None:
    """Path checks of position.py:98-114 in the positions dtype; raises PathError."""
    dt = positions.dtype.type
    valid = np.broadcast_to((kpos[None, :] <= qpos[:, None])[None], positions.shape)
    if attention_mask is not None:
        am = attention_mask if attention_mask.ndim == 3 else attention_mask[None]
        valid = valid & am
    eps = dt(np.finfo(dt).eps)
    rounding = (eps * np.abs(positions)).astype(dt)
    tol = (dt(atol) + rounding).astype(dt)
    if ((positions < -tol) & valid).any():
        raise PathError("nonnegative")
    available = (qpos[:, None] - kpos[None, :]).astype(dt)
    available = (np.maximum(available, dt(-1)) + dt(1)).astype(dt)
    upper = ((available[None] + dt(atol)).astype(dt) + rounding).astype(dt)
    if ((positions > upper) & valid).any():
        raise PathError("available")
    pairs = valid[..., :-1] & valid[..., 1:]
    diff = (positions[..., :-1] - positions[..., 1:]).astype(dt)
    gaps = (kpos[1:] - kpos[:-1]).astype(dt)
    pair_tol = ((dt(atol) + rounding[..., :-1]).astype(dt) + rounding[..., 1:]).astype(dt)
    if ((diff < -pair_tol) & pairs).any():
        raise PathError("nonincreasing")
    if ((diff > (gaps + pair_tol).astype(dt)) & pairs).any():
        raise PathError("gap")


def canonical_policy(contextual, queries, keys, fixed_indices, canonical, profile_query_ordinals,
                     strict: bool):
    """CanonicalPositionPolicy.__call__ (attention.py:32-57) with a lowered
    profile: canonical [H, F_rows, F] rows indexed through profile_query_ordinals."""
    ordinal = {int(p): i for i, p in enumerate(fixed_indices)}
    known = {int(o): r for r, o in enumerate(profile_query_ordinals)}
    rows = [i for i, p in enumerate(queries.tolist()) if p in ordinal]
    if not rows:
        return contextual
    cols = [j for j, p in enumerate(keys.tolist()) if p in ordinal]
    col_ord = [ordinal[int(keys[j])] for j in cols]
    result = contextual.copy()
    for r in rows:
        prow = known[ordinal[int(queries[r])]]
        result[:, r, cols] = canonical[:, prow, col_ord].astype(result.dtype)
    if strict:
        validate_contextual_path(result, queries, keys)
    return result


def selected_visibility(queries, keys, fixed_indices, selected_indices) -> np.ndarray:
    """SelectedAssociationPolicy.__call__ (attention.py:65-72)."""
    selected = np.isin(queries, selected_indices)
    fixed = np.isin(keys, np.asarray(fixed_indices, dtype=np.int64))
    return (~selected[:, None]) | (~fixed[None, :]) | (queries[:, None] == keys[None, :])
