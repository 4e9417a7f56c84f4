"""Request layouts and WCA parameters on the CPU.

RequestPlan follows src/cacheslide_vllm/contracts.py:26-181 (schema version 1,
canonical-JSON SHA-256 identities); WCAConfig follows policy.py:21-45.
"""

from __future__ import annotations

import hashlib
import json

import pytest

from cacheslide_amd import RequestPlan, WCAConfig
from cacheslide_amd.contracts import digest


def meta(*chunks, **top):
    doc = {"version": 1, "operation": "reuse", "namespace": "ns", "task_id": "t"}
    doc.update(top)
    doc["chunks"] = [{"id": i, "role": r, "start": s, "end": e} for i, r, s, e in chunks]
    return doc


LAYOUT = (("sys", "reuse", 0, 3), ("doc", "reuse", 3, 5), ("q", "recompute", 5, 7))
TOKENS = [5, 6, 7, 8, 9, 10, 11]


def test_digest_is_sha256_of_canonical_json():
    assert digest([1, 2]) == hashlib.sha256(b"[1,2]").hexdigest()
    assert digest({"b": 1, "a": "x"}) == hashlib.sha256(b'{"a":"x","b":1}').hexdigest()
    with pytest.raises(ValueError):
        digest(float("nan"))


def test_plan_indices_layout_and_round_trip():
    plan = RequestPlan.parse(meta(*LAYOUT), TOKENS)
    assert plan.fixed_indices == (0, 1, 2, 3, 4)
    assert plan.mandatory_indices == (5, 6)
    assert plan.fixed_layout == (("sys", digest((5, 6, 7)), 3), ("doc", digest((8, 9)), 2))
    assert RequestPlan.parse(plan.to_json(), TOKENS) == plan
    assert RequestPlan.parse(json.dumps(meta(*LAYOUT)), TOKENS) == plan
    # a reused last chunk still makes the last token mandatory
    tail = RequestPlan.parse(meta(("q", "recompute", 0, 2), ("doc", "reuse", 2, 4)), [1, 2, 3, 4])
    assert tail.mandatory_indices == (0, 1, 3)


def test_identities_follow_the_ordered_fixed_template():
    plan = RequestPlan.parse(meta(*LAYOUT), TOKENS)
    longer_query = RequestPlan.parse(meta(*LAYOUT[:2], ("q", "recompute", 5, 9)), TOKENS + [12, 13])
    assert plan.cache_key("m", 3) == longer_query.cache_key("m", 3)
    assert plan.profile_key("m", 3) == longer_query.profile_key("m", 3)
    swapped = RequestPlan.parse(meta(("doc", "reuse", 0, 2), ("sys", "reuse", 2, 5), LAYOUT[2]),
                                [8, 9, 5, 6, 7, 10, 11])
    assert swapped.cache_key("m", 3) != plan.cache_key("m", 3)
    edited = RequestPlan.parse(meta(*LAYOUT), [5, 6, 7, 8, 99, 10, 11])
    assert edited.cache_key("m", 3) != plan.cache_key("m", 3)
    assert plan.cache_key("m", 3) != plan.cache_key("m", 4) != plan.cache_key("other", 4)
    assert plan.profile_key("m", 3) != plan.cache_key("m", 3)


@pytest.mark.parametrize("doc, tokens, message", [
    (meta(*LAYOUT, version=2), TOKENS, "schema version"),
    (meta(*LAYOUT, version=True), TOKENS, "schema version"),
    (meta(*LAYOUT, extra=1), TOKENS, "schema version"),
    (meta(*LAYOUT, operation="train"), TOKENS, "operation must be"),
    (meta(*LAYOUT, namespace=""), TOKENS, "namespace must be a nonempty string"),
    (meta(*LAYOUT, task_id="a\nb"), TOKENS, "control characters"),
    (meta(*LAYOUT), [], "prompt token ids"),
    (meta(*LAYOUT), [1, -2, 3, 4, 5, 6, 7], "prompt token ids"),
    (meta(), TOKENS, "nonempty list"),
    (meta(("a", "reuse", 0, 3), ("b", "recompute", 4, 7)), TOKENS, "without gaps"),
    (meta(("a", "reuse", 0, 3), ("b", "recompute", 3, 8)), TOKENS, "without gaps"),
    (meta(("a", "reuse", 0, 3), ("a", "recompute", 3, 7)), TOKENS, "duplicate chunk id"),
    (meta(("a", "other", 0, 7)), TOKENS, "invalid role"),
    (meta(("a", "reuse", 0, 6)), TOKENS, "every prompt token"),
    (meta(("a", "reuse", True, 7)), TOKENS, "integer token offsets"),
    ({"version": 1, "operation": "reuse", "namespace": "n", "task_id": "t",
      "chunks": [{"id": "a", "role": "reuse", "start": 0}]}, TOKENS, "exactly id, role, start, end"),
    ("[1, 2]", TOKENS, "JSON object"),
])
def test_invalid_requests_raise_value_errors(doc, tokens, message):
    with pytest.raises(ValueError, match=message):
        RequestPlan.parse(doc, tokens)


def test_chunk_count_and_metadata_size_limits():
    many = meta(*((f"c{i}", "recompute", i, i + 1) for i in range(1025)))
    with pytest.raises(ValueError, match="at most 1024 chunks"):
        RequestPlan.parse(many, list(range(1025)))
    with pytest.raises(ValueError, match="exceeds 1 MiB"):
        RequestPlan.parse(" " * (1 << 20) + json.dumps(meta(*LAYOUT)), TOKENS)


def test_wca_config_defaults_and_validation():
    config = WCAConfig()
    assert (config.correction_fraction, config.epsilon, config.gate_interval,
            config.convergence_threshold, config.convergence_mode, config.weight_update,
            config.clamp_alpha) == (0.26, 1e-8, 4, 0.12, "paper_cosine_lt", "previous_layer", False)
    for kwargs, message in (
        ({"correction_fraction": True}, "not a boolean"),
        ({"epsilon": float("inf")}, "finite real number"),
        ({"convergence_threshold": 10 ** 400}, "finite real number"),
        ({"correction_fraction": 1.5}, r"\[0, 1\]"),
        ({"epsilon": 0.0}, "finite and positive"),
        ({"gate_interval": 0}, "positive integer"),
        ({"gate_interval": 2.0}, "positive integer"),
        ({"clamp_alpha": 1}, "boolean"),
        ({"convergence_mode": "cosine"}, "convergence_mode"),
        ({"weight_update": "next_layer"}, "weight_update"),
    ):
        with pytest.raises(ValueError, match=message):
            WCAConfig(**kwargs)
    assert WCAConfig(correction_fraction=1, convergence_mode="distance_lt",
                     weight_update="same_layer", clamp_alpha=True).correction_fraction == 1
