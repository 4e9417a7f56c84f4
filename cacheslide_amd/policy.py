"""WCA parameters (src/cacheslide_vllm/policy.py:21-45), pure Python.

Same fields, defaults, accepted values and ValueError messages as the
reference's WCAConfig; the checks are table-driven here.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal


def _finite_number(name: str, value: object) -> None:
    """Accept an int or float (bool, str and complex are not) with a finite value."""
    if type(value) not in (int, float):
        raise ValueError(f"{name} must be a finite real number, not a boolean")
    try:
        finite = math.isfinite(value)
    except OverflowError:  # an int beyond the float range
        finite = False
    if not finite:
        raise ValueError(f"{name} must be a finite real number")


# name -> (test, message) for each scalar field after the finiteness checks
_RULES = (
    ("correction_fraction", lambda x: 0 <= x <= 1, "correction_fraction must be in [0, 1]"),
    ("epsilon", lambda x: x > 0, "epsilon must be finite and positive"),
    ("gate_interval", lambda x: type(x) is int and x >= 1, "gate_interval must be a positive integer"),
    ("clamp_alpha", lambda x: type(x) is bool, "clamp_alpha must be a boolean"),
    ("convergence_mode", lambda x: x in ("paper_cosine_lt", "distance_lt"), "unknown convergence_mode"),
    ("weight_update", lambda x: x in ("previous_layer", "same_layer"), "unknown weight_update"),
)


@dataclass(frozen=True)
class WCAConfig:
    correction_fraction: float = 0.26
    epsilon: float = 1e-8
    gate_interval: int = 4
    convergence_threshold: float = 0.12
    convergence_mode: Literal["paper_cosine_lt", "distance_lt"] = "paper_cosine_lt"
    weight_update: Literal["previous_layer", "same_layer"] = "previous_layer"
    clamp_alpha: bool = False

    def __post_init__(self) -> None:
        for name in ("correction_fraction", "epsilon", "convergence_threshold"):
            _finite_number(name, getattr(self, name))
        for name, test, message in _RULES:
            if not test(getattr(self, name)):
                raise ValueError(message)
