"""CCPE profile artifacts: the on-disk format of src/cacheslide_vllm/profiles.py.

A profile directory holds ``manifest.json`` and ``profiles.safetensors``.  The
manifest (format ``cacheslide-profiles-v1``) names the adapter identity, the
model geometry, one entry per profile key (layer, ordered fixed chunks,
histogram bin width, sample count), the SHA-256 of the tensor file and its
own canonical-JSON digest.  The tensor file holds, per key, the canonical
positions ``[heads, F, F]`` fp32 and the ordinal query/key vectors ``[F]``
int64.  Files written by the reference load here and files written here load
there: the manifest fields, checksums, tensor names, dtypes and the
ValueError messages are the reference's (profiles.py:19-251, 346-401).

* ``ProfileBundle`` validates a directory completely (sizes, checksums,
  fields, geometry, tensor headers, canonical ordinals, bounded and causal
  positions) before it builds any profile; ``get`` selects by the request's
  profile key and checks the ordered fixed layout (profiles.py:112-251).
* ``save_profiles`` writes the artifact of already calibrated profiles into
  a new directory (the save half of ``calibrate_profiles``, profiles.py:346-401).
* ``calibrate_from_forward`` is ``calibrate_profiles`` (profiles.py:254-401)
  for a caller that owns the model: it budgets the run, drives the caller's
  forward with an observer that takes each layer's device trace through
  ``CoPE.position_trace`` and ``project``, calibrates each profile key on the
  device (``CCPEProfile.calibrate``) and saves the artifact.
"""

from __future__ import annotations

import hashlib
import json
import math
import re
from collections.abc import Callable, Mapping, Sequence
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .contracts import RequestPlan, digest
from .position import CCPEProfile, ChunkIdentity, CoPE, CoPEPositionTrace

PROFILE_FORMAT = "cacheslide-profiles-v1"
_MAX_JSON_BYTES = 8 * 1024 * 1024
_HEX64 = re.compile(r"[0-9a-f]{64}")
_MANIFEST_FIELDS = frozenset((
    "format", "adapter_identity", "trained_profile_version", "num_layers", "query_heads",
    "max_positions", "profiles", "tensors_sha256", "manifest_sha256",
))
_ENTRY_FIELDS = frozenset(("layer", "chunks", "histogram_bin_width", "sample_count"))
_CHUNK_FIELDS = frozenset(("role", "content_hash", "length"))


# ---------------------------------------------------------------- field checks
def _int_at_least(value: object, name: str, minimum: int = 1) -> int:
    if type(value) is not int or value < minimum:
        raise ValueError(f"{name} must be an integer >= {minimum}")
    return value


def _text(value: object, name: str) -> str:
    ok = (isinstance(value, str) and value.strip() != "" and len(value) <= 256
          and all(ord(ch) >= 32 for ch in value))
    if not ok:
        raise ValueError(f"invalid {name}")
    return value


def _sha(value: object, name: str) -> str:
    if not (isinstance(value, str) and _HEX64.fullmatch(value)):
        raise ValueError(f"invalid {name} SHA-256")
    return value


def _exact_fields(value: object, fields: frozenset, name: str) -> dict:
    if not (isinstance(value, dict) and set(value) == fields):
        raise ValueError(f"invalid {name} fields")
    return value


def _no_duplicates(pairs: list[tuple[str, object]]) -> dict:
    seen: dict = {}
    for name, value in pairs:
        if name in seen:
            raise ValueError(f"duplicate JSON field: {name}")
        seen[name] = value
    return seen


def _reject_constant(token: str) -> None:
    raise ValueError(f"nonfinite JSON value: {token}")


def file_sha256(path: Path) -> str:
    """Hex SHA-256 of a file's bytes, read in 8 MiB blocks."""
    h = hashlib.sha256()
    with path.open("rb") as stream:
        for block in iter(lambda: stream.read(8 << 20), b""):
            h.update(block)
    return h.hexdigest()


def _regular_file(directory: Path, name: str) -> Path:
    path = directory / name
    if path.is_symlink() or not path.is_file():
        raise ValueError(f"artifact requires a regular, non-symlink {name}")
    return path


def _plan_chunks(plan: RequestPlan) -> tuple[ChunkIdentity, ...]:
    return tuple(ChunkIdentity(cid, content, length) for cid, content, length in plan.fixed_layout)


def _manifest(path: Path) -> dict:
    if path.stat().st_size > _MAX_JSON_BYTES:
        raise ValueError("profile metadata exceeds size budget")
    doc = json.loads(path.read_text(), object_pairs_hook=_no_duplicates,
                     parse_constant=_reject_constant)
    _exact_fields(doc, _MANIFEST_FIELDS, "profile manifest")
    claimed = _sha(doc["manifest_sha256"], "manifest")
    if digest({k: v for k, v in doc.items() if k != "manifest_sha256"}) != claimed:
        raise ValueError("profile manifest checksum mismatch")
    return doc


def _entry_spec(key: str, entry: object, layers: int) -> tuple[dict, tuple[ChunkIdentity, ...], int]:
    """One manifest entry -> (entry, ordered chunks, fixed token count)."""
    _sha(key, "profile key")
    entry = _exact_fields(entry, _ENTRY_FIELDS, "profile entry")
    if _int_at_least(entry["layer"], "layer", 0) >= layers:
        raise ValueError("profile layer outside model geometry")
    raw = entry["chunks"]
    if not (isinstance(raw, list) and 1 <= len(raw) <= 1024):
        raise ValueError("profile requires ordered fixed chunks")
    chunks = []
    for item in raw:
        item = _exact_fields(item, _CHUNK_FIELDS, "chunk identity")
        chunks.append(ChunkIdentity(_text(item["role"], "chunk role"), _sha(item["content_hash"], "chunk"),
                                    _int_at_least(item["length"], "chunk length")))
    if len({chunk.role for chunk in chunks}) != len(chunks):
        raise ValueError("duplicate ordered fixed chunk identity")
    width = entry["histogram_bin_width"]
    if type(width) not in (int, float) or not math.isfinite(width) or width <= 0:
        raise ValueError("invalid histogram bin width")
    _int_at_least(entry["sample_count"], "sample_count")
    return entry, tuple(chunks), sum(chunk.length for chunk in chunks)


class ProfileBundle:
    """Canonical CCPE profiles of one adapter, validated before any tensor is read.

    ``max_elements`` bounds the sum of all stored tensor elements (positions
    and both ordinal vectors).  ``get`` returns None on a miss; callers then use
    contextual attention (no extrapolation).
    """

    def __init__(self, path: str | Path, adapter_identity: str, max_elements: int = 1_000_000):
        _int_at_least(max_elements, "max_elements")
        _sha(adapter_identity, "adapter identity")
        self.path = Path(path).resolve(strict=True)
        doc = _manifest(_regular_file(self.path, "manifest.json"))
        if doc["format"] != PROFILE_FORMAT:
            raise ValueError("unsupported CacheSlide profile format version")
        if doc["adapter_identity"] != adapter_identity:
            raise ValueError("profile adapter identity mismatch")
        version = _text(doc["trained_profile_version"], "profile version")
        layers = _int_at_least(doc["num_layers"], "num_layers")
        heads = _int_at_least(doc["query_heads"], "query_heads")
        max_positions = _int_at_least(doc["max_positions"], "max_positions", 2)
        entries = doc["profiles"]
        if not (isinstance(entries, dict) and entries):
            raise ValueError("profile manifest requires nonempty profiles")

        specs: dict[str, tuple[dict, tuple[ChunkIdentity, ...], int]] = {}
        layout: dict[str, tuple[tuple[int, ...], str]] = {}
        elements = 0
        for key, raw in entries.items():
            specs[key] = spec = _entry_spec(key, raw, layers)
            count = spec[2]
            elements += heads * count * count + 2 * count
            if elements > max_elements:
                raise ValueError("profile tensors exceed max_elements budget")
            layout[f"{key}.positions"] = ((heads, count, count), "F32")
            layout[f"{key}.query_positions"] = ((count,), "I64")
            layout[f"{key}.key_positions"] = ((count,), "I64")

        tensor_file = _regular_file(self.path, "profiles.safetensors")
        if tensor_file.stat().st_size > max_elements * 8 + _MAX_JSON_BYTES:
            raise ValueError("profile tensor file exceeds size budget")
        if file_sha256(tensor_file) != _sha(doc["tensors_sha256"], "tensor"):
            raise ValueError("profile tensor checksum mismatch")

        self._profiles: dict[str, CCPEProfile] = {}
        with safe_open(tensor_file, framework="pt", device="cpu") as source:
            if set(source.keys()) != set(layout):
                raise ValueError("profile tensor keys mismatch")
            # headers first: shapes and dtypes of every tensor before any data
            for name, (shape, dtype) in layout.items():
                header = source.get_slice(name)
                if tuple(header.get_shape()) != shape or header.get_dtype() != dtype:
                    raise ValueError("profile tensor layout/dtype mismatch")
            for key, (entry, chunks, count) in specs.items():
                table = source.get_tensor(f"{key}.positions")
                rows = source.get_tensor(f"{key}.query_positions")
                cols = source.get_tensor(f"{key}.key_positions")
                ordinals = torch.arange(count)
                if not (torch.equal(rows, ordinals) and torch.equal(cols, ordinals)):
                    raise ValueError("profile query/key layout must be canonical ordinals")
                bounded = bool(torch.isfinite(table).all()) and not bool((table < 0).any()) \
                    and not bool((table > max_positions - 1).any())
                if not bounded:
                    raise ValueError("profile positions must be finite and bounded")
                if table.triu(diagonal=1).count_nonzero():
                    raise ValueError("profile has noncausal canonical positions")
                self._profiles[key] = CCPEProfile(
                    trained_profile_version=version, checkpoint_id=adapter_identity, chunks=chunks,
                    query_positions=rows, key_positions=cols, canonical_positions=table,
                    max_positions=max_positions, histogram_bin_width=float(entry["histogram_bin_width"]),
                    sample_count=entry["sample_count"],
                )
        self.metadata = doc
        self.identity = digest(doc)
        self.adapter_identity = adapter_identity

    def get(self, plan: RequestPlan, layer: int) -> CCPEProfile | None:
        """The profile of the request's namespace/task/ordered fixed layout at ``layer``."""
        _int_at_least(layer, "layer", 0)
        key = plan.profile_key(self.adapter_identity, layer)
        profile = self._profiles.get(key)
        if profile is None:
            return None
        if self.metadata["profiles"][key]["layer"] != layer:
            raise ValueError("profile key refers to a different layer")
        ordinals = torch.arange(len(plan.fixed_indices))
        profile.lookup(_plan_chunks(plan), ordinals, ordinals, checkpoint_id=self.adapter_identity,
                       trained_profile_version=self.metadata["trained_profile_version"])
        return profile


def save_profiles(
    output: str | Path,
    profiles: Mapping[str, tuple[int, CCPEProfile]],
    *,
    adapter_identity: str,
    num_layers: int,
    query_heads: int,
    max_positions: int,
    trained_profile_version: str,
) -> Path:
    """Write ``{profile key: (layer, profile)}`` as a new profile directory.

    The directory is created only here and never overwritten; tensors are
    saved in key order, the manifest last.
    """
    output = Path(output)
    if output.exists() or output.is_symlink():
        raise FileExistsError(f"profile output already exists: {output}")
    if not profiles:
        raise ValueError("profile manifest requires nonempty profiles")
    tensors: dict[str, torch.Tensor] = {}
    entries: dict[str, dict] = {}
    for key in sorted(profiles):
        layer, profile = profiles[key]
        _sha(key, "profile key")
        tensors[f"{key}.positions"] = profile.canonical_positions.detach().float().cpu().contiguous()
        tensors[f"{key}.query_positions"] = profile.query_positions.detach().cpu().contiguous()
        tensors[f"{key}.key_positions"] = profile.key_positions.detach().cpu().contiguous()
        entries[key] = {
            "layer": layer,
            "chunks": [{"role": c.role, "content_hash": c.content_hash, "length": c.length}
                       for c in profile.chunks],
            "histogram_bin_width": profile.histogram_bin_width,
            "sample_count": profile.sample_count,
        }
    output.mkdir(parents=True, exist_ok=False)
    tensor_file = output / "profiles.safetensors"
    save_file(tensors, str(tensor_file))
    doc = {
        "format": PROFILE_FORMAT,
        "adapter_identity": adapter_identity,
        "trained_profile_version": trained_profile_version,
        "num_layers": num_layers,
        "query_heads": query_heads,
        "max_positions": max_positions,
        "profiles": entries,
        "tensors_sha256": file_sha256(tensor_file),
    }
    doc["manifest_sha256"] = digest(doc)
    (output / "manifest.json").write_text(json.dumps(doc, indent=2) + "\n")
    return output


Observer = Callable[[int, torch.Tensor, torch.Tensor, CoPE], None]


def calibrate_from_forward(
    forward: Callable[[RequestPlan, Observer], None],
    requests: Sequence[RequestPlan],
    output: str | Path,
    *,
    adapter_identity: str,
    num_layers: int,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    max_positions: int,
    max_elements: int = 1_000_000,
    trained_profile_version: str = "v1",
) -> Path:
    """Calibrate and save the CCPE profiles of ``requests`` (profiles.py:254-401).

    ``forward(plan, observer)`` runs the caller's frozen model on the plan's
    full prompt and calls ``observer(layer, query, key, cope)`` once per
    attention layer with that layer's ``[T, Hq, D]`` queries and ``[T, Hkv, D]``
    keys.  The whole run is budgeted before any trace exists; each layer's
    fixed x fixed positions are traced on the device; traces never reach the
    artifact.
    """
    _int_at_least(max_elements, "max_elements")
    _text(trained_profile_version, "trained_profile_version")
    _sha(adapter_identity, "adapter identity")
    output = Path(output)
    if output.exists() or output.is_symlink():
        raise FileExistsError(f"profile output already exists: {output}")
    if not requests:
        raise ValueError("calibration requires at least one request")
    plans: list[RequestPlan] = []
    for request in requests:
        if not isinstance(request, RequestPlan):
            raise ValueError("calibration requires validated RequestPlan inputs")
        plan = RequestPlan.parse(request.to_json(), request.token_ids)
        if not plan.fixed_indices:
            raise ValueError("each calibration request needs a reusable fixed chunk")
        plans.append(plan)

    # budget: every source trace plus every stored profile, before any trace
    key_layer: dict[str, int] = {}
    key_chunks: dict[str, tuple[ChunkIdentity, ...]] = {}
    budget = 0
    for plan in plans:
        tokens, fixed = len(plan.token_ids), len(plan.fixed_indices)
        budget += num_layers * query_heads * (tokens * tokens + fixed * fixed)
        for layer in range(num_layers):
            key = plan.profile_key(adapter_identity, layer)
            if key not in key_chunks:
                budget += query_heads * fixed * fixed + 2 * fixed
                key_chunks[key] = _plan_chunks(plan)
                key_layer[key] = layer
        if budget > max_elements:
            raise ValueError("CCPE calibration source traces exceed max_elements budget")

    traces: dict[str, list[CoPEPositionTrace]] = {key: [] for key in key_chunks}
    for plan in plans:
        tokens = len(plan.token_ids)
        fixed = torch.tensor(plan.fixed_indices, dtype=torch.long)
        seen: set[int] = set()

        def observer(layer: int, query: torch.Tensor, key: torch.Tensor, cope: CoPE) -> None:
            if type(layer) is not int or not 0 <= layer < num_layers or layer in seen:
                raise ValueError("reference observer emitted an invalid/repeated layer")
            if tuple(query.shape) != (tokens, query_heads, head_dim) or \
                    tuple(key.shape) != (tokens, kv_heads, head_dim):
                raise ValueError("reference observer Q/K layout mismatch")
            trace = cope.position_trace(query, key, torch.arange(tokens, device=query.device),
                                        checkpoint_id=adapter_identity, max_elements=max_elements)
            traces[plan.profile_key(adapter_identity, layer)].append(
                trace.project(fixed, fixed, canonical_positions=True))
            seen.add(layer)

        with torch.inference_mode():
            forward(plan, observer)
        if seen != set(range(num_layers)):
            raise ValueError("reference model did not observe every attention layer")

    calibrated = {
        key: (key_layer[key], CCPEProfile.calibrate(samples, key_chunks[key],
                                                    trained_profile_version=trained_profile_version,
                                                    max_elements=max_elements))
        for key, samples in traces.items()
    }
    return save_profiles(output, calibrated, adapter_identity=adapter_identity, num_layers=num_layers,
                         query_heads=query_heads, max_positions=max_positions,
                         trained_profile_version=trained_profile_version)
