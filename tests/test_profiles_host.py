"""CCPE profile artifacts on the CPU: the format of src/cacheslide_vllm/profiles.py.

Round trip through ``save_profiles`` and ``ProfileBundle``, then every check
the reference loader makes (profiles.py:80-251): manifest fields and digest,
duplicate/nonfinite JSON, symlinks, the tensor checksum, tensor keys, shapes
and dtypes, canonical ordinals, bounded and causal positions, geometry,
budgets, and selection by the request's profile key.
"""

from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file, save_file

from cacheslide_amd import CCPEProfile, ChunkIdentity, RequestPlan
from cacheslide_amd.contracts import digest
from cacheslide_amd.profiles import PROFILE_FORMAT, ProfileBundle, file_sha256, save_profiles

ADAPTER = hashlib.sha256(b"adapter").hexdigest()
TOKENS = [11, 12, 13, 14, 15, 16]


def plan(tokens=TOKENS):
    doc = {"version": 1, "operation": "reuse", "namespace": "ns", "task_id": "t",
           "chunks": [{"id": "sys", "role": "reuse", "start": 0, "end": 3},
                      {"id": "doc", "role": "reuse", "start": 3, "end": 5},
                      {"id": "q", "role": "recompute", "start": 5, "end": 6}]}
    return RequestPlan.parse(doc, tokens)


def profile_of(p: RequestPlan, heads=2, max_positions=8, version="v1") -> CCPEProfile:
    fixed = len(p.fixed_indices)
    table = torch.tril(torch.arange(heads * fixed * fixed, dtype=torch.float32).reshape(heads, fixed, fixed)
                       % max_positions)
    chunks = tuple(ChunkIdentity(cid, content, length) for cid, content, length in p.fixed_layout)
    return CCPEProfile(trained_profile_version=version, checkpoint_id=ADAPTER, chunks=chunks,
                       query_positions=torch.arange(fixed), key_positions=torch.arange(fixed),
                       canonical_positions=table, max_positions=max_positions,
                       histogram_bin_width=0.25, sample_count=3)


def write(tmp_path: Path, layers=2, heads=2, max_positions=8) -> Path:
    p = plan()
    profiles = {p.profile_key(ADAPTER, layer): (layer, profile_of(p, heads, max_positions))
                for layer in range(layers)}
    return save_profiles(tmp_path / "profiles", profiles, adapter_identity=ADAPTER, num_layers=layers,
                         query_heads=heads, max_positions=max_positions, trained_profile_version="v1")


def rewrite_manifest(path: Path, edit) -> None:
    """Apply edit(doc) and recompute the manifest digest (a well-formed forgery)."""
    doc = json.loads((path / "manifest.json").read_text())
    edit(doc)
    doc.pop("manifest_sha256", None)
    doc["manifest_sha256"] = digest(doc)
    (path / "manifest.json").write_text(json.dumps(doc))


def rewrite_tensors(path: Path, edit) -> None:
    tensors = load_file(str(path / "profiles.safetensors"))
    edit(tensors)
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(path / "profiles.safetensors"))
    rewrite_manifest(path, lambda d: d.update(tensors_sha256=file_sha256(path / "profiles.safetensors")))


def test_round_trip_and_selection(tmp_path):
    out = write(tmp_path)
    doc = json.loads((out / "manifest.json").read_text())
    assert doc["format"] == PROFILE_FORMAT
    assert set(doc) == {"format", "adapter_identity", "trained_profile_version", "num_layers",
                        "query_heads", "max_positions", "profiles", "tensors_sha256", "manifest_sha256"}
    assert doc["tensors_sha256"] == hashlib.sha256((out / "profiles.safetensors").read_bytes()).hexdigest()
    bundle = ProfileBundle(out, ADAPTER)
    p = plan()
    for layer in range(2):
        got = bundle.get(p, layer)
        want = profile_of(p)
        assert torch.equal(got.canonical_positions, want.canonical_positions)
        assert got.chunks == want.chunks and got.sample_count == 3 and got.histogram_bin_width == 0.25
        assert got.checkpoint_id == ADAPTER and got.trained_profile_version == "v1"
    assert bundle.get(p, 2) is None                       # no profile for that layer
    assert bundle.get(plan([11, 12, 99, 14, 15, 16]), 0) is None  # other fixed content
    with pytest.raises(ValueError, match="layer must be an integer"):
        bundle.get(p, -1)
    assert bundle.identity == digest(doc)
    with pytest.raises(FileExistsError):
        write(tmp_path)


@pytest.mark.parametrize("edit, message", [
    (lambda d: d.update(format="cacheslide-profiles-v0"), "unsupported CacheSlide profile format"),
    (lambda d: d.update(num_layers=1), "profile layer outside model geometry"),
    (lambda d: d.update(max_positions=1), "max_positions must be an integer >= 2"),
    (lambda d: d.update(trained_profile_version=" "), "invalid profile version"),
    (lambda d: d.update(profiles={}), "requires nonempty profiles"),
    (lambda d: d.update(extra=1), "invalid profile manifest fields"),
    (lambda d: next(iter(d["profiles"].values())).update(histogram_bin_width=0), "invalid histogram bin width"),
    (lambda d: next(iter(d["profiles"].values())).update(sample_count=0), "sample_count must be an integer"),
    (lambda d: next(iter(d["profiles"].values())).update(chunks=[]), "ordered fixed chunks"),
    (lambda d: next(iter(d["profiles"].values()))["chunks"][1].update(role="sys"), "duplicate ordered fixed chunk"),
    (lambda d: next(iter(d["profiles"].values()))["chunks"][0].update(content_hash="x"), "invalid chunk SHA-256"),
    (lambda d: d["profiles"].update({"nothex": d["profiles"].pop(next(iter(d["profiles"])))}),
     "invalid profile key SHA-256"),
])
def test_invalid_manifest_rejected_even_with_new_checksum(tmp_path, edit, message):
    out = write(tmp_path)
    rewrite_manifest(out, edit)
    with pytest.raises(ValueError, match=message):
        ProfileBundle(out, ADAPTER)


def test_manifest_integrity(tmp_path):
    out = write(tmp_path)
    with pytest.raises(ValueError, match="adapter identity mismatch"):
        ProfileBundle(out, hashlib.sha256(b"other").hexdigest())
    with pytest.raises(ValueError, match="invalid adapter identity SHA-256"):
        ProfileBundle(out, "adapter")
    text = (out / "manifest.json").read_text()
    (out / "manifest.json").write_text(text.replace('"num_layers": 2', '"num_layers": 3'))
    with pytest.raises(ValueError, match="manifest checksum mismatch"):
        ProfileBundle(out, ADAPTER)
    (out / "manifest.json").write_text('{"format": 1, "format": 2}')
    with pytest.raises(ValueError, match="duplicate JSON field: format"):
        ProfileBundle(out, ADAPTER)
    (out / "manifest.json").write_text('{"format": NaN}')
    with pytest.raises(ValueError, match="nonfinite JSON value: NaN"):
        ProfileBundle(out, ADAPTER)


def test_tensor_file_integrity(tmp_path):
    out = write(tmp_path)
    data = bytearray((out / "profiles.safetensors").read_bytes())
    data[-1] ^= 1
    (out / "profiles.safetensors").write_bytes(bytes(data))
    with pytest.raises(ValueError, match="tensor checksum mismatch"):
        ProfileBundle(out, ADAPTER)


@pytest.mark.parametrize("edit, message", [
    (lambda t: t.update({k: v.double() for k, v in t.items() if k.endswith(".positions")}),
     "tensor layout/dtype mismatch"),
    (lambda t: t.update({k: v[:, :-1] for k, v in t.items() if k.endswith(".positions")}),
     "tensor layout/dtype mismatch"),
    (lambda t: t.update(extra=torch.zeros(1)), "tensor keys mismatch"),
    (lambda t: t.update({k: v.flip(0) for k, v in t.items() if k.endswith(".query_positions")}),
     "canonical ordinals"),
    (lambda t: t.update({k: torch.ones_like(v) for k, v in t.items() if k.endswith(".positions")}),
     "noncausal canonical positions"),
    (lambda t: t.update({k: v * 100 for k, v in t.items() if k.endswith(".positions")}),
     "finite and bounded"),
    (lambda t: t.update({k: v - 1 for k, v in t.items() if k.endswith(".positions")}),
     "finite and bounded"),
    (lambda t: t.update({k: v.masked_fill(v == 1, float("nan")) for k, v in t.items() if k.endswith(".positions")}),
     "finite and bounded"),
])
def test_corrupt_tensor_layout_rejected_even_with_new_checksum(tmp_path, edit, message):
    out = write(tmp_path)
    rewrite_tensors(out, edit)
    with pytest.raises(ValueError, match=message):
        ProfileBundle(out, ADAPTER)


def test_budgets(tmp_path):
    out = write(tmp_path)
    # 2 layers x (2 heads x 5 x 5 + 2 x 5) = 120 elements
    ProfileBundle(out, ADAPTER, max_elements=120)
    with pytest.raises(ValueError, match="exceed max_elements budget"):
        ProfileBundle(out, ADAPTER, max_elements=119)
    with pytest.raises(ValueError, match="max_elements must be an integer >= 1"):
        ProfileBundle(out, ADAPTER, max_elements=0)


def test_files_cannot_be_symlinks(tmp_path):
    out = write(tmp_path)
    elsewhere = tmp_path / "elsewhere.json"
    os.replace(out / "manifest.json", elsewhere)
    (out / "manifest.json").symlink_to(elsewhere)
    with pytest.raises(ValueError, match="regular, non-symlink manifest.json"):
        ProfileBundle(out, ADAPTER)
    os.remove(out / "manifest.json")
    os.replace(elsewhere, out / "manifest.json")
    tensors = tmp_path / "elsewhere.safetensors"
    os.replace(out / "profiles.safetensors", tensors)
    (out / "profiles.safetensors").symlink_to(tensors)
    with pytest.raises(ValueError, match="regular, non-symlink profiles.safetensors"):
        ProfileBundle(out, ADAPTER)
