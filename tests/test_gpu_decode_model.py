"""End-to-end decode steps of the paged decoder (cacheslide_amd/decode_model.py)
against a float32 restatement on the CPU whose attention is the oracle's
cope_attention over the request's gathered keys (the decode call of
src/cacheslide_vllm/runtime.py:489-508 over paged.py:433-472).

Workload: 2 layers, hidden 512 (4 query heads, 2 KV heads, head_dim 128), FFN
1024, vocab 1000, CoPE P = 64, bf16 weights N(0, 0.02); three requests with
contexts of 300, 170 and 45 keys drawn N(0, 1) into a paged cache of block 16
with a shuffled block table; 4 decode steps, teacher-forced with the tokens of
the device run.  Logits agree within 3e-2 (bf16 activations between the
GEMMs against float32 throughout).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd import _hip
from cacheslide_amd.ccpe import decode_workspace, raise_flags
from cacheslide_amd.decode_model import MISTRAL_7B, DecoderShape, PagedDecoder
from oracle import ccpe as orc

SHAPE = DecoderShape(layers=2, hidden=512, heads=4, kv_heads=2, ffn=1024, vocab=1000, npos=64)
LENS = [300, 170, 45]
STEPS = 4
BS = 16


def test_mistral_shape_parameter_count():
    # 7,241,732,096 parameters: 14.48 GB of bf16 weights read per decode step
    assert MISTRAL_7B.parameters == 7_241_732_096
    with pytest.raises(ValueError):
        DecoderShape(hidden=4000)
    with pytest.raises(ValueError):
        DecoderShape(heads=32, kv_heads=2)


def layout(device):
    gen = torch.Generator().manual_seed(404)
    per = [(n + STEPS + BS - 1) // BS for n in LENS]
    cols = max(per)
    perm = torch.randperm(sum(per), generator=gen)
    table = torch.zeros((len(LENS), cols), dtype=torch.int32)
    at = 0
    for b, p in enumerate(per):
        table[b, :p] = perm[at:at + p].to(torch.int32)
        at += p
    return sum(per), table.to(device)


def gathered(cache, table_row, n):
    """[n, Hkv, 2 x 128] records of keys 0..n-1 of one request (float32, CPU)."""
    blocks = cache[table_row.long()].permute(0, 2, 1, 3).reshape(-1, cache.shape[1], cache.shape[3])
    return blocks[:n].float().cpu()


def reference_step(model, ids, kv, heads, kv_heads):
    """float32 layer loop of the decoder with oracle attention; kv[l][b] holds
    the request's [n, Hkv, 256] records and gains this token's."""
    w = lambda t: t.detach().float().cpu()  # noqa: E731
    s = model.shape
    x = w(model.embed)[ids.cpu()]
    residual = None
    for li, layer in enumerate(model.layers):
        residual = x if residual is None else x + residual
        h = torch.nn.functional.rms_norm(residual, (s.hidden,), w(layer.in_norm), s.eps)
        qkv = h @ w(layer.qkv).T
        q = qkv[:, :heads * 128].view(-1, heads, 128)
        k = qkv[:, heads * 128:(heads + kv_heads) * 128].view(-1, kv_heads, 128)
        v = qkv[:, (heads + kv_heads) * 128:].view(-1, kv_heads, 128)
        e = w(layer.cope.position_embeddings).numpy()
        rows = []
        for b in range(len(ids)):
            kv[li][b] = torch.cat([kv[li][b], torch.cat([k[b], v[b]], dim=-1)[None]])
            rec = kv[li][b].numpy()
            n = rec.shape[0]
            rows.append(torch.from_numpy(orc.cope_attention(q[b:b + 1].numpy(), rec[..., :128], rec[..., 128:], e,
                                                            np.array([n - 1]))))
        attn = torch.cat(rows).reshape(len(ids), s.hidden)
        residual = attn @ w(layer.o).T + residual
        h = torch.nn.functional.rms_norm(residual, (s.hidden,), w(layer.post_norm), s.eps)
        gate, up = (h @ w(layer.gate_up).T).split(s.ffn, dim=-1)
        x = (torch.nn.functional.silu(gate) * up) @ w(layer.down).T
    h = torch.nn.functional.rms_norm(x + residual, (s.hidden,), w(model.norm), s.eps)
    return h @ w(model.lm_head).T


@pytest.mark.gpu
def test_decode_steps_match_float32_reference(device):
    model = PagedDecoder(SHAPE, device, seed=17)
    nblocks, table = layout(device)
    caches = model.new_caches(nblocks, BS)
    gen = torch.Generator(device=device).manual_seed(18)
    for c in caches:
        c.normal_(generator=gen)
    kv = [[gathered(c, table[b], n) for b, n in enumerate(LENS)] for c in caches]
    max_context = max(LENS) + STEPS
    ws = decode_workspace(len(LENS), SHAPE.heads, max_context, 1024, device)
    flags = _hip.new_flags(device)
    ids = torch.tensor([3, 500, 999], device=device)
    positions = torch.tensor(LENS, dtype=torch.long, device=device)
    for step in range(STEPS):
        got = model.step(ids, positions, caches, table, max_context=max_context, workspace=ws, flags=flags)
        want = reference_step(model, ids, kv, SHAPE.heads, SHAPE.kv_heads)
        torch.testing.assert_close(got.float().cpu(), want, atol=3e-2, rtol=3e-2, msg=f"step {step}")
        ids = got.argmax(-1)
        positions += 1
    raise_flags(flags)
    # the new tokens' records sit in their slots of every layer's cache
    for li, c in enumerate(caches):
        for b, n in enumerate(LENS):
            rec = gathered(c, table[b], n + STEPS)
            torch.testing.assert_close(rec[n:], kv[li][b][n:].to(torch.bfloat16).float(), atol=2e-2, rtol=2e-2)


MISTRAL_LENS = [600, 250]


@pytest.mark.gpu
def test_mistral_shaped_decode_steps_match_float32_reference(device):
    """The Mistral-7B layer shape (hidden 4096, 32 query / 8 KV heads, FFN
    14336, vocab 32000) at 2 layers: two requests with contexts of 600 and
    250 keys, 2 decode steps teacher-forced with the device's tokens, against
    the float32 restatement.  Tolerance 6e-2 absolute and relative on the
    logits: bf16 activations between the GEMMs of a 4096-wide model against
    float32 throughout."""
    shape = DecoderShape(layers=2)
    steps = 2
    model = PagedDecoder(shape, device, seed=23)
    gen = torch.Generator().manual_seed(405)
    per = [(n + steps + BS - 1) // BS for n in MISTRAL_LENS]
    perm = torch.randperm(sum(per), generator=gen)
    table = torch.zeros((len(MISTRAL_LENS), max(per)), dtype=torch.int32)
    at = 0
    for b, p in enumerate(per):
        table[b, :p] = perm[at:at + p].to(torch.int32)
        at += p
    table = table.to(device)
    caches = model.new_caches(sum(per), BS)
    dgen = torch.Generator(device=device).manual_seed(24)
    for c in caches:
        c.normal_(generator=dgen)
    kv = [[gathered(c, table[b], n) for b, n in enumerate(MISTRAL_LENS)] for c in caches]
    max_context = max(MISTRAL_LENS) + steps
    ws = decode_workspace(len(MISTRAL_LENS), shape.heads, max_context, 1024, device)
    flags = _hip.new_flags(device)
    ids = torch.tensor([7, 31999], device=device)
    positions = torch.tensor(MISTRAL_LENS, dtype=torch.long, device=device)
    for step in range(steps):
        got = model.step(ids, positions, caches, table, max_context=max_context, workspace=ws, flags=flags)
        want = reference_step(model, ids, kv, shape.heads, shape.kv_heads)
        assert bool(torch.isfinite(got.float()).all())
        torch.testing.assert_close(got.float().cpu(), want, atol=6e-2, rtol=6e-2, msg=f"step {step}")
        ids = got.argmax(-1)
        positions += 1
    raise_flags(flags)


@pytest.mark.gpu
def test_generate_is_greedy_over_step_and_checks_flags_once(device):
    model = PagedDecoder(SHAPE, device, seed=19)
    nblocks, table = layout(device)
    caches = model.new_caches(nblocks, BS)
    gen = torch.Generator(device=device).manual_seed(20)
    for c in caches:
        c.normal_(generator=gen)
    saved = [c.clone() for c in caches]
    first = torch.tensor([7, 8, 9], device=device)
    lengths = torch.tensor(LENS, dtype=torch.int32, device=device)
    max_context = max(LENS) + STEPS
    tokens = model.generate(first, lengths, caches, table, STEPS, max_context=max_context)
    # the same loop through step() from the saved caches
    ws = decode_workspace(len(LENS), SHAPE.heads, max_context, 1024, device)
    flags = _hip.new_flags(device)
    ids, positions = first, lengths.long()
    for t in range(STEPS):
        ids = model.step(ids, positions, saved, table, max_context=max_context, workspace=ws,
                         flags=flags).argmax(-1)
        assert torch.equal(ids, tokens[t])
        positions = positions + 1
    # a context beyond max_context is reported once, at the end of the loop
    with pytest.raises(ValueError, match="exceeds max_context"):
        model.generate(first, lengths, caches, table, 2, max_context=100)


@pytest.mark.gpu
def test_step_over_shared_runs_matches_per_request_decode(device):
    """``PagedDecoder.step`` with ``shared`` (the batch's reused chunks read once
    per layer, ccpe_decode_shared) against the same step with the per-request
    decode, from the same state: 4 requests holding 3 of 4 shared runs of 512
    keys in their own orders and 20-50 keys of their own; logits within 3e-2
    of the largest logit."""
    from cacheslide_amd.ccpe import SharedRuns, decode_shared_workspace

    b, n_runs, run_blocks, slots = 4, 4, 32, 3
    model = PagedDecoder(SHAPE, device, seed=77)
    own = [20 + 10 * i for i in range(b)]
    own_blocks = max((n + 1 + BS - 1) // BS for n in own)
    shared_blocks = n_runs * run_blocks
    caches = model.new_caches(shared_blocks + b * own_blocks, BS)
    gen = torch.Generator(device=device).manual_seed(78)
    for cache in caches:
        cache.normal_(generator=gen)
    runs = torch.arange(shared_blocks, dtype=torch.int32).view(n_runs, run_blocks)
    order = torch.tensor([[(i + j) % n_runs for j in range(slots)] for i in range(b)])
    table = torch.cat([runs[order].reshape(b, -1),
                       shared_blocks + torch.arange(b * own_blocks, dtype=torch.int32).view(b, own_blocks)], 1)
    table = table.to(device)
    lengths = torch.tensor([slots * run_blocks * BS + n for n in own], device=device)
    max_context = int(lengths.max()) + 1
    shared = SharedRuns(table, runs, order, BS, margin=256)
    ids = torch.tensor([5, 17, 301, 999], device=device)
    flags = _hip.new_flags(device)
    la = model.step(ids, lengths, caches, table, max_context=max_context, flags=flags,
                    workspace=decode_workspace(b, SHAPE.heads, max_context, 1024, device)).float()
    lb = model.step(ids, lengths, caches, table, max_context=max_context, flags=flags, shared=shared,
                    workspace=decode_shared_workspace(b, SHAPE.heads, shared, max_context, 1024, device)).float()
    raise_flags(flags)
    assert float((la - lb).abs().max()) <= 3e-2 * float(la.abs().max())
