#!/usr/bin/env python3
"""Benchmark of the CCPE reuse-attention hot path on one MI355X.

Workload (the headline configuration): single-layer CCPE prefill attention at
Mistral-7B head shape -- batch 8 x (4 chunks x 1024 tokens), 32 query / 8 KV
heads, head dim 128, bf16, Q/K/V ~ N(0, 1), CoPE table [128, 64] ~ N(0, 0.02),
paged KV with block size 16 and seeded random-permutation block tables.  One
step is one launch of the fused MFMA prefill kernel over the whole batch,
reading K/V through the block table.

Also reported, each in a sub-record of the same JSON line: the decode
kernel at the 64-request x 32k-context shape (one layer's distinct KV, 8.6 GB
per call, one request checked against the oracle), end-to-end greedy decoding
of a random Mistral-7B-shaped model over 64 x 32k-token reused contexts, the
reuse call's attention with both runtime policies (MFMA path and generic
kernel on the same call), the SLIDE relocation step,
the WCA update, the selective-prefill rows and the layer-snapshot reads.  The
CPU baselines time the torch CPU restatement of the reference path
(oracle/torch_cpu.py, the reference's op order) on bounded samples of the
same workloads, with all host threads torch uses and with one thread.

Prints one JSON line.  Only one GPU is used: --gpus above 1 exits.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "CCPE decode tok/s + HBM TB/s %peak; prefill TFLOP/s %MFMA peak, 1 MI355X"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


def seed_gen(cfg: int, j: int):
    import torch

    return torch.Generator("cpu").manual_seed(1000 * cfg + j)


def prefill_flops(b, hq, n, d, p) -> float:
    """4 B Hq D N(N+1)/2 (QK^T and PV over the causal triangle) + 2 B Hq N D P (Q.E)."""
    return 4.0 * b * hq * d * n * (n + 1) / 2 + 2.0 * b * hq * n * d * p


def traffic_from_profiles(name: str):
    """HBM bytes per launch recorded in profiles/<name>.md ('traffic_bytes_per_launch: N')."""
    path = ROOT / "profiles" / f"{name}.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def build_prefill(device):
    import torch

    from cacheslide_amd import _hip
    from cacheslide_amd.paged import HipSlotMover

    B, CH, L, HQ, HKV, D, P, BS = 8, 4, 1024, 32, 8, 128, 64, 16
    N = CH * L
    q = torch.randn((B, N, HQ, D), generator=seed_gen(2, 0)).to(torch.bfloat16)
    k = torch.randn((B, N, HKV, D), generator=seed_gen(2, 1)).to(torch.bfloat16)
    v = torch.randn((B, N, HKV, D), generator=seed_gen(2, 2)).to(torch.bfloat16)
    e = torch.randn((D, P), generator=seed_gen(2, 3)) * 0.02
    nblocks = B * N // BS
    table = torch.randperm(nblocks, generator=seed_gen(2, 4)).to(torch.int32).view(B, N // BS)
    cache = torch.empty((nblocks, HKV, BS, 2 * D), dtype=torch.bfloat16, device=device)
    mover = HipSlotMover()
    tok = torch.arange(N)
    for b in range(B):
        slots = (table[b, tok // BS].long() * BS + tok % BS).tolist()
        mover.scatter(cache, None, None, slots, k[b].to(device), v[b].to(device))
    torch.cuda.synchronize()
    inputs = dict(
        q=q.to(device), cache=cache, table=table.to(device), e=e.to(device).contiguous(),
        qpos=torch.arange(N, device=device).repeat(B, 1).contiguous(),
        nk=torch.full((B,), N, dtype=torch.int32, device=device),
        out=torch.empty((B, N, HQ, D), dtype=torch.bfloat16, device=device),
        flags=_hip.new_flags(device),
    )
    shape = dict(B=B, N=N, HQ=HQ, HKV=HKV, D=D, P=P, BS=BS)
    host = dict(q=q, k=k, v=v, e=e)
    return inputs, shape, host


def prefill_launcher(inputs, shape, device):
    from cacheslide_amd import _hip
    from cacheslide_amd.ccpe import _paged_source

    lib = _hip.load()
    src = _paged_source(inputs["cache"], inputs["table"])
    q, qpos = inputs["q"], inputs["qpos"]
    args = (
        _hip.ptr(q), q.stride(0), q.stride(1), q.stride(2), _hip.ptr(qpos), qpos.stride(0),
        shape["B"], shape["N"], shape["HQ"], shape["HKV"], _hip.ptr(inputs["nk"]), src,
        _hip.ptr(inputs["e"]), shape["P"], _hip.ptr(inputs["out"]), _hip.ptr(inputs["flags"]),
        _hip.stream_of(device),
    )

    def step():
        status = lib.cs_ccpe_prefill_bf16(*args)
        if status:
            _hip.check(status, "cs_ccpe_prefill_bf16")

    return step


def time_steps(step, steps: int, warmup: int):
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms


def spot_check_prefill(inputs, host, shape):
    """A few rows of batch 0 / GQA group 0 against the oracle (guards the number)."""
    import numpy as np

    from oracle import ccpe as orc

    rows = [0, 777, shape["N"] - 1]
    out = inputs["out"][0, rows, :4].float().cpu().numpy()
    k = host["k"][0, :, :1].float().numpy()
    v = host["v"][0, :, :1].float().numpy()
    worst = 0.0
    for i, r in enumerate(rows):
        q = host["q"][0, r : r + 1, :4].float().numpy()
        exp = orc.cope_attention(q, k[: r + 1], v[: r + 1], host["e"].numpy(), np.array([r]))
        worst = max(worst, float(np.abs(out[i] - exp[0]).max()))
    return worst


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_median_s(fn, repeats: int = 3) -> float:
    """One warm-up call, then the median wall time of ``repeats`` calls."""
    fn()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def with_threads(n: int, fn):
    import torch

    old = torch.get_num_threads()
    torch.set_num_threads(n)
    try:
        return fn()
    finally:
        torch.set_num_threads(old)


def rows_flops(rows, heads: int, d: int, p: int) -> float:
    """Causal-triangle FLOPs of the given query rows: 4 heads D (r + 1) per
    row for QK^T and PV plus 2 heads D P per row for Q.E (the prefill formula
    restricted to a row subset)."""
    return float(sum(4.0 * heads * d * (int(r) + 1) + 2.0 * heads * d * p for r in rows))


def cpu_baseline(host, shape) -> dict:
    """The torch CPU restatement of cope_attention (oracle/torch_cpu.py, the
    reference's op order with 64-row query chunks) on the box's host cores:
    batch item 0 of the prefill workload, all 32 query heads, every fourth of
    its 4096 rows (each against all keys, as the reference computes them);
    one warm-up, median of 3.  The one-thread figure runs one GQA group
    (4 query heads) over every eighth row."""
    import torch

    from oracle import torch_cpu as tc

    N, D, P = shape["N"], shape["D"], shape["P"]
    q, k, v, e = host["q"][0], host["k"][0], host["v"][0], host["e"]
    rows4, rows8 = torch.arange(0, N, 4), torch.arange(0, N, 8)
    threads = torch.get_num_threads()
    t_all = cpu_median_s(lambda: tc.cope_attention(q[rows4], k, v, e, rows4))
    t_one = with_threads(1, lambda: cpu_median_s(
        lambda: tc.cope_attention(q[rows8, :4], k[:, :1], v[:, :1], e, rows8)))
    flops_all = rows_flops(rows4.tolist(), shape["HQ"], D, P)
    flops_one = rows_flops(rows8.tolist(), 4, D, P)
    return {
        "value": round(flops_all / t_all / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle/torch_cpu.py cope_attention (torch on the CPU, reference op order, 64-row "
                  f"query chunks) on batch item 0 of the workload: 32 heads x every 4th of {N} rows, "
                  f"{flops_all / 1e9:.0f} of the workload's "
                  f"{prefill_flops(8, shape['HQ'], N, D, P) / 1e9:.0f} GFLOP; median of 3 after one "
                  f"warm-up: {t_all:.2f} s",
        "one_thread_value": round(flops_one / t_one / 1e12, 6),
        "one_thread_sample": f"4 query heads (one GQA group) x every 8th row, median {t_one:.2f} s",
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def cpu_decode_leg(ctx: int = 32769, requests: int = 2) -> dict:
    """The reference decode step on the host (oracle/torch_cpu.py decode_step:
    advanced-indexing gather of the request's canonical slots, then
    cope_attention at one row) for ``requests`` of the 64 requests of one layer,
    32q/8kv heads, bf16 cache; scaled to one layer-step of 64 requests."""
    import torch

    from oracle import torch_cpu as tc

    BS, HQ, HKV, D, P = 16, 32, 8, 128, 64
    per = (ctx + BS - 1) // BS
    g = torch.Generator().manual_seed(5100)
    cache = torch.randn((requests * per, HKV, BS, 2 * D), generator=g).to(torch.bfloat16)
    table = torch.randperm(requests * per, generator=g).to(torch.int32).view(requests, per)
    q = torch.randn((requests, 1, HQ, D), generator=g).to(torch.bfloat16)
    e = torch.randn((D, P), generator=g) * 0.02

    def run(n_req):
        for b in range(n_req):
            tc.decode_step(cache, table[b], ctx, q[b], e)

    threads = torch.get_num_threads()
    t_all = cpu_median_s(lambda: run(requests))
    t_one = with_threads(1, lambda: cpu_median_s(lambda: run(1)))
    kv = ctx * HKV * D * 2 * 2
    return {
        "value_GBs": round(requests * kv / t_all / 1e9, 3),
        "layer_step_ms_64_requests": round(t_all / requests * 64 * 1e3, 1),
        "tok_per_s_32_layers": round(64 / (32 * t_all / requests * 64), 3),
        "cores": threads,
        "one_thread_GBs": round(kv / t_one / 1e9, 3),
        "kind": "port",
        "sample": f"{requests} of 64 requests x {ctx} keys (one layer), median of 3 after one warm-up; "
                  f"64-request layer-step time scaled linearly",
    }


def cpu_slide_leg(blocks: int = 10_000, chunks: int = 51) -> dict:
    """The relocation step on the host (oracle/torch_cpu.py relocate: advanced
    indexing on the [blocks, 8, 16, 256] bf16 layout, the map update and the
    freed slots) for one layer of 10k blocks and 51 chunks of 64..2048 tokens
    (a tenth of the device workload's chunks, one of its 32 layers)."""
    import numpy as np
    import torch

    from oracle import torch_cpu as tc

    BS, HKV, REC = 16, 8, 256
    rng = np.random.default_rng(3100)
    lens = rng.integers(64, 2049, chunks)
    pages = [(int(n) + BS - 1) // BS for n in lens]
    perm = rng.permutation(blocks)
    need = sum(pages)
    src_blk, dst_blk = perm[:need], perm[need:2 * need]
    fs, fd, ps, pd, slot_all = [], [], [], [], []
    at = 0
    for n, pg in zip(lens.tolist(), pages):
        sb, db = src_blk[at:at + pg], dst_blk[at:at + pg]
        at += pg
        nfull = n // BS
        fs += sb[:nfull].tolist()
        fd += db[:nfull].tolist()
        for t in range(nfull * BS, n):
            ps.append(int(sb[t // BS]) * BS + t % BS)
            pd.append(int(db[t // BS]) * BS + t % BS)
        slot_all += (np.repeat(db, BS)[:n] * BS + np.tile(np.arange(BS), pg)[:n]).tolist()
    T = int(lens.sum())
    cache = torch.empty((blocks, HKV, BS, REC), dtype=torch.bfloat16)
    cache.view(torch.int16).random_(generator=torch.Generator().manual_seed(3101))
    L = lambda xs: torch.tensor(xs, dtype=torch.long)  # noqa: E731
    fs, fd, ps, pd, slots = L(fs), L(fd), L(ps), L(pd), L(slot_all)
    tokens = torch.arange(T)
    mapping = torch.full((T,), -1, dtype=torch.long)
    step = lambda: tc.relocate(cache, fs, fd, ps, pd, mapping, tokens, slots)  # noqa: E731
    threads = torch.get_num_threads()
    t_all = cpu_median_s(step)
    t_one = with_threads(1, lambda: cpu_median_s(step))
    moved = (fs.numel() * BS + ps.numel()) * HKV * REC * 2
    traffic = 2 * moved + T * 8 * 3
    return {
        "value_GBs": round(traffic / t_all / 1e9, 3),
        "cores": threads,
        "one_thread_GBs": round(traffic / t_one / 1e9, 3),
        "kind": "port",
        "sample": f"1 layer x [{blocks} blocks, 8, 16, 256] bf16, {chunks} chunks ({T} tokens), "
                  f"median of 3 after one warm-up",
    }


def cpu_wca_leg(layers: int = 31) -> dict:
    """WCA on the host (oracle/torch_cpu.py WCA, float64 as wca.py): one
    request of 16384 tokens x 8 heads x 128, bf16, fraction 0.15: initialize,
    then ``layers`` layer updates with the runtime's finite checks."""
    import torch

    from oracle import torch_cpu as tc

    T, H, D = 16384, 8, 128
    g = torch.Generator().manual_seed(4100)
    new_k = torch.randn((T, H, D), generator=g).to(torch.bfloat16)
    new_v = torch.randn((T, H, D), generator=g).to(torch.bfloat16)
    old_k = (new_k.float() + 0.05 * torch.randn((T, H, D), generator=g)).to(torch.bfloat16)
    old_v = (new_v.float() + 0.05 * torch.randn((T, H, D), generator=g)).to(torch.bfloat16)
    reused = torch.ones(T, dtype=torch.bool)
    reused[-1] = False
    mandatory = ~reused
    state = {}

    def init():
        state["st"] = tc.WCA(old_k, new_k, reused, mandatory)

    def updates(count=layers):
        st = tc.WCA(old_k, new_k, reused, mandatory)
        for layer in range(2, 2 + count):
            idx = st.active
            st.update(layer, old_k, old_v, new_k[idx], new_v[idx])

    threads = torch.get_num_threads()
    t_init = cpu_median_s(init)
    t_traj = cpu_median_s(updates)
    t_upd = (t_traj - t_init) / layers
    a = int(state["st"].active.numel())
    upd_bytes = 2 * T * H * D * 2 + 6 * a * H * D * 2
    # one thread: a 7-layer trajectory (layers 2..8, two of them gate layers)
    short = lambda: updates(7)  # noqa: E731
    t_one_init = with_threads(1, lambda: cpu_median_s(init))
    t_one_upd = (with_threads(1, lambda: cpu_median_s(short)) - t_one_init) / 7
    return {
        "update_ms_per_layer": round(t_upd * 1e3, 3),
        "update_GBs": round(upd_bytes / t_upd / 1e9, 3),
        "initialize_ms_per_request": round(t_init * 1e3, 2),
        "cores": threads,
        "one_thread_update_ms_per_layer": round(t_one_upd * 1e3, 3),
        "one_thread_initialize_ms_per_request": round(t_one_init * 1e3, 2),
        "kind": "port",
        "sample": f"1 of 4 requests: initialize + {layers} layer updates (one thread: 7), median of 3 "
                  f"after one warm-up",
    }


def decode_measure(device, steps: int, warmup: int):
    """Decode kernel at 64 requests x 32k context (position 32768), 32q/8kv, d 128,
    one layer's distinct KV (8.6 GB)."""
    import torch

    from cacheslide_amd import CoPE, _hip
    from cacheslide_amd.ccpe import _paged_source, decode_workspace

    B, CTX, HQ, HKV, D, P, BS, SPLIT = 64, 32769, 32, 8, 128, 64, 16, 1024
    per = (CTX + BS - 1) // BS
    nblocks = B * per
    gen = torch.Generator(device=device).manual_seed(5005)
    cache = torch.empty((nblocks, HKV, BS, 2 * D), dtype=torch.bfloat16, device=device)
    cache.normal_(generator=gen)
    table = torch.randperm(nblocks, generator=seed_gen(5, 1)).to(torch.int32).view(B, per).to(device)
    q = torch.randn((B, HQ, D), generator=seed_gen(5, 2)).to(torch.bfloat16).to(device)
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.randn((D, P), generator=seed_gen(5, 3)) * 0.02)
    nk = torch.full((B,), CTX, dtype=torch.int32, device=device)
    ws = decode_workspace(B, HQ, CTX, SPLIT, device)
    out = torch.empty((B, HQ, D), dtype=torch.bfloat16, device=device)
    flags = _hip.new_flags(device)
    src = _paged_source(cache, table)
    lib = _hip.load()
    e = cope.position_embeddings.detach()
    args = (_hip.ptr(q), q.stride(0), q.stride(1), B, HQ, HKV, _hip.ptr(nk), CTX, src, _hip.ptr(e), P,
            SPLIT, _hip.ptr(ws), ws.numel(), _hip.ptr(out), _hip.ptr(flags), _hip.stream_of(device))

    def step():
        status = lib.cs_ccpe_decode_bf16(*args)
        if status:
            _hip.check(status, "cs_ccpe_decode_bf16")

    ms = time_steps(step, steps, warmup)
    kv_bytes = B * CTX * HKV * D * 2 * 2
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    # sampled parity: request 0 at full context against the oracle
    import numpy as np

    from oracle import ccpe as orc

    recs = cache[table[0].long()].permute(0, 2, 1, 3).reshape(-1, HKV, 2 * D)[:CTX].float().cpu().numpy()
    expected = orc.cope_attention(q[:1].float().cpu().numpy(), recs[..., :D], recs[..., D:],
                                  e.float().cpu().numpy(), np.array([CTX - 1]))
    check_err = float(np.abs(out[:1].float().cpu().numpy() - expected).max())
    ceilings = read_ceilings(cache, table, B, HKV, BS, D, device)
    del cache
    torch.cuda.empty_cache()
    return {
        "workload": "ccpe_decode_paged: 64 requests x 32769 keys, 32q/8kv heads, head_dim 128, "
                    "P=64, block 16, split 1024, one layer of distinct KV",
        "ms_per_call": round(ms, 4),
        "kv_bytes_per_call": kv_bytes,
        "achieved_GBs": round(gbs, 1),
        "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
        "tok_per_s_attention_32_layers": round(B / (32 * ms * 1e-3), 1),
        "spot_check_max_abs_err": round(check_err, 5),
        **ceilings,
        "frac_of_pattern_read_rate": round(gbs / ceilings["read_rate_pattern_GBs"], 4),
    }


def read_ceilings(cache, table, B: int, HKV: int, BS: int, D: int, device) -> dict:
    """What this device reads per second from the decode's 8.6 GB cache
    (cs_read_probe): streamed once, and in the decode kernel's pattern -- per
    workgroup the 64 blocks x (16 keys x 512 B) of one KV head of a 1024-key
    split, split-major, through the same random block tables (each request's
    2049 blocks padded to 33 x 64 by wrapping)."""
    import torch

    from cacheslide_amd import _hip

    lib = _hip.load()
    # the probe is measurement support: bound here, not in the package's binding
    probe = lib.cs_read_probe
    probe.restype = ctypes.c_int
    probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                      ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    per = table.shape[1]
    chunk = BS * 2 * D * 2                                  # one KV head's records of a block
    splits = (per + 63) // 64
    cols = torch.arange(splits * 64, device=device) % per
    blocks = table.long()[:, cols].view(B, splits, 64).permute(1, 0, 2)        # [split, request, 64]
    offsets = (blocks[:, :, None, :] * (HKV * chunk)
               + torch.arange(HKV, device=device)[None, None, :, None] * chunk).reshape(-1).contiguous()
    groups = offsets.numel() // 64
    sink = torch.empty(groups * 256, dtype=torch.int32, device=device)
    nbytes = cache.numel() * cache.element_size()
    stream = _hip.stream_of(device)

    def streamed():
        _hip.check(probe(_hip.ptr(cache), nbytes, None, 0, 0, 0, _hip.ptr(sink), sink.numel(), stream),
                   "cs_read_probe")

    def pattern():
        _hip.check(probe(_hip.ptr(cache), nbytes, _hip.ptr(offsets), offsets.numel(), 64, chunk,
                         _hip.ptr(sink), sink.numel(), stream), "cs_read_probe")

    ms_stream = time_steps(streamed, 10, 3)
    ms_pattern = time_steps(pattern, 10, 3)
    return {
        "read_rate_stream_GBs": round(nbytes / (ms_stream * 1e-3) / 1e9, 1),
        "read_rate_pattern_GBs": round(offsets.numel() * chunk / (ms_pattern * 1e-3) / 1e9, 1),
    }


def decode_e2e_measure(device, tokens: int = 128, warmup: int = 4) -> dict:
    """End-to-end greedy decoding at the Mistral-7B shape (32 layers, d_model
    4096, 32q/8kv heads x 128, FFN 14336, vocab 32000, bf16 weights N(0, 0.02)):
    64 requests, each a 32k context of 16 reused chunks of 2048 tokens shared by
    every request in a request-specific rotation (chunk-shifted reuse), then
    ``tokens`` generated tokens.  One paged cache per layer (block 16): the
    2048 shared chunk blocks (K/V ~ N(0, 1)) plus 8 private decode blocks per
    request.  Timed: ``tokens`` decode steps of the whole batch (projections
    as library GEMMs, the K/V write through cs_slot_scatter, attention through
    the fused decode), after ``warmup`` untimed steps."""
    import torch

    from cacheslide_amd.ccpe import SharedRuns
    from cacheslide_amd.decode_model import MISTRAL_7B, PagedDecoder

    B, CTX, CHUNKS, BS = 64, 32768, 16, 16
    shape = MISTRAL_7B
    chunk_blocks = CTX // CHUNKS // BS
    shared = CHUNKS * chunk_blocks
    own = (tokens + BS - 1) // BS
    model = PagedDecoder(shape, device, seed=5050)
    caches = model.new_caches(shared + B * own, BS)
    gen = torch.Generator(device=device).manual_seed(5051)
    for cache in caches:
        cache[:shared].normal_(generator=gen)
        cache[shared:].zero_()
    rotation = (torch.arange(CHUNKS)[None, :] + torch.arange(B)[:, None]) % CHUNKS
    chunk_rows = (rotation[:, :, None] * chunk_blocks + torch.arange(chunk_blocks)).reshape(B, -1)
    private = shared + torch.arange(B * own).view(B, own)
    table = torch.cat([chunk_rows, private], dim=1).to(torch.int32).to(device)
    first = torch.randint(0, shape.vocab, (B,), generator=seed_gen(5, 4)).to(device)
    lengths = torch.full((B,), CTX, dtype=torch.int32, device=device)
    max_context = CTX + tokens
    model.generate(first, lengths, caches, table, warmup, max_context=max_context)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = model.generate(first, lengths, caches, table, tokens, max_context=max_context)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    # the same generation with the shared chunks read once per step for the
    # batch (ccpe_decode_shared): runs = the 16 chunks, each request's slots
    # its rotation; the last 256 shared keys and the request's own keys exact
    runs = SharedRuns(table, torch.arange(shared, dtype=torch.int32).view(CHUNKS, chunk_blocks), rotation, BS,
                      margin=256, pieces=2)
    model.generate(first, lengths, caches, table, warmup, max_context=max_context, shared=runs)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out_shared = model.generate(first, lengths, caches, table, tokens, max_context=max_context, shared=runs)
    torch.cuda.synchronize()
    seconds_shared = time.perf_counter() - t0
    # one step from the same state both ways: the logits agree to the bf16
    # level (greedy runs of a random-weight model then part at near-ties)
    from cacheslide_amd import _hip
    from cacheslide_amd.ccpe import decode_shared_workspace, decode_workspace
    flags = _hip.new_flags(device)
    pos = lengths.to(torch.long)
    la = model.step(first, pos, caches, table, max_context=max_context, flags=flags,
                    workspace=decode_workspace(B, shape.heads, max_context, 1024, device)).float()
    lb = model.step(first, pos, caches, table, max_context=max_context, flags=flags, shared=runs,
                    workspace=decode_shared_workspace(B, shape.heads, runs, max_context, 1024, device)).float()
    # control: the exact per-request decode against itself with another split
    # (only the summation order of the attention differs)
    lc = model.step(first, pos, caches, table, max_context=max_context, flags=flags, split=512,
                    workspace=decode_workspace(B, shape.heads, max_context, 512, device)).float()
    logit_rel = float((la - lb).abs().max() / la.abs().max())
    control_rel = float((la - lc).abs().max() / la.abs().max())
    top1 = float((la.argmax(-1) == lb.argmax(-1)).float().mean())
    control_top1 = float((la.argmax(-1) == lc.argmax(-1)).float().mean())
    top2_gap = float((la.topk(2, dim=-1).values.diff(dim=-1).abs() / la.abs().max()).median())
    del out_shared
    kv_bytes_step = sum(B * (CTX + t + 1) * shape.kv_heads * 128 * 2 * 2 for t in range(tokens)) / tokens
    hbm_ideal_ms = (shape.layers * kv_bytes_step + 2 * shape.parameters) / PEAK_HBM_GBS / 1e6
    distinct = len(set(out[:, 0].tolist()))
    del caches, model
    torch.cuda.empty_cache()
    return {
        "workload": "greedy decoding, Mistral-7B shape (32 layers, 4096, 32q/8kv x 128, FFN 14336, vocab 32000, "
                    "bf16 random weights), 64 requests x 32768-token contexts of 16 shared 2048-token chunks "
                    f"in per-request rotation, {tokens} tokens each, paged KV block 16",
        "tokens_per_request": tokens,
        "seconds": round(seconds, 3),
        "ms_per_step": round(seconds * 1e3 / tokens, 3),
        "tok_per_s": round(B * tokens / seconds, 1),
        "hbm_ideal_ms_per_step": round(hbm_ideal_ms, 2),
        "hbm_ideal_tok_per_s": round(B / (hbm_ideal_ms * 1e-3), 1),
        "note": "the ideal counts every K/V byte from HBM; the 16 shared chunks are 134 MB per layer, "
                "so most K/V reads can hit the 256 MB Infinity Cache",
        "distinct_tokens_request_0": distinct,
        "shared_runs": {
            "seconds": round(seconds_shared, 3),
            "ms_per_step": round(seconds_shared * 1e3 / tokens, 3),
            "tok_per_s": round(B * tokens / seconds_shared, 1),
            "one_step_logits_max_rel_diff": round(logit_rel, 6),
            "one_step_argmax_equal": round(top1, 4),
            "control_split_512_logits_max_rel_diff": round(control_rel, 6),
            "control_split_512_argmax_equal": round(control_top1, 4),
            "one_step_median_top2_gap_rel": round(top2_gap, 6),
            "note": "ccpe_decode_shared: each of the 16 chunks read once per layer and step for the 64 requests "
                    "(positions P-1), every request's last 256 chunk keys and own keys with exact positions, the "
                    "two softmax states merged; the exact decode runs where a tail's gate mass stays below P-1",
        },
    }


def reuse_measure(device, steps: int = 5) -> dict:
    """The reuse call of runtime.py:576-609 at a 16384-token context: 8 reused
    chunks of 2016 tokens (16128 fixed) and a recomputed 256-token question;
    the active rows are 15% of the fixed rows (2420, seeded, as WCA selects
    them) and the question's rows, 32q/8kv heads x 128, bf16 Q/K/V ~ N(0, 1),
    CoPE P = 64 (table N(0, 0.1)), strict_contextual canonical positions from
    a [32, 16128, 16128] fp32 profile (one calibration-like path 0.5 per token
    shared by the heads, a broadcast view), updated_and_self visibility.  Timed:
    cope_attention on the MFMA policy path (``steps`` calls) and, once, the same
    call on the generic kernel (explicit key coordinates); the two outputs
    are compared."""
    import math

    import torch

    from cacheslide_amd import (CCPEProfile, CanonicalPositionPolicy, ChunkIdentity, CoPE, RequestPlan,
                                SelectedAssociationPolicy, cope_attention)

    CH, CHUNKS, DYN, HQ, HKV, D, P = 2016, 8, 256, 32, 8, 128, 64
    F = CH * CHUNKS
    n = F + DYN
    spec = [{"id": f"C{i}", "role": "reuse", "start": i * CH, "end": (i + 1) * CH} for i in range(CHUNKS)]
    spec.append({"id": "question", "role": "recompute", "start": F, "end": n})
    plan = RequestPlan.parse({"version": 1, "namespace": "bench", "task_id": "reuse", "operation": "reuse",
                              "chunks": spec}, [(7 * i) % 32000 for i in range(n)])
    gen = torch.Generator(device=device).manual_seed(6006)
    q_all = torch.randn((n, HQ, D), generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn((n, HKV, D), generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn((n, HKV, D), generator=gen, device=device).to(torch.bfloat16)
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.randn((D, P), generator=seed_gen(6, 1)) * 0.1)
    n_sel = math.ceil(0.15 * F)
    sel = torch.randperm(F, generator=seed_gen(6, 2))[:n_sel].sort().values
    rows = torch.cat([sel, torch.arange(F, n)]).to(device)
    ords = torch.arange(F, device=device, dtype=torch.float32)
    path = ((ords[:, None] - ords[None, :] + 1) * 0.5).clamp_(0, P - 1)
    path.masked_fill_(ords[None, :] > ords[:, None], 0.0)        # future keys: in bounds, never validated
    profile = CCPEProfile(trained_profile_version="v1", checkpoint_id="ckpt",
                          chunks=tuple(ChunkIdentity(*c) for c in plan.fixed_layout),
                          query_positions=torch.arange(F), key_positions=torch.arange(F),
                          canonical_positions=path.expand(HQ, F, F), max_positions=P, histogram_bin_width=0.25,
                          sample_count=1)
    policy = CanonicalPositionPolicy(plan, profile, "ckpt", mode="strict_contextual")
    visibility = SelectedAssociationPolicy(plan.fixed_indices, sel.to(device))
    q = q_all[rows].contiguous()
    keys = torch.arange(n, device=device)

    def run(explicit_keys=False):
        return cope_attention(q, k, v, cope, rows, keys if explicit_keys else None, positions_transform=policy,
                              visibility_transform=visibility, query_chunk_size=64)

    out = run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    t0 = time.perf_counter()
    ref = run(explicit_keys=True)
    torch.cuda.synchronize()
    ms_generic = (time.perf_counter() - t0) * 1e3
    err = float((out.float() - ref.float()).abs().max())
    causal = float((rows.double() + 1).sum())
    flops = 4.0 * HQ * D * causal + 2.0 * HQ * D * P * len(rows)
    canon_bytes = n_sel * HQ * F * 4
    # the same rows on a layer without a profile (SelectedAssociationPolicy
    # alone): no checker runs beside the attention, whose row blocks that walk
    # every causal key (the question rows) are then split over the keys
    def run_selected():
        return cope_attention(q, k, v, cope, rows, None, visibility_transform=visibility, query_chunk_size=64)

    run_selected()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run_selected()
    torch.cuda.synchronize()
    ms_selected = (time.perf_counter() - t0) * 1e3 / steps
    del profile, policy
    # the same call with a per-head profile in HBM (head h: a path of
    # 0.4 + 0.01 h per token, 33.3 GB), so every canonical row the call reads
    # is its own bytes rather than one row shared by the heads
    del path
    base = (ords[:, None] - ords[None, :] + 1).clamp_(min=0)   # q - k + 1 up to the diagonal, 0 above
    per_head = torch.empty((HQ, F, F), dtype=torch.float32, device=device)
    for h in range(HQ):
        torch.mul(base, 0.4 + 0.01 * h, out=per_head[h]).clamp_(0, P - 1)
    del base
    profile_h = CCPEProfile(trained_profile_version="v1", checkpoint_id="ckpt",
                            chunks=tuple(ChunkIdentity(*c) for c in plan.fixed_layout),
                            query_positions=torch.arange(F), key_positions=torch.arange(F),
                            canonical_positions=per_head, max_positions=P, histogram_bin_width=0.25,
                            sample_count=1)
    policy = CanonicalPositionPolicy(plan, profile_h, "ckpt", mode="strict_contextual")
    run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    ms_per_head = (time.perf_counter() - t0) * 1e3 / steps
    del profile_h, policy, per_head
    torch.cuda.empty_cache()
    return {
        "workload": "cope_attention reuse call: 16384 keys (8 reused chunks x 2016 + 256 recomputed), 2676 active "
                    "rows (2420 selected fixed + 256), 32q/8kv heads x 128, bf16, P=64, strict canonical profile "
                    "[32, 16128, 16128] fp32, updated_and_self visibility",
        "ms_per_call": round(ms, 3),
        "generic_ms_per_call": round(ms_generic, 2),
        "speedup_vs_generic": round(ms_generic / ms, 1),
        "max_abs_diff_vs_generic": round(err, 5),
        "reference_flop_per_call": flops,
        "reference_equivalent_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
        "canonical_bytes_checked": canon_bytes,
        "canonical_GBs_whole_call": round(canon_bytes / (ms * 1e-3) / 1e9, 1),
        "selected_only_ms_per_call": round(ms_selected, 3),
        "per_head_profile_ms_per_call": round(ms_per_head, 3),
        "per_head_profile_canonical_GBs_whole_call": round(canon_bytes / (ms_per_head * 1e-3) / 1e9, 1),
        "note": "the timed profile is one [16128, 16128] path broadcast to the 32 heads (its canonical rows are "
                "re-read from L2); per_head_profile_* times the same call with a [32, 16128, 16128] profile "
                "stored per head (33.3 GB in HBM, head h's path 0.4 + 0.01 h per token); selected_only_* the "
                "same rows on a layer without a profile (no checker; the question rows' blocks split over the keys)",
    }


def calibration_measure(device, steps: int = 5) -> dict:
    """The calibration-layer reuse call (runtime.py:448-454, 594-600): before
    WCA has selected rows, every row of the request attends with a
    CanonicalPositionPolicy and no SelectedAssociationPolicy (the same call
    is every layer's under selected_attention "all").  2 reused chunks of 2048
    tokens (4096 fixed) and a 256-token recomputed question, all 4352 rows in
    order, 32q/8kv heads x 128, bf16 Q/K/V ~ N(0, 1), CoPE P = 64 (table
    N(0, 0.1)), strict_contextual positions from a per-head [32, 4096, 4096]
    fp32 profile (head h: a path of 0.4 + 0.01 h per token; 2 GiB, no
    broadcast).  Timed: cope_attention on the MFMA policy path (``steps``
    calls) and, once, the same call on the generic kernel (explicit key
    coordinates); the two outputs are compared."""
    import torch

    from cacheslide_amd import CCPEProfile, CanonicalPositionPolicy, ChunkIdentity, CoPE, RequestPlan, cope_attention

    CH, CHUNKS, DYN, HQ, HKV, D, P = 2048, 2, 256, 32, 8, 128, 64
    F = CH * CHUNKS
    n = F + DYN
    spec = [{"id": f"C{i}", "role": "reuse", "start": i * CH, "end": (i + 1) * CH} for i in range(CHUNKS)]
    spec.append({"id": "question", "role": "recompute", "start": F, "end": n})
    plan = RequestPlan.parse({"version": 1, "namespace": "bench", "task_id": "calibration", "operation": "reuse",
                              "chunks": spec}, [(11 * i) % 32000 for i in range(n)])
    gen = torch.Generator(device=device).manual_seed(6306)
    q = torch.randn((n, HQ, D), generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn((n, HKV, D), generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn((n, HKV, D), generator=gen, device=device).to(torch.bfloat16)
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.randn((D, P), generator=seed_gen(7, 1)) * 0.1)
    ords = torch.arange(F, device=device, dtype=torch.float32)
    canon = torch.empty((HQ, F, F), dtype=torch.float32, device=device)
    for h in range(HQ):
        canon[h] = ((ords[:, None] - ords[None, :] + 1) * (0.4 + 0.01 * h)).clamp_(0, P - 1)
        canon[h].masked_fill_(ords[None, :] > ords[:, None], 0.0)
    profile = CCPEProfile(trained_profile_version="v1", checkpoint_id="ckpt",
                          chunks=tuple(ChunkIdentity(*c) for c in plan.fixed_layout),
                          query_positions=torch.arange(F), key_positions=torch.arange(F),
                          canonical_positions=canon, max_positions=P, histogram_bin_width=0.25, sample_count=1)
    policy = CanonicalPositionPolicy(plan, profile, "ckpt", mode="strict_contextual")
    rows = torch.arange(n, device=device)
    keys = torch.arange(n, device=device)

    def run(explicit_keys=False):
        return cope_attention(q, k, v, cope, rows, keys if explicit_keys else None, positions_transform=policy,
                              query_chunk_size=64)

    out = run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    t0 = time.perf_counter()
    ref = run(explicit_keys=True)
    torch.cuda.synchronize()
    ms_generic = (time.perf_counter() - t0) * 1e3
    err = float((out.float() - ref.float()).abs().max())
    causal = float((rows.double() + 1).sum())
    flops = 4.0 * HQ * D * causal + 2.0 * HQ * D * P * n
    canon_bytes = HQ * F * (F + 1) // 2 * 4           # the causal fixed x fixed cells, once each
    del canon, profile, policy
    torch.cuda.empty_cache()
    return {
        "workload": "cope_attention calibration-layer call: 4352 keys (2 reused chunks x 2048 + 256 recomputed), "
                    "all 4352 rows, 32q/8kv heads x 128, bf16, P=64, strict per-head canonical profile "
                    "[32, 4096, 4096] fp32, no selected set",
        "ms_per_call": round(ms, 3),
        "generic_ms_per_call": round(ms_generic, 2),
        "speedup_vs_generic": round(ms_generic / ms, 1),
        "max_abs_diff_vs_generic": round(err, 5),
        "reference_flop_per_call": flops,
        "reference_equivalent_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
        "canonical_bytes_read": canon_bytes,
        "canonical_GBs_whole_call": round(canon_bytes / (ms * 1e-3) / 1e9, 1),
    }


def tiny_e2e_measure(device) -> dict:
    """The tiny end-to-end flow (the reference's CPU smoke, workflow_smoke.py:
    117-324): a 2-layer random decoder (d_model 64, 4 heads x 16, vocab 512,
    CoPE P = 64) on SelectiveRuntime with SLIDE arenas on paged caches;
    profiles calibrated from the model's own forward, then populate,
    recompute, same-context reuse, a shifted chunk under strict CCPE (fallback)
    and under mixed_bias_override (reuse), each a prefill and 5 greedy decode
    steps.  Wall clock per case, device synchronized around it, on a second
    pass with a fresh store and runtimes (the first pass pays the one-time
    costs)."""
    import pathlib
    import tempfile

    import torch

    from tests._e2e import CASES, device_runtimes, invoke, tiny_plan

    plan = tiny_plan(32)
    with tempfile.TemporaryDirectory() as root:
        for tag in ("warm", "timed"):
            store, runtimes = device_runtimes(device, pathlib.Path(root), plan, layers=2, calibration_layer=0,
                                              tag=tag)
            times, receipts, tokens = [], [], []
            for i, (op, dyn, mode) in enumerate(CASES):
                rt, model = runtimes[mode]
                torch.cuda.synchronize(device)
                t0 = time.perf_counter()
                _, ids, receipt = invoke(rt, model, tiny_plan(dyn), op, f"req-{i}")
                torch.cuda.synchronize(device)
                times.append((time.perf_counter() - t0) * 1e3)
                receipts.append(receipt)
                tokens.append(ids)
            for rt, _ in runtimes.values():
                rt.close()
            store.close()
    return {
        "workload": "tiny end-to-end: 2-layer random decoder (d_model 64, 4 heads x 16, vocab 512, CoPE P=64), "
                    "5 cases (populate, recompute, reuse, shifted strict -> fallback, shifted mixed -> reuse), "
                    "each a prefill + 5 greedy decode steps, paged SLIDE arenas",
        "cases": [f"{op}/{dyn}/{mode}" for op, dyn, mode in CASES],
        "wall_ms_per_case": [round(t, 2) for t in times],
        "decisions": [{"cache_hit": r["cache_hit"], "fallback": r["fallback"],
                       "position_policy_fallback": r["position_policy_fallback"]} for r in receipts],
        "tokens": tokens,
    }


def cpu_tiny_e2e_leg(gpu_tokens) -> dict:
    """The oracle runtime (oracle/runtime.py) on the host, driven through the
    same five cases on the same model and plans: wall clock per case (after a
    first pass), and whether its greedy tokens equal the device run's."""
    from tests._e2e import CASES, invoke, oracle_runtimes, tiny_plan

    plan = tiny_plan(32)
    for _ in range(2):
        runtimes = oracle_runtimes(plan, layers=2, calibration_layer=0)
        times, tokens = [], []
        for i, (op, dyn, mode) in enumerate(CASES):
            rt, model = runtimes[mode]
            t0 = time.perf_counter()
            _, ids, _ = invoke(rt, model, tiny_plan(dyn), op, f"req-{i}")
            times.append((time.perf_counter() - t0) * 1e3)
            tokens.append(ids)
    return {"value": round(sum(times), 1), "unit": "ms for the 5 cases", "cores": 1, "kind": "port",
            "sample": "the whole workload", "wall_ms_per_case": [round(t, 1) for t in times],
            "tokens_equal_device": tokens == gpu_tokens}


def note(message: str) -> None:
    """Progress line on stderr (stdout carries only the JSON record)."""
    print(f"bench: {message}", file=sys.stderr, flush=True)


def slide_measure(device, steps: int, layers: int = 32) -> dict:
    """SLIDE relocation step on a stacked paged cache [L, 100000 blocks, 8 heads,
    16, 256] bf16: 512 reused chunks of 64..2048 tokens move from their current
    slots to a seeded random permutation of free blocks -- whole pages by page
    copy, the partial last page by slot copy -- then the token -> slot map is
    rewritten (scatter) and read back (gather), and the source slots return to
    the free list.  Moves are byte copies; the step is checked bit-exact."""
    import numpy as np
    import torch

    from cacheslide_amd import relocate

    NB, HKV, BS, REC, CHUNKS = 100_000, 8, 16, 256, 512
    rng = np.random.default_rng(3000)
    lens = rng.integers(64, 2049, CHUNKS)
    pages = [(int(n) + BS - 1) // BS for n in lens]
    perm = rng.permutation(NB)
    need = sum(pages)
    src_blk = perm[:need]
    dst_blk = perm[need:2 * need]
    full_src, full_dst, part_src, part_dst, tok_all, slot_all = [], [], [], [], [], []
    at, tok0 = 0, 0
    for n, pg in zip(lens.tolist(), pages):
        sb, db = src_blk[at:at + pg], dst_blk[at:at + pg]
        at += pg
        nfull = n // BS
        full_src.extend(sb[:nfull].tolist())
        full_dst.extend(db[:nfull].tolist())
        for t in range(nfull * BS, n):
            part_src.append(int(sb[t // BS]) * BS + t % BS)
            part_dst.append(int(db[t // BS]) * BS + t % BS)
        slots = (np.repeat(db, BS)[:n] * BS + np.tile(np.arange(BS), pg)[:n]).tolist()
        tok_all.extend(range(tok0, tok0 + n))
        slot_all.extend(slots)
        tok0 += n
    T = int(lens.sum())
    torch.cuda.empty_cache()
    cache = torch.empty((layers, NB, HKV, BS, REC), dtype=torch.bfloat16, device=device)
    cache.view(torch.int16).random_(generator=torch.Generator(device=device).manual_seed(3001))
    dev = lambda xs: torch.tensor(xs, dtype=torch.long, device=device)  # noqa: E731
    fs, fd, ps, pd = dev(full_src), dev(full_dst), dev(part_src), dev(part_dst)
    tokens, slots = dev(tok_all), dev(slot_all)
    mapping = torch.full((T,), -1, dtype=torch.long, device=device)
    free = relocate.SlotFreeList(NB * BS, device)
    src_slots = dev((np.repeat(src_blk, BS) * BS + np.tile(np.arange(BS), need)).tolist())

    def step():
        relocate.copy_pages(cache, fs, fd, check=False)  # disjoint by construction (two halves of one permutation)
        relocate.copy_slots(cache, ps, pd, check=False)
        relocate.scatter_mapping(mapping, tokens, slots)
        relocate.gather_mapping(mapping, tokens)
        free.release(src_slots)

    ms = time_steps(step, steps, 2)
    rec_bytes = layers * HKV * 2 * REC  # K and V of one token over all layers
    moved = (len(full_src) * BS + len(part_src)) * rec_bytes
    traffic = 2 * moved + T * 8 * 3 + src_slots.numel() * 8
    bits = cache.view(torch.int16)  # compare bit patterns (random fill holds NaN encodings)
    exact = bool(torch.equal(bits[:, fd[:64]], bits[:, fs[:64]]))
    if ps.numel():
        s_, d_ = ps[:64], pd[:64]
        exact = exact and bool(torch.equal(bits[:, d_ // BS, :, d_ % BS], bits[:, s_ // BS, :, s_ % BS]))
    exact = exact and bool(torch.equal(mapping, slots))
    del cache
    torch.cuda.empty_cache()
    gbs = traffic / (ms * 1e-3) / 1e9
    return {
        "workload": f"slide relocation: {layers} layers x [100000 blocks, 8 heads, 16, 256] bf16, "
                    f"512 chunks of 64..2048 tokens ({T} tokens) per step",
        "ms_per_step": round(ms, 4),
        "bytes_per_step": traffic,
        "achieved_GBs": round(gbs, 1),
        "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
        "bit_exact": exact,
    }


def wca_measure(device, layers: int = 31) -> dict:
    """WCA at Mistral-7B KV shape: 4 requests x 8 reused chunks of 2048 tokens
    (T = 16384), 8 KV heads x 128, bf16; cached KV = recomputed KV + N(0, 0.05)
    drift; correction fraction 0.15, gate every 4 layers.  Times
    WCAState.initialize (full-T deviation scoring and top-k selection) and the
    per-layer WCAState.update (score, weights, blend, gate, commit, promote),
    host checks included, as the runtime calls them."""
    import torch

    from cacheslide_amd import WCAConfig, WCAState

    R, T, H, D = 4, 16384, 8, 128
    gen = torch.Generator(device=device).manual_seed(4000)
    config = WCAConfig(correction_fraction=0.15)
    reqs = []
    for _ in range(R):
        new_k = torch.randn((T, H, D), generator=gen, device=device).to(torch.bfloat16)
        new_v = torch.randn((T, H, D), generator=gen, device=device).to(torch.bfloat16)
        old_k = (new_k.float() + 0.05 * torch.randn((T, H, D), generator=gen, device=device)).to(torch.bfloat16)
        old_v = (new_v.float() + 0.05 * torch.randn((T, H, D), generator=gen, device=device)).to(torch.bfloat16)
        reused = torch.ones(T, dtype=torch.bool, device=device)
        reused[-1] = False
        mandatory = ~reused
        reqs.append((new_k, new_v, old_k, old_v, reused, mandatory))
    # untimed warm-up: first-call library and allocator set-up
    n_k, n_v, o_k, o_v, ru, ma = reqs[0]
    warm = WCAState.initialize(o_k, n_k, ru, ma, config)
    idx = warm.active_indices
    warm.update(2, o_k, o_v, n_k.index_select(0, idx), n_v.index_select(0, idx))
    del warm
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    states = [WCAState.initialize(o_k, n_k, ru, ma, config) for n_k, n_v, o_k, o_v, ru, ma in reqs]
    torch.cuda.synchronize()
    init_ms = (time.perf_counter() - t0) * 1e3 / R
    upd_s, upd_bytes, rows = 0.0, 0, 0
    for layer in range(2, 2 + layers):
        for st, (n_k, n_v, o_k, o_v, _, _) in zip(states, reqs):
            idx = st.active_indices
            rk, rv = n_k.index_select(0, idx), n_v.index_select(0, idx)
            computed = idx.clone()  # the caller's row positions (runtime.py:535-537)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            st.update(layer, o_k, o_v, rk, rv, computed_indices=computed)
            torch.cuda.synchronize()
            upd_s += time.perf_counter() - t0
            a = idx.numel()
            rows += a
            # finite checks of the whole cached K and V, then old and new K, V rows
            # read and fused K, V written
            upd_bytes += 2 * T * H * D * 2 + 6 * a * H * D * 2
    n_upd = layers * R
    return {
        "workload": "wca: 4 requests x 8 chunks x 2048 tokens, 8 kv heads x 128, bf16, "
                    f"fraction 0.15, layer 1 full then {layers} layer updates each",
        "initialize_ms_per_request": round(init_ms, 4),
        "initialize_GBs": round(2 * T * H * D * 2 / (init_ms * 1e-3) / 1e9, 1),
        "update_ms_per_layer": round(upd_s * 1e3 / n_upd, 4),
        "active_rows_per_update": round(rows / n_upd, 1),
        "update_GBs": round(upd_bytes / upd_s / 1e9, 1),
        "update_hbm_frac": round(upd_bytes / upd_s / 1e9 / PEAK_HBM_GBS, 4),
        "note": "wall-clock per call, host validation and the one status readback per call "
                "included (transactional API); update bytes = finite checks of the cached K/V "
                "plus 6 row passes",
    }


def rows_measure(device, steps: int = 50) -> dict:
    """Selective-prefill row bookkeeping (runtime.py:408-456) at Mistral-7B
    hidden size: T = 16384 tokens, hidden 4096 bf16, 13926 fixed tokens; the
    previous layer ran 2459 rows (15% of the fixed tokens plus 370 dynamic
    ones), the next one runs 2459 rows of which 246 are newly promoted fixed
    tokens restored from the snapshot.  Times the remap kernel (hidden and
    residual rows) through the C ABI with prebuilt arguments, and the final
    zero-filled [T, H] scatter; HIP events on the launch stream."""
    import ctypes

    import torch

    from cacheslide_amd import _hip

    T, H, F = 16384, 4096, 13926
    g = torch.Generator().manual_seed(5000)
    perm = torch.randperm(T, generator=g)
    fixed = perm[:F].sort().values
    dynamic = perm[F:F + 370].sort().values
    sel = fixed[torch.randperm(F, generator=g)[:2089]]
    previous = torch.cat([sel, dynamic]).sort().values
    promoted = fixed[~torch.isin(fixed, previous)][torch.randperm(F - 2089, generator=g)[:246]]
    keep = previous[torch.randperm(len(previous), generator=g)[246:]]
    active = torch.cat([keep, promoted]).sort().values
    dev = lambda x: x.to(device).contiguous()
    fixed, previous, active = dev(fixed), dev(previous), dev(active)
    hidden = torch.randn(len(previous), H, device=device, dtype=torch.bfloat16)
    residual = torch.randn_like(hidden)
    snap_h = torch.randn(F, H, device=device, dtype=torch.bfloat16)
    snap_r = torch.randn_like(snap_h)
    out_h = torch.empty(len(active), H, device=device, dtype=torch.bfloat16)
    out_r = torch.empty_like(out_h)
    final = torch.empty(T, H, device=device, dtype=torch.bfloat16)
    restored = torch.zeros(1, dtype=torch.long, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    lib = _hip.load()
    views = [_hip.view(x) for x in (hidden, residual, snap_h, snap_r, out_h, out_r, final)]
    refs = [ctypes.byref(v) for v in views]
    stream = _hip.stream_of(device)
    P = _hip.ptr

    # arguments built once, as a caller's loop holds them: the timed calls
    # measure the launches, not the building of ctypes values
    remap_args = (refs[0], refs[1], refs[2], refs[3], refs[4], refs[5], P(previous), len(previous), P(active),
                  len(active), P(fixed), F, P(restored), P(flags), stream)
    scatter_args = (refs[4], P(active), len(active), refs[6], P(flags), stream)

    def remap():
        status = lib.cs_rows_remap(*remap_args)
        if status:
            _hip.check(status, "cs_rows_remap")

    def scatter():
        status = lib.cs_rows_scatter(*scatter_args)
        if status:
            _hip.check(status, "cs_rows_scatter")

    ms_remap = time_steps(remap, steps, 5)
    ms_scatter = time_steps(scatter, steps, 5)
    torch.cuda.synchronize()
    ok = int(flags.item()) == 0 and int(restored.item()) == 246 * (steps + 5)
    remap_bytes = 2 * 2 * len(active) * H * 2           # hidden + residual rows, read and written
    scatter_bytes = len(active) * H * 2 + T * H * 2     # rows read, the whole output written
    return {
        "workload": "selective prefill rows: 16384 tokens, hidden 4096 bf16, 2459 active rows "
                    "(246 restored from the fixed-token snapshot), final [16384, 4096] scatter",
        "remap_us_per_call": round(ms_remap * 1e3, 2),
        "remap_GBs": round(remap_bytes / (ms_remap * 1e-3) / 1e9, 1),
        "scatter_us_per_call": round(ms_scatter * 1e3, 2),
        "scatter_GBs": round(scatter_bytes / (ms_scatter * 1e-3) / 1e9, 1),
        "hbm_frac_remap": round(remap_bytes / (ms_remap * 1e-3) / 8e12, 4),
        "checked": ok,
    }


def snapshot_measure(device, reps: int = 5) -> dict:
    """Layer K/V snapshot reads (runtime.py:192-272) at Mistral-7B geometry: one
    page holds the 13926 fixed tokens' K and V, 8 kv heads x 128, bf16 (57 MB).

    Wall clock per page, page bytes already in host memory:
    * decode: bytes -> checked device tensors through SnapshotUploader
      (staging, DMA, device finite check, flag readback);
    * reference_decode: the reference's steps on the same bytes
      (safetensors load, torch.isfinite on the CPU, .to(device)), synchronized;
    * store_read: TieredPageStore.read of a resident page (its sha256 check),
      the same cost in both implementations;
    * h2d_GBs: the bare pinned-to-HBM DMA of the data region, HIP events on its stream;
    * layer_loop: 32 layers of (read this layer's page, prefetch the next, a GPU
      compute stand-in), wall clock per layer: compute alone, the reference's
      flow (decode and the next page's checksum on the compute thread), and
      LayerSnapshots at prefetch depth 1 (the reference's policy), 4 and 8.
    """
    import ctypes
    import tempfile
    import time

    import torch
    from safetensors.torch import load as st_load

    from cacheslide_amd import RequestPlan, _hip
    from cacheslide_amd.snapshot import LayerSnapshots, SnapshotUploader, encode_snapshot
    from cacheslide_amd.pagestore import PageStore

    F, HKV, D = 13926, 8, 128
    shapes = {"k": (F, HKV, D), "v": (F, HKV, D)}
    g = torch.Generator(device=device).manual_seed(6000)
    kv = {n: torch.randn(F, HKV, D, device=device, generator=g).bfloat16() for n in ("k", "v")}
    data = encode_snapshot(kv)
    region = 2 * F * HKV * D * 2
    uploader = SnapshotUploader(device)

    def wall(fn, n=reps):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3

    def ours():
        SnapshotUploader.take(uploader.submit(lambda: data, shapes, torch.bfloat16))

    def reference():
        tensors = st_load(data)
        for t in tensors.values():
            if not torch.isfinite(t).all():
                raise ValueError("nonfinite")
        return {n: t.to(device=device, dtype=torch.bfloat16) for n, t in tensors.items()}

    got = SnapshotUploader.take(uploader.submit(lambda: data, shapes, torch.bfloat16))
    ok = all(torch.equal(got[n].view(torch.int16), kv[n].view(torch.int16)) for n in kv)
    ms_ours, ms_ref = wall(ours), wall(reference)

    # bare DMA from pinned memory on a side stream
    pinned = torch.empty(region, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(region, dtype=torch.uint8, device=device)
    side = torch.cuda.Stream(device)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h = ctypes.c_void_p(side.cuda_stream)
    copy = lambda: _hip.call("cs_copy_async", _hip.ptr(dst), ctypes.c_void_p(pinned.data_ptr()), region,
                             _hip.COPY_H2D, h)
    copy()
    ev0.record(side)
    for _ in range(reps):
        copy()
    ev1.record(side)
    ev1.synchronize()
    ms_dma = ev0.elapsed_time(ev1) / reps

    doc = {"version": 1, "operation": "reuse", "namespace": "bench", "task_id": "snapshot",
           "chunks": [{"id": "fixed", "role": "reuse", "start": 0, "end": F},
                      {"id": "q", "role": "recompute", "start": F, "end": F + 64}]}
    plan = RequestPlan.parse(doc, list(range(F + 64)))
    L = 32  # Mistral-7B's layer count
    busy = torch.randn(8192, 8192, device=device, dtype=torch.bfloat16)
    work = lambda: [busy @ busy for _ in range(8)]             # per-layer compute stand-in

    def per_layer(loop):
        loop()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loop()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / L * 1e3

    with tempfile.TemporaryDirectory() as root:
        store = PageStore(root + "/pages", cpu_budget_bytes=(L + 1) * len(data),
                                disk_budget_bytes=(L + 1) * len(data))
        key = lambda layer: plan.cache_key("bench", layer) + "/kv"
        for layer in range(L):
            store.put(key(layer), data)
        ms_store = wall(lambda: store.read(key(0)))

        def compute_only():
            for _ in range(L):
                work()

        def reference_flow():
            # runtime.py:531-536 on the compute thread: _read (decode) then
            # _prefetch (a resident page is checksummed inside submit_load)
            future = store.submit_load(key(0))
            for layer in range(L):
                future.result()
                reference()
                if layer + 1 < L:
                    future = store.submit_load(key(layer + 1))
                work()

        def our_flow(depth):
            snaps = LayerSnapshots(store, plan, "bench", device, layers=L, kv_heads=HKV, head_dim=D,
                                   hidden_size=4096, prefetch_depth=depth)

            def loop():
                snaps.prefetch(0, torch.bfloat16)
                for layer in range(L):
                    snaps.read(layer, "kv", torch.bfloat16)
                    snaps.prefetch(layer + 1, torch.bfloat16)
                    work()
            return snaps, loop

        ms_compute = per_layer(compute_only)
        ms_ref_loop = per_layer(reference_flow)
        loops = {}
        for depth in (1, 4, 8):
            snaps, loop = our_flow(depth)
            loops[depth] = per_layer(loop)
            snaps.uploader.close()
        store.close()
    uploader.close()
    return {
        "workload": "layer K/V snapshot page: 13926 fixed tokens x 8 kv heads x 128 x (K, V), bf16, "
                    f"{region / 1e6:.1f} MB data region, page bytes in host memory",
        "decode_ms_per_page": round(ms_ours, 3),
        "decode_GBs": round(region / (ms_ours * 1e-3) / 1e9, 2),
        "reference_decode_ms_per_page": round(ms_ref, 3),
        "speedup_vs_reference_steps": round(ms_ref / ms_ours, 2),
        "h2d_dma_GBs": round(region / (ms_dma * 1e-3) / 1e9, 2),
        "pcie_frac": round(region / (ms_dma * 1e-3) / 64e9, 3),
        "store_read_ms_per_page": round(ms_store, 3),
        "layer_loop": {
            "layers": L,
            "compute_only_ms_per_layer": round(ms_compute, 3),
            "reference_flow_ms_per_layer": round(ms_ref_loop, 3),
            "prefetch_depth1_ms_per_layer": round(loops[1], 3),
            "prefetch_depth4_ms_per_layer": round(loops[4], 3),
            "prefetch_depth8_ms_per_layer": round(loops[8], 3),
        },
        "checked": ok,
        "note": "wall clock; the reference steps run here on the same bytes (safetensors load, "
                "CPU isfinite, .to(device)); every read includes the store's sha256 check of the "
                "page; PCIe 5.0 x16 is 64 GB/s per direction",
    }


def copy_calibration(device, nbytes: int, steps: int) -> dict:
    """A plain device copy of a known size, for scaling HBM counters
    (FETCH_SIZE / WRITE_SIZE) read under rocprofv3 --pmc."""
    import torch

    n = nbytes // 2
    src = torch.ones(n, dtype=torch.bfloat16, device=device)
    dst = torch.empty_like(src)
    ms = time_steps(lambda: dst.copy_(src), steps, 2)
    return {"copy_bytes_read": n * 2, "copy_bytes_written": n * 2, "ms_per_copy": round(ms, 4),
            "GBs": round(2 * n * 2 / (ms * 1e-3) / 1e9, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only time a plain device copy of BYTES (counter calibration)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end decoding run")
    ap.add_argument("--no-reuse", action="store_true", help="skip the reuse-call attention")
    ap.add_argument("--e2e-tokens", type=int, default=128)
    ap.add_argument("--no-slide", action="store_true")
    ap.add_argument("--slide-layers", type=int, default=32)
    ap.add_argument("--no-wca", action="store_true")
    ap.add_argument("--no-rows", action="store_true")
    ap.add_argument("--no-snapshot", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: cacheslide_amd has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        return 2
    import torch

    device = torch.device("cuda", 0)
    if args.copy_calibration:
        print(json.dumps(copy_calibration(device, args.copy_calibration, args.steps)), flush=True)
        return 0
    inputs, shape, host = build_prefill(device)
    step = prefill_launcher(inputs, shape, device)
    ms = time_steps(step, args.steps, args.warmup)
    flops = prefill_flops(shape["B"], shape["HQ"], shape["N"], shape["D"], shape["P"])
    tflops = flops / (ms * 1e-3) / 1e12
    note(f"prefill: {ms:.3f} ms/step")
    check_err = spot_check_prefill(inputs, host, shape)
    if check_err > 2e-2:
        print(f"prefill spot check failed: max abs error {check_err}", file=sys.stderr)
        return 1
    record = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) Q/K/V, CoPE table N(0,0.02), random-permutation block tables",
        "config": {
            "workload": "ccpe_prefill_paged: batch 8 x 4 chunks x 1024 tokens, 32q/8kv heads, "
                        "head_dim 128, CoPE P=64, paged KV block 16",
            "batch": shape["B"],
            "tokens_per_request": shape["N"],
            "flop_per_step": flops,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic_from_profiles("ccpe_prefill_paged_mistral7b"),
        },
        "spot_check_max_abs_err": round(check_err, 5),
    }
    del inputs
    torch.cuda.empty_cache()
    if not args.no_decode:
        record["decode"] = decode_measure(device, max(5, args.steps // 5), 5)
        note(f"decode: {record['decode']['ms_per_call']} ms/call")
    if not args.no_e2e:
        record["decode_e2e"] = decode_e2e_measure(device, args.e2e_tokens)
        note(f"decode e2e: {record['decode_e2e']['tok_per_s']} tok/s")
    if not args.no_e2e:
        record["tiny_e2e"] = tiny_e2e_measure(device)
        note(f"tiny e2e: {record['tiny_e2e']['wall_ms_per_case']} ms per case")
    if not args.no_reuse:
        record["reuse"] = reuse_measure(device)
        note(f"reuse: {record['reuse']['ms_per_call']} ms/call (generic {record['reuse']['generic_ms_per_call']})")
        record["calibration_call"] = calibration_measure(device)
        note(f"calibration call: {record['calibration_call']['ms_per_call']} ms/call "
             f"(generic {record['calibration_call']['generic_ms_per_call']})")
    if not args.no_slide:
        try:
            record["slide"] = slide_measure(device, max(3, args.steps // 10), args.slide_layers)
        except torch.cuda.OutOfMemoryError as error:  # pragma: no cover - depends on the device
            record["slide"] = {"error": f"out of memory: {error}"}
            torch.cuda.empty_cache()
        note(f"slide: {record['slide'].get('ms_per_step')} ms/step")
    if not args.no_wca:
        record["wca"] = wca_measure(device)
        note(f"wca: {record['wca']['update_ms_per_layer']} ms/layer update")
    if not args.no_rows:
        record["rows"] = rows_measure(device)
        note(f"rows: remap {record['rows']['remap_us_per_call']} us, "
             f"scatter {record['rows']['scatter_us_per_call']} us")
    if not args.no_snapshot:
        record["snapshot"] = snapshot_measure(device)
        note(f"snapshot: decode {record['snapshot']['decode_ms_per_page']} ms/page, "
             f"layer loop {record['snapshot']['layer_loop']}")
    if not args.no_cpu_baseline:
        note("cpu baseline: prefill")
        record["cpu_baseline"] = cpu_baseline(host, shape)
        if "decode" in record:
            note("cpu baseline: decode")
            record["decode"]["cpu_baseline"] = cpu_decode_leg()
        if "slide" in record:
            note("cpu baseline: slide")
            record["slide"]["cpu_baseline"] = cpu_slide_leg()
        if "wca" in record:
            note("cpu baseline: wca")
            record["wca"]["cpu_baseline"] = cpu_wca_leg()
        if "tiny_e2e" in record:
            note("cpu baseline: tiny e2e")
            record["tiny_e2e"]["cpu_baseline"] = cpu_tiny_e2e_leg(record["tiny_e2e"]["tokens"])
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
