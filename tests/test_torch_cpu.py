"""The torch CPU restatement that bench.py times as its CPU baseline equals
the numpy oracle (CPU only)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import ccpe as orc
from oracle import slide as oslide
from oracle import torch_cpu as tc
from oracle import wca as owca


def test_cope_attention_matches_oracle():
    g = torch.Generator().manual_seed(1)
    q = torch.randn((150, 8, 32), generator=g)
    k = torch.randn((150, 2, 32), generator=g)
    v = torch.randn((150, 2, 32), generator=g)
    e = torch.randn((32, 64), generator=g) * 0.3
    rows = torch.randperm(150, generator=g)[:70]
    got = tc.cope_attention(q[rows], k, v, e, rows, query_chunk_size=16)
    want = orc.cope_attention(q[rows].numpy(), k.numpy(), v.numpy(), e.numpy(), rows.numpy())
    np.testing.assert_allclose(got.numpy(), want, atol=2e-5, rtol=2e-5)
    # bf16 inputs: the cast back to the value dtype, as the reference does
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    got = tc.cope_attention(qb[rows], kb, vb, e, rows)
    want = orc.cope_attention(qb[rows].float().numpy(), kb.float().numpy(), vb.float().numpy(), e.numpy(),
                              rows.numpy())
    np.testing.assert_allclose(got.float().numpy(), orc.bf16_round(want), atol=1e-2, rtol=1e-2)


def test_decode_step_reads_the_canonical_slots():
    g = torch.Generator().manual_seed(2)
    cache = torch.randn((20, 2, 16, 64), generator=g)
    row = torch.randperm(20, generator=g)[:12].to(torch.int32)
    n = 180
    q = torch.randn((1, 4, 32), generator=g)
    e = torch.randn((32, 16), generator=g) * 0.1
    got = tc.decode_step(cache, row, n, q, e)
    t = np.arange(n)
    slots = row.numpy()[t // 16].astype(np.int64) * 16 + t % 16
    rec = cache.numpy()[slots // 16, :, slots % 16]
    want = orc.cope_attention(q.numpy(), rec[..., :32], rec[..., 32:], e.numpy(), np.array([n - 1]))
    np.testing.assert_allclose(got.numpy(), want, atol=2e-5, rtol=2e-5)


def test_relocate_matches_oracle_moves():
    g = torch.Generator().manual_seed(3)
    cache = torch.randn((30, 2, 4, 8), generator=g)
    ref = cache.numpy()[None].copy()
    perm = torch.randperm(30, generator=g)
    sb, db = perm[:6], perm[6:12]
    slots = (perm[12:20, None] * 4 + torch.arange(4)).reshape(-1)
    ss, ds = slots[:10], slots[10:20]
    mapping = torch.full((40,), -1, dtype=torch.long)
    tokens, new_slots = torch.arange(0, 40, 3), torch.arange(0, 40, 3) * 7
    freed = tc.relocate(cache, sb, db, ss, ds, mapping, tokens, new_slots)
    oslide.page_copy(ref, sb.tolist(), db.tolist())
    oslide.slot_copy(ref, ss.tolist(), ds.tolist())
    np.testing.assert_array_equal(cache.numpy(), ref[0])
    assert mapping[tokens].tolist() == new_slots.tolist() and int((mapping >= 0).sum()) == len(tokens)
    assert sorted(freed.tolist()) == sorted((sb[:, None] * 4 + torch.arange(4)).reshape(-1).tolist() + ss.tolist())


def test_wca_trajectory_matches_oracle():
    T, H, D = 400, 4, 16
    g = torch.Generator().manual_seed(4)
    fresh = torch.randn((T, H, D), generator=g).double()
    cached = fresh + 0.05 * torch.randn((T, H, D), generator=g).double()
    reused = torch.ones(T, dtype=torch.bool)
    mandatory = torch.zeros(T, dtype=torch.bool)
    mandatory[-1] = True
    st = tc.WCA(cached, fresh, reused, mandatory, gate_interval=2, threshold=0.5)
    ost = owca.State(cached.numpy(), fresh.numpy(), reused.numpy(), mandatory.numpy(), fraction=0.15,
                     gate_interval=2, threshold=0.5, dtype="float64")
    assert st.budget == ost.budget
    assert st.active.tolist() == ost.active.tolist()
    for layer in range(2, 8):
        ck = torch.randn((T, H, D), generator=g).double()
        cv = torch.randn((T, H, D), generator=g).double()
        idx = st.active
        rk = ck[idx] + 0.3 * torch.randn((len(idx), H, D), generator=g).double()
        rk[::5] = torch.randn((len(rk[::5]), H, D), generator=g).double()     # some rows far off
        rv = cv[idx] + 0.3 * torch.randn((len(idx), H, D), generator=g).double()
        idx_t, fk, fv, rem, prom = st.update(layer, ck, cv, rk, rv)
        o_idx, ofk, ofv, _, orem, oprom, _ = ost.update(layer, ck.numpy(), cv.numpy(), rk.numpy(), rv.numpy())
        assert idx_t.tolist() == o_idx.tolist()
        # weights differ from the exact sums in the last ulp (torch reduces in tree order)
        np.testing.assert_allclose(fk.numpy(), ofk, rtol=1e-12, atol=1e-12)
        assert rem.tolist() == orem.tolist() and prom.tolist() == oprom.tolist()
