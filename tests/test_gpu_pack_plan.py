"""lia_pack_plan_device (packing and the plan in two launches, the plan built from the packing's
inputs) against lia_pack_device followed by lia_attention_plan: the same metadata, status, plan
bytes and attention outputs, bit for bit; and a rejected step (packing failures of every kind)
writes neither the output nor the pool, as the reference rejects a batch before anything runs
(src/inference/paging.rs:118-186)."""
import numpy as np
import pytest
import torch

import gpu_data as G

pytestmark = pytest.mark.gpu

E_ROWS, E_PAGE_RANGE, E_POSITION, E_MISSING_PAGE, E_DUPLICATE = 1, 6, 8, 10, 11


def _inputs(b):
    return (G.u32_dev(np.arange(b.n_seqs)), G.u32_dev(b.q_len), G.u32_dev(b.cached))


def _run(lia, b, case, fused, flat, cfg, fill_ws=0, fused_append=True):
    """One step: packing (+ plan), fused append + attention, merge.  Returns everything the step
    writes, as host arrays."""
    g = b.geom
    rows, W = b.n_rows, g.hkv * g.d
    seq_slots, q_lens, cached = _inputs(b)
    dflat = G.u32_dev(flat)
    cu = torch.full((b.n_seqs + 1,), -7, dtype=torch.int32, device="cuda")
    meta = [torch.full((cfg.max_rows,), -7, dtype=torch.int32, device="cuda") for _ in range(3)]
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    ws = torch.full((lia.workspace_bytes(cfg),), fill_ws, dtype=torch.uint8, device="cuda")
    kc = G.to_dev(case.kc, torch.int16).clone()
    vc = G.to_dev(case.vc, torch.int16).clone()
    out = torch.full((rows, g.hq, g.d), 7.0, dtype=torch.bfloat16, device="cuda")
    newk = G.to_dev(case.kc.reshape(-1, W)[:rows].copy(), torch.int16).view(torch.bfloat16)
    newv = G.to_dev(case.vc.reshape(-1, W)[:rows].copy(), torch.int16).view(torch.bfloat16)
    context = b.stride * g.page_size
    if fused:
        lia.pack_plan_device(cfg, seq_slots, q_lens, cached, dflat, rows, context, cu, meta[0],
                             meta[1], meta[2], status, ws)
    else:
        lia.pack_device(seq_slots, q_lens, cached, dflat, b.stride, g.page_size, b.pool_pages, context,
                        cfg.max_rows, cu, meta[0], meta[1], meta[2], status)
        lia.attention_plan(cfg, b.n_seqs, rows, cu, meta[0], meta[1], ws, pages=dflat)
    q = G.to_dev(case.q_store, torch.bfloat16)
    if fused_append:
        lia.attention_partial_append(cfg, b.n_seqs, dflat, meta[2], q, newk, newv, kc, vc, out, ws)
    else:
        lia.attention_partial(cfg, b.n_seqs, dflat, q, kc, vc, out, ws)
    lia.attention_merge(cfg, b.n_seqs, rows, out, ws)
    torch.cuda.synchronize()
    u = lambda t: t.cpu().numpy().view(np.uint32)
    return dict(status=int(status.item()), cu=u(cu), positions=u(meta[0]), sequences=u(meta[1]),
                slots=u(meta[2]), out=out.view(torch.int16).cpu().numpy(),
                kc=kc.cpu().numpy(), vc=vc.cpu().numpy(), header=u(ws[:32].view(torch.int32)))


def _cases(wl):
    rng = np.random.default_rng(31)
    k = rng.integers(1, 4, size=12)
    return [
        ("decode", wl.custom([17, 300, 5000, 12000, 64, 1], [1] * 6, seed=31)),
        ("mtp", wl.custom(rng.integers(20, 4000, size=12), 1 + k, seed=32)),
        ("prefill", wl.custom([64, 430, 1200, 777, 1500, 33], [64, 130, 200, 1, 1, 1], seed=33)),
        ("config2", wl.config2(seed=2)),
        ("config4", wl.config4(seed=1)),
    ]


@pytest.mark.parametrize("idx", range(5))
def test_pack_plan_matches_pack_then_plan(lia, wl, idx):
    name, b = _cases(wl)[idx]
    print(f"[case] pack+plan {name}: seqs={b.n_seqs} rows={b.n_rows}", flush=True)
    case = G.Case(b, seed=40 + idx)
    cfg = case.config(lia)
    flat = b.flat_table()
    ref = _run(lia, b, case, False, flat, cfg)
    got = _run(lia, b, case, True, flat, cfg, fill_ws=0xA5)
    assert ref["status"] == 0 and got["status"] == 0
    for key in ("cu", "positions", "sequences", "slots", "out", "kc", "vc"):
        assert np.array_equal(got[key], ref[key]), (name, key)
    assert np.array_equal(got["header"][:5], ref["header"][:5]), name  # units, blocks, ranges, overflow, verdict
    assert got["header"][4] == 0


def _reject_cases(b):
    """(label, table edit, expected status): each makes the step fail a packing check."""
    P = b.geom.page_size
    flat = b.flat_table()
    s = b.stride
    out = []
    f = flat.copy(); f[2 * s + 1] = b.pool_pages + 3
    out.append(("page outside the pool", f, E_PAGE_RANGE))
    f = flat.copy(); f[1 * s + 0] = 0xFFFFFFFF  # a page under sequence 1's cached keys
    out.append(("missing cached page", f, E_MISSING_PAGE))
    # sequences 0 and 2 add one row each at positions 699 and 1499 (both at offset 11 of their
    # page): sequence 2's page of that row aliased to sequence 0's gives both rows one slot
    p0, p2 = int(b.cached[0]), int(b.cached[2])
    assert p0 % P == p2 % P and b.q_len[0] == b.q_len[2] == 1
    f = flat.copy(); f[2 * s + p2 // P] = f[0 * s + p0 // P]
    out.append(("duplicate slot", f, E_DUPLICATE))
    return out


@pytest.mark.parametrize("wide", [False, True])
def test_pack_plan_rejected_step_writes_nothing(lia, wl, wide):
    q_last = 64 if wide else 2
    b = wl.custom([700, 43, 1500, 2000 + q_last], [1, 3, 1, q_last], seed=41)
    case = G.Case(b, seed=41)
    cfg = case.config(lia)
    clean = _run(lia, b, case, False, b.flat_table(), cfg)
    for label, flat, want in _reject_cases(b):
        print(f"[case] rejected step ({label}), wide={wide}", flush=True)
        for fused in (False, True):
            r = _run(lia, b, case, fused, flat, cfg, fill_ws=0xA5 if fused else 0)
            assert r["status"] == want, (label, fused, r["status"])
            assert np.all(r["out"] == np.int16(0x40E0)), (label, fused)  # bf16 7.0: untouched
            assert np.array_equal(r["kc"], case.kc.view(np.int16)), (label, fused)
            assert np.array_equal(r["vc"], case.vc.view(np.int16)), (label, fused)
            if fused:
                assert r["header"][4] == want
    # and the step after a rejected one runs normally on the same inputs
    ok = _run(lia, b, case, True, b.flat_table(), cfg)
    assert ok["status"] == 0 and np.array_equal(ok["out"], clean["out"])


def test_pack_plan_rows_over_capacity_and_row_count_mismatch(lia, wl):
    b = wl.custom([300, 900], [5, 7], seed=42)
    case = G.Case(b, seed=42)
    g = b.geom
    cfg = case.config(lia, max_rows=12)
    seq_slots, q_lens, cached = _inputs(b)
    dflat = G.u32_dev(b.flat_table())
    for q, n_rows, want in ((np.array([5, 8], np.uint32), 12, E_ROWS),   # 13 rows > max_rows 12
                            (np.array([5, 6], np.uint32), 12, 0)):        # 11 rows, n_rows 12
        cu = torch.zeros(3, dtype=torch.int32, device="cuda")
        meta = [torch.zeros(12, dtype=torch.int32, device="cuda") for _ in range(3)]
        status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        ws = torch.full((lia.workspace_bytes(cfg),), 0xA5, dtype=torch.uint8, device="cuda")
        lia.pack_plan_device(cfg, seq_slots, G.u32_dev(q), cached, dflat, n_rows, b.stride * g.page_size,
                             cu, meta[0], meta[1], meta[2], status, ws)
        torch.cuda.synchronize()
        hdr = ws[:32].view(torch.int32).cpu().numpy()
        assert int(status.item()) == want
        # nothing planned: an over-capacity batch (rejected) and a row count other than n_rows
        assert hdr[0] == 0 and hdr[2] == 0, (q, hdr)
