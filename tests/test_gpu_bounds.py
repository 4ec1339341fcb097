"""Page ids outside the pool, missing pages and duplicate slots on the device path.

Engine::run_paged rejects a table entry outside the pool (src/inference/paging.rs:139-144)
and a second write to one slot (paging.rs:163-166) before anything runs.  The device
packing makes the same checks and, on failure, leaves cu_seqlens empty and every slot
unset, so the plan schedules nothing: the step's output and the pool stay untouched.
Independently of packing, the attention kernels never base a load on a table entry outside
the pool: such a page reads as zero keys.  Pools here are allocated with slack pages past
`pool_pages` filled with NaN, so even a kernel without the bound would read mapped memory
(and show NaN) instead of faulting."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF
E_ROWS, E_PAGE_RANGE, E_POSITION, E_MISSING_PAGE, E_DUPLICATE = 1, 6, 8, 10, 11


def _pack(lia, slots, q_lens, cached, table, stride, P, pool_pages, context, max_rows):
    n = len(slots)
    cu = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    out = [torch.full((max_rows,), -7, dtype=torch.int32, device="cuda") for _ in range(3)]
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    lia.pack_device(G.u32_dev(slots), G.u32_dev(q_lens), G.u32_dev(cached),
                    G.u32_dev(np.asarray(table, np.uint32)), stride, P, pool_pages, context,
                    max_rows, cu, out[0], out[1], out[2], status)
    torch.cuda.synchronize()
    u = lambda t: t.cpu().numpy().view(np.uint32)
    return int(status.item()), u(cu), u(out[0]), u(out[1]), u(out[2])


def _rejected(cu, slots, rows):
    return np.all(cu == 0) and np.all(slots[:rows] == NONE)


def test_pack_rejects_table_entry_outside_pool_before_row_checks(lia):
    """Sequence 1's cached page 0 is page 40 of a 32-page pool; sequence 0's row has a
    position past the context.  The table check comes first, as in paging.rs."""
    stride, P = 4, 16
    table = [3, 4, 10, 11, 40, 7, NONE, NONE]
    st, cu, pos, seq, slots = _pack(lia, [0, 1], [1, 1], [70, 20], table, stride, P, 32, 64, 4)
    assert st == E_PAGE_RANGE
    assert _rejected(cu, slots, 2)
    # without the bad entry the row error is reported
    table[4] = 9
    st, cu, *_ = _pack(lia, [0, 1], [1, 1], [70, 20], table, stride, P, 32, 64, 4)
    assert st == E_POSITION


def test_pack_reports_missing_cached_page(lia):
    stride, P = 4, 16
    # sequence 0 fine (rows 0, 1); sequence 1 (rows 2, 3) attends cached page 0, marked missing
    table = [3, 4, NONE, NONE, NONE, 7, NONE, NONE]
    st, cu, pos, seq, slots = _pack(lia, [0, 1], [2, 2], [5, 16], table, stride, P, 32, 64, 8)
    assert st == E_MISSING_PAGE
    assert _rejected(cu, slots, 4)


def test_pack_table_checks_come_before_row_checks_and_after_the_row_count(lia):
    stride, P = 4, 16
    # sequence 0's cached page is missing; sequence 1's row is past the context
    table = [NONE, 4, NONE, NONE, 5, 6, NONE, NONE]
    st, cu, pos, seq, slots = _pack(lia, [0, 1], [1, 1], [20, 70], table, stride, P, 32, 64, 4)
    assert st == E_MISSING_PAGE and _rejected(cu, slots, 4)
    # an out-of-pool entry outranks the missing page
    table[5] = 99
    st, *_ = _pack(lia, [0, 1], [1, 1], [20, 40], table, stride, P, 32, 64, 4)
    assert st == E_PAGE_RANGE
    # more rows than max_rows outranks both
    st, cu, pos, seq, slots = _pack(lia, [0, 1], [3, 3], [20, 40], table, stride, P, 32, 64, 4)
    assert st == E_ROWS and _rejected(cu, slots, 4)


def test_pack_rejects_duplicate_slots_across_sequences(lia):
    stride, P = 4, 16
    # both sequences append at positions 16, 17 into physical page 4
    table = [3, 4, NONE, NONE, 5, 4, NONE, NONE]
    st, cu, pos, seq, slots = _pack(lia, [0, 1], [2, 2], [16, 16], table, stride, P, 32, 64, 8)
    assert st == E_DUPLICATE
    assert _rejected(cu, slots, 4)


def test_pack_rejects_duplicate_slots_within_a_sequence(lia):
    stride, P = 4, 16
    table = [6, 6, NONE, NONE]  # logical pages 0 and 1 are the same physical page
    st, cu, *_ = _pack(lia, [0], [32], [0], table, stride, P, 32, 64, 32)
    assert st == E_DUPLICATE


def test_pack_duplicate_check_over_several_hash_passes(lia):
    """More rows than one LDS hash pass holds (4,100 rows): the only duplicate pair is the
    last page's slots against page 3's, found in whichever pass holds them."""
    P, n = 16, 4100
    stride = -(-n // P)
    rng = np.random.default_rng(3)
    pool = stride + 8
    table = rng.permutation(pool)[:stride].astype(np.uint32)
    st, cu, pos, seq, slots = _pack(lia, [0], [n], [0], table, stride, P, pool, stride * P, n)
    assert st == 0
    assert len(np.unique(slots[:n])) == n
    table[stride - 1] = table[3]
    st, cu, pos, seq, slots = _pack(lia, [0], [n], [0], table, stride, P, pool, stride * P, n)
    assert st == E_DUPLICATE
    assert _rejected(cu, slots, n)


def _slack_case(wl, seed, wide=True):
    """Decode, MTP and (wide) a 64-row chunk: the batch runs on the prefill kernel when wide,
    else on the decode kernel."""
    q_last = 64 if wide else 2
    b = wl.custom([700, 40 + 3, 1500, 2000 + q_last], [1, 3, 1, q_last], seed=seed)
    case = G.Case(b, seed=seed)
    g = b.geom
    W = g.hkv * g.d
    slack = 8
    nan = 0x7FC0  # bf16 quiet NaN
    kc = np.concatenate([case.kc.reshape(-1, W), np.full((slack * g.page_size, W), nan, np.uint16)])
    vc = np.concatenate([case.vc.reshape(-1, W), np.full((slack * g.page_size, W), nan, np.uint16)])
    return b, case, kc, vc


@pytest.mark.parametrize("wide", [False, True])
def test_step_with_out_of_pool_page_writes_nothing(lia, wl, wide):
    """A step whose block table names a page past the pool (in the slack): device packing
    reports it, the plan schedules nothing, the output keeps its sentinel and the pool,
    slack included, keeps its bytes."""
    b, case, kc, vc = _slack_case(wl, 41, wide)
    g = b.geom
    P, W = g.page_size, g.hkv * g.d
    flat = b.flat_table()
    flat[2 * b.stride + 5] = b.pool_pages + 2  # a cached page of sequence 2
    dkc, dvc = G.to_dev(kc.reshape(-1), torch.int16), G.to_dev(vc.reshape(-1), torch.int16)
    dflat = G.u32_dev(flat)
    rows = b.n_rows
    cu = torch.zeros(b.n_seqs + 1, dtype=torch.int32, device="cuda")
    positions, sequences, slots = (torch.zeros(rows, dtype=torch.int32, device="cuda") for _ in range(3))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    cfg = case.config(lia)
    ws = G.dirty_workspace(lia, cfg)
    out = torch.full((rows, g.hq, g.d), 7.0, dtype=torch.bfloat16, device="cuda")
    newk = torch.ones((rows, W), dtype=torch.bfloat16, device="cuda")
    lia.pack_device(G.u32_dev(np.arange(b.n_seqs)), G.u32_dev(b.q_len), G.u32_dev(b.cached), dflat,
                    b.stride, P, b.pool_pages, b.stride * P, rows, cu, positions, sequences, slots,
                    status)
    lia.attention_plan(cfg, b.n_seqs, rows, cu, positions, sequences, ws, pages=dflat)
    lia.attention_partial_append(cfg, b.n_seqs, dflat, slots, G.to_dev(case.q_store, torch.bfloat16),
                                 newk, newk, dkc, dvc, out, ws)
    lia.attention_merge(cfg, b.n_seqs, rows, out, ws)
    torch.cuda.synchronize()
    assert status.item() == E_PAGE_RANGE
    assert torch.all(out == 7.0).item()
    assert np.array_equal(dkc.cpu().numpy().view(np.uint16), kc.reshape(-1))
    assert np.array_equal(dvc.cpu().numpy().view(np.uint16), vc.reshape(-1))


@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("logical", [0, 5, 40])
def test_attention_reads_no_page_outside_the_pool(lia, wl, logical, wide):
    """Host-packed metadata (no packing check) with one table entry past the pool: the
    attention kernels read that page as zero keys - never the NaN slack behind it - so the
    result equals the float64 oracle over a pool whose page there is all zero.  Logical page
    0 is also the first page of a workgroup's range (the plan's preloaded pages)."""
    b, case, kc, vc = _slack_case(wl, 42 + logical, wide)
    g = b.geom
    flat = b.flat_table()
    seq = 3 if logical == 40 else 2
    flat[seq * b.stride + logical] = b.pool_pages + 2
    case.flat = flat
    W = g.hkv * g.d
    dev = case.device()
    dev["kc"] = G.to_dev(kc.reshape(-1), torch.int16)
    dev["vc"] = G.to_dev(vc.reshape(-1), torch.int16)
    got = case.run(lia, dev)
    # the oracle reads the same table over a pool whose slack is zero
    zk = kc.copy()
    zv = vc.copy()
    zk[b.pool_pages * g.page_size:] = 0
    zv[b.pool_pages * g.page_size:] = 0
    case.kc, case.vc = zk.reshape(-1), zv.reshape(-1)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] out-of-pool page at logical {logical} wide={wide}: max_abs={mx:.3e} mean_abs={mean:.3e}",
          flush=True)
    assert np.all(np.isfinite(got))
    assert mx < 2e-2 and mean < 2e-3
