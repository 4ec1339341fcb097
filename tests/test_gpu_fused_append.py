"""GPU parity of lia_attention_partial_append (KV append fused into the attention launch).

Each case takes a batch whose pool already holds every key (the CPU oracle's input), lifts
the step's new rows out of the pool into new_k / new_v, overwrites their pool slots with
garbage on the device and runs plan -> partial_append -> merge.  The output must match the
float64 oracle on the original pool (same tolerances as the unfused path) and the pool
afterwards must equal the original bytes, i.e. what lia_kv_append writes."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, F16, F32, FP8

pytestmark = pytest.mark.gpu

TOL = {BF16: (2e-2, 2e-3), F16: (2e-2, 2e-3)}


def _run_fused(case, lia, seed, garbage=True):
    b, g = case.batch, case.g
    dev = case.device()
    W = g.hkv * g.d
    slots = b.slot_mapping().astype(np.int64)
    kc = case.kc.reshape(-1, W)
    vc = case.vc.reshape(-1, W)
    newk, newv = kc[slots].copy(), vc[slots].copy()
    dkc, dvc = dev["kc"].view(-1, W), dev["vc"].view(-1, W)
    if garbage:
        rng = np.random.default_rng(seed + 7)
        junk = rng.integers(0, 65535, newk.shape).astype(np.uint16)
        idx = torch.from_numpy(slots).cuda()
        dkc[idx] = G.to_dev(junk, torch.int16)
        dvc[idx] = G.to_dev(junk[::-1].copy(), torch.int16)
    cfg = case.config(lia)
    ws = G.dirty_workspace(lia, cfg)
    odt = torch.float32 if g.out_dtype == F32 else torch.bfloat16
    out = torch.full((b.n_rows, g.hq, g.d), float("nan"), dtype=odt, device="cuda")
    lia.attention_plan(cfg, b.n_seqs, b.n_rows, dev["cu"], dev["positions"], dev["sequences"], ws,
                       pages=dev["pages"])
    lia.attention_partial_append(cfg, b.n_seqs, dev["pages"], G.u32_dev(slots), dev["q"],
                                 G.to_dev(newk, torch.int16), G.to_dev(newv, torch.int16),
                                 dev["kc"], dev["vc"], out, ws)
    lia.attention_merge(cfg, b.n_seqs, b.n_rows, out, ws)
    torch.cuda.synchronize()
    return (out.float().cpu().numpy(), dev["kc"].cpu().numpy().view(np.uint16),
            dev["vc"].cpu().numpy().view(np.uint16))


def _check(case, lia, label, seed):
    print(f"[case] fused {label}: seqs={case.batch.n_seqs} rows={case.batch.n_rows} "
          f"ctx={case.batch.ctx.tolist()[:8]} q_len={case.batch.q_len.tolist()[:8]}", flush=True)
    got, kpool, vpool = _run_fused(case, lia, seed)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] fused {label}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)), label
    tol_max, tol_mean = TOL[case.g.kv_dtype]
    assert mx < tol_max and mean < tol_mean, (label, mx, mean)
    assert np.array_equal(kpool, case.kc) and np.array_equal(vpool, case.vc), label


def test_fused_config2_decode(lia, wl):
    _check(G.Case(wl.config2(seed=0, layers=1), seed=0), lia, "cfg2", 0)


@pytest.mark.parametrize("kv", [BF16, F16])
@pytest.mark.parametrize("d,hq,hkv,page", [(128, 16, 2, 16), (64, 8, 2, 32), (128, 32, 2, 64)])
def test_fused_decode_edge_contexts(lia, wl, kv, d, hq, hkv, page):
    ctx = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 511, 1000, 2049, 4097]
    g = wl.Geometry(hq=hq, hkv=hkv, d=d, page_size=page, kv_dtype=kv, q_dtype=F32, out_dtype=F32)
    b = wl.custom(ctx, [1] * len(ctx), geom=g, seed=13)
    _check(G.Case(b, seed=13), lia, f"edge kv={kv} d={d} page={page}", 13)


def test_fused_mtp_verify(lia, wl):
    rng = np.random.default_rng(14)
    k = rng.integers(1, 4, size=12)
    ctx = rng.integers(20, 3000, size=12)
    _check(G.Case(wl.custom(ctx, 1 + k, seed=14), seed=14), lia, "mtp", 14)


@pytest.mark.parametrize("hq,hkv", [(16, 2), (8, 8), (32, 2), (16, 1)])
def test_fused_prefill_chunks(lia, wl, hq, hkv):
    """Prefill from scratch (no cached keys), prefix-cached chunks whose new keys span
    many blocks and column blocks, and decode rows in one batch."""
    g = wl.Geometry(hq=hq, hkv=hkv, d=128)
    ctx = [64, 300 + 130, 1000 + 200, 777, 1500, 33, 97]
    q = [64, 130, 200, 1, 1, 1, 97]
    _check(G.Case(wl.custom(ctx, q, geom=g, seed=15), seed=15), lia, f"prefill hq={hq} hkv={hkv}", 15)


@pytest.mark.parametrize("q_len", [[1, 0, 3, 0, 1], [0, 2, 0, 64, 0]])
def test_fused_sequences_without_rows(lia, wl, q_len):
    """Sequences adding no rows next to decode, MTP and prefill rows, through the fused launch."""
    ctx = [500, 300, 1000 + 200, 64 + 64, 4097]
    _check(G.Case(wl.custom(ctx, q_len, seed=18), seed=18), lia, f"no-row sequences {q_len}", 18)


def test_fused_matches_unfused(lia, wl):
    """Same output as kv_append + partial + merge to within accumulation order."""
    b = wl.custom([5000, 17, 900, 64], [1, 1, 3, 64], seed=16)
    case = G.Case(b, seed=16)
    fused, _, _ = _run_fused(case, lia, 16)
    plain = case.run(lia)
    assert np.max(np.abs(fused - plain)) < 1e-2


@pytest.mark.parametrize("kv", [BF16, F16])
def test_fused_append_canonicalises_nan_like_kv_append(lia, wl, O, kv):
    """NaN payloads in the new rows land in the pool exactly as lia_kv_append stores
    them (canonical quiet NaN with the sign kept); other values are copied unchanged."""
    g = wl.Geometry(hq=16, hkv=2, d=128, kv_dtype=kv)
    b = wl.custom([40, 700], [3, 1], geom=g, seed=17)
    case = G.Case(b, seed=17)
    W = g.hkv * g.d
    slots = b.slot_mapping().astype(np.int64)
    rng = np.random.default_rng(17)
    newk = case.kc.reshape(-1, W)[slots].copy()
    newv = case.vc.reshape(-1, W)[slots].copy()
    nan = 0x7f81 if kv == BF16 else 0x7c01
    for arr in (newk, newv):
        pick = rng.choice(arr.size, 50, replace=False)
        arr.reshape(-1)[pick] = (nan + rng.integers(0, 60, 50)) | (rng.integers(0, 2, 50) << 15)
    # expected pool: the oracle append (src dtype = pool dtype) into the original pool
    kexp, vexp = case.kc.copy(), case.vc.copy()
    layout = O.KVLayout(g.hkv, g.d, g.page_size, b.pool_pages, kv)
    O.kv_append(layout, b.positions(), b.sequences(), b.flat_table(), b.stride, newk, newv,
                kexp, vexp, src_dtype=kv, slot_mapping=b.slot_mapping())
    dev = case.device()
    cfg = case.config(lia)
    ws = G.dirty_workspace(lia, cfg)
    out = torch.empty((b.n_rows, g.hq, g.d), dtype=torch.bfloat16, device="cuda")
    lia.attention_plan(cfg, b.n_seqs, b.n_rows, dev["cu"], dev["positions"], dev["sequences"], ws,
                       pages=dev["pages"])
    lia.attention_partial_append(cfg, b.n_seqs, dev["pages"], G.u32_dev(b.slot_mapping()),
                                 dev["q"], G.to_dev(newk, torch.int16), G.to_dev(newv, torch.int16),
                                 dev["kc"], dev["vc"], out, ws)
    torch.cuda.synchronize()
    assert np.array_equal(dev["kc"].cpu().numpy().view(np.uint16), kexp)
    assert np.array_equal(dev["vc"].cpu().numpy().view(np.uint16), vexp)


@pytest.mark.parametrize("seed", [0, 1])
def test_config3_full_step_with_shared_prefix_pages(lia, wl, O, seed):
    """BASELINE config 3 at full size as a step: device packing builds cu_seqlens, positions,
    sequences and the slot mapping from per-sequence counts (bit-exact against the oracle's
    host packing), the plan, the attention launch with the new K/V appended into the pool,
    and the merge.  The prefill chunks and decode rows share a 256-page cached prefix by
    reference count.  Outputs against the float64 oracle; the pool against lo_kv_append of
    the new rows into the pool as it was before the step."""
    b = wl.config3(seed=seed)
    assert b.shared, "config 3 shares prefix pages"
    case = G.Case(b, seed=seed)
    g = b.geom
    P, W = g.page_size, g.hkv * g.d
    print(f"[case] cfg3 step: rows={b.n_rows} seqs={b.n_seqs} {b.notes}", flush=True)
    slots_h = b.slot_mapping()
    kc0, vc0 = case.kc.reshape(-1, W), case.vc.reshape(-1, W)
    newk, newv = kc0[slots_h.astype(np.int64)].copy(), vc0[slots_h.astype(np.int64)].copy()
    # the pool before the step: the new rows' slots hold junk
    rng = np.random.default_rng(33)
    before_k, before_v = kc0.copy(), vc0.copy()
    before_k[slots_h.astype(np.int64)] = rng.integers(0, 65535, newk.shape).astype(np.uint16)
    before_v[slots_h.astype(np.int64)] = rng.integers(0, 65535, newv.shape).astype(np.uint16)
    dkc = G.to_dev(before_k.reshape(-1), torch.int16)
    dvc = G.to_dev(before_v.reshape(-1), torch.int16)
    flat = G.u32_dev(b.flat_table())
    rows = b.n_rows
    cu = torch.zeros(b.n_seqs + 1, dtype=torch.int32, device="cuda")
    positions = torch.zeros(rows, dtype=torch.int32, device="cuda")
    sequences = torch.zeros_like(positions)
    slots = torch.zeros_like(positions)
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    cfg = case.config(lia)
    ws = G.dirty_workspace(lia, cfg)
    out = torch.full((rows, g.hq, g.d), float("nan"), dtype=torch.bfloat16, device="cuda")
    lia.pack_device(G.u32_dev(np.arange(b.n_seqs)), G.u32_dev(b.q_len), G.u32_dev(b.cached), flat,
                    b.stride, P, b.pool_pages, b.stride * P, rows, cu, positions, sequences, slots,
                    status)
    lia.attention_plan(cfg, b.n_seqs, rows, cu, positions, sequences, ws, pages=flat)
    lia.attention_partial_append(cfg, b.n_seqs, flat, slots, G.to_dev(case.q_store, torch.bfloat16),
                                 G.to_dev(newk, torch.int16), G.to_dev(newv, torch.int16), dkc, dvc,
                                 out, ws)
    lia.attention_merge(cfg, b.n_seqs, rows, out, ws)
    torch.cuda.synchronize()
    assert status.item() == 0
    # packing: the oracle's host packing of the same rows
    lim = O.PagingLimits(b.n_seqs, b.stride * P, P, b.pool_pages, 1, rows)
    st, packed = O.pack_rows(lim, [(0, int(p), int(s)) for p, s in zip(b.positions(), b.sequences())],
                             [t.tolist() for t in b.tables], [])
    assert st == 0
    assert np.array_equal(cu.cpu().numpy().view(np.uint32), packed["cu_seqlens"])
    assert np.array_equal(positions.cpu().numpy().view(np.uint32), packed["positions"])
    assert np.array_equal(sequences.cpu().numpy().view(np.uint32), packed["sequences"])
    assert np.array_equal(slots.cpu().numpy().view(np.uint32), packed["slot_mapping"])
    # pool: lo_kv_append of the step's rows into the pool as it was before
    kexp, vexp = before_k.reshape(-1).copy(), before_v.reshape(-1).copy()
    layout = O.KVLayout(g.hkv, g.d, P, b.pool_pages, g.kv_dtype)
    O.kv_append(layout, packed["positions"], packed["sequences"], b.flat_table(), b.stride, newk,
                newv, kexp, vexp, src_dtype=g.kv_dtype)
    assert np.array_equal(dkc.cpu().numpy().view(np.uint16), kexp)
    assert np.array_equal(dvc.cpu().numpy().view(np.uint16), vexp)
    got = out.float().cpu().numpy()
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] cfg3 step: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got))
    assert mx < 2e-2 and mean < 2e-3


@pytest.mark.parametrize("case_name", ["decode_mtp_prefill", "config5_head", "prefill_chunks"])
def test_fused_fp8_append(lia, wl, O, case_name):
    """lia_attention_partial_append_fp8: the step's bf16 rows are quantised into the FP8 pool
    exactly as lia_kv_append(src bf16) stores them - bytes and per-(page, head) scales, fresh
    pages (scale 0) taking scale 1 - and attended with those quantised values (float64
    oracle over the pool after the append, FP8 tolerance)."""
    if case_name == "config5_head":
        b5 = wl.config5(seed=0)
        keep = 8
        ctx, q_len = b5.ctx[:keep], b5.q_len[:keep]
        g = b5.geom
    elif case_name == "prefill_chunks":
        # prefill chunks after cached prefixes next to decode rows: 152 rows per sequence on
        # average, so the prefill kernel attends the FP8 pool
        ctx, q_len = [300, 1000 + 200, 2048 + 260, 700, 1500], [300, 200, 260, 1, 1]
        g = wl.Geometry(kv_dtype=FP8)
    else:
        # decode rows at and past page boundaries (fresh pages), MTP rows crossing a page,
        # a prefill chunk of 40 rows after 16 cached keys
        ctx, q_len = [17, 33, 100, 16 + 3, 16 + 40, 900], [1, 1, 1, 3, 40, 2]
        g = wl.Geometry(kv_dtype=FP8)
    b = wl.custom(ctx, q_len, geom=g, seed=71)
    P, W = g.page_size, g.hkv * g.d
    rng = np.random.default_rng(71)
    tokens = b.pool_pages * P
    layout = O.KVLayout(g.hkv, g.d, P, b.pool_pages, FP8)
    kc = np.zeros(tokens * W, np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros(b.pool_pages * g.hkv, np.float32)
    vs = np.zeros_like(ks)
    kf = rng.standard_normal((b.pool_pages, P, g.hkv, g.d)).astype(np.float32)
    vf = rng.standard_normal((b.pool_pages, P, g.hkv, g.d)).astype(np.float32)
    # quantise the pages holding cached keys; pages holding only new rows stay fresh (scale 0)
    cached_pages = set()
    for s, t in enumerate(b.tables):
        for lp in range(-(-int(b.cached[s]) // P)):
            cached_pages.add(int(t[lp]))
    ids = np.array(sorted(cached_pages), np.uint32)
    O.kv_quantize_pages(layout, ids, kf[ids], vf[ids], kc, vc, ks, vs)
    newk = O.from_f32(rng.standard_normal((b.n_rows, W)).astype(np.float32) * 2, BF16)
    newv = O.from_f32(rng.standard_normal((b.n_rows, W)).astype(np.float32), BF16)
    # expected pool after the step
    kexp, vexp, ksx, vsx = kc.copy(), vc.copy(), ks.copy(), vs.copy()
    O.kv_append(layout, b.positions(), b.sequences(), b.flat_table(), b.stride, newk, newv, kexp,
                vexp, src_dtype=BF16, k_scales=ksx, v_scales=vsx)
    assert (ksx != ks).any(), "some page was fresh"
    dkc, dvc = G.to_dev(kc, torch.uint8), G.to_dev(vc, torch.uint8)
    dks, dvs = G.to_dev(ks), G.to_dev(vs)
    qf = O.from_f32(rng.standard_normal((b.n_rows, g.hq, g.d)).astype(np.float32), BF16)
    cfg = lia.AttentionConfig(g.hq, g.hkv, g.d, P, b.pool_pages, b.stride, g.q_dtype, g.kv_dtype,
                              g.out_dtype, g.scale, b.n_seqs, b.n_rows, int(b.ctx.max()))
    ws = G.dirty_workspace(lia, cfg)
    out = torch.full((b.n_rows, g.hq, g.d), float("nan"), dtype=torch.bfloat16, device="cuda")
    flat = G.u32_dev(b.flat_table())
    print(f"[case] fused fp8 {case_name}: seqs={b.n_seqs} rows={b.n_rows}", flush=True)
    lia.attention_plan(cfg, b.n_seqs, b.n_rows, G.u32_dev(b.cu_seqlens()), G.u32_dev(b.positions()),
                       G.u32_dev(b.sequences()), ws, pages=flat)
    lia.attention_partial_append_fp8(cfg, b.n_seqs, flat, G.u32_dev(b.slot_mapping()),
                                     G.to_dev(qf, torch.bfloat16), G.to_dev(newk, torch.bfloat16),
                                     G.to_dev(newv, torch.bfloat16), dkc, dvc, dks, dvs, out, ws)
    lia.attention_merge(cfg, b.n_seqs, b.n_rows, out, ws)
    torch.cuda.synchronize()
    assert np.array_equal(dks.cpu().numpy(), ksx) and np.array_equal(dvs.cpu().numpy(), vsx)
    assert np.array_equal(dkc.cpu().numpy(), kexp) and np.array_equal(dvc.cpu().numpy(), vexp)
    geom = O.geom(g.hq, g.hkv, g.d, P, b.stride, FP8, g.scale)
    ref = O.attention_f64(geom, b.positions(), b.sequences(), b.flat_table(), O.to_f32(qf, BF16),
                          kexp, vexp, ksx, vsx)
    got = out.float().cpu().numpy()
    mx, mean = G.errors(got, ref)
    print(f"[case] fused fp8 {case_name}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)) and mx < 5e-2 and mean < 5e-3
