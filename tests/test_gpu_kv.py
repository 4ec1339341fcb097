"""GPU parity of packing, slot mapping, KV append and FP8 page quantisation: bit-exact
against the CPU oracle (through the C ABI)."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, F16, F32, FP8

pytestmark = pytest.mark.gpu


def _append_case(O, lia, wl, kv, src, page, use_slots, rows_per_seq=(1, 3, 40), seed=0):
    rng = np.random.default_rng(seed)
    g = wl.Geometry(hq=16, hkv=2, d=128, page_size=page, kv_dtype=kv)
    ctx = [50, 300, 1000]
    b = wl.custom(ctx, list(rows_per_seq), geom=g, seed=seed)
    n = b.n_rows
    W = g.hkv * g.d
    kf = rng.standard_normal((n, W)).astype(np.float32)
    vf = rng.standard_normal((n, W)).astype(np.float32)
    if src == BF16:
        ks, vs = O.from_f32(kf, BF16), O.from_f32(vf, BF16)
        kd, vd = G.to_dev(ks, torch.bfloat16), G.to_dev(vs, torch.bfloat16)
    elif src == F16:
        ks, vs = O.from_f32(kf, F16), O.from_f32(vf, F16)
        kd, vd = G.to_dev(ks, torch.float16), G.to_dev(vs, torch.float16)
    else:
        ks, vs = kf, vf
        kd, vd = G.to_dev(kf), G.to_dev(vf)
    tokens = b.pool_pages * page
    store = np.uint8 if kv == FP8 else np.uint16
    fill = rng.integers(0, 255 if kv == FP8 else 65535, tokens * W).astype(store)
    kc, vc = fill.copy(), fill[::-1].copy()
    k_scales = v_scales = None
    if kv == FP8:
        k_scales = rng.uniform(0.005, 0.02, b.pool_pages * g.hkv).astype(np.float32)
        v_scales = rng.uniform(0.005, 0.02, b.pool_pages * g.hkv).astype(np.float32)
        # pages never quantised (scale 0) take scale 1, which the append records
        k_scales[rng.random(k_scales.size) < 0.3] = 0.0
        v_scales[rng.random(v_scales.size) < 0.3] = 0.0
    layout_o = O.KVLayout(g.hkv, g.d, page, b.pool_pages, kv)
    layout_p = lia.KVLayout(g.hkv, g.d, page, b.pool_pages, kv)
    pos, seq, flat, slots = b.positions(), b.sequences(), b.flat_table(), b.slot_mapping()
    dkc = G.to_dev(kc, torch.uint8 if kv == FP8 else torch.int16)
    dvc = G.to_dev(vc, torch.uint8 if kv == FP8 else torch.int16)
    dks = G.to_dev(k_scales) if k_scales is not None else None
    dvs = G.to_dev(v_scales) if v_scales is not None else None
    O.kv_append(layout_o, pos, seq, flat, b.stride, ks, vs, kc, vc, src_dtype=src,
                slot_mapping=slots if use_slots else None, k_scales=k_scales, v_scales=v_scales)
    if use_slots:
        lia.kv_append(layout_p, kd, vd, dkc, dvc, slot_mapping=G.u32_dev(slots),
                      k_scales=dks, v_scales=dvs)
    else:
        lia.kv_append(layout_p, kd, vd, dkc, dvc, positions=G.u32_dev(pos), sequences=G.u32_dev(seq),
                      pages=G.u32_dev(flat), stride=b.stride, k_scales=dks, v_scales=dvs)
    torch.cuda.synchronize()
    gk = dkc.cpu().numpy().view(store)
    gv = dvc.cpu().numpy().view(store)
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)
    if kv == FP8:
        assert np.array_equal(dks.cpu().numpy(), k_scales) and np.array_equal(dvs.cpu().numpy(), v_scales)


@pytest.mark.parametrize("kv", [F16, BF16, FP8])
@pytest.mark.parametrize("src", [F32, BF16, F16])
@pytest.mark.parametrize("page", [16, 32])
def test_kv_append_bit_exact(O, lia, wl, kv, src, page):
    print(f"[case] append kv={kv} src={src} page={page}", flush=True)
    _append_case(O, lia, wl, kv, src, page, use_slots=False)
    _append_case(O, lia, wl, kv, src, page, use_slots=True, seed=1)


def test_kv_append_reference_fixture(O, lia):
    """llama_cache_paged addressing on the reference's rotary fixture rows
    (src/gpu/kernels/llama_position.rs:132-152): f16 pool, 32-token pages, stride 4096."""
    positions = np.array([0, 31, 32, 8191, 131071], np.uint32)
    sequences = np.array([0, 1, 0, 1, 0], np.uint32)
    tables = np.zeros(2 * 4096, np.uint32)
    for row, page in enumerate([5, 3, 2, 7, 1]):
        tables[sequences[row] * 4096 + positions[row] // 32] = page
    j = np.arange(5 * 256)
    k = ((j * 43 % 997) / 256.0 - 2.0).astype(np.float32).reshape(5, 256)
    v = ((j * 17 % 509) / 128.0 - 2.0).astype(np.float32).reshape(5, 256)
    ek = np.zeros(8 * 32 * 256, np.uint16)
    ev = np.zeros_like(ek)
    O.kv_append(O.KVLayout(2, 128, 32, 8, F16), positions, sequences, tables, 4096, k, v, ek, ev)
    dk = torch.zeros(ek.size, dtype=torch.int16, device="cuda")
    dv = torch.zeros_like(dk)
    lia.kv_append(lia.KVLayout(2, 128, 32, 8, F16), G.to_dev(k), G.to_dev(v), dk, dv,
                  positions=G.u32_dev(positions), sequences=G.u32_dev(sequences),
                  pages=G.u32_dev(tables), stride=4096)
    torch.cuda.synchronize()
    assert np.array_equal(dk.cpu().numpy().view(np.uint16), ek)
    assert np.array_equal(dv.cpu().numpy().view(np.uint16), ev)


def test_pack_device_matches_host(lia, wl, O):
    for cfg in (wl.config1(seed=2), wl.config3(seed=2), wl.config4(seed=2)):
        print(f"[case] pack_device {cfg.name}", flush=True)
        n = cfg.n_seqs
        rows = cfg.n_rows
        P = cfg.geom.page_size
        context = int(cfg.stride * P)
        dev_out = {k: torch.full((rows + (k == "cu"),), -7, dtype=torch.int32, device="cuda")
                   for k in ("cu", "positions", "sequences", "slots")}
        status = torch.full((1,), -7, dtype=torch.int32, device="cuda")
        lia.pack_device(G.u32_dev(np.arange(n)), G.u32_dev(cfg.q_len), G.u32_dev(cfg.cached),
                        G.u32_dev(cfg.flat_table()), cfg.stride, P, cfg.pool_pages, context, rows,
                        dev_out["cu"], dev_out["positions"], dev_out["sequences"], dev_out["slots"],
                        status)
        torch.cuda.synchronize()
        assert status.item() == 0
        host_rows = [(0, int(p), int(s)) for p, s in zip(cfg.positions(), cfg.sequences())]
        lim = lia.PagingLimits(max(n, 1), context, P, cfg.pool_pages, 1, max(rows, 1))
        packed = lia.pack_rows(lim, host_rows, [t.tolist() for t in cfg.tables])
        got = {k: v.cpu().numpy().view(np.uint32) for k, v in dev_out.items()}
        assert np.array_equal(got["positions"], packed["positions"])
        assert np.array_equal(got["sequences"], packed["sequences"])
        assert np.array_equal(got["slots"], packed["slot_mapping"])
        assert np.array_equal(got["cu"][:n + 1], packed["cu_seqlens"])


def test_pack_device_reports_missing_page(lia):
    pages = G.u32_dev(np.array([3, 0xFFFFFFFF], np.uint32))
    out = [torch.zeros(4, dtype=torch.int32, device="cuda") for _ in range(4)]
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    lia.pack_device(G.u32_dev([0]), G.u32_dev([2]), G.u32_dev([15]), pages, 2, 16, 8, 32, 4,
                    out[0], out[1], out[2], out[3], status)
    torch.cuda.synchronize()
    assert status.item() == 10  # -LIA_E_MISSING_PAGE


@pytest.mark.parametrize("order,expect", [((0, 1), 10), ((1, 0), 8)])
def test_pack_device_reports_first_failing_row(lia, order, expect):
    """Two failing sequences: the status is the error of the earlier row in packed order
    (sequence A: its second row needs a missing page; sequence B: position 40 >= context)."""
    pages = G.u32_dev(np.array([3, 0xFFFFFFFF, 4, 5], np.uint32))  # stride 2: rows 0 and 1
    seqs = {0: (0, 2, 15), 1: (1, 1, 40)}  # (table row, q_len, cached)
    slot, q_len, cached = zip(*[seqs[i] for i in order])
    out = [torch.zeros(8, dtype=torch.int32, device="cuda") for _ in range(4)]
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    lia.pack_device(G.u32_dev(slot), G.u32_dev(q_len), G.u32_dev(cached), pages, 2, 16, 8, 32, 8,
                    out[0], out[1], out[2], out[3], status)
    torch.cuda.synchronize()
    assert status.item() == expect  # 10: -LIA_E_MISSING_PAGE, 8: -LIA_E_POSITION


def test_kv_quantize_pages_bit_exact(O, lia):
    rng = np.random.default_rng(12)
    H, D, P, pool = 2, 128, 16, 40
    n = 9
    k = rng.standard_normal((n, P, H, D)).astype(np.float32) * 3
    v = rng.standard_normal((n, P, H, D)).astype(np.float32)
    v[3] = 0
    ids = rng.permutation(pool)[:n].astype(np.uint32)
    kc = np.zeros(pool * P * H * D, np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros(pool * H, np.float32)
    vs = np.zeros_like(ks)
    O.kv_quantize_pages(O.KVLayout(H, D, P, pool, FP8), ids, k, v, kc, vc, ks, vs)
    dkc = torch.zeros(kc.size, dtype=torch.uint8, device="cuda")
    dvc = torch.zeros_like(dkc)
    dks = torch.zeros(ks.size, dtype=torch.float32, device="cuda")
    dvs = torch.zeros_like(dks)
    lia.kv_quantize_pages(lia.KVLayout(H, D, P, pool, FP8), G.u32_dev(ids), G.to_dev(k), G.to_dev(v),
                          dkc, dvc, dks, dvs)
    torch.cuda.synchronize()
    assert np.array_equal(dks.cpu().numpy(), ks) and np.array_equal(dvs.cpu().numpy(), vs)
    assert np.array_equal(dkc.cpu().numpy(), kc) and np.array_equal(dvc.cpu().numpy(), vc)


def test_engine_step_append_then_attend(lia, wl, O):
    """Engine mirror: stage (host packing + upload), append this step's K/V, attend."""
    g = wl.Geometry(hq=16, hkv=2, d=128, page_size=32, kv_dtype=BF16, q_dtype=BF16,
                    out_dtype=F32)
    eng = lia.Engine(16, 2, 128, pool_tokens=4096, layers=2, page_size=32, kv_dtype=BF16,
                     q_dtype=BF16, out_dtype=F32, prefill_batch=256)
    eng.configure_paging(4, 2048)
    rng = np.random.default_rng(13)
    pool_k = O.from_f32(rng.standard_normal((4096, 2, 128)).astype(np.float32), BF16)
    pool_v = O.from_f32(rng.standard_normal((4096, 2, 128)).astype(np.float32), BF16)
    eng.k[1].copy_(G.to_dev(pool_k, torch.int16).view(4096, 2, 128))
    eng.v[1].copy_(G.to_dev(pool_v, torch.int16).view(4096, 2, 128))
    tables = [[int(x) for x in rng.permutation(128)[:k]] for k in (10, 3)]
    tables[1] = [p for p in range(128) if p not in tables[0]][:3]
    rows = [(5, p, 0) for p in range(290, 300)] + [(7, 70, 1)]
    packed = eng.stage(rows, tables, outputs=[9, 10])
    n = len(rows)
    q = O.from_f32(rng.standard_normal((n, 16, 128)).astype(np.float32), BF16)
    k = O.from_f32(rng.standard_normal((n, 256)).astype(np.float32), BF16)
    v = O.from_f32(rng.standard_normal((n, 256)).astype(np.float32), BF16)
    out = eng.attention(1, G.to_dev(q, torch.bfloat16), G.to_dev(k, torch.bfloat16),
                        G.to_dev(v, torch.bfloat16))
    torch.cuda.synchronize()
    kc, vc = pool_k.reshape(-1).copy(), pool_v.reshape(-1).copy()
    O.kv_append(O.KVLayout(2, 128, 32, 128, BF16), packed["positions"], packed["sequences"],
                packed["flat"], packed["stride"], k, v, kc, vc, src_dtype=BF16)
    assert np.array_equal(eng.k[1].cpu().numpy().view(np.uint16).reshape(-1), kc)
    geom = O.geom(16, 2, 128, 32, packed["stride"], BF16)
    ref = O.attention_f64(geom, packed["positions"], packed["sequences"], packed["flat"],
                          O.to_f32(q, BF16), kc, vc)
    err = np.abs(out.cpu().numpy() - ref)
    assert err.max() < 2e-2 and err.mean() < 2e-3
