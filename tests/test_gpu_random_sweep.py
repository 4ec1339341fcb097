"""Seeded random sweep of lia_paged_attention against the f64 oracle.

Each case draws a geometry (head_dim 64 / 128, 1-8 KV heads, GQA groups 1-16, pages of 16-64
tokens), a pool type (bf16, f16, FP8 e4m3 with per-page scales), query / output types, and a
batch: pure decode, MTP-verify rows, mixed prefill chunks over cached prefixes with decode rows,
or tiny contexts.  Contexts are drawn log-uniformly, so page boundaries, single keys and long
prefixes all occur.  Every case runs the whole entry point (plan, split attention, combine)
and is held to the parity bar of test_gpu_attention.py: bf16 / f16 KV max-abs 2e-2 and mean-abs
2e-3, FP8 KV max-abs 5e-2, against the float64 softmax of the stored K/V."""
import numpy as np
import pytest

import gpu_data as G
from gpu_data import BF16, F16, F32, FP8

pytestmark = pytest.mark.gpu

TOL = {BF16: (2e-2, 2e-3), F16: (2e-2, 2e-3), FP8: (5e-2, 5e-3)}
CASES = 48
# the oracle's work per case (attended row-keys x query heads x head_dim) is kept below this
MAX_WORK = 4e8


def draw_case(wl, i):
    rng = np.random.default_rng(7919 * (i + 1))
    d = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 6, 8, 16]))
    page = int(rng.choice([16, 32, 64]))
    kv = int(rng.choice([BF16, F16, FP8]))
    q_dtype, out_dtype = [(BF16, BF16), (F32, F32), (BF16, F32), (F32, BF16)][int(rng.integers(4))]
    kind = ["decode", "mtp", "mixed", "tiny"][i % 4]
    if kind == "decode":
        n = int(rng.integers(1, 65))
        q = np.ones(n, np.int64)
        ctx = np.exp(rng.uniform(0, np.log(20000), n)).astype(np.int64) + 1
    elif kind == "mtp":
        n = int(rng.integers(1, 33))
        q = rng.integers(2, 5, n)
        ctx = q + np.exp(rng.uniform(0, np.log(12000), n)).astype(np.int64)
    elif kind == "mixed":
        n_pre, n_dec = int(rng.integers(1, 4)), int(rng.integers(0, 6))
        q = np.concatenate([rng.integers(17, 600, n_pre), np.ones(n_dec, np.int64)])
        prefix = np.concatenate([rng.integers(0, 3000, n_pre),
                                 np.exp(rng.uniform(0, np.log(8000), n_dec)).astype(np.int64)])
        ctx = q + prefix
    else:
        n = int(rng.integers(1, 9))
        q = rng.integers(1, 4, n)
        ctx = q + rng.integers(0, 40, n)
    g = wl.Geometry(hq=hkv * group, hkv=hkv, d=d, page_size=page, kv_dtype=kv, q_dtype=q_dtype,
                    out_dtype=out_dtype)
    # keep the oracle's work bounded: halve the cached keys, and once none are left the rows
    # (every pass shrinks the work until it fits or each sequence has one row and one key)
    while float(np.dot(q, ctx)) * g.hq * d > MAX_WORK and ctx.max() > 1:
        if (ctx > q).any():
            ctx = np.maximum(q, q + (ctx - q) // 2)
        else:
            q = np.maximum(1, q // 2)
            ctx = q.copy()
    perm = rng.permutation(len(q))  # prefill and decode rows interleaved in the batch
    return kind, wl.custom(ctx[perm], q[perm], geom=g, seed=i, pool_slack=int(rng.integers(0, 64)))


@pytest.mark.parametrize("i", range(CASES))
def test_random_batch(lia, wl, i):
    kind, b = draw_case(wl, i)
    g = b.geom
    print(f"[case] sweep {i} {kind}: d={g.d} hq={g.hq} hkv={g.hkv} page={g.page_size} kv={g.kv_dtype} "
          f"q/o={g.q_dtype}/{g.out_dtype} seqs={b.n_seqs} rows={b.n_rows} "
          f"ctx={b.ctx.tolist()[:6]} q_len={b.q_len.tolist()[:6]}", flush=True)
    case = G.Case(b, seed=i)
    got = case.run(lia)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] sweep {i}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)), i
    tol_max, tol_mean = TOL[g.kv_dtype]
    assert mx < tol_max and mean < tol_mean, (i, kind, mx, mean)


STEP_CASES = 24


@pytest.mark.parametrize("i", range(STEP_CASES))
def test_random_step_device_packing_fused_append(lia, wl, i):
    """The serving step on a random batch (16-bit pools; FP8 draws use bf16): the batch packed on
    the device from its per-sequence inputs with the plan beside it (lia_pack_plan_device), the
    step's rows appended by the attention launch itself (lia_attention_partial_append) and the
    combine.  cu_seqlens, positions, sequences and the slot mapping must equal the host
    packing bit for bit, the pool afterwards must hold exactly the original bytes (the rows'
    slots were overwritten with garbage first), and the output is held to the parity bar."""
    import torch
    kind, b = draw_case(wl, 100 + i)
    if b.geom.kv_dtype == FP8:
        b.geom = wl.Geometry(hq=b.geom.hq, hkv=b.geom.hkv, d=b.geom.d, page_size=b.geom.page_size,
                             kv_dtype=BF16, q_dtype=b.geom.q_dtype, out_dtype=b.geom.out_dtype)
    g = b.geom
    print(f"[case] step {i} {kind}: d={g.d} hq={g.hq} hkv={g.hkv} page={g.page_size} kv={g.kv_dtype} "
          f"q/o={g.q_dtype}/{g.out_dtype} seqs={b.n_seqs} rows={b.n_rows} "
          f"ctx={b.ctx.tolist()[:6]} q_len={b.q_len.tolist()[:6]}", flush=True)
    case = G.Case(b, seed=100 + i)
    dev = case.device()
    W = g.hkv * g.d
    slots = b.slot_mapping().astype(np.int64)
    newk = case.kc.reshape(-1, W)[slots].copy()
    newv = case.vc.reshape(-1, W)[slots].copy()
    junk = np.random.default_rng(i).integers(0, 65535, newk.shape).astype(np.uint16)
    idx = torch.from_numpy(slots).cuda()
    dev["kc"].view(-1, W)[idx] = G.to_dev(junk, torch.int16)
    dev["vc"].view(-1, W)[idx] = G.to_dev(junk[::-1].copy(), torch.int16)
    cfg = case.config(lia)
    ws = G.dirty_workspace(lia, cfg)
    rows = b.n_rows
    cu = torch.full((b.n_seqs + 1,), -1, dtype=torch.int32, device="cuda")
    positions = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    sequences = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    slot_map = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    lia.pack_plan_device(cfg, G.u32_dev(np.arange(b.n_seqs)), G.u32_dev(b.q_len), G.u32_dev(b.cached),
                         dev["pages"], rows, b.stride * g.page_size, cu, positions, sequences, slot_map,
                         status, ws)
    odt = torch.float32 if g.out_dtype == F32 else torch.bfloat16
    out = torch.full((rows, g.hq, g.d), float("nan"), dtype=odt, device="cuda")
    lia.attention_partial_append(cfg, b.n_seqs, dev["pages"], slot_map, dev["q"],
                                 G.to_dev(newk, torch.int16), G.to_dev(newv, torch.int16),
                                 dev["kc"], dev["vc"], out, ws)
    lia.attention_merge(cfg, b.n_seqs, rows, out, ws)
    torch.cuda.synchronize()
    assert status.item() == 0
    u32 = lambda t: t.cpu().numpy().view(np.uint32)
    assert np.array_equal(u32(cu), b.cu_seqlens())
    assert np.array_equal(u32(positions), b.positions())
    assert np.array_equal(u32(sequences), b.sequences())
    assert np.array_equal(u32(slot_map), b.slot_mapping())
    assert np.array_equal(dev["kc"].cpu().numpy().view(np.uint16), case.kc)
    assert np.array_equal(dev["vc"].cpu().numpy().view(np.uint16), case.vc)
    got = out.float().cpu().numpy()
    mx, mean = G.errors(got, case.f64())
    print(f"[case] step {i}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)), i
    tol_max, tol_mean = TOL[g.kv_dtype]
    assert mx < tol_max and mean < tol_mean, (i, kind, mx, mean)


FP8_STEP_CASES = 16


@pytest.mark.parametrize("i", range(FP8_STEP_CASES))
def test_random_fp8_step(lia, wl, O, i):
    """The serving step on an FP8 pool for a random batch: device packing with the plan beside it,
    lia_attention_partial_append_fp8 (the step's bf16 rows quantised into the pool with their
    pages' scales, fresh pages taking scale 1, then attended) and the combine.  The packed
    metadata must equal the host packing, the pool bytes and per-(page, head) scales must equal
    what the oracle's lia_kv_append stores, and the output is held to the FP8 bar against the
    float64 oracle over the pool after the append."""
    import torch
    kind, b0 = draw_case(wl, 200 + i)
    g0 = b0.geom
    g = wl.Geometry(hq=g0.hq, hkv=g0.hkv, d=g0.d, page_size=g0.page_size, kv_dtype=FP8, q_dtype=BF16,
                    out_dtype=g0.out_dtype)
    b = wl.custom(b0.ctx, b0.q_len, geom=g, seed=200 + i, pool_slack=8)
    P, W = g.page_size, g.hkv * g.d
    print(f"[case] fp8 step {i} {kind}: d={g.d} hq={g.hq} hkv={g.hkv} page={P} out={g.out_dtype} "
          f"seqs={b.n_seqs} rows={b.n_rows} ctx={b.ctx.tolist()[:6]} q_len={b.q_len.tolist()[:6]}",
          flush=True)
    rng = np.random.default_rng(300 + i)
    tokens = b.pool_pages * P
    layout = O.KVLayout(g.hkv, g.d, P, b.pool_pages, FP8)
    kc = np.zeros(tokens * W, np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros(b.pool_pages * g.hkv, np.float32)
    vs = np.zeros_like(ks)
    # pages holding cached keys are quantised from float pages; pages holding only new rows stay
    # fresh (scale 0) for the append to initialise
    cached_pages = sorted({int(t[lp]) for s, t in enumerate(b.tables)
                           for lp in range(-(-int(b.cached[s]) // P))})
    if cached_pages:
        ids = np.array(cached_pages, np.uint32)
        kf = rng.standard_normal((len(ids), P, g.hkv, g.d)).astype(np.float32)
        vf = rng.standard_normal((len(ids), P, g.hkv, g.d)).astype(np.float32)
        O.kv_quantize_pages(layout, ids, kf, vf, kc, vc, ks, vs)
    newk = O.from_f32(rng.standard_normal((b.n_rows, W)).astype(np.float32), BF16)
    newv = O.from_f32(rng.standard_normal((b.n_rows, W)).astype(np.float32), BF16)
    kexp, vexp, ksx, vsx = kc.copy(), vc.copy(), ks.copy(), vs.copy()
    O.kv_append(layout, b.positions(), b.sequences(), b.flat_table(), b.stride, newk, newv, kexp,
                vexp, src_dtype=BF16, k_scales=ksx, v_scales=vsx)
    dkc, dvc = G.to_dev(kc, torch.uint8), G.to_dev(vc, torch.uint8)
    dks, dvs = G.to_dev(ks), G.to_dev(vs)
    qf = O.from_f32(rng.standard_normal((b.n_rows, g.hq, g.d)).astype(np.float32), BF16)
    cfg = lia.AttentionConfig(g.hq, g.hkv, g.d, P, b.pool_pages, b.stride, g.q_dtype, g.kv_dtype,
                              g.out_dtype, g.scale, b.n_seqs, b.n_rows, int(b.ctx.max()))
    ws = G.dirty_workspace(lia, cfg)
    rows = b.n_rows
    cu = torch.full((b.n_seqs + 1,), -1, dtype=torch.int32, device="cuda")
    positions = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    sequences = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    slot_map = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    flat = G.u32_dev(b.flat_table())
    lia.pack_plan_device(cfg, G.u32_dev(np.arange(b.n_seqs)), G.u32_dev(b.q_len), G.u32_dev(b.cached),
                         flat, rows, b.stride * P, cu, positions, sequences, slot_map, status, ws)
    odt = torch.float32 if g.out_dtype == F32 else torch.bfloat16
    out = torch.full((rows, g.hq, g.d), float("nan"), dtype=odt, device="cuda")
    lia.attention_partial_append_fp8(cfg, b.n_seqs, flat, slot_map, G.to_dev(qf, torch.bfloat16),
                                     G.to_dev(newk, torch.bfloat16), G.to_dev(newv, torch.bfloat16),
                                     dkc, dvc, dks, dvs, out, ws)
    lia.attention_merge(cfg, b.n_seqs, rows, out, ws)
    torch.cuda.synchronize()
    assert status.item() == 0
    u32 = lambda t: t.cpu().numpy().view(np.uint32)
    assert np.array_equal(u32(cu), b.cu_seqlens())
    assert np.array_equal(u32(positions), b.positions())
    assert np.array_equal(u32(sequences), b.sequences())
    assert np.array_equal(u32(slot_map), b.slot_mapping())
    assert np.array_equal(dks.cpu().numpy(), ksx) and np.array_equal(dvs.cpu().numpy(), vsx)
    assert np.array_equal(dkc.cpu().numpy(), kexp) and np.array_equal(dvc.cpu().numpy(), vexp)
    geom = O.geom(g.hq, g.hkv, g.d, P, b.stride, FP8, g.scale)
    ref = O.attention_f64(geom, b.positions(), b.sequences(), b.flat_table(), O.to_f32(qf, BF16),
                          kexp, vexp, ksx, vsx)
    got = out.float().cpu().numpy()
    mx, mean = G.errors(got, ref)
    print(f"[case] fp8 step {i}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)), i
    assert mx < TOL[FP8][0] and mean < TOL[FP8][1], (i, kind, mx, mean)
