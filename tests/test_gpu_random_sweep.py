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
    ws = torch.zeros(lia.workspace_bytes(cfg), dtype=torch.uint8, device="cuda")
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
