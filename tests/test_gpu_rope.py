"""GPU parity of the RoPE table and the fused RoPE + KV append (through the C ABI), bit-exact
against the CPU oracle: the coefficient table equals the oracle's, and the fused kernel,
given the oracle's table, writes the oracle's query and pool bytes
(src/gpu/kernels/llama_position.rs:36-118, fixture at :128-239)."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, F16, F32, FP8

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d", [64, 128])
def test_coefficients_bit_exact(lia, O, d):
    positions = np.array([0, 1, 17, 31, 32, 4095, 8191, 65535, 131071, 100003], np.uint32)
    print(f"[case] rope coefficients d={d}", flush=True)
    ref = O.rope_coefficients(positions, d)
    out = torch.zeros(ref.size, dtype=torch.float32, device="cuda")
    lia.rope_coefficients(G.u32_dev(positions), d, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _run(lia, O, hq, hkv, d, kv, qdt, page, use_slots, seed):
    rng = np.random.default_rng(seed)
    stride, rows = 64, 9
    pool_pages = stride * 2
    seqs = rng.integers(0, 2, rows).astype(np.uint32)
    tables = np.stack([rng.permutation(pool_pages)[:stride] for _ in range(2)]).astype(np.uint32)
    positions = np.zeros(rows, np.uint32)
    for s in range(2):
        idx = np.where(seqs == s)[0]
        positions[idx] = np.sort(rng.choice(stride * page, idx.size, replace=False))
    flat = tables.reshape(-1)
    slots = np.array([flat[s * stride + p // page] * page + p % page for s, p in zip(seqs, positions)],
                     np.uint32)
    combined = rng.uniform(-4, 4, (rows, (hq + 2 * hkv) * d)).astype(np.float32)
    coeffs = O.rope_coefficients(positions, d)
    layout_o = O.KVLayout(hkv, d, page, pool_pages, kv)
    store = np.uint8 if kv == FP8 else np.uint16
    W = hkv * d
    kc = rng.integers(0, 255 if kv == FP8 else 65535, pool_pages * page * W).astype(store)
    vc = kc[::-1].copy()
    k_scales = v_scales = None
    if kv == FP8:
        k_scales = rng.uniform(0.005, 0.03, pool_pages * hkv).astype(np.float32)
        v_scales = rng.uniform(0.005, 0.03, pool_pages * hkv).astype(np.float32)
        k_scales[rng.random(k_scales.size) < 0.3] = 0.0  # never quantised: take scale 1
        v_scales[rng.random(v_scales.size) < 0.3] = 0.0
    qref = np.zeros(rows * hq * d, np.uint16 if qdt == BF16 else np.float32)
    kref, vref = kc.copy(), vc.copy()
    # device copies first: the oracle records the scales of never-quantised pages in place
    dks = G.to_dev(k_scales) if k_scales is not None else None
    dvs = G.to_dev(v_scales) if v_scales is not None else None
    O.rope_kv_append(layout_o, hq, positions, seqs, flat, stride, coeffs, combined, qref, qdt, kref,
                     vref, slot_mapping=slots if use_slots else None, k_scales=k_scales,
                     v_scales=v_scales)
    dt = torch.uint8 if kv == FP8 else torch.int16
    dkc, dvc = G.to_dev(kc, dt), G.to_dev(vc, dt)
    q = torch.zeros((rows, hq, d), dtype=torch.bfloat16 if qdt == BF16 else torch.float32, device="cuda")
    layout = lia.KVLayout(hkv, d, page, pool_pages, kv)
    kw = dict(slot_mapping=G.u32_dev(slots)) if use_slots else dict(
        positions=G.u32_dev(positions), sequences=G.u32_dev(seqs), pages=G.u32_dev(flat), stride=stride)
    lia.rope_kv_append(layout, hq, G.to_dev(coeffs), G.to_dev(combined), q, dkc, dvc,
                       k_scales=dks, v_scales=dvs, **kw)
    torch.cuda.synchronize()
    qgot = q.view(torch.int16).cpu().numpy().view(np.uint16) if qdt == BF16 else q.cpu().numpy()
    if qdt == BF16:
        assert np.array_equal(qgot.reshape(-1), qref)
    else:
        assert np.array_equal(qgot.reshape(-1).view(np.uint32), qref.view(np.uint32))
    assert np.array_equal(dkc.cpu().numpy().view(store), kref)
    assert np.array_equal(dvc.cpu().numpy().view(store), vref)
    if kv == FP8:  # the oracle's arrays hold the recorded scales
        assert np.array_equal(dks.cpu().numpy(), k_scales) and np.array_equal(dvs.cpu().numpy(), v_scales)


def test_reference_geometry(lia, O):
    """16 q / 2 kv heads, d 128, f16 pool, 32-token pages, f32 queries, table addressing."""
    print("[case] rope reference geometry", flush=True)
    _run(lia, O, 16, 2, 128, F16, F32, 32, False, 1)


@pytest.mark.parametrize("hq,hkv,d,kv,qdt,page,slots", [
    (16, 2, 128, BF16, BF16, 16, True),
    (8, 2, 64, BF16, F32, 16, False),
    (16, 2, 128, FP8, BF16, 16, True),
    (16, 1, 128, F16, F32, 64, True),
    (4, 4, 64, FP8, F32, 32, False),
])
def test_generalised(lia, O, hq, hkv, d, kv, qdt, page, slots):
    print(f"[case] rope hq={hq} hkv={hkv} d={d} kv={kv} q={qdt} page={page} slots={slots}", flush=True)
    _run(lia, O, hq, hkv, d, kv, qdt, page, slots, hq + d + kv)
