"""Pool slots outside every sequence's context hold NaN: a fresh or recycled KV page can hold any
bytes past its sequence's last key, and pages no block table names can hold anything.  The
attention kernels must not let them reach the output: every output stays finite and matches the
f64 oracle, which reads only attended keys (src/gpu/llama_attention.rs:253-284)."""
import numpy as np
import pytest

import gpu_data as G
from gpu_data import BF16, F16, F32, FP8

pytestmark = pytest.mark.gpu

TOL = {BF16: (2e-2, 2e-3), F16: (2e-2, 2e-3), FP8: (5e-2, 5e-3)}


def _poison(case):
    """NaN (bf16 / f16 0xFFFF, e4m3 0x7F) in every K and V slot no sequence attends."""
    b, g = case.batch, case.g
    P = g.page_size
    tokens = b.pool_pages * P
    live = np.zeros(tokens, bool)
    for table, c in zip(b.tables, b.ctx):
        k = np.arange(int(c))
        live[np.asarray(table, np.int64)[k // P] * P + k % P] = True
    nan = 0x7F if g.kv_dtype == FP8 else 0xFFFF
    for plane in (case.kc, case.vc):
        plane.reshape(tokens, -1)[~live] = nan
    return int((~live).sum())


CASES = {
    # decode rows over contexts ending at every position in a page
    "decode": ([1, 2, 15, 16, 17, 31, 32, 33, 100, 511, 1000, 2049], [1] * 12),
    # verify rows and short chunks (two-tile units)
    "mixed": ([40, 1200, 17, 5000, 300], [3, 1, 2, 4, 1]),
    # prefill chunks, with and without a prefix (the prefill kernel)
    "prefill": ([300, 1077, 2040], [300, 77, 40]),
}


@pytest.mark.parametrize("kv", [BF16, F16, FP8])
@pytest.mark.parametrize("kind", list(CASES))
def test_nan_outside_contexts(lia, wl, kind, kv):
    ctx, q_len = CASES[kind]
    g = wl.Geometry(kv_dtype=kv)
    b = wl.custom(ctx, q_len, geom=g, seed=51)
    case = G.Case(b, seed=51)
    dead = _poison(case)
    print(f"[case] dead slots NaN: {kind} kv={kv} dead={dead}", flush=True)
    got = case.run(lia)
    ref = case.f64()
    assert np.all(np.isfinite(ref))
    assert np.all(np.isfinite(got)), (kind, kv)
    mx, mean = G.errors(got, ref)
    print(f"[case] dead slots NaN: {kind} kv={kv} max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert mx < TOL[kv][0] and mean < TOL[kv][1]
