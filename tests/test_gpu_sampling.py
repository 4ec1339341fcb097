"""GPU tests of sparse paged sampling through the C ABI: the candidates kernel bit-exact
against the oracle's records (oracle/sampling.py: ids and f32 bits of all 21 slots, part
maxima exact, f64 masses within 1e-12 relative - the reduction order differs), and
lia_sample_paged's tokens equal to the oracle's on the reference's GPU test rows
(src/sampling/nucleus.rs:183-231) and on MiniCPM5-width vocabularies."""
import math

import numpy as np
import pytest
import torch

from oracle import sampling as OS
from test_sampling import reference_gpu_rows

pytestmark = pytest.mark.gpu


def _records(lia, logits, temps):
    rows, vocab = logits.shape
    parts = -(-vocab // 1024)
    lg = torch.from_numpy(logits).cuda()
    t = torch.tensor(temps, dtype=torch.float64, device="cuda")
    cand = torch.full((rows, parts, 21), -1, dtype=torch.int64, device="cuda")
    norm = torch.full((rows, parts, 2), -7.0, dtype=torch.float64, device="cuda")
    lia.nucleus_candidates(t, lg, cand, norm)
    torch.cuda.synchronize()
    return cand.cpu().numpy().view(np.uint64), norm.cpu().numpy()


def _check_records(lia, logits, temps, label):
    print(f"[case] candidates {label} rows={logits.shape[0]} vocab={logits.shape[1]}", flush=True)
    cand, norm = _records(lia, logits, temps)
    want_c, want_n = OS.nucleus_candidates(logits, temps)
    assert np.array_equal(cand, want_c), label
    assert np.array_equal(norm[..., 0], want_n[..., 0]), label
    a, b = norm[..., 1], want_n[..., 1]
    assert np.array_equal(np.isnan(a), np.isnan(b)), label
    ok = ~np.isnan(b)
    assert np.all(np.abs(a[ok] - b[ok]) <= 1e-12 * np.maximum(np.abs(b[ok]), 1e-300)), label


def test_candidates_reference_rows(lia):
    logits, temps = reference_gpu_rows()
    _check_records(lia, logits, temps, "reference rows")


def test_candidates_special_values_and_ragged_vocab(lia):
    rng = np.random.default_rng(7)
    for vocab in (1000, 1024, 2049, 5000):
        x = (rng.standard_normal((5, vocab)) * 4).astype(np.float32)
        x[0, 3] = np.nan
        x[1, 7] = np.inf
        x[2, :] = -np.inf                             # a row with no finite entry
        x[3, :300] = 2.5                              # ties: larger ids first
        x[3, 300] = np.float32(-0.0)
        x[3, 301] = np.float32(0.0)
        x[4, 10] = np.uint32(0xFFFFFFFF).view(np.float32)    # all-ones NaN: never selected
        x[4, 11] = np.uint32(0x7FC00000).view(np.float32)    # a positive NaN: largest key
        _check_records(lia, x, [1.0, 0.5, 1.0, 2.0, 0.0], f"special vocab={vocab}")


def test_candidates_minicpm5_vocabulary(lia):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((2, 130560)) * 3).astype(np.float32)
    _check_records(lia, x, [1.0, 0.7], "vocab 130560")


def test_sample_paged_reference_rows(lia):
    print("[case] sample_paged reference rows", flush=True)
    logits, temps = reference_gpu_rows()
    ps = lia.PagedSampler(logits.shape[1], 8)
    samplers = [lia.Sampler(temps[i], 0, 0.95, 42) for i in range(4)]
    got = ps.sample(torch.from_numpy(logits).cuda(), samplers, [1, 2, 3, 4])
    want, fallbacks = OS.sample_rows(logits, [OS.Sampling(temps[i], 0, 0.95, 42)
                                              for i in range(4)], [1, 2, 3, 4])
    assert got == want and ps.fallbacks == fallbacks == 2
    bad = logits.copy()
    bad[0, 37] = np.nan
    with pytest.raises(lia.LiaError) as e:
        ps.sample(torch.from_numpy(bad).cuda(), samplers, [1, 2, 3, 4])
    assert e.value.status == -26


def test_sample_paged_mixed_samplers_match_oracle(lia):
    print("[case] sample_paged mixed samplers vocab 130560", flush=True)
    rng = np.random.default_rng(9)
    V = 130560
    logits = (rng.standard_normal((6, V)) * 2).astype(np.float32)
    logits[0, 5000:5010] = 12.0
    logits[3, :] = -30.0
    logits[3, 77777] = 5.0
    configs = [None, (1.0, 0, 0.9, 1, False), (0.6, 7, 1.0, 2, False), (1.0, 0, 0.05, 3, True),
               (1.5, 0, 1.0, 4, False), (0.8, 20, 0.5, 5, True)]
    positions = [11, 22, 33, 44, 55, 66]
    ps = lia.PagedSampler(V, 8)
    got = ps.sample(torch.from_numpy(logits).cuda(),
                    [None if c is None else lia.Sampler(*c) for c in configs], positions)
    want, fallbacks = OS.sample_rows(logits, [None if c is None else OS.Sampling(*c)
                                              for c in configs], positions)
    assert got == want and ps.fallbacks == fallbacks
    assert got[0] == 5009
