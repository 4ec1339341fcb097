"""CPU tests of sparse paged sampling.

The oracle (oracle/sampling.py) is pinned by the reference's own tests, case for case:
src/sampling/random.rs:52-71 (published MT19937 vector, reference doubles),
src/sampling.rs:192-313, src/sampling/nucleus.rs:127-231 (including the host half of the
GPU candidates test: which rows may be sampled sparsely and that every row's distribution
equals the full one), src/sampling/gumbel.rs:98-110.  The product's host sampler
(lia_sampler_*, lia_sample_host) is then compared with the oracle bit for bit."""
import math

import numpy as np
import pytest

from oracle import sampling as OS


# ------------------------------------------------------------------ oracle pinning

def test_mt19937_published_vector_and_reference_doubles():
    r = OS.Random(5489)
    assert [r.next() for _ in range(10)] == [
        3499211612, 581869302, 3890346734, 3586334585, 545404204, 4161255391, 3922919429,
        949333985, 2715962298, 1323567403]
    r = OS.Random(5489)
    for _ in range(9999):
        r.next()
    assert r.next() == 4123659995
    assert OS.f32_bits(OS.Random(42).uniform_f32()) == OS.f32_bits(0.37454012)
    r = OS.Random(42)
    assert abs(r.uniform() - 0.796542984287846) < 1e-15
    assert abs(r.uniform() - 0.18343478789336848) < 1e-15


def test_unrestricted_nucleus_uses_the_full_vocabulary():
    full = OS.Sampling(1.0, 0, 1.0, 42)
    assert len(full.distribution([(i, 0.0) for i in range(32)])) == 32
    half = OS.Sampling(1.0, 0, 0.5, 42)
    assert len(half.distribution([(i, 0.0) for i in range(32)])) == 16
    with pytest.raises(OS.Error):
        full.distribution([(7, 0.0), (7, 1.0)])


def _at(entries, sample):
    c = 0.0
    for i, p in entries:
        c += p
        if sample < c:
            return i
    return entries[-1][0]


def test_temperature_top_k_and_nucleus():
    s = OS.Sampling(2.0, 3, 1.0, 42)
    d = s.distribution([(0, 0.0), (1, 2.0), (2, 4.0), (3, -100.0)])
    z = 1.0 + math.exp(-1.0) + math.exp(-2.0)
    for (i, p), (ei, ep) in zip(d, [(2, 1 / z), (1, math.exp(-1.0) / z), (0, math.exp(-2.0) / z)]):
        assert i == ei and abs(p - ep) < 1e-14
    s = OS.Sampling(1.0, 20, 0.7, 0)
    d = s.distribution([(0, 0.0), (1, 0.0), (2, 0.0), (3, 0.0)])
    assert [i for i, _ in d] == [3, 2, 1]
    assert _at(d, 0.0) == 3 and _at(d, 1 / 3) == 2 and _at(d, 0.99999) == 1


def test_invalid_and_extreme_distributions():
    for args in [(0.0, 20, 0.95, 0), (1.0, 21, 0.95, 0), (1.0, 20, 0.0, 0)]:
        with pytest.raises(OS.Error):
            OS.Sampling(*args)
    s = OS.Sampling(2.2250738585072014e-308, 20, 1.0, 0)
    for bad in ([], [(0, math.nan)], [(0, math.inf)], [(0, -math.inf)], [(1, 0.0), (1, 1.0)]):
        with pytest.raises(OS.Error):
            s.distribution(bad)
    fmax = float(np.finfo(np.float32).max)
    assert _at(s.distribution([(0, -fmax), (1, fmax)]), 0.999999) == 1


def _partial_logits():
    """sampling.rs:256-268: ((id * 73 % 997) as f32 - 498.0) * 0.03 in f32, with -inf, -0.0
    and 0.0 at id % 41 == 0, 1, 2."""
    out = []
    for i in range(4860):
        m = i % 41
        if m == 0:
            v = -math.inf
        elif m == 1:
            v = -0.0
        elif m == 2:
            v = 0.0
        else:
            v = float((np.float32(i * 73 % 997) - np.float32(498.0)) * np.float32(0.03))
        out.append((i, v))
    return out


def test_partial_selection_matches_full_sort():
    logits = _partial_logits()
    ordered = sorted(logits, key=OS._order_key)
    for top_k in (1, 2, 7, 20):
        for top_p in (0.01, 0.7, 0.95, 1.0):
            s = OS.Sampling(1.0, top_k, top_p, 42)
            assert s.distribution(logits) == s.distribution(ordered[:top_k])


def _nucleus_logits():
    return [float(np.float32(((i * 173 % 4096) - 2048.0) / 64.0)) for i in range(4096)]


def test_partial_nucleus_selection_matches_independent_full_sort():
    logits = _nucleus_logits()
    for temperature in (0.2, 1.0, 2.0):
        for top_p in (0.01, 0.5, 0.95, 1.0):
            s = OS.Sampling(temperature, 0, top_p, 42)
            want = s.distribution(list(enumerate(logits)))
            got = s.distribution_logits(np.array(logits, np.float32))
            assert [i for i, _ in got] == [i for i, _ in want]
            assert max(abs(a[1] - b[1]) for a, b in zip(got, want)) < 1e-12


def test_omitted_high_scores_and_ambiguous_boundaries_force_fallback():
    s = OS.Sampling(1.0, 0, 0.5, 42)
    assert s.checked_nucleus([(0, 0.0), (1, -1.0)], 0.0, 2.0, 0.1) is None
    assert s.checked_nucleus([(0, 0.0), (1, -1.0)], 0.0, 2.0, -10.0) is None
    assert s.checked_nucleus([(0, 0.0), (1, -1.0)], 0.0, 1.5, -10.0) is not None


def reference_gpu_rows():
    """The four rows of the reference's GPU candidates test (nucleus.rs:192-206)."""
    V = 3073
    rows = [np.zeros(V, np.float32),
            np.array([20.0 if i == 2048 else -20.0 for i in range(V)], np.float32),
            np.array([1.0 if i < 300 else -20.0 for i in range(V)], np.float32),
            np.array([np.float32(1.0) - np.float32(i % 1024) * np.float32(0.2)
                      + np.float32(i // 1024) * np.float32(0.03) if i % 1024 < 4 else -50.0
                      for i in range(V)], np.float32)]
    return np.stack(rows), [1.0, 1.0, 1.0, 0.7]


def test_reference_candidates_case_sparse_pattern_and_exact_distributions():
    logits, temps = reference_gpu_rows()
    cand, norm = OS.nucleus_candidates(logits, temps)
    rows = OS.read_rows(cand, norm, temps, logits.shape[1])
    for index, (c, mx, total, omitted) in enumerate(rows):
        s = OS.Sampling(temps[index], 0, 0.95, 42)
        want = s.distribution(list(enumerate(float(x) for x in logits[index])))
        sparse = s.checked_nucleus(c, mx, total, omitted)
        assert (sparse is not None) == [False, True, False, True][index]
        got = sparse if sparse is not None else s.distribution_logits(logits[index])
        assert [i for i, _ in got] == [i for i, _ in want]
        assert max(abs(a[1] - b[1]) for a, b in zip(got, want)) < 1e-12
    bad = logits.copy()
    bad[0, 37] = np.nan
    cand, norm = OS.nucleus_candidates(bad, temps)
    with pytest.raises(OS.Error):
        OS.read_rows(cand, norm, temps, bad.shape[1])


def test_gumbel_max_reproduces_categorical_mass():
    entries = [(0, 0.2), (1, 0.3), (2, 0.5)]
    counts = [0, 0, 0]
    for seed in range(30000):
        counts[OS.gumbel_draw(entries, seed, 2050)] += 1
    for c, e in zip(counts, (0.2, 0.3, 0.5)):
        assert abs(c / 30000 - e) < 0.015


def test_candidates_are_the_top21_by_total_order():
    """Closed form of the kernel's records: the 21 largest entries of each part by the total
    order of their f32 bits (ties: larger id), and the part's f64 mass."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 2500)).astype(np.float32)
    x[0, 5] = np.float32(-0.0)
    x[0, 6] = np.float32(0.0)
    x[1, :40] = 3.0                                  # ties across ids
    cand, norm = OS.nucleus_candidates(x, [1.0, 0.0])
    for r in range(2):
        for p in range(3):
            seg = x[r, p * 1024:(p + 1) * 1024]
            bits = seg.view(np.int32).astype(np.int64)
            key = np.where(bits < 0, bits ^ 0x7FFFFFFF, bits)
            ids = np.arange(p * 1024, p * 1024 + len(seg))
            order = np.lexsort((-ids, -key))[:21]
            got_ids = (cand[r, p] >> np.uint64(32)).astype(np.int64)
            assert list(got_ids) == list(ids[order])
            assert norm[r, p, 0] == float(seg.max())
    tail = x[0, 2048:].astype(np.float64)
    assert abs(norm[0, 2, 1] - math.fsum(np.exp(tail - tail.max()))) < 1e-12
    assert norm[1, 0, 1] == 0.0                      # temperature 0: no mass


# ------------------------------------------------------------------ product vs oracle

def test_sampler_settings_validation(lia):
    for args in [(0.0, 20, 0.95, 0), (1.0, 21, 0.95, 0), (1.0, 20, 0.0, 0), (math.nan, 0, 1.0, 0),
                 (1.0, 0, 1.5, 0)]:
        with pytest.raises(lia.LiaError) as e:
            lia.Sampler(*args)
        assert e.value.status == -25


def test_sampler_distribution_matches_oracle(lia):
    rng = np.random.default_rng(2)
    cases = [_partial_logits()[:300], list(enumerate(_nucleus_logits()[:500]))]
    for _ in range(20):
        n = int(rng.integers(1, 200))
        vals = rng.standard_normal(n).astype(np.float32) * 3
        vals[rng.random(n) < 0.1] = -np.inf
        vals[rng.random(n) < 0.1] = 1.25
        cases.append(list(zip(rng.permutation(10000)[:n].tolist(), [float(v) for v in vals])))
    for cands in cases:
        if all(v == -math.inf for _, v in cands):
            continue
        for t, k, p in [(1.0, 0, 1.0), (0.7, 5, 0.9), (2.0, 20, 0.5), (1.3, 0, 0.3)]:
            got = lia.Sampler(t, k, p, 0).distribution(cands)
            want = OS.Sampling(t, k, p, 0).distribution(cands)
            assert got == want


def test_sampler_errors(lia):
    s = lia.Sampler(1.0, 0, 1.0, 0)
    for bad, code in [([], -27), ([(0, math.nan)], -26), ([(0, math.inf)], -26),
                      ([(0, -math.inf)], -27), ([(1, 0.0), (1, 1.0)], -28)]:
        with pytest.raises(lia.LiaError) as e:
            s.distribution(bad)
        assert e.value.status == code


@pytest.mark.parametrize("keyed", [False, True])
def test_draws_match_oracle(lia, keyed):
    rng = np.random.default_rng(3)
    for seed in (0, 42, 2026, 2**40 + 7):
        a = lia.Sampler(0.8, 0, 0.9, seed, position_keyed=keyed)
        b = OS.Sampling(0.8, 0, 0.9, seed, position_keyed=keyed)
        for step in range(50):
            n = int(rng.integers(1, 30))
            d = b.distribution([(int(i), float(v)) for i, v in
                                zip(rng.permutation(5000)[:n], rng.standard_normal(n))])
            if keyed and step % 7 == 0:
                a.set_position(1000 + step)
                b.set_position(1000 + step)
            assert a.draw(d) == b.draw(d)


def _sample_case(lia, logits, configs, positions):
    temps = [((t if k == 0 else 0.0) if t is not None else 0.0) for t, k, p, seed, keyed in configs]
    cand, norm = OS.nucleus_candidates(logits, temps)
    mk = lambda f: [None if c[0] is None else f(*c) for c in configs]
    got = lia.sample_host(logits.shape[1], mk(lambda t, k, p, s, kd: lia.Sampler(t, k, p, s, kd)),
                          positions, cand, norm, logits)
    want = OS.sample_rows(logits, mk(lambda t, k, p, s, kd: OS.Sampling(t, k, p, s, kd)),
                          positions)
    return got, tuple(want)


def test_sample_host_matches_oracle_on_reference_rows(lia):
    logits, temps = reference_gpu_rows()
    configs = [(temps[i], 0, 0.95, 42, False) for i in range(4)]
    got, want = _sample_case(lia, logits, configs, [5, 6, 7, 8])
    assert got == want and got[1] == 2        # rows 0 and 2 read their full logits


def test_sample_host_mixed_samplers_match_oracle(lia):
    rng = np.random.default_rng(4)
    V = 2600
    logits = (rng.standard_normal((6, V)) * 2).astype(np.float32)
    logits[1, 100:110] = 9.0                      # tied peak
    logits[2] = -np.inf
    logits[2, 2000] = 1.0
    configs = [(None, 0, 1.0, 0, False), (None, 0, 1.0, 0, False), (1.0, 0, 0.9, 1, False),
               (0.6, 7, 1.0, 2, False), (1.0, 0, 0.2, 3, True), (1.5, 0, 1.0, 4, False)]
    got, want = _sample_case(lia, logits, configs, [10, 20, 30, 40, 50, 60])
    assert got == want
    assert got[0][1] in range(100, 110) and got[0][1] == 109   # ties: larger id wins
