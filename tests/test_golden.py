"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py)
against the CPU oracle: the oracle must reproduce them bit for bit, and the config-1
outputs are checked once more against a float64 softmax written here in numpy from the
stored K/V (src/gpu/llama_attention.rs:253-284)."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as MG  # noqa: E402

GOLDEN = os.path.join(HERE, "golden")


def _load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def rebuilt():
    return MG.build_all()


@pytest.mark.parametrize("name", ["cfg1.npz", "reference_attention.npz", "reference_merge.npz",
                                  "reference_rotary.npz"])
def test_oracle_reproduces_fixture(rebuilt, name):
    want = _load(name)
    got = rebuilt[name]
    assert sorted(want) == sorted(got), name
    for k, w in want.items():
        g = np.asarray(got[k])
        assert g.dtype == w.dtype and g.shape == w.shape, (name, k)
        if g.dtype.kind == "f":
            assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), (name, k)
        else:
            assert np.array_equal(g, w), (name, k)


def test_cfg1_fixture_against_numpy_softmax(O, wl):
    fx = _load("cfg1.npz")
    b, kc, vc, q_store = MG.cfg1_inputs(O, wl)
    assert MG.digest(kc, vc, q_store) == str(fx["inputs_sha256"])
    g = b.geom
    P = g.page_size
    kf = O.to_f32(kc, MG.BF16).astype(np.float64).reshape(-1, g.hkv, g.d)
    vf = O.to_f32(vc, MG.BF16).astype(np.float64).reshape(-1, g.hkv, g.d)
    qf = O.to_f32(q_store, MG.BF16).astype(np.float64).reshape(-1, g.hq, g.d)
    group = g.hq // g.hkv
    stride = int(fx["stride"])
    for r in range(b.n_rows):
        s, n = int(fx["sequences"][r]), int(fx["positions"][r]) + 1
        tok = np.arange(n)
        phys = fx["flat"][s * stride + tok // P].astype(np.int64) * P + tok % P
        for h in range(g.hq):
            sc = kf[phys, h // group] @ qf[r, h] * g.scale
            w = np.exp(sc - sc.max())
            ref = (w / w.sum()) @ vf[phys, h // group]
            assert np.max(np.abs(ref - fx["out_f64"][r, h])) < 1e-12
    assert np.max(np.abs(fx["out_split_f32"] - fx["out_f64"])) < 3e-5
    # packing: the workload's own closed forms
    assert np.array_equal(fx["cu_seqlens"], b.cu_seqlens())
    assert np.array_equal(fx["slot_mapping"], b.slot_mapping())


def test_merge_fixture_against_numpy():
    fx = _load("reference_merge.npz")
    for parts in MG.MERGE_PARTS:
        pr = MG.merge_partial(parts).reshape(48, parts, 130).astype(np.float64)
        m, l = pr[:, :, 128], pr[:, :, 129]
        M = np.max(np.where(l > 0, m, -np.inf), axis=1, keepdims=True)
        w = np.where(l > 0, np.exp(m - M), 0.0)
        ref = (w[:, :, None] * pr[:, :, :128]).sum(1) / (w * l).sum(1, keepdims=True)
        out = fx[f"out_parts{parts}"]
        assert np.max(np.abs(out[5:8].reshape(48, 128) - ref)) < 1e-5, parts
        assert np.all(out[:5] == 7.0) and np.all(out[8:] == 7.0)
