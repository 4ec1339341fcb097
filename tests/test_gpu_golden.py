"""The HIP library against the committed golden fixtures (tests/golden/*.npz), with no
oracle call: inputs are regenerated from their closed forms or seeds and checked against
the fixtures' SHA-256 digests, then packing (bit-exact), attention (max-abs 2e-2 and
mean-abs 2e-3 for the bf16 case; 1e-3 / 1e-4 for the reference's f16 case with f32
queries) and the fused RoPE + append (bit-exact) are compared with the stored outputs."""
import os
import sys

import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, F16, F32

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as MG  # noqa: E402

pytestmark = pytest.mark.gpu


def _load(name):
    with np.load(os.path.join(HERE, "golden", name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _attend(lia, g, n_seqs, n_rows, pool_pages, stride, max_ctx, cu, pos, seq, flat, q, kc, vc):
    cfg = lia.AttentionConfig(g.hq, g.hkv, g.d, g.page_size, pool_pages, stride, g.q_dtype,
                              g.kv_dtype, g.out_dtype, g.scale, n_seqs, n_rows, max_ctx)
    ws = G.dirty_workspace(lia, cfg)
    odt = torch.float32 if g.out_dtype == F32 else torch.bfloat16
    out = torch.full((n_rows, g.hq, g.d), float("nan"), dtype=odt, device="cuda")
    lia.paged_attention(cfg, n_seqs, G.u32_dev(cu), G.u32_dev(pos), G.u32_dev(seq), G.u32_dev(flat),
                        q, kc, vc, out, ws, None, None)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_cfg1_pack_and_attention(lia, wl, O):
    print("[case] golden cfg1", flush=True)
    fx = _load("cfg1.npz")
    b, kc, vc, q_store = MG.cfg1_inputs(O, wl)
    assert MG.digest(kc, vc, q_store) == str(fx["inputs_sha256"])
    n, rows = len(fx["ctx"]), int(fx["q_len"].sum())
    P, stride = b.geom.page_size, int(fx["stride"])
    dev = {k: torch.full((rows + (k == "cu"),), -7, dtype=torch.int32, device="cuda")
           for k in ("cu", "positions", "sequences", "slots")}
    status = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    lia.pack_device(G.u32_dev(np.arange(n)), G.u32_dev(fx["q_len"]), G.u32_dev(fx["cached"]),
                    G.u32_dev(fx["flat"]), stride, P, int(fx["pool_pages"]), stride * P, rows,
                    dev["cu"], dev["positions"], dev["sequences"], dev["slots"], status)
    torch.cuda.synchronize()
    assert status.item() == 0
    got = {k: v.cpu().numpy().view(np.uint32) for k, v in dev.items()}
    assert np.array_equal(got["cu"][:n + 1], fx["cu_seqlens"])
    assert np.array_equal(got["positions"], fx["positions"])
    assert np.array_equal(got["sequences"], fx["sequences"])
    assert np.array_equal(got["slots"], fx["slot_mapping"])
    out = _attend(lia, b.geom, n, rows, int(fx["pool_pages"]), stride, int(fx["ctx"].max()),
                  fx["cu_seqlens"], fx["positions"], fx["sequences"], fx["flat"],
                  G.to_dev(q_store, torch.bfloat16), G.to_dev(kc, torch.int16), G.to_dev(vc, torch.int16))
    mx, mean = G.errors(out, fx["out_f64"])
    print(f"[case] golden cfg1: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(out)) and mx < 2e-2 and mean < 2e-3
    assert np.max(np.abs(out - fx["out_split_f32"])) < 2e-2


def test_reference_known_answer_attention(lia, wl):
    print("[case] golden reference attention", flush=True)
    fx = _load("reference_attention.npz")
    from test_oracle import _reference_vectors
    stride, pos, seq, tables, keys, vals, q, _ = _reference_vectors()
    kc = keys.astype(np.float16).view(np.uint16)
    vc = vals.astype(np.float16).view(np.uint16)
    assert MG.digest(kc, vc, q, tables) == str(fx["inputs_sha256"])
    g = wl.Geometry(hq=16, hkv=2, d=128, page_size=32, kv_dtype=F16, q_dtype=F32, out_dtype=F32)
    cu = np.array([0, 8, 16, 17], np.uint32)  # three runs of consecutive positions
    out = _attend(lia, g, 3, 17, 2 * stride, stride, 16385, cu, pos, seq, tables, G.to_dev(q),
                  G.to_dev(kc.reshape(-1), torch.int16), G.to_dev(vc.reshape(-1), torch.int16))
    mx, mean = G.errors(out, fx["out_f32"])
    print(f"[case] golden reference attention: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert mx < 1e-3 and mean < 1e-4


def test_reference_rotary_fixture(lia):
    print("[case] golden rotary cache", flush=True)
    fx = _load("reference_rotary.npz")
    positions, sequences, tables, combined, slots = MG.rotary_inputs()
    assert MG.digest(combined, tables) == str(fx["inputs_sha256"])
    coeffs = torch.zeros(5 * 128, dtype=torch.float32, device="cuda")
    lia.rope_coefficients(G.u32_dev(positions), 128, coeffs)
    kc = torch.zeros(8 * 32 * 256, dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    q = torch.zeros((5, 16, 128), dtype=torch.float32, device="cuda")
    layout = lia.KVLayout(2, 128, 32, 8, F16)
    lia.rope_kv_append(layout, 16, coeffs, G.to_dev(combined.reshape(5, -1)), q, kc, vc,
                       positions=G.u32_dev(positions), sequences=G.u32_dev(sequences),
                       pages=G.u32_dev(tables), stride=4096)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy().reshape(-1).view(np.uint32), fx["query_bits"])
    k = kc.cpu().numpy().view(np.uint16).reshape(-1, 256)
    v = vc.cpu().numpy().view(np.uint16).reshape(-1, 256)
    assert np.array_equal(k[fx["slots"]], fx["k_rows"]) and np.array_equal(v[fx["slots"]], fx["v_rows"])
    others = np.setdiff1d(np.arange(k.shape[0]), fx["slots"])
    assert not k[others].any() and not v[others].any()
