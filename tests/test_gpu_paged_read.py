"""lia_paged_read, the decode kernel's loads without its arithmetic (the paged-read ceiling the
bench times beside the kernel): each wave folds the words it loaded of the keys inside its
range, so over a decode batch the XOR of the sink words equals the XOR of every attended key's
K words (all KV heads), and on FP8 pools of its V words too, which the host computes from the
pool and the block tables."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, F16, FP8

pytestmark = pytest.mark.gpu


def _host_fold(case):
    b, g = case.batch, case.g
    P = g.page_size
    planes = [case.kc] + ([case.vc] if g.kv_dtype == FP8 else [])
    acc = np.uint32(0)
    for plane in planes:
        words = plane.view(np.uint32).reshape(b.pool_pages * P, -1)  # one slot's row per line
        for s in range(b.n_seqs):
            t = np.arange(int(b.ctx[s]))  # keys attended by the sequence's row
            slots = np.asarray(b.tables[s], np.int64)[t // P] * P + t % P
            acc ^= np.bitwise_xor.reduce(words[slots].reshape(-1))
    return int(acc)


def _fold(lia, case):
    b = case.batch
    dev = case.device()
    cfg = case.config(lia)
    ws = G.dirty_workspace(lia, cfg)
    lia.attention_plan(cfg, b.n_seqs, b.n_rows, dev["cu"], dev["positions"], dev["sequences"], ws,
                       pages=dev["pages"])
    sink = torch.zeros(lia.paged_read_sink_words(cfg), dtype=torch.int32, device="cuda")
    lia.paged_read(cfg, b.n_seqs, dev["pages"], dev["q"], dev["kc"], dev["vc"], sink, ws,
                   dev["k_scales"], dev["v_scales"])
    torch.cuda.synchronize()
    return int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))


@pytest.mark.parametrize("kv", [BF16, F16, FP8])
@pytest.mark.parametrize("d,hq,hkv,page", [(128, 16, 2, 16), (64, 8, 2, 16), (128, 16, 2, 32),
                                           (128, 8, 1, 16)])
def test_paged_read_loads_every_key_once(lia, wl, kv, d, hq, hkv, page):
    ctx = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 511, 1000, 2049, 4097]
    g = wl.Geometry(hq=hq, hkv=hkv, d=d, page_size=page, kv_dtype=kv)
    b = wl.custom(ctx, [1] * len(ctx), geom=g, seed=5)
    case = G.Case(b, seed=5, fill="fp8_codes") if kv == FP8 else G.Case(b, seed=5, fill="uniform")
    print(f"[case] paged_read kv={kv} d={d} hq={hq} hkv={hkv} page={page}", flush=True)
    assert _fold(lia, case) == _host_fold(case)


def test_paged_read_config2_full_size(lia, wl):
    case = G.Case(wl.config2(seed=0), seed=0, fill="uniform")
    print(f"[case] paged_read config 2 sum ctx {int(case.batch.ctx.sum())}", flush=True)
    assert _fold(lia, case) == _host_fold(case)


def test_paged_read_config5_full_size(lia, wl):
    case = G.Case(wl.config5(seed=0), seed=0, fill="fp8_codes")
    print(f"[case] paged_read config 5 sum ctx {int(case.batch.ctx.sum())}", flush=True)
    assert _fold(lia, case) == _host_fold(case)
