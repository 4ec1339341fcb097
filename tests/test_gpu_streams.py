"""Attention launches on two streams at once, each with its own workspace, pool and output: the
library keeps no device state between calls other than the caller's workspace, so the
concurrent results equal each batch's results run alone, bit for bit, and the oracle."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, FP8

pytestmark = pytest.mark.gpu


def _setup(lia, wl, ctx, q_len, kv, seed):
    b = wl.custom(ctx, q_len, geom=wl.Geometry(kv_dtype=kv), seed=seed)
    case = G.Case(b, seed=seed)
    cfg = case.config(lia)
    dev = case.device()
    ws = G.dirty_workspace(lia, cfg)
    out = torch.full((b.n_rows, case.g.hq, case.g.d), float("nan"), dtype=torch.bfloat16, device="cuda")
    return case, cfg, dev, ws, out


def _launch(lia, case, cfg, dev, ws, out, stream):
    lia.paged_attention(cfg, case.batch.n_seqs, dev["cu"], dev["positions"], dev["sequences"],
                        dev["pages"], dev["q"], dev["kc"], dev["vc"], out, ws, dev["k_scales"],
                        dev["v_scales"], stream=stream)


def test_two_streams_concurrent(lia, wl):
    batches = [
        ([28000, 9000, 17, 3000, 1200, 64, 5000, 700], [1] * 8, BF16, 61),  # decode kernel
        ([300, 1077, 2040], [300, 77, 40], BF16, 62),                       # prefill kernel
        ([4000, 250, 9000, 33], [1, 3, 2, 1], FP8, 63),                      # two-tile, FP8 pool
    ]
    sets = [_setup(lia, wl, *b) for b in batches]
    alone = []
    for case, cfg, dev, ws, out in sets:
        _launch(lia, case, cfg, dev, ws, out, None)
        torch.cuda.synchronize()
        got = out.clone()
        mx, mean = G.errors(got.float().cpu().numpy(), case.f64())
        tol = (5e-2, 5e-3) if case.g.kv_dtype == FP8 else (2e-2, 2e-3)
        print(f"[case] alone seqs={case.batch.n_seqs}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
        assert mx < tol[0] and mean < tol[1]
        alone.append(got)
    streams = [torch.cuda.Stream() for _ in sets]
    for rep in range(3):
        print(f"[case] concurrent round {rep}", flush=True)
        for (case, cfg, dev, ws, out), st in zip(sets, streams):
            out.fill_(float("nan"))
        torch.cuda.synchronize()
        # each stream runs every batch twice in a row, interleaved with the other streams
        for _ in range(2):
            for (case, cfg, dev, ws, out), st in zip(sets, streams):
                _launch(lia, case, cfg, dev, ws, out, st)
        torch.cuda.synchronize()
        for (case, cfg, dev, ws, out), ref in zip(sets, alone):
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep
