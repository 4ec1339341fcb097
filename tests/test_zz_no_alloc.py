"""lia_paged_attention_static (the entry point that allocates nothing) against
lia_paged_attention (caller workspace): two calls in a row through the C ABI, the second
with a smaller batch, each bit-identical to the workspace entry point's output (the same
kernels and plan run on the same inputs).  Also: a configuration whose workspace exceeds the
static array is rejected."""
import ctypes as C

import numpy as np
import pytest
import torch

import gpu_data as G

pytestmark = pytest.mark.gpu


def _static(lia, case, dev, out):
    b = case.batch
    cfg = case.config(lia)
    p = lambda t: None if t is None else C.c_void_p(t.data_ptr())
    st = lia.lib().lia_paged_attention_static(
        C.byref(cfg), b.n_seqs, b.n_rows, p(dev["cu"]), p(dev["positions"]), p(dev["sequences"]),
        p(dev["pages"]), p(dev["q"]), p(dev["kc"]), p(dev["vc"]), p(dev["k_scales"]),
        p(dev["v_scales"]), p(out), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, st


@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_static_workspace_matches_caller_workspace(lia, wl, kind):
    if kind == "decode":
        batches = [wl.config2(seed=0, layers=1), wl.custom([900, 33, 4000], [1, 1, 1], seed=61)]
    else:
        # prefill workspaces hold 128-column records: a batch of 165 rows fits the array
        batches = [wl.custom([64, 1500 + 100, 700], [64, 100, 1], seed=62),
                   wl.custom([200, 40], [50, 1], seed=63)]
    for i, b in enumerate(batches):
        print(f"[case] static workspace {kind} call {i}: seqs={b.n_seqs} rows={b.n_rows}", flush=True)
        case = G.Case(b, seed=60 + i)
        assert lia.workspace_bytes(case.config(lia)) <= lia.lib().lia_static_workspace_bytes()
        dev = case.device()
        ref = torch.from_numpy(case.run(lia, dev)).to(torch.bfloat16).cuda()
        out = torch.full_like(ref, float("nan"))
        _static(lia, case, dev, out)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (kind, i)
        want = case.f64()
        mx, mean = G.errors(out.float().cpu().numpy(), want)
        assert mx < 2e-2 and mean < 2e-3


def test_static_workspace_limit(lia, wl):
    b = wl.config3(seed=0)  # thousands of prefill rows: more records than the array holds
    case = G.Case.__new__(G.Case)
    case.batch, case.g = b, b.geom
    cfg = case.config(lia)
    assert lia.workspace_bytes(cfg) > lia.lib().lia_static_workspace_bytes()
    fake = C.c_void_p(0x100000)
    st = lia.lib().lia_paged_attention_static(C.byref(cfg), b.n_seqs, b.n_rows, *([fake] * 7),
                                              None, None, fake, None)
    assert st == -22  # LIA_E_WORKSPACE, before anything is launched
