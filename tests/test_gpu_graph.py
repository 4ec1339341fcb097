"""Graph capture of a whole paged step and the output-row gather.

The step (device packing, plan, the KV append - fused into the attention launch on 16-bit
pools, the quantising append on FP8 pools - partial attention, merge) is captured once
and replayed several times with new queries written between replays by ordinary eager work;
every replay must equal the eager execution of the same step bit for bit (the reference
replays captured paged graphs the same way, src/inference/paging.rs:215-259)."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, FP8

pytestmark = pytest.mark.gpu


BATCHES = {
    # decode, MTP-like and prefill rows mixed (the decode kernel)
    "mixed": (([300, 1200, 17, 5000, 64], [1, 1, 3, 1, 64]), BF16),
    # long chunks with prefixes (the prefill kernel and its combine)
    "prefill": (([300, 1000 + 77, 2000 + 40], [300, 77, 40]), BF16),
    # an FP8 pool: quantising append, then attention over e4m3 pages
    "fp8": (([300, 1200, 17, 5000, 64], [1, 1, 3, 1, 64]), FP8),
}


def _setup(lia, wl, kind, seed):
    (ctx, q_len), kv = BATCHES[kind]
    b = wl.custom(ctx, q_len, geom=wl.Geometry(kv_dtype=kv), seed=seed)
    case = G.Case(b, seed=seed)
    g = b.geom
    dev = case.device()
    W = g.hkv * g.d
    slots = b.slot_mapping().astype(np.int64)
    if kv == FP8:
        rng = np.random.default_rng(seed)
        newk = G.to_dev(G.O.from_f32(rng.standard_normal((b.n_rows, W), dtype=np.float32) * 0.01, BF16),
                        torch.bfloat16)
        newv = G.to_dev(G.O.from_f32(rng.standard_normal((b.n_rows, W), dtype=np.float32) * 0.01, BF16),
                        torch.bfloat16)
    else:
        newk = G.to_dev(case.kc.reshape(-1, W)[slots].copy(), torch.bfloat16)
        newv = G.to_dev(case.vc.reshape(-1, W)[slots].copy(), torch.bfloat16)
    cfg = case.config(lia)
    layout = lia.KVLayout(g.hkv, g.d, g.page_size, b.pool_pages, kv)
    ws = G.dirty_workspace(lia, cfg)
    meta = dict(
        seq_slots=G.u32_dev(np.arange(b.n_seqs)), q_lens=G.u32_dev(b.q_len), cached=G.u32_dev(b.cached),
        cu=torch.zeros(b.n_seqs + 1, dtype=torch.int32, device="cuda"),
        positions=torch.zeros(b.n_rows, dtype=torch.int32, device="cuda"),
        sequences=torch.zeros(b.n_rows, dtype=torch.int32, device="cuda"),
        slots=torch.zeros(b.n_rows, dtype=torch.int32, device="cuda"),
        status=torch.zeros(1, dtype=torch.int32, device="cuda"))
    out = torch.zeros((b.n_rows, g.hq, g.d), dtype=torch.bfloat16, device="cuda")

    def step():
        lia.pack_device(meta["seq_slots"], meta["q_lens"], meta["cached"], dev["pages"], b.stride,
                        g.page_size, b.pool_pages, b.stride * g.page_size, b.n_rows, meta["cu"],
                        meta["positions"], meta["sequences"], meta["slots"], meta["status"])
        lia.attention_plan(cfg, b.n_seqs, b.n_rows, meta["cu"], meta["positions"], meta["sequences"],
                           ws, pages=dev["pages"])
        if kv == FP8:
            lia.kv_append(layout, newk, newv, dev["kc"], dev["vc"], slot_mapping=meta["slots"],
                          k_scales=dev["k_scales"], v_scales=dev["v_scales"])
            lia.attention_partial(cfg, b.n_seqs, dev["pages"], dev["q"], dev["kc"], dev["vc"], out, ws,
                                  k_scales=dev["k_scales"], v_scales=dev["v_scales"])
        else:
            lia.attention_partial_append(cfg, b.n_seqs, dev["pages"], meta["slots"], dev["q"], newk,
                                         newv, dev["kc"], dev["vc"], out, ws)
        lia.attention_merge(cfg, b.n_seqs, b.n_rows, out, ws)
    return b, case, dev, step, out, meta


@pytest.mark.parametrize("kind", list(BATCHES))
def test_graph_replays_equal_eager(lia, wl, kind):
    b, case, dev, step, out, meta = _setup(lia, wl, kind, 31)
    pool_k, pool_v = dev["kc"].clone(), dev["vc"].clone()
    rng = np.random.default_rng(5)
    qs = [G.to_dev(G.O.from_f32(rng.standard_normal(tuple(dev["q"].shape), dtype=np.float32), BF16),
                   torch.bfloat16) for _ in range(4)]
    # eager results per query set
    expected = []
    for q in qs:
        dev["q"].copy_(q)
        dev["kc"].copy_(pool_k)
        dev["vc"].copy_(pool_v)
        step()
        torch.cuda.synchronize()
        assert meta["status"].item() == 0
        expected.append((out.clone(), dev["kc"].clone()))
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            step()
    torch.cuda.synchronize()
    for i, q in enumerate(qs):
        print(f"[case] graph replay {kind} {i}", flush=True)
        dev["q"].copy_(q)
        dev["kc"].copy_(pool_k)
        dev["vc"].copy_(pool_v)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), expected[i][0].view(torch.int16)), i
        assert torch.equal(dev["kc"], expected[i][1]), i
    # the replayed output is also right against the f64 oracle on the pool the step left
    # (last query set)
    store = np.uint8 if case.g.kv_dtype == FP8 else np.uint16
    case.kc = dev["kc"].cpu().numpy().view(store).reshape(-1)
    case.vc = dev["vc"].cpu().numpy().view(store).reshape(-1)
    case.q_store = qs[-1].view(torch.int16).cpu().numpy().view(np.uint16)
    case.q32 = G.O.to_f32(case.q_store, BF16)
    mx, mean = G.errors(out.float().cpu().numpy(), case.f64())
    tol = (5e-2, 5e-3) if case.g.kv_dtype == FP8 else (2e-2, 2e-3)
    print(f"[case] graph {kind}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert mx < tol[0] and mean < tol[1]


@pytest.mark.parametrize("width,offset", [(2048, 0), (2048 + 4, 0), (7, 0), (256, 1)])
def test_gather_rows(lia, O, width, offset):
    """llama_gather_hidden generalised: vector path (rows of 4k words, aligned) and the
    word path (odd widths, misaligned pointers)."""
    rng = np.random.default_rng(width + offset)
    rows, count = 37, 11
    src = rng.standard_normal(rows * width + offset).astype(np.float32)
    idx = rng.integers(0, rows, count).astype(np.uint32)
    ref = O.gather(idx, src[offset:], width)
    dsrc = G.to_dev(src)[offset:].view(rows, width)
    dst = torch.zeros(count * width + offset, dtype=torch.float32, device="cuda")[offset:].view(count, width)
    lia.gather_rows(G.u32_dev(idx), dsrc, dst)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy().reshape(-1).view(np.uint32), ref.view(np.uint32))


GROWING = {
    # decode rows: every step one key longer per sequence (the decode kernel, one tile)
    "decode": ([300, 1200, 17, 5000, 64], [1, 1, 1, 1, 1]),
    # verify rows and short chunks (the decode kernel's two-tile path)
    "mixed": ([2000, 1200, 5000, 900], [8, 1, 3, 2]),
    # prefill chunks over growing prefixes (the prefill kernel and its merge)
    "prefill": ([3000, 2500], [256, 128]),
}


@pytest.mark.parametrize("kind", list(GROWING))
def test_graph_replays_follow_growing_contexts(lia, wl, kind):
    """A serving loop over one captured step: device packing and plan in one launch
    (lia_pack_plan_device), the fused append + attention, the merge.  Between replays only the
    packing's inputs (each sequence's cached keys, advanced by its rows), the step's new K/V
    rows and nothing else change, so the device plan - units, block ranges, merge descriptors,
    split records - is rebuilt under the same graph every step, over a workspace that still
    holds the previous step's plan.  Each replay equals the eager step bit for bit, and every
    eager step matches the f64 oracle."""
    import dataclasses
    ctx_final, q_len = GROWING[kind]
    S = 3
    final = wl.custom(ctx_final, q_len, seed=41)
    steps = [dataclasses.replace(final, ctx=final.ctx - (S - 1 - i) * final.q_len) for i in range(S)]
    cases = [G.Case(b, seed=41) for b in steps]
    g, case = final.geom, cases[-1]
    rows, W = final.n_rows, g.hkv * g.d
    cfg = case.config(lia)
    dev = case.device()
    ws = G.dirty_workspace(lia, cfg)
    seq_slots, q_lens = G.u32_dev(np.arange(final.n_seqs)), G.u32_dev(final.q_len)
    cached = G.u32_dev(steps[0].cached)
    cu = torch.zeros(final.n_seqs + 1, dtype=torch.int32, device="cuda")
    meta = [torch.zeros(rows, dtype=torch.int32, device="cuda") for _ in range(3)]
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    newk = torch.zeros((rows, W), dtype=torch.bfloat16, device="cuda")
    newv = torch.zeros_like(newk)
    out = torch.zeros((rows, g.hq, g.d), dtype=torch.bfloat16, device="cuda")
    context = final.stride * g.page_size

    def set_step(i):
        # the step's rows are the pool's own values at their slots, so the append rewrites
        # what the pool holds and every step attends the same pool contents
        slots = steps[i].slot_mapping().astype(np.int64)
        cached.copy_(G.u32_dev(steps[i].cached))
        newk.copy_(G.to_dev(case.kc.reshape(-1, W)[slots].copy(), torch.bfloat16))
        newv.copy_(G.to_dev(case.vc.reshape(-1, W)[slots].copy(), torch.bfloat16))

    def step():
        lia.pack_plan_device(cfg, seq_slots, q_lens, cached, dev["pages"], rows, context, cu, meta[0],
                             meta[1], meta[2], status, ws)
        lia.attention_partial_append(cfg, final.n_seqs, dev["pages"], meta[2], dev["q"], newk, newv,
                                     dev["kc"], dev["vc"], out, ws)
        lia.attention_merge(cfg, final.n_seqs, rows, out, ws)

    expected = []
    for i in range(S):
        set_step(i)
        step()
        torch.cuda.synchronize()
        assert status.item() == 0, i
        got = out.float().cpu().numpy()
        mx, mean = G.errors(got, cases[i].f64())
        print(f"[case] growing {kind} eager step {i}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
        assert mx < 2e-2 and mean < 2e-3, i
        expected.append(out.clone())
    set_step(0)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            step()
    torch.cuda.synchronize()
    for rep in range(2):
        for i in range(S):
            print(f"[case] growing {kind} replay {rep} step {i}", flush=True)
            set_step(i)
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert status.item() == 0, i
            assert torch.equal(out.view(torch.int16), expected[i].view(torch.int16)), (rep, i)
