"""Benchmark of the paged decode-attention hot path on one MI355X.

Workload: ragged bf16 decode, batch 8, contexts U[1024, 32768]
(seeded), 16 query / 2 KV heads, head_dim 128, 16-token pages scattered by a seeded
permutation, N(0,1) data, 40 layers as independent KV slices.

One step = device packing of the batch (cu_seqlens, positions, slot mapping) and the work
plan (lia_pack_plan_device: the plan runs beside the packing, then the table checks), then per
layer: the split attention kernel with the KV append of the 8 new tokens
fused in (lia_attention_partial_append: the new keys are read from the step's rows and
scattered into the pool by the same launch) and the split combine.  The step is captured once as a HIP graph and replayed (the reference
replays CUDA graphs of the paged forward, src/inference/paging.rs:238-259).

value = decode tokens/s of the whole step (8 tokens per step).  The roofline object
covers the dominant kernel (the split attention kernel), timed alone with HIP events on
its stream; its algorithmic bytes are K/V of every attended key + Q + O + block table +
the appended rows it writes.  Beside it, the same run times two ceilings of those bytes:
`read_ceiling`, a contiguous read (lia_hbm_read), and `paged_read_ceiling`, the kernel's own
plan, loads and pipeline with the attention arithmetic left out (lia_paged_read).

`side` holds configs 3, 4 and 5 (parity workloads, timed for the record): a one-layer step,
the attention launch alone, for 4 and 5 the kernel's loads alone, and a 40-layer model step
per layer; every layer has its own KV pool, so no timed launch re-reads a pool the 256 MB
last-level cache could still hold.  `cpu_baseline` is the reference algorithm (the oracle's
f32 split-K + merge) on the host cores, a bounded sample scaled to the step.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0   # dense MFMA, MI355X
METRIC = "decode-attn tokens/s + achieved HBM GB/s (% peak), ragged batch 8, 1 GPU"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-side", action="store_true",
                    help="skip the one-layer steps of configs 3, 4 and 5 in the default run")
    ap.add_argument("--side-steps", type=int, default=20,
                    help="graph replays timed per side configuration (10 steps each)")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles",
                                                    "attention_decode_cfg2_traffic.json"),
                    help="HBM traffic per launch measured by rocprofv3 --pmc (JSON summary)")
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5),
                    help="3, 4 or 5: time one layer of that BASELINE configuration's attention "
                         "(a parity workload, not the headline line) and print its own JSON line")
    ap.add_argument("--kv", default=None, choices=("fp8",),
                    help="with --config 3 or 4: the same batch on an FP8 e4m3 pool (per-page scales)")
    return ap.parse_args()


def load_traffic(path, kernel_us, layer_bytes):
    """traffic = (FETCH_SIZE + WRITE_SIZE per dispatch of the kernel) x calibration factor."""
    if not path or not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return round((t["fetch_kib"] * t["fetch_scale"] + t["write_kib"] * t["write_scale"]) * 1024)


SIDE_NAMES = {3: "mixed chunked-prefill + decode attention step", 4: "MTP-verify attention step",
              5: "FP8-KV decode attention step"}


def side_measure(config, seed, steps, warmup, reps, kv=None, layers=40):
    """One layer of BASELINE config 3 (mixed prefill + decode, MFMA-bound), 4 (MTP verify) or
    5 (FP8 decode) on resident synthetic data, timed as a step of its own: device packing,
    the plan, the KV append of the step's rows (fused into the attention launch on 16-bit
    pools; on FP8 pools quantised by the append launch of the same call, just before the
    attention launch), split attention and the combine, replayed from a graph (`reps` steps
    per graph).  The attention launch alone is timed the same way (a graph of `reps` launches
    on one plan).  Every layer has its own KV pool, queries and rows, and the `reps` steps or
    launches of a graph go to `reps` different layers, so no timed launch re-reads a pool the
    256 MB last-level cache may still hold (config 3's pool is 101 MB, config 4's 274 MB).
    Returns the step and kernel times with their rooflines: MFMA for config 3, HBM (and MFMA)
    for configs 4 and 5, against the layer's algorithmic work.  It also times a model step as
    config 2's is: the packing and plan once, then per layer the attention launch and the
    combine, `layers` layers in one graph; reported per layer."""
    import torch
    from __graft_entry__ import package
    lia = package()
    import lia_rs_amd.workloads as wl
    b = getattr(wl, "config%d" % config)(seed=seed)
    if kv == "fp8":
        b.geom = wl.Geometry(kv_dtype=wl.FP8)
    g = b.geom
    P = g.page_size
    tokens = b.pool_pages * P
    dev = "cuda"
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    fp8 = g.kv_dtype == lia.FP8
    rows = b.n_rows
    reps = max(reps, 1)
    L = max(layers, reps)

    def layer():
        if fp8:
            kp = torch.randint(0, 120, (tokens, g.hkv, g.d), generator=gen, dtype=torch.uint8, device=dev)
            vp = torch.randint(0, 120, (tokens, g.hkv, g.d), generator=gen, dtype=torch.uint8, device=dev)
        else:
            kp = torch.randn((tokens, g.hkv, g.d), generator=gen, device=dev).to(torch.bfloat16)
            vp = torch.randn((tokens, g.hkv, g.d), generator=gen, device=dev).to(torch.bfloat16)
        return dict(kp=kp, vp=vp,
                    newk=torch.randn((rows, g.hkv * g.d), generator=gen, device=dev).to(torch.bfloat16),
                    newv=torch.randn((rows, g.hkv * g.d), generator=gen, device=dev).to(torch.bfloat16),
                    q=torch.randn((rows, g.hq, g.d), generator=gen, device=dev).to(torch.bfloat16),
                    out=torch.empty((rows, g.hq, g.d), dtype=torch.bfloat16, device=dev))

    pools = [layer() for _ in range(L)]
    ks = torch.full((b.pool_pages * g.hkv,), 0.01, device=dev) if fp8 else None
    vs = ks.clone() if fp8 else None
    i32 = lambda a: torch.from_numpy(np.asarray(a, np.uint32).view(np.int32)).to(dev)
    seq_slots, q_lens, cached = i32(np.arange(b.n_seqs)), i32(b.q_len), i32(b.cached)
    flat = i32(b.flat_table())
    cu = torch.zeros(b.n_seqs + 1, dtype=torch.int32, device=dev)
    positions = torch.zeros(rows, dtype=torch.int32, device=dev)
    sequences = torch.zeros(rows, dtype=torch.int32, device=dev)
    slots = torch.zeros(rows, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    cfg = lia.AttentionConfig(g.hq, g.hkv, g.d, P, b.pool_pages, b.stride, g.q_dtype, g.kv_dtype,
                              g.out_dtype, g.scale, b.n_seqs, rows, int(b.ctx.max()))
    ws = torch.zeros(lia.workspace_bytes(cfg), dtype=torch.uint8, device=dev)
    context = b.stride * P

    def pack():
        lia.pack_plan_device(cfg, seq_slots, q_lens, cached, flat, rows, context, cu, positions,
                             sequences, slots, status, ws)

    def attend(i):
        t = pools[i]
        if fp8:
            lia.attention_partial_append_fp8(cfg, b.n_seqs, flat, slots, t["q"], t["newk"], t["newv"],
                                             t["kp"], t["vp"], ks, vs, t["out"], ws)
        else:
            lia.attention_partial_append(cfg, b.n_seqs, flat, slots, t["q"], t["newk"], t["newv"],
                                         t["kp"], t["vp"], t["out"], ws)

    def merge(i):
        lia.attention_merge(cfg, b.n_seqs, rows, pools[i]["out"], ws)

    def step(i):
        pack()
        attend(i)
        merge(i)

    def timed(body, n=reps):
        """Average time of body(i) over graphs of n calls on layers 0 .. n-1."""
        graph, stream = torch.cuda.CUDAGraph(), torch.cuda.Stream()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for i in range(n):
                    body(i)
        for _ in range(max(warmup, 1)):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream()
        e0.record(cur)
        for _ in range(steps):
            graph.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (steps * n)

    step(0)
    torch.cuda.synchronize()
    if status.item() != 0:
        raise RuntimeError(f"device packing failed: status {status.item()}")
    us = timed(step)
    # the attention launch alone, on the plan the steps left (the FP8 call includes its append
    # launch: the two launches of lia_attention_partial_append_fp8)
    kus = timed(attend)
    # the appended rows: read from the step's rows (bf16) and written to the pool
    append_bytes = rows * g.hkv * g.d * 2 * (2 + (1 if fp8 else 2))
    nbytes, flops = b.algorithmic_bytes() + append_bytes, b.flops()
    mfma = config == 3

    # the decode kernel's loads alone (lia_paged_read) on the same plan, against the attention
    # launch alone (on FP8 pools without its append launch)
    paged = None
    if not mfma:
        sink = torch.zeros(lia.paged_read_sink_words(cfg), dtype=torch.int32, device=dev)
        rus = timed(lambda i: lia.paged_read(cfg, b.n_seqs, flat, pools[i]["q"], pools[i]["kp"],
                                             pools[i]["vp"], sink, ws, ks, vs))
        aus = timed(lambda i: lia.attention_partial(cfg, b.n_seqs, flat, pools[i]["q"], pools[i]["kp"],
                                                    pools[i]["vp"], pools[i]["out"], ws, ks, vs)) \
            if fp8 else kus
        rbytes = b.algorithmic_bytes()
        paged = {"us": round(rus, 3), "GBps": round(rbytes / (rus * 1e-6) / 1e9, 1),
                 "frac_of_peak": round(rbytes / (rus * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
                 "attention_us": round(aus, 3), "kernel_frac_of_paged_read": round(rus / aus, 4)}

    # a model step: the batch's packing and plan once, then every layer over its own pool
    model = None
    if layers > 1:
        def model_step(_):
            pack()
            for i in range(layers):
                attend(i)
                merge(i)

        mus = timed(model_step, 1) / layers
        model = {"layers": layers, "step_us": round(mus * layers, 3), "per_layer_us": round(mus, 3)}
    del pools

    def roof(t_us):
        gbps, tflops = nbytes / (t_us * 1e-6) / 1e9, flops / (t_us * 1e-6) / 1e12
        r = {"bound": "mfma" if mfma else "hbm", "achieved": round(tflops if mfma else gbps, 1),
             "peak": PEAK_BF16_TFLOPS if mfma else PEAK_HBM_GBPS, "unit": "TFLOP/s" if mfma else "GB/s",
             "frac": round((tflops / PEAK_BF16_TFLOPS) if mfma else (gbps / PEAK_HBM_GBPS), 4)}
        if config == 4:  # MTP verify also reports its matrix-unit rate
            r["mfma_TFLOPs"] = round(tflops, 1)
            r["mfma_frac"] = round(tflops / PEAK_BF16_TFLOPS, 4)
        return r

    return {
        "metric": f"{SIDE_NAMES[config]}, us per layer (pack + plan + append + split attention + combine)",
        "workload": f"BASELINE config {config}" + (" on an FP8 pool" if kv == "fp8" and config != 5 else ""),
        "dtype": "fp8-e4m3 KV, bf16 Q" if fp8 else "bf16", "rows": rows, "sequences": b.n_seqs,
        "sum_ctx": int(b.ctx.sum()), "bytes_per_layer": nbytes, "flops_per_layer": flops,
        "step_us": round(us, 3), "step_roofline": roof(us),
        "kernel_us": round(kus, 3), "kernel_roofline": roof(kus),
        "paged_read_ceiling": paged,
        "model_step": dict(model, roofline=roof(model["per_layer_us"])) if model else None,
        "kernel": ("append_kernel + " if fp8 else "") +
                  ("wide_kernel (prefill)" if mfma else "attention_kernel (decode, fused append)"
                   if not fp8 else "attention_kernel (decode)"),
    }


def side_config(args):
    """bench.py --config 3|4|5: the side measurement of that configuration on its own JSON line."""
    r = side_measure(args.config, args.seed, args.steps, args.warmup, args.kernel_reps, args.kv)
    log(f"config {args.config}: step {r['step_us']:.2f} us, attention {r['kernel_us']:.2f} us")
    print(json.dumps({
        "metric": r["metric"], "value": r["step_us"], "unit": "us", "higher_is_better": False,
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "dtype": r["dtype"],
        "data": "synthetic (seeded, resident in HBM)",
        "config": {"workload": r["workload"], "rows": r["rows"], "sequences": r["sequences"],
                   "sum_ctx": r["sum_ctx"]},
        "roofline": dict(r["step_roofline"], bytes_per_layer=r["bytes_per_layer"],
                         flops_per_layer=r["flops_per_layer"]),
        "kernel": {"name": r["kernel"], "us": r["kernel_us"], "roofline": r["kernel_roofline"]},
    }), flush=True)


def read_ceiling(lia, layer_bytes, L, reps):
    """The contiguous-read ceiling on this device: lia_hbm_read of layer_bytes, timed exactly
    as the attention kernel is (a graph of L back-to-back launches, replayed `reps` times, HIP
    events on the replaying stream), over rotating buffers totalling >= 1 GiB so the 256 MB
    last-level cache cannot serve them.  The best of three grid sizes; plus the rate of 1 GiB
    reads."""
    import torch
    cus = lia.lib().lia_device_cus() or 256

    def timed(nbytes, nbuf, wgs):
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
        sink = torch.empty(wgs, dtype=torch.int32, device="cuda")
        graph, stream = torch.cuda.CUDAGraph(), torch.cuda.Stream()
        with torch.cuda.stream(stream):
            lia.hbm_read(bufs[0], wgs, sink, stream=stream)
            with torch.cuda.graph(graph, stream=stream):
                for i in range(L):
                    lia.hbm_read(bufs[i % nbuf], wgs, sink, stream=stream)
        torch.cuda.synchronize()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream()
        e0.record(cur)
        for _ in range(reps):
            graph.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        del bufs
        return e0.elapsed_time(e1) * 1e3 / (reps * L)

    nbuf = max(4, -(-(1 << 30) // layer_bytes))
    runs = {wgs: timed(layer_bytes, nbuf, wgs) for wgs in (2 * cus, 4 * cus, 8 * cus)}
    wgs, us = min(runs.items(), key=lambda kv: kv[1])
    us_1g = min(timed(1 << 30, 3, w) for w in (4 * cus, 8 * cus))
    torch.cuda.empty_cache()
    gbps = layer_bytes / (us * 1e-6) / 1e9
    return {"bytes": layer_bytes, "us": round(us, 3), "GBps": round(gbps, 1),
            "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4), "workgroups": wgs,
            "us_by_workgroups": {str(k): round(v, 3) for k, v in runs.items()},
            "GBps_1GiB": round((1 << 30) / (us_1g * 1e-6) / 1e9, 1),
            "kernel": "hbm_read_kernel (lia_hbm_read: contiguous, 16-byte non-temporal loads)"}


def host_cpus():
    """The host's CPU count as this process sees it (its affinity set: the cores the job may
    run on), the machine's count, the OpenMP thread setting of the environment and the model."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": len(os.sched_getaffinity(0)), "machine_cpus": os.cpu_count(),
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model}


def cpu_baseline(args, b, g, kpool, vpool, q, layer_bytes, L):
    """The oracle's scalar split-K + merge (kernels/llama.rs:63-159, 201-290) on one layer of
    the batch, compiled here at -O3 -march=native with OpenMP over (row, head, split): one
    warm-up run, then at least 5 timed runs (more until args.cpu_seconds), median reported."""
    import tempfile
    import torch
    from oracle import build as OB
    from oracle import oracle as O
    path = OB.build_baseline(os.path.join(tempfile.mkdtemp(prefix="lia_cpu_"), "baseline.so"))
    blib = O.baseline_lib(path)
    kc = kpool.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    vc = vpool.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    q32 = q.float().cpu().numpy()
    geom = O.geom(g.hq, g.hkv, g.d, g.page_size, b.stride, g.kv_dtype, g.scale)
    pos_h, seq_h, flat_h = b.positions(), b.sequences(), b.flat_table()
    run = lambda: O.paged_attention_f32(geom, pos_h, seq_h, flat_h, q32, kc, vc, span=256, lib_=blib)
    run()  # warm-up
    times, t_start = [], time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 4 * L):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    per_layer = float(np.median(times))
    threads = int(blib.lo_omp_threads())
    return {"value": round(b.n_rows / (per_layer * L), 4), "unit": "tokens/s",
            "cores": threads, "kind": "port", **host_cpus(),
            "sample": f"median of {len(times)} runs (after 1 warm-up) of one layer of the config-2 "
                      f"batch (8 rows, sum ctx {int(b.ctx.sum())}) in f32 split-K (span 256) + merge, "
                      f"gcc -O3 -march=native, OpenMP {threads} threads, scaled to {L} layers; "
                      f"{per_layer * 1e3:.1f} ms/layer, {layer_bytes / per_layer / 1e9:.2f} GB/s"}


def main():
    args = parse()
    if args.config != 2:
        side_config(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path shards by sequence / KV "
              "head with no cross-GPU exchange); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from __graft_entry__ import package
    lia = package()
    import lia_rs_amd.workloads as wl

    torch.cuda.set_device(0)
    dev = "cuda"
    b = wl.config2(seed=args.seed, layers=args.layers)
    g = b.geom
    L = args.layers
    P = g.page_size
    tokens = b.pool_pages * P
    log(f"config2: ctx={b.ctx.tolist()} sum={int(b.ctx.sum())} pool_pages={b.pool_pages} "
        f"layers={L}; {b.notes}")

    # ---- resident inputs: per-layer KV pools, queries and this step's new K/V rows
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    kpool, vpool, qs, newk, newv = [], [], [], [], []
    for layer in range(L):
        kpool.append(torch.randn((tokens, g.hkv, g.d), generator=gen, device=dev).to(torch.bfloat16))
        vpool.append(torch.randn((tokens, g.hkv, g.d), generator=gen, device=dev).to(torch.bfloat16))
        qs.append(torch.randn((b.n_rows, g.hq, g.d), generator=gen, device=dev).to(torch.bfloat16))
        newk.append(torch.randn((b.n_rows, g.hkv * g.d), generator=gen, device=dev).to(torch.bfloat16))
        newv.append(torch.randn((b.n_rows, g.hkv * g.d), generator=gen, device=dev).to(torch.bfloat16))
    outs = [torch.empty((b.n_rows, g.hq, g.d), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    i32 = lambda a: torch.from_numpy(np.asarray(a, np.uint32).view(np.int32)).to(dev)
    seq_slots, q_lens, cached = i32(np.arange(b.n_seqs)), i32(b.q_len), i32(b.cached)
    flat = i32(b.flat_table())
    rows = b.n_rows
    cu = torch.zeros(b.n_seqs + 1, dtype=torch.int32, device=dev)
    positions = torch.zeros(rows, dtype=torch.int32, device=dev)
    sequences = torch.zeros(rows, dtype=torch.int32, device=dev)
    slots = torch.zeros(rows, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    cfg = lia.AttentionConfig(g.hq, g.hkv, g.d, P, b.pool_pages, b.stride, g.q_dtype, g.kv_dtype,
                              g.out_dtype, g.scale, b.n_seqs, rows, int(b.ctx.max()))
    ws = torch.zeros(lia.workspace_bytes(cfg), dtype=torch.uint8, device=dev)
    context = b.stride * P
    torch.cuda.synchronize()

    def step():
        lia.pack_plan_device(cfg, seq_slots, q_lens, cached, flat, rows, context, cu, positions,
                             sequences, slots, status, ws)
        for layer in range(L):
            lia.attention_partial_append(cfg, b.n_seqs, flat, slots, qs[layer], newk[layer],
                                         newv[layer], kpool[layer], vpool[layer], outs[layer], ws)
            lia.attention_merge(cfg, b.n_seqs, rows, outs[layer], ws)

    # eager step once (validates arguments, checks the packing status)
    step()
    torch.cuda.synchronize()
    if status.item() != 0:
        raise RuntimeError(f"device packing failed: status {status.item()}")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    # ---- timed region: K graph replays of the whole step
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(stop) / args.steps
    log(f"step: {ms_step:.4f} ms (wall {wall * 1e3 / args.steps:.4f} ms)")

    # ---- dominant kernel alone: one graph of L fused append + split-attention launches
    kgraph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(kgraph, stream=stream):
            for layer in range(L):
                lia.attention_partial_append(cfg, b.n_seqs, flat, slots, qs[layer], newk[layer],
                                             newv[layer], kpool[layer], vpool[layer],
                                             outs[layer], ws)
    torch.cuda.synchronize()
    for _ in range(3):
        kgraph.replay()
    torch.cuda.synchronize()
    ks, ke = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    ks.record(cur)
    for _ in range(args.kernel_reps):
        kgraph.replay()
    ke.record(cur)
    torch.cuda.synchronize()
    kernel_us = ks.elapsed_time(ke) * 1e3 / (args.kernel_reps * L)
    # attended K/V (the new keys read from the step's rows) + Q + O + table, plus the
    # appended K/V rows the fused launch writes into the pool
    layer_bytes = b.algorithmic_bytes() + rows * g.hkv * g.d * 2 * 2
    achieved = layer_bytes / (kernel_us * 1e-6) / 1e9
    step_bytes = layer_bytes * L
    step_gbps = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"attention kernel: {kernel_us:.2f} us/launch, {achieved:.1f} GB/s "
        f"({achieved / PEAK_HBM_GBPS:.1%} of peak), layer bytes {layer_bytes}")

    # ---- the kernel's own loads without its arithmetic (lia_paged_read: same plan, ranges,
    # loads and pipeline waits), timed the same way: the ceiling of its access pattern
    sink = torch.zeros(lia.paged_read_sink_words(cfg), dtype=torch.int32, device=dev)
    rgraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(rgraph, stream=stream):
            for layer in range(L):
                lia.paged_read(cfg, b.n_seqs, flat, qs[layer], kpool[layer], vpool[layer], sink, ws,
                               stream=stream)
    torch.cuda.synchronize()
    for _ in range(3):
        rgraph.replay()
    torch.cuda.synchronize()
    ks.record(cur)
    for _ in range(args.kernel_reps):
        rgraph.replay()
    ke.record(cur)
    torch.cuda.synchronize()
    read_us = ks.elapsed_time(ke) * 1e3 / (args.kernel_reps * L)
    read_gbps = layer_bytes / (read_us * 1e-6) / 1e9
    paged = {"us": round(read_us, 3), "GBps": round(read_gbps, 1),
             "frac_of_peak": round(read_gbps / PEAK_HBM_GBPS, 4),
             "kernel_frac_of_paged_read": round(read_us / kernel_us, 4),
             "kernel": "attention_kernel<128,1,bf16> read-only variant (lia_paged_read: the "
                       "kernel's plan, loads and pipeline waits, no attention arithmetic)"}
    log(f"paged read (the kernel's loads alone): {read_us:.2f} us/launch, {read_gbps:.1f} GB/s "
        f"({read_gbps / PEAK_HBM_GBPS:.1%} of peak); attention kernel at {read_us / kernel_us:.1%} of it")

    # ---- the same bytes read contiguously on this device: the ceiling the kernel is held to
    ceiling = read_ceiling(lia, layer_bytes, L, args.kernel_reps)
    log(f"contiguous read of {layer_bytes} B: {ceiling['us']:.2f} us/launch, {ceiling['GBps']:.1f} GB/s "
        f"({ceiling['frac_of_peak']:.1%} of peak; 1 GiB reads {ceiling['GBps_1GiB']:.1f} GB/s); "
        f"attention kernel at {achieved / ceiling['GBps']:.1%} of it")

    # ---- the reference algorithm on the host cores (bounded sample, one layer repeated)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, b, g, kpool[0], vpool[0], qs[0], layer_bytes, L)
        log(f"cpu baseline: {cpu}")

    # ---- one-layer steps of configs 3, 4 and 5 (parity workloads, timed for the record)
    side = {}
    if not args.no_side:
        del kpool, vpool, qs, newk, newv
        torch.cuda.empty_cache()
        for c in (3, 4, 5):
            side["config%d" % c] = side_measure(c, args.seed, args.side_steps, 3, 10)
            torch.cuda.empty_cache()
            log(f"config {c}: step {side['config%d' % c]['step_us']:.2f} us, attention "
                f"{side['config%d' % c]['kernel_us']:.2f} us")

    out = {
        "metric": METRIC,
        "value": round(b.n_rows / (ms_step * 1e-3), 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/Q, random-permutation block tables)",
        "config": {
            "workload": "BASELINE config 2: ragged bf16 paged decode, batch 8, ctx U[1024,32768] "
                        "seed %d, 16q/2kv heads, head_dim 128, page 16, %d layers as independent "
                        "KV slices; step = device pack and plan (two launches) + per layer (split attention "
                        "with the KV append fused in + combine), HIP-graph replay" % (args.seed, L),
            "batch": b.n_seqs, "layers": L, "ctx": b.ctx.tolist(), "sum_ctx": int(b.ctx.sum()),
            "page_size": P, "pool_pages": b.pool_pages,
            "step_hbm_GBps": round(step_gbps, 1),
            "step_hbm_frac": round(step_gbps / PEAK_HBM_GBPS, 4),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": load_traffic(args.traffic, kernel_us, layer_bytes),
            "kernel": "attention_kernel<128,1,bf16> (fused append)", "kernel_us": round(kernel_us, 3),
            "bytes_per_launch": layer_bytes,
            "read_ceiling": dict(ceiling, kernel_frac_of_ceiling=round(achieved / ceiling["GBps"], 4)),
            "paged_read_ceiling": paged,
        },
        "cpu_baseline": cpu,
        "side": side or None,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
