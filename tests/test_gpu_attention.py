"""GPU parity of lia_paged_attention against the CPU oracle (through the C ABI).

Tolerances: bf16 / f16 KV max-abs 2e-2 and mean-abs 2e-3, FP8 KV max-abs 5e-2, against
the float64 softmax of the stored (rounded) K/V - the reference's own oracle form
(src/gpu/llama_attention.rs:253-284).  The f16 reference-format case also reports its
error against the reference's 3e-5 bar for its f16 tensor-core kernels."""
import numpy as np
import pytest
import torch

import gpu_data as G
from gpu_data import BF16, F16, F32, FP8

pytestmark = pytest.mark.gpu

TOL = {BF16: (2e-2, 2e-3), F16: (2e-2, 2e-3), FP8: (5e-2, 5e-3)}


def _check(case, lia, label):
    print(f"[case] {label}: seqs={case.batch.n_seqs} rows={case.batch.n_rows} "
          f"ctx={case.batch.ctx.tolist()[:8]} q_len={case.batch.q_len.tolist()[:8]}", flush=True)
    got = case.run(lia)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] {label}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)), label
    tol_max, tol_mean = TOL[case.g.kv_dtype]
    assert mx < tol_max and mean < tol_mean, (label, mx, mean)
    return got, ref


def test_config1_plumbing_vs_reference_cpu_path(lia, wl, O):
    b = wl.config1(seed=0)
    case = G.Case(b, seed=0)
    got, ref = _check(case, lia, "cfg1")
    # the scalar split-K CPU path (the reference algorithm in f32) agrees too
    cpu = O.paged_attention_f32(case.oracle_geom(), case.positions, case.sequences, case.flat,
                                case.q32, case.kc, case.vc, span=32)
    assert np.max(np.abs(cpu - ref)) < 1e-5
    assert np.max(np.abs(got - cpu)) < 2e-2


@pytest.mark.parametrize("kv", [BF16, F16, FP8])
@pytest.mark.parametrize("qo", [(BF16, BF16), (F32, F32)])
@pytest.mark.parametrize("d,hq,hkv,page", [(128, 16, 2, 16), (64, 8, 2, 16), (128, 16, 2, 32)])
def test_decode_edge_contexts(lia, wl, kv, qo, d, hq, hkv, page):
    ctx = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 511, 1000, 2049, 4097]
    g = wl.Geometry(hq=hq, hkv=hkv, d=d, page_size=page, kv_dtype=kv, q_dtype=qo[0],
                    out_dtype=qo[1])
    b = wl.custom(ctx, [1] * len(ctx), geom=g, seed=3)
    _check(G.Case(b, seed=3), lia, f"edge kv={kv} q/o={qo} d={d} page={page}")


def test_reference_known_answer_vectors(lia, wl):
    """Inputs of the reference's f64 attention test (src/gpu/llama_attention.rs:212-252):
    f16 KV in 32-token pages with reversed tables, f32 queries and outputs."""
    from test_oracle import _reference_vectors
    stride, pos, seq, tables, keys, vals, q, _ = _reference_vectors()
    g = wl.Geometry(hq=16, hkv=2, d=128, page_size=32, kv_dtype=F16, q_dtype=F32, out_dtype=F32)
    # rows are grouped by sequence with consecutive positions: 3 groups
    ctx = np.array([4098, 16385, 8192])
    b = wl.Batch(g, ctx, np.array([8, 8, 1]), pool_pages=2 * stride, tables=[], stride=stride)
    case = G.Case.__new__(G.Case)
    case.batch, case.g = b, g
    case.kc = keys.astype(np.float16).view(np.uint16).reshape(-1)
    case.vc = vals.astype(np.float16).view(np.uint16).reshape(-1)
    case.k_scales = case.v_scales = None
    case.q_store = case.q32 = q
    case.positions, case.sequences = pos, seq
    case.cu = np.array([0, 8, 16, 17], np.uint32)
    case.flat = tables
    got = case.run(lia)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] reference vectors: max_abs={mx:.3e} mean_abs={mean:.3e} (reference bar 3e-5)",
          flush=True)
    assert mx < 3e-5 and mean < 1e-5  # the reference's own bar (llama_attention.rs:393)


def test_mtp_verify_rows(lia, wl):
    rng = np.random.default_rng(4)
    k = rng.integers(1, 4, size=12)
    ctx = rng.integers(20, 3000, size=12)
    b = wl.custom(ctx, 1 + k, seed=4)
    _check(G.Case(b, seed=4), lia, "mtp")


def test_mixed_prefill_and_decode(lia, wl):
    ctx = [64, 300 + 130, 1000 + 200, 777, 1500, 33]
    q = [64, 130, 200, 1, 1, 1]
    b = wl.custom(ctx, q, seed=5)
    _check(G.Case(b, seed=5), lia, "mixed")


@pytest.mark.parametrize("kv", [BF16, FP8])
def test_prefill_group_sizes(lia, wl, kv):
    for hq, hkv in [(16, 2), (8, 8), (32, 2), (16, 1)]:
        g = wl.Geometry(hq=hq, hkv=hkv, d=128, kv_dtype=kv)
        b = wl.custom([40, 700], [40, 9], geom=g, seed=6)
        _check(G.Case(b, seed=6), lia, f"groups hq={hq} hkv={hkv} kv={kv}")


@pytest.mark.parametrize("hq,hkv", [(6, 2), (10, 2)])
def test_odd_group_sizes(lia, wl, hq, hkv):
    """GQA groups of 3 and 5: rows per column block (16 NT / group, 128 / group on the prefill
    kernel) are not powers of two, so the plan's block offsets take the general floor-sum.
    Decode rows, MTP-like rows and prefill chunks with prefixes."""
    g = wl.Geometry(hq=hq, hkv=hkv, d=128)
    for ctx, q, name in [([17, 300, 2049, 64], [1, 1, 1, 1], "decode"),
                         ([40, 700, 1500], [3, 2, 4], "mtp"),
                         ([300, 1077, 40, 513], [300, 77, 40, 33], "prefill")]:
        b = wl.custom(ctx, q, geom=g, seed=13)
        _check(G.Case(b, seed=13), lia, f"group {hq // hkv} {name}")


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("rows", ["decode", "mtp"])
def test_batch_sizes_reversed_tables(lia, wl, n, rows):
    """The reference's small-batch and long-context checks (tests/minicpm5.rs:248-288,
    tests/minicpm5_long_context.rs:5-97): batches of 1-5 and 8 sequences with contexts up to
    16k, their block tables handed out from the top of the pool downward and each sequence's
    pages in reverse logical order (as the reference's reversed tables, llama_attention.rs:
    222-236); one new row per sequence, or 2-4 verify rows."""
    ctx = np.array([16384, 3000, 777, 12000, 48, 9000, 1, 5000][:n], np.int64)
    q = np.ones(n, np.int64) if rows == "decode" else np.array([2, 4, 3, 2, 4, 3, 1, 2][:n], np.int64)
    ctx = np.maximum(ctx, q)
    g = wl.Geometry()
    P = g.page_size
    need = [-(-int(c) // P) for c in ctx]
    pool = sum(need) + 3
    tables, top = [], pool
    for k in need:
        tables.append(np.arange(top - k, top, dtype=np.uint32)[::-1].copy())
        top -= k
    b = wl.Batch(g, ctx, q, pool, tables, stride=max(need))
    _check(G.Case(b, seed=70 + n), lia, f"batch {n} {rows} reversed tables")


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_config2_full_size_one_layer(lia, wl, seed):
    """North-star shape: batch 8, contexts U[1k, 32k], one layer against the oracle; seeds
    other than the bench's draw other contexts and page tables."""
    b = wl.config2(seed=seed, layers=1)
    _check(G.Case(b, seed=seed), lia, f"cfg2 layer seed {seed}")


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config4_mtp_full_size(lia, wl, seed):
    b = wl.config4(seed=seed)
    _check(G.Case(b, seed=seed), lia, f"cfg4 seed {seed}")


def test_config5_fp8_long_contexts(lia, wl):
    """The FP8 decode workload of BASELINE config 5 on its first 8 sequences (contexts from
    its log-uniform [1k, 128k] draw; the full 64-sequence pool takes a minute to build on the
    host): e4m3 pages with per-page scales, long contexts split over many workgroups."""
    full = wl.config5(seed=0)
    ctx = [int(c) for c in full.ctx[:8]]
    b = wl.custom(ctx, [1] * len(ctx), geom=wl.Geometry(kv_dtype=FP8), seed=11)
    _check(G.Case(b, seed=11), lia, f"cfg5 first 8 (sum ctx {sum(ctx)})")


def test_config5_fp8_full_size(lia, wl):
    """BASELINE config 5 at full size: 64 sequences, contexts log-uniform in [1k, 128k]
    (1.68M keys), e4m3 pools drawn as codes with per-(page, head) scales."""
    b = wl.config5(seed=0)
    print(f"[case] cfg5 full: building {int(b.ctx.sum())} keys", flush=True)
    got, ref = _check(G.Case(b, seed=0, fill="fp8_codes"), lia, "cfg5 full")
    # outputs of these pools are small (|out| < 0.2): hold them to 1 % of that as well
    assert np.max(np.abs(got - ref)) < 2e-3


@pytest.mark.parametrize("q_len", [[1, 0, 3, 0, 1], [0, 0, 200, 0, 1], [0, 1, 0, 0, 0],
                                   [3, 0, 4, 0, 2]])
def test_sequences_without_rows(lia, wl, q_len):
    """Sequences that add no rows this step (repeated cu_seqlens entries) next to decode, MTP
    and prefill rows: device packing equals the host packing and attention the oracle."""
    ctx = [500, 300, 1000 + 200, 64, 4097]
    b = wl.custom(ctx, q_len, seed=21)
    case = G.Case(b, seed=21)
    print(f"[case] sequences without rows q_len={q_len}", flush=True)
    n, rows, P = b.n_seqs, b.n_rows, b.geom.page_size
    dev = {k: torch.full((rows + (k == "cu"),), -7, dtype=torch.int32, device="cuda")
           for k in ("cu", "positions", "sequences", "slots")}
    dev["cu"] = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    status = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    lia.pack_device(G.u32_dev(np.arange(n)), G.u32_dev(b.q_len), G.u32_dev(b.cached),
                    G.u32_dev(b.flat_table()), b.stride, P, b.pool_pages, b.stride * P, rows,
                    dev["cu"], dev["positions"], dev["sequences"], dev["slots"], status)
    torch.cuda.synchronize()
    assert status.item() == 0
    got = {k: v.cpu().numpy().view(np.uint32) for k, v in dev.items()}
    assert np.array_equal(got["cu"], b.cu_seqlens())
    assert np.array_equal(got["positions"], b.positions())
    assert np.array_equal(got["sequences"], b.sequences())
    assert np.array_equal(got["slots"], b.slot_mapping())
    _check(case, lia, f"no-row sequences {q_len}")


@pytest.mark.parametrize("kv", [BF16, FP8])
@pytest.mark.parametrize("page", [64, 128])
def test_large_pages(lia, wl, kv, page):
    """Pages of 64 and 128 tokens (a 32-token chunk inside one page): decode and MTP rows with
    contexts around page and chunk edges, then prefill chunks with prefixes."""
    g = wl.Geometry(kv_dtype=kv, page_size=page)
    b = wl.custom([1, 63, 64, 65, 700, 4100], [1, 1, 2, 3, 1, 1], geom=g, seed=23)
    _check(G.Case(b, seed=23), lia, f"pages of {page} kv={kv} decode/MTP")
    b = wl.custom([300, 1000 + 77, 129], [300, 77, 129], geom=g, seed=24)
    _check(G.Case(b, seed=24), lia, f"pages of {page} kv={kv} prefill")


@pytest.mark.parametrize("hq,hkv", [(32, 1), (24, 1), (64, 2), (16, 16), (16, 8), (32, 16)])
def test_group_extremes(lia, wl, hq, hkv):
    """GQA groups of 24 and 32 (the largest accepted: two 16-column tiles hold one row, or
    128 / group rows in a prefill unit) and of 1 and 2 (8 and 16 KV heads: 8-16 rows per tile)."""
    g = wl.Geometry(hq=hq, hkv=hkv, d=128)
    b = wl.custom([1, 17, 700, 4100], [1, 1, 3, 1], geom=g, seed=25)
    _check(G.Case(b, seed=25), lia, f"group {hq // hkv} decode/MTP")
    b = wl.custom([300, 1000 + 77], [300, 77], geom=g, seed=26)
    _check(G.Case(b, seed=26), lia, f"group {hq // hkv} prefill")


@pytest.mark.parametrize("kv", [BF16, FP8])
def test_maximum_context(lia, wl, kv):
    """The reference's longest request (131,072 tokens, models/minicpm5.rs:15) decoding next to
    a 4-row MTP sequence ending at the same length, plus a short one."""
    g = wl.Geometry(kv_dtype=kv)
    b = wl.custom([131072, 131072, 33], [1, 4, 1], geom=g, seed=27)
    print(f"[case] maximum context kv={kv}", flush=True)
    _check(G.Case(b, seed=27), lia, f"context 131072 kv={kv}")


def test_capacity_does_not_change_results(lia, wl):
    """A configuration sized for far more rows and sequences than the batch (a larger
    workspace, more unit and record slots) gives bit-identical outputs."""
    b = wl.custom([5000, 17, 900, 64, 300], [1, 1, 3, 64, 0], seed=28)
    case = G.Case(b, seed=28)
    dev = case.device()
    g = b.geom
    outs = []
    for max_seqs, max_rows in ((b.n_seqs, b.n_rows), (64, 4096)):
        cfg = lia.AttentionConfig(g.hq, g.hkv, g.d, g.page_size, b.pool_pages, b.stride, g.q_dtype,
                                  g.kv_dtype, g.out_dtype, g.scale, max_seqs, max_rows, int(b.ctx.max()))
        ws = G.dirty_workspace(lia, cfg)
        out = torch.full((b.n_rows, g.hq, g.d), float("nan"), dtype=torch.bfloat16, device="cuda")
        lia.paged_attention(cfg, b.n_seqs, dev["cu"], dev["positions"], dev["sequences"], dev["pages"],
                            dev["q"], dev["kc"], dev["vc"], out, ws)
        torch.cuda.synchronize()
        outs.append(out.view(torch.int16).cpu().numpy())
    print("[case] capacity", flush=True)
    assert np.array_equal(outs[0], outs[1])
    got = torch.from_numpy(outs[1]).view(torch.bfloat16).float().numpy()
    mx, mean = G.errors(got, case.f64())
    assert mx < 2e-2 and mean < 2e-3


@pytest.mark.parametrize("rows_kind", ["decode", "mixed"])
def test_many_sequences(lia, wl, rows_kind):
    """1,500 sequences: more than the 1,024 the plan keeps in LDS (its general path) and than
    one packing workgroup covers; decode only, and mixed with sequences adding 0 or 3 rows."""
    rng = np.random.default_rng(29)
    n = 1500
    q = np.ones(n, np.int64) if rows_kind == "decode" else rng.choice([0, 1, 1, 3], n)
    ctx = rng.integers(1, 300, n) + q
    b = wl.custom(ctx, q, seed=29)
    print(f"[case] many sequences {rows_kind}: rows {b.n_rows}", flush=True)
    P = b.geom.page_size
    dev = {k: torch.full((b.n_rows,), -7, dtype=torch.int32, device="cuda")
           for k in ("positions", "sequences", "slots")}
    dev["cu"] = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    status = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    lia.pack_device(G.u32_dev(np.arange(n)), G.u32_dev(b.q_len), G.u32_dev(b.cached),
                    G.u32_dev(b.flat_table()), b.stride, P, b.pool_pages, b.stride * P, b.n_rows,
                    dev["cu"], dev["positions"], dev["sequences"], dev["slots"], status)
    torch.cuda.synchronize()
    assert status.item() == 0
    got = {k: v.cpu().numpy().view(np.uint32) for k, v in dev.items()}
    assert np.array_equal(got["cu"], b.cu_seqlens())
    assert np.array_equal(got["positions"], b.positions())
    assert np.array_equal(got["sequences"], b.sequences())
    assert np.array_equal(got["slots"], b.slot_mapping())
    _check(G.Case(b, seed=29), lia, f"many sequences {rows_kind}")


@pytest.mark.parametrize("kv", [BF16, F16, FP8])
def test_prefill_few_units_long_prefix(lia, wl, kv):
    """A short chunk after a long prefix on the prefill kernel: one or two 128-column units per
    KV head take every workgroup, so each unit leaves hundreds of split records and the
    combine runs many record batches."""
    g = wl.Geometry(kv_dtype=kv)
    for ctx, q, seed in (([65536 + 32], [32], 30), ([30000 + 16, 20000 + 40], [16, 40], 31)):
        got, ref = _check(G.Case(wl.custom(ctx, q, geom=g, seed=seed), seed=seed), lia,
                          f"chunks {q} after {ctx} kv={kv}")
        # averages over tens of thousands of keys are small: also within 2 % of their scale
        scale = float(np.max(np.abs(ref)))
        print(f"[case] max |ref| {scale:.3e}", flush=True)
        assert np.max(np.abs(got - ref)) < 2e-2 * scale


@pytest.mark.parametrize("d,q", [(128, 4), (64, 2), (128, 1)])
def test_single_sequence_small_merge(lia, wl, d, q):
    """One long sequence verifying a few draft rows (or decoding): the merge grid is small, so
    each record row is merged by two workgroups, on the two-tile and the one-tile path."""
    g = wl.Geometry(d=d, hq=16 if d == 128 else 8)
    b = wl.custom([20000 + q], [q], geom=g, seed=32)
    _check(G.Case(b, seed=32), lia, f"single sequence d={d} rows={q}")


def test_prefill_weighted_ranges_in_launch_order(lia, wl):
    """A 64-row chunk after 1,536 cached keys: 8 prefill units of about 50 blocks each, about 400
    blocks in all.  That is fewer blocks than the launch's prefill workgroups (two per CU), so
    ranges run on workgroups in launch order rather than XCD-major, and more ranges than CUs, so
    the ranges of workgroups past the first dispatch round get the plan's smaller weight."""
    b = wl.custom([1536 + 64], [64], seed=33)
    case = G.Case(b, seed=33)
    _check(case, lia, "weighted ranges in launch order")
    units, blocks, ranges, overflow = case.last_ws[:16].view(torch.int32).cpu().tolist()
    cus = lia.lib().lia_device_cus()
    print(f"[case] units={units} blocks={blocks} ranges={ranges} cus={cus}", flush=True)
    assert overflow == 0 and units == 8 and ranges == blocks
    assert cus < ranges < 2 * cus


@pytest.mark.parametrize("prefix", [8200, 9000, 9100])
def test_prefill_xcd_major_at_the_weight_boundary(lia, wl, prefix):
    """A 16-row chunk after `prefix` cached keys: 2 prefill units of 258-286 blocks, so the plan
    has as many ranges as the launch's prefill workgroups (XCD-major ranges) and a total cost
    (blocks plus the units' start charges) of 532, 582 or 588.  The dispatch-round weights need
    588 here for every range to keep a block: below it the plan uses equal shares, at 588 the
    weighted ranges are just over one block wide.  The workspace starts dirty, so a range left
    without blocks inside a unit would show in the output."""
    b = wl.custom([prefix + 16], [16], seed=34)
    case = G.Case(b, seed=34)
    _check(case, lia, f"prefill 16 rows after {prefix} keys")
    units, blocks, ranges, overflow = case.last_ws[:16].view(torch.int32).cpu().tolist()
    print(f"[case] units={units} blocks={blocks} ranges={ranges}", flush=True)
    assert overflow == 0 and units == 2 and blocks >= ranges == 512


def test_repeat_calls_are_identical(lia, wl):
    b = wl.custom([5000, 17, 900], [1, 1, 3], seed=8)
    case = G.Case(b, seed=8)
    dev = case.device()
    a = case.run(lia, dev)
    c = case.run(lia, dev)
    assert np.array_equal(a, c)


def test_config3_mixed_prefill_full_size(lia, wl):
    """BASELINE config 3 at full size: chunks (512, 0), (1024, 4096), (2048, 8192) and five
    decode rows in one batch (the prefill kernel's 128-column units)."""
    _check(G.Case(wl.config3(seed=0), seed=0), lia, "cfg3")


def test_prefill_bf16_values_beyond_f16_range(lia, wl):
    """A bf16 pool with |V| around 2e5 (beyond f16's 65504) through the prefill kernel's split
    records and their combine: the records keep the pool's type, so nothing overflows."""
    b = wl.custom([300, 1000 + 77, 2000 + 40], [300, 77, 40], seed=12)
    case = G.Case(b, seed=12, v_scale=2e5)
    print("[case] prefill bf16 |V| ~ 2e5", flush=True)
    got = case.run(lia)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] prefill bf16 |V| ~ 2e5: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got))
    assert mx < 2e-2 * 2e5 and mean < 2e-3 * 2e5


@pytest.mark.parametrize("kv,d,page", [(F16, 128, 32), (BF16, 64, 16), (FP8, 128, 16),
                                       (FP8, 128, 32), (FP8, 64, 16)])
def test_prefill_kernel_geometries(lia, wl, kv, d, page):
    """Prefill units of 128 columns over other page sizes, head_dim 64, f16 and FP8 pools, with
    chunks that are not multiples of the unit's rows and prefixes not page-aligned."""
    g = wl.Geometry(hq=16, hkv=2, d=d, page_size=page, kv_dtype=kv, q_dtype=F32, out_dtype=F32)
    b = wl.custom([300, 1000 + 77, 40, 513], [300, 77, 40, 33], geom=g, seed=9)
    _check(G.Case(b, seed=9), lia, f"prefill kv={kv} d={d} page={page}")


@pytest.mark.parametrize("kv", [BF16, F16])
def test_f32_output_split_records_keep_f32_precision(lia, wl, O, kv):
    """Long contexts split over many workgroups, f32 queries and outputs: the split records
    are f32 (no 16-bit rounding of partial rows), so the error against the float64 oracle
    stays at the level of the kernel's 16-bit MFMA operands, and the same batch with bf16
    output (16-bit records) is no closer than that."""
    g = wl.Geometry(hq=16, hkv=2, d=128, kv_dtype=kv, q_dtype=F32, out_dtype=F32)
    b = wl.custom([30000, 12000, 4096], [1, 1, 1], geom=g, seed=51)
    case = G.Case(b, seed=51)
    got = case.run(lia)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    cpu = O.paged_attention_f32(case.oracle_geom(), case.positions, case.sequences, case.flat,
                                case.q32, case.kc, case.vc, span=256)
    cmx, _ = G.errors(cpu, ref)
    print(f"[case] f32 out split kv={kv}: max_abs={mx:.3e} mean_abs={mean:.3e} "
          f"(oracle f32 split-K {cmx:.3e})", flush=True)
    # measured 2.2e-4 (bf16 pool) and 3.0e-5 (f16 pool): the 16-bit MFMA operands, not the
    # records, set the error
    assert mx < (5e-4 if kv == BF16 else 1e-4) and mean < (1e-4 if kv == BF16 else 1e-5)


@pytest.mark.parametrize("d,out", [(128, F32), (128, BF16), (64, F32)])
def test_merge_one_column_per_wave(lia, wl, d, out):
    """Many decode sequences (about six split records per unit: the combine merges one column
    per wave) with one 100k-token context among them, whose units hold far more records than
    one pass of a wave covers.  f32 outputs keep f32 records; over these 131k outputs their
    error is that of the kernel's 16-bit MFMA operands (measured 1.2e-3 max, 8.3e-5 mean, the
    same with the workgroup-per-column merge); bf16 outputs are held to the usual bar."""
    rng = np.random.default_rng(61)
    ctx = np.concatenate([rng.integers(200, 3000, 63), [100000]])
    g = wl.Geometry(hq=16 if d == 128 else 8, hkv=2, d=d, kv_dtype=BF16, q_dtype=out, out_dtype=out)
    b = wl.custom(ctx, np.ones(64, np.int64), geom=g, seed=61)
    case = G.Case(b, seed=61)
    got, ref = _check(case, lia, f"wave-per-column merge d={d} out={out}")
    if out == F32:
        mx, mean = G.errors(got, ref)
        assert mx < 2e-3 and mean < 1e-4, (mx, mean)


def test_f16_split_records_saturate_at_the_f16_maximum(lia, wl):
    """An f16 pool whose V values sit at +-65504 over units split across workgroups, bf16
    output (f16 records): a record row may exceed max |V| by a rounding step; it saturates
    instead of becoming infinite, so the merged output stays finite and within tolerance."""
    g = wl.Geometry(hq=16, hkv=2, d=128, kv_dtype=F16, q_dtype=BF16, out_dtype=BF16)
    b = wl.custom([20000, 9000], [1, 1], geom=g, seed=52)
    case = G.Case(b, seed=52)
    v = np.where(np.random.default_rng(52).random(case.vc.size) < 0.5, 65504.0, -65504.0)
    case.vc = v.astype(np.float16).view(np.uint16)
    got = case.run(lia)
    ref = case.f64()
    mx, mean = G.errors(got, ref)
    print(f"[case] f16 V at +-65504: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got))
    assert mx < 2e-2 * 65504 and mean < 2e-3 * 65504


def test_fp8_decode_large_v_scales(lia, wl):
    """FP8 pool with V page scales of about 1-4 (V amax ~ 1000) and queries scaled by 4, so the
    lazily raised softmax reference trails the scores by up to 8 log2 units (weights up to
    2^8): the f16 weights of P.V stay finite for every page scale below 256.  Errors are
    relative to the output's scale."""
    from oracle import oracle as O
    g = wl.Geometry(hq=16, hkv=2, d=128, kv_dtype=FP8)
    b = wl.custom([4000, 9000, 700, 20000], [1, 1, 1, 1], geom=g, seed=25)
    case = G.Case(b, seed=25, v_scale=250.0)
    assert 0.5 < float(np.median(case.v_scales)) < 8.0
    case.q_store = O.from_f32((case.q32 * 4.0).astype(np.float32), BF16)
    case.q32 = O.to_f32(case.q_store, BF16)
    print(f"[case] fp8 large V scales: v_scales {case.v_scales.min():.2f}..{case.v_scales.max():.2f}",
          flush=True)
    got = case.run(lia)
    ref = case.f64()
    assert np.all(np.isfinite(got))
    scale = float(np.max(np.abs(ref)))
    mx, mean = G.errors(got, ref)
    print(f"[case] fp8 large V scales: max_abs/scale={mx / scale:.3e} mean/scale={mean / scale:.3e}",
          flush=True)
    assert mx / scale < 5e-2 and mean / scale < 5e-3
