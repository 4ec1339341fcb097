"""Pins the CPU oracle (oracle/lia_oracle.c) before anything is compared against it.

Each check is independent of the oracle's own formulas: IEEE/OCP conversions against
numpy and torch, packing against a brute-force restatement of paging.rs, attention
against the reference's own known-answer inputs (src/gpu/llama_attention.rs:212-284)
evaluated with numpy in float64, the merge against the reference's merge vectors
(src/gpu/kernels/llama_merge.rs:91-108) and the identity "merge of any split equals the
unsplit softmax", and the fused RoPE + append against the separate path on the
reference's fixture (src/gpu/kernels/llama_position.rs:128-239).
"""
import numpy as np
import pytest
import torch

F32, F16, BF16, FP8 = 0, 1, 2, 3


# ------------------------------------------------------------------ conversions

def test_f16_decode_exhaustive(O):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = O.to_f32(bits, F16)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


def _interesting_f32(n, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(n).astype(np.float32) * np.float32(10) ** rng.integers(-9, 6, n).astype(np.float32)
    b = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    b = b[np.isfinite(b)]
    # ties and boundaries of the f16 / bf16 / e4m3 grids
    c = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 2**-24, 2**-25, 3 * 2**-26,
                  2**-14, 448.0, 464.0, 2**-9, 2**-10, 3 * 2**-11, 1.0625, 1.1875],
                 dtype=np.float32)
    return np.concatenate([a, b, c, -c])


def test_f16_encode_matches_numpy_rne(O):
    x = _interesting_f32(200000, 1)
    got = O.from_f32(x, F16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_matches_torch_rne(O):
    x = _interesting_f32(200000, 2)
    got = O.from_f32(x, BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = O.to_f32(got, BF16)
    assert np.array_equal(back, torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_e4m3_decode_all_codes(O):
    codes = np.arange(256, dtype=np.uint8)
    got = O.to_f32(codes, FP8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])


def test_e4m3_encode_rne_and_saturation(O):
    x = _interesting_f32(200000, 3)
    x = x[np.abs(x) < 448.0]
    got = O.from_f32(x, FP8)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)
    # saturating beyond the largest finite value (448)
    big = np.array([448.0, 460.0, 464.0, 1e6, -500.0], np.float32)
    assert list(O.from_f32(big, FP8)) == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE]


# ------------------------------------------------------------------ packing

def _limits(O, max_sequences=4, context=256, page_size=32, pool_pages=32, vocabulary=1000,
            prefill_batch=64):
    return O.PagingLimits(max_sequences, context, page_size, pool_pages, vocabulary, prefill_batch)


def _brute_pack(rows, tables, P):
    """Straight restatement of paging.rs:148-186 for valid inputs."""
    groups, slots = [], []
    for i, (tok, pos, seq) in enumerate(rows):
        slots.append(tables[seq][pos // P] * P + pos % P)
        if groups and rows[i - 1][2] == seq:
            groups[-1][1] += 1
            groups[-1][2] = pos + 1
        else:
            groups.append([i, 1, pos + 1])
    return groups, slots


def test_pack_valid_batch_matches_brute_force(O):
    lim = _limits(O)
    tables = [[5, 3], [7], [2, 9, 11]]
    rows = [(1, 30, 0), (2, 31, 0), (3, 32, 0), (4, 3, 1), (5, 70, 2), (6, 71, 2)]
    st, out = O.pack_rows(lim, rows, tables, outputs=[2, 3, 5])
    assert st == 0
    groups, slots = _brute_pack(rows, tables, 32)
    assert out["groups"].tolist() == groups
    assert out["slot_mapping"].tolist() == slots
    assert out["cu_seqlens"].tolist() == [g[0] for g in groups] + [len(rows)]
    stride = 8
    flat = out["flat"].reshape(4, stride)
    assert flat[0, :2].tolist() == [5, 3] and flat[0, 2:].tolist() == [0xFFFFFFFF] * 6
    assert flat[3].tolist() == [0xFFFFFFFF] * 8
    assert out["maximum"] == 72 and not out["decoding"]
    assert out["span"] == 256 and out["parts"] == 1


def test_pack_decode_rule(O):
    lim = _limits(O, context=8192, pool_pages=300)
    tables = [list(range(0, 100)), list(range(100, 200))]
    rows = [(1, 3000, 0), (1, 10, 1)]
    st, out = O.pack_rows(lim, rows, tables, outputs=[0, 1])
    assert st == 0 and out["decoding"]
    assert out["span"] == 64  # 2048 < 3001 <= 8192
    assert out["parts"] == 48  # ceil(3001/64) = 47 -> next multiple of 16


@pytest.mark.parametrize("case,expected", [
    ("rows0", -1), ("outcount", -2), ("outrow", -3), ("tables", -4), ("tablelen", -5),
    ("pagerange", -6), ("token", -7), ("position", -8), ("missingtable", -9),
    ("missingpage", -10), ("duplicate", -11), ("nonconsecutive", -12)])
def test_pack_errors(O, case, expected):
    lim = _limits(O)
    tables = [[1, 2], [3]]
    rows = [(1, 0, 0), (1, 1, 0)]
    outputs = []
    if case == "rows0":
        rows = []
    elif case == "outcount":
        outputs = [0, 0, 0, 0, 0]
    elif case == "outrow":
        outputs = [2]
    elif case == "tables":
        tables = [[1]] * 5
    elif case == "tablelen":
        tables = [list(range(9))]
    elif case == "pagerange":
        tables = [[1, 32]]
    elif case == "token":
        rows = [(1000, 0, 0)]
    elif case == "position":
        rows = [(1, 256, 0)]
    elif case == "missingtable":
        rows = [(1, 0, 2)]
    elif case == "missingpage":
        rows = [(1, 40, 1)]
    elif case == "duplicate":
        tables = [[1], [1]]
        rows = [(1, 0, 0), (1, 0, 1)]
    elif case == "nonconsecutive":
        rows = [(1, 0, 0), (1, 2, 0)]
    st, _ = O.pack_rows(lim, rows, tables, outputs)
    assert st == expected


def test_decode_span_parts_closed_form(O):
    for tokens in [1, 100, 2048, 2049, 8192, 8193, 32768, 131072]:
        span = 32 if tokens <= 2048 else 64 if tokens <= 8192 else 160
        assert O.decode_span(tokens) == span
        count = -(-tokens // span)
        parts = 1 << (count - 1).bit_length() if count <= 16 else -(-count // 16) * 16
        assert O.decode_parts(tokens, span) == parts


# ------------------------------------------------------------------ KV append

@pytest.mark.parametrize("dtype", [F16, BF16])
def test_kv_append_brute_force(O, dtype):
    rng = np.random.default_rng(5)
    H, D, P, pool = 2, 64, 16, 12
    layout = O.KVLayout(H, D, P, pool, dtype)
    tables = [[7, 2, 9], [4, 11]]
    stride = 3
    flat = np.full(2 * stride, 0xFFFFFFFF, np.uint32)
    flat[:3] = tables[0]
    flat[3:5] = tables[1]
    positions = np.array([15, 16, 17, 31, 0], np.uint32)
    sequences = np.array([0, 0, 0, 1, 1], np.uint32)
    k = rng.standard_normal((5, H * D)).astype(np.float32)
    v = rng.standard_normal((5, H * D)).astype(np.float32)
    kc = np.zeros(pool * P * H * D, np.uint16)
    vc = np.zeros_like(kc)
    O.kv_append(layout, positions, sequences, flat, stride, k, v, kc, vc)
    ek, ev = np.zeros_like(kc), np.zeros_like(vc)
    conv = (lambda a: a.astype(np.float16).view(np.uint16)) if dtype == F16 else \
        (lambda a: torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    for r in range(5):
        page = tables[sequences[r]][positions[r] // P]
        at = (page * P + positions[r] % P) * H * D
        ek[at:at + H * D] = conv(k[r])
        ev[at:at + H * D] = conv(v[r])
    assert np.array_equal(kc, ek) and np.array_equal(vc, ev)


def test_fp8_append_scale_rule(O):
    """FP8 append: values divided by the page's scale and rounded to e4m3 (torch's
    float8_e4m3fn cast); a page whose scale is 0 (never quantised) takes scale 1 and the
    append writes 1 into the scale arrays, pages not appended to keep 0."""
    rng = np.random.default_rng(8)
    H, D, P, pool = 2, 64, 16, 6
    layout = O.KVLayout(H, D, P, pool, FP8)
    slots = np.array([0 * P + 3, 2 * P + 5, 2 * P + 6, 4 * P + 0], np.uint32)
    k = rng.standard_normal((4, H * D)).astype(np.float32)
    v = rng.standard_normal((4, H * D)).astype(np.float32)
    ks = np.zeros(pool * H, np.float32)
    vs = np.zeros(pool * H, np.float32)
    ks[2 * H:3 * H] = [0.01, 0.02]   # page 2 quantised before, pages 0 and 4 never
    vs[2 * H:3 * H] = [0.03, 0.04]
    kc = np.zeros(pool * P * H * D, np.uint8)
    vc = np.zeros_like(kc)
    zeros = np.zeros(4, np.uint32)
    O.kv_append(layout, zeros, zeros, zeros, 0, k, v, kc, vc, slot_mapping=slots, k_scales=ks, v_scales=vs)
    want_k = np.zeros(pool * H, np.float32)
    want_v = np.zeros(pool * H, np.float32)
    want_k[[0, 1, 8, 9]] = 1.0
    want_v[[0, 1, 8, 9]] = 1.0
    want_k[4:6], want_v[4:6] = [0.01, 0.02], [0.03, 0.04]
    assert np.array_equal(ks, want_k) and np.array_equal(vs, want_v)
    e4m3 = lambda a: torch.from_numpy(a).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    for r, slot in enumerate(slots):
        page = slot // P
        scale_k = np.repeat(ks[page * H:(page + 1) * H], D)
        scale_v = np.repeat(vs[page * H:(page + 1) * H], D)
        at = slot * H * D
        assert np.array_equal(kc[at:at + H * D], e4m3(k[r] / scale_k))
        assert np.array_equal(vc[at:at + H * D], e4m3(v[r] / scale_v))


def test_kv_quantize_pages_closed_form(O):
    rng = np.random.default_rng(6)
    H, D, P, pool = 2, 64, 16, 6
    layout = O.KVLayout(H, D, P, pool, FP8)
    k = rng.standard_normal((2, P, H, D)).astype(np.float32)
    v = rng.standard_normal((2, P, H, D)).astype(np.float32)
    v[1] = 0.0
    kc = np.zeros(pool * P * H * D, np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros(pool * H, np.float32)
    vs = np.zeros_like(ks)
    O.kv_quantize_pages(layout, [4, 1], k, v, kc, vc, ks, vs)
    for n, page in enumerate([4, 1]):
        for h in range(H):
            s = np.abs(k[n, :, h, :]).max() / np.float32(448)
            assert ks[page * H + h] == np.float32(s)
            q = kc.reshape(pool, P, H, D)[page, :, h, :]
            ref = torch.from_numpy(k[n, :, h, :] / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(q, ref)
    assert vs[1 * H] == 1.0 and not vc.reshape(pool, P, H, D)[1].any()


# ------------------------------------------------------------------ attention

def _reference_vectors(capacity=16416, page=32):
    """Inputs of scalar_and_tensor_paged_attention_match_independent_f64_reference
    (src/gpu/llama_attention.rs:212-252), generated from their closed forms."""
    stride = capacity // page
    positions = np.array(list(range(4090, 4098)) + list(range(16377, 16385)) + [8191], np.uint32)
    sequences = np.array([0] * 8 + [1] * 8 + [0], np.uint32)
    tables = np.array([(1 - s) * stride + stride - 1 - p for s in range(2) for p in range(stride)],
                      np.uint32)

    def value(s, t, h, c, plane):
        return ((s * 7 + t * 17 + h * 23 + c * 13 + plane * 11) % 257) / 256.0 - 0.5

    tok = np.arange(capacity)
    keys = np.zeros((capacity * 2, 2, 128), np.float32)  # [physical][head][col]
    vals = np.zeros_like(keys)
    h = np.arange(2)[:, None]
    c = np.arange(128)[None, :]
    for s in range(2):
        phys = tables[s * stride + tok // page].astype(np.int64) * page + tok % page
        for plane, dst in ((0, keys), (1, vals)):
            dst[phys] = ((s * 7 + tok[:, None, None] * 17 + h[None] * 23 + c[None] * 13 + plane * 11)
                         % 257) / 256.0 - 0.5
    q = ((np.arange(len(positions) * 2048) * 19 % 61) / 64.0 - 30.0 / 64.0).astype(np.float32)
    return stride, positions, sequences, tables, keys, vals, q.reshape(-1, 16, 128), value


@pytest.fixture(scope="module")
def refcase(O):
    stride, pos, seq, tables, keys, vals, q, value = _reference_vectors()
    kc = keys.astype(np.float16).view(np.uint16)
    vc = vals.astype(np.float16).view(np.uint16)
    g = O.geom(16, 2, 128, 32, stride, F16, 1.0 / np.sqrt(128.0))
    f64 = O.attention_f64(g, pos, seq, tables, q, kc, vc)
    return dict(stride=stride, pos=pos, seq=seq, tables=tables, kc=kc, vc=vc, q=q, g=g, f64=f64,
                keys=keys, vals=vals, value=value)


def test_attention_f64_matches_independent_numpy(refcase):
    rc = refcase
    kf = rc["kc"].view(np.float16).astype(np.float64).reshape(-1, 2, 128)
    vf = rc["vc"].view(np.float16).astype(np.float64).reshape(-1, 2, 128)
    P, stride = 32, rc["stride"]
    for r in [0, 7, 8, 15, 16]:
        n = int(rc["pos"][r]) + 1
        s = int(rc["seq"][r])
        tok = np.arange(n)
        phys = rc["tables"][s * stride + tok // P].astype(np.int64) * P + tok % P
        for h in [0, 5, 8, 15]:
            scores = kf[phys, h // 8] @ rc["q"][r, h].astype(np.float64) / np.sqrt(128.0)
            w = np.exp(scores - scores.max())
            w /= w.sum()
            ref = w @ vf[phys, h // 8]
            assert np.max(np.abs(ref - rc["f64"][r, h])) < 1e-12


def test_attention_partial_merge_matches_f64(O, refcase):
    """The reference's scalar configuration (parts 144, span 128) and its 3e-5 bar."""
    rc = refcase
    rows = len(rc["pos"])
    part = O.attention_partial(rc["g"], 0, rows, 144, 128, rc["pos"], rc["seq"], rc["tables"],
                               rc["q"], rc["kc"], rc["vc"])
    out = np.zeros((rows, 16, 128), np.float32)
    O.merge(16, 128, 0, rows, 144, part, out)
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - rc["f64"])) < 3e-5


def test_split_invariance_and_baseline(O, refcase):
    rc = refcase
    for span in (32, 160, 4096, 32768):
        out = O.paged_attention_f32(rc["g"], rc["pos"], rc["seq"], rc["tables"], rc["q"], rc["kc"],
                                    rc["vc"], span=span)
        assert np.max(np.abs(out - rc["f64"])) < 3e-5, span


def test_merge_reference_vectors(O):
    """Vectors of warp_reduction_matches_block_reduction_bits
    (src/gpu/kernels/llama_merge.rs:91-108), merged in float64 with numpy."""
    for parts in [1, 2, 3, 4, 8, 16]:
        partial = np.zeros((3 * 16 * parts, 130), np.float32)
        for group in range(48):
            for p in range(parts):
                at = group * parts + p
                partial[at, :128] = ((group * 7 + p * 13 + np.arange(128) * 17) % 59) / 32.0 - 1.0
                valid = p == 0 or (group + p) % 3 != 0
                partial[at, 128] = (group % 7 + p) / 8.0 if valid else -np.inf
                partial[at, 129] = 0.25 + p / 16.0 if valid else 0.0
        out = np.full((9, 16, 128), 7.0, np.float32)  # guard rows around query_start 5
        O.merge(16, 128, 5, 3, parts, partial, out)
        pr = partial.reshape(48, parts, 130).astype(np.float64)
        m = pr[:, :, 128]
        l = pr[:, :, 129]
        M = np.max(np.where(l > 0, m, -np.inf), axis=1, keepdims=True)
        w = np.where(l > 0, np.exp(m - M), 0.0)
        ref = (w[:, :, None] * pr[:, :, :128]).sum(1) / (w * l).sum(1, keepdims=True)
        assert np.max(np.abs(out[5:8].reshape(48, 128) - ref)) < 1e-5, parts
        assert np.all(out[:5] == 7.0) and np.all(out[8:] == 7.0)


def test_empty_parts_are_skipped(O):
    rng = np.random.default_rng(9)
    P, H, D = 16, 1, 64
    pool = 8
    kc = O.from_f32(rng.standard_normal((pool * P, H, D)).astype(np.float32), BF16)
    vc = O.from_f32(rng.standard_normal((pool * P, H, D)).astype(np.float32), BF16)
    g = O.geom(2, 1, D, P, 8, BF16)
    q = rng.standard_normal((1, 2, D)).astype(np.float32)
    pos = np.array([20], np.uint32)
    seq = np.array([0], np.uint32)
    tables = np.array([3, 6, 0, 0, 0, 0, 0, 0], np.uint32)
    part = O.attention_partial(g, 0, 1, 8, 16, pos, seq, tables, q, kc, vc)
    rec = part.reshape(2, 8, D + 2)
    assert np.all(rec[:, 2:, D] == -np.inf) and np.all(rec[:, 2:, D + 1] == 0.0)
    out = np.zeros((1, 2, D), np.float32)
    O.merge(2, D, 0, 1, 8, part, out)
    ref = O.attention_f64(g, pos, seq, tables, q, kc, vc)
    assert np.max(np.abs(out - ref)) < 1e-5


# ------------------------------------------------------------------ RoPE + append

def test_rotary_cache_matches_separate_rope_and_append(O):
    """Fixture of combined_rotary_cache_matches_separate_operators
    (src/gpu/kernels/llama_position.rs:128-239): bit-equal Q and K/V."""
    positions = np.array([0, 31, 32, 8191, 131071], np.uint32)
    sequences = np.array([0, 1, 0, 1, 0], np.uint32)
    tables = np.zeros(2 * 4096, np.uint32)
    for row, page in enumerate([5, 3, 2, 7, 1]):
        tables[sequences[row] * 4096 + positions[row] // 32] = page
    i = np.arange(5 * 2048)
    q = ((i * 37 % 1021) / 128.0 - 4.0).astype(np.float32)
    j = np.arange(5 * 256)
    k = ((j * 43 % 997) / 256.0 - 2.0).astype(np.float32)
    v = ((j * 17 % 509) / 128.0 - 2.0).astype(np.float32)
    combined = np.concatenate([np.concatenate([q[r * 2048:(r + 1) * 2048], k[r * 256:(r + 1) * 256],
                                               v[r * 256:(r + 1) * 256]]) for r in range(5)])
    qr = O.rope(16, positions, q)
    kr = O.rope(2, positions, k)
    layout = O.KVLayout(2, 128, 32, 8, F16)
    ek = np.zeros(8 * 32 * 256, np.uint16)
    ev = np.zeros_like(ek)
    O.kv_append(layout, positions, sequences, tables, 4096, kr.reshape(5, 256), v.reshape(5, 256), ek, ev)
    coeffs = O.coefficients(positions)
    query = np.zeros(5 * 2048, np.float32)
    keys = np.zeros_like(ek)
    values = np.zeros_like(ev)
    O.rotary_cache(5, 4096, 32, positions, sequences, tables, coeffs, combined, query, keys, values)
    assert np.array_equal(query.view(np.uint32), qr.view(np.uint32))
    assert np.array_equal(keys, ek) and np.array_equal(values, ev)


def test_coefficients_against_float64(O):
    """coefficients (llama_position.rs:36-47): angle = f32(pos * f32(1 / f32(base^(2i/128))))
    with correctly rounded f32 steps; cos/sin checked in float64 on that angle."""
    positions = np.array([0, 1, 17, 4095, 131071], np.uint32)
    got = O.coefficients(positions).reshape(5, 64, 2)
    x = (np.float32(2.0) * np.arange(64, dtype=np.float32)) / np.float32(128.0)
    p32 = np.power(np.float64(5e6), x.astype(np.float64)).astype(np.float32)
    inv = (np.float32(1.0) / p32).astype(np.float32)
    angle = (positions[:, None].astype(np.float32) * inv[None, :]).astype(np.float32)
    assert np.max(np.abs(got[:, :, 0] - np.cos(angle.astype(np.float64)))) < 5e-7
    assert np.max(np.abs(got[:, :, 1] - np.sin(angle.astype(np.float64)))) < 5e-7


def _rope_fixture(rows, hq, hkv, d, seed):
    rng = np.random.default_rng(seed)
    combined = rng.uniform(-4, 4, (rows, (hq + 2 * hkv) * d)).astype(np.float32)
    return combined


def test_rope_kv_append_equals_rotary_cache_on_reference_geometry(O):
    """The generalised restatement reproduces rotary_cache's bits (16 q / 2 kv heads, d 128,
    f16 pool in 32-token pages, f32 queries, llama_position.rs:49-118)."""
    positions = np.array([0, 31, 32, 8191, 131071], np.uint32)
    sequences = np.array([0, 1, 0, 1, 0], np.uint32)
    tables = np.zeros(2 * 4096, np.uint32)
    for row, page in enumerate([5, 3, 2, 7, 1]):
        tables[sequences[row] * 4096 + positions[row] // 32] = page
    combined = _rope_fixture(5, 16, 2, 128, 21)
    coeffs = O.coefficients(positions)
    q1 = np.zeros(5 * 2048, np.float32)
    k1 = np.zeros(8 * 32 * 256, np.uint16)
    v1 = np.zeros_like(k1)
    O.rotary_cache(5, 4096, 32, positions, sequences, tables, coeffs, combined, q1, k1, v1)
    layout = O.KVLayout(2, 128, 32, 8, 1)
    q2 = np.zeros_like(q1)
    k2 = np.zeros_like(k1)
    v2 = np.zeros_like(v1)
    O.rope_kv_append(layout, 16, positions, sequences, tables, 4096, coeffs, combined, q2, 0, k2, v2)
    assert np.array_equal(q1.view(np.uint32), q2.view(np.uint32))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def _fma32(a, b, c):
    # f32 fma: the product of two f32 is exact in longdouble (64-bit significand)
    L = np.longdouble
    return (a.astype(L) * b.astype(L) + c.astype(L)).astype(np.float32)


@pytest.mark.parametrize("hq,hkv,d,kv,qdt", [(8, 2, 64, 2, 2), (16, 1, 128, 1, 0), (4, 4, 64, 1, 0)])
def test_rope_kv_append_generalised(O, hq, hkv, d, kv, qdt):
    """Rotation restated in numpy (rounded products, fma in extended precision), queries
    rounded to the requested type, K/V through the pinned lo_kv_append."""
    rows, P, stride = 6, 16, 64
    rng = np.random.default_rng(hq * 100 + d)
    positions = rng.integers(0, stride * P, rows).astype(np.uint32)
    sequences = np.zeros(rows, np.uint32)
    positions = np.unique(positions)[:rows]
    rows = positions.size
    sequences = np.zeros(rows, np.uint32)
    tables = rng.permutation(stride).astype(np.uint32)
    combined = _rope_fixture(rows, hq, hkv, d, 22)
    coeffs = O.rope_coefficients(positions, d).reshape(rows, d // 2, 2)
    half = d // 2
    x = combined.reshape(rows, hq + 2 * hkv, d)
    c = coeffs[:, None, :, 0]
    s = coeffs[:, None, :, 1]
    left, right = x[:, :hq + hkv, :half], x[:, :hq + hkv, half:]
    a = _fma32(left, np.broadcast_to(c, left.shape), -(right * s))
    b = _fma32(right, np.broadcast_to(c, right.shape), left * s)
    rot = np.concatenate([a, b], axis=2)
    layout = O.KVLayout(hkv, d, P, stride, kv)
    kexp = np.zeros(stride * P * hkv * d, np.uint16)
    vexp = np.zeros_like(kexp)
    O.kv_append(layout, positions, sequences, tables, stride, rot[:, hq:].reshape(rows, -1),
                x[:, hq + hkv:].reshape(rows, -1), kexp, vexp)
    qexp = rot[:, :hq].reshape(-1)
    qout = np.zeros(rows * hq * d, np.uint16 if qdt == 2 else np.float32)
    kc = np.zeros_like(kexp)
    vc = np.zeros_like(vexp)
    O.rope_kv_append(layout, hq, positions, sequences, tables, stride, coeffs, combined, qout, qdt,
                     kc, vc)
    if qdt == 2:
        assert np.array_equal(qout, O.from_f32(qexp, 2))
    else:
        assert np.array_equal(qout.view(np.uint32), qexp.view(np.uint32))
    assert np.array_equal(kc, kexp) and np.array_equal(vc, vexp)


def test_rope_coefficients_generalise_the_reference_table(O):
    positions = np.array([0, 5, 4095, 131071], np.uint32)
    assert np.array_equal(O.rope_coefficients(positions, 128).view(np.uint32),
                          O.coefficients(positions).view(np.uint32))
    got = O.rope_coefficients(positions, 64).reshape(4, 32, 2)
    x = (np.float32(2.0) * np.arange(32, dtype=np.float32)) / np.float32(64.0)
    inv = (np.float32(1.0) / np.power(np.float64(5e6), x.astype(np.float64)).astype(np.float32)).astype(np.float32)
    angle = (positions[:, None].astype(np.float32) * inv[None, :]).astype(np.float32)
    assert np.array_equal(got[:, :, 0], np.cos(angle.astype(np.float64)).astype(np.float32))
    assert np.array_equal(got[:, :, 1], np.sin(angle.astype(np.float64)).astype(np.float32))


# ------------------------------------------------------------------ RoPE: the mathematics
#
# The checks above compare the fused and separate restatements with each other.  These pin
# the rotation itself with facts the mathematics fixes, independently of the oracle's
# formula: a rotation by angle 0 is the identity, a rotation keeps each (i, i + d/2) pair's
# length, rotating basis vectors gives (cos, sin) columns at exactly the "rotate half"
# positions with the reference's signs (src/gpu/kernels/llama.rs:33-60: lane i < d/2 pairs
# with i + d/2 and takes -sin), and the dot product of a rotated query and key depends only
# on the distance between their positions.

def _rope_all(O, positions, x, d, hq=1):
    """Rotate rows x[rows][hq][d] (queries) with the generalised restatement; f32 output."""
    positions = np.asarray(positions, np.uint32)
    rows = positions.size
    hkv = 1
    combined = np.zeros((rows, hq + 2 * hkv, d), np.float32)
    combined[:, :hq] = x
    coeffs = O.rope_coefficients(positions, d)
    layout = O.KVLayout(hkv, d, 16, rows, F16)
    qout = np.zeros(rows * hq * d, np.float32)
    kc = np.zeros(rows * 16 * hkv * d, np.uint16)
    O.rope_kv_append(layout, hq, positions, np.zeros(rows, np.uint32),
                     np.arange(rows, dtype=np.uint32), 1, coeffs, combined.reshape(rows, -1), qout,
                     F32, kc, np.zeros_like(kc), slot_mapping=np.arange(rows, dtype=np.uint32) * 16)
    return qout.reshape(rows, hq, d)


@pytest.mark.parametrize("d", [64, 128])
def test_rope_position_zero_is_identity(O, d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((4, 3, d)).astype(np.float32) * 10
    x[0, 0, :4] = [0.0, -0.0, np.float32(1e-30), np.float32(-3e38)]
    got = _rope_all(O, np.zeros(4, np.uint32), x, d, hq=3)
    # bit-equal; a zero may change sign (x*1 - y*0 is -0 + +0 = +0 for x = -0, y < 0)
    nz = x != 0
    assert np.array_equal(got[nz].view(np.uint32), x[nz].view(np.uint32))
    assert np.all(got[~nz] == 0)
    if d == 128:  # the reference-geometry restatement (16 heads x 128 dims)
        q = rng.standard_normal(2 * 16 * 128).astype(np.float32)
        assert np.array_equal(O.rope(16, np.zeros(2, np.uint32), q).view(np.uint32), q.view(np.uint32))


@pytest.mark.parametrize("d", [64, 128])
def test_rope_basis_vectors_rotate_half(O, d):
    """e_i -> cos(a_i) e_i + sin(a_i) e_{i+d/2};  e_{i+d/2} -> -sin(a_i) e_i + cos(a_i) e_{i+d/2},
    with a_i = f32(pos * f32(1 / f32(5e6^(2i/d)))) evaluated here in numpy."""
    half = d // 2
    positions = np.array([1, 7, 1000, 131071], np.uint32)
    x = np.zeros((positions.size, d, d), np.float32)
    for i in range(d):
        x[:, i, i] = 1.0
    got = _rope_all(O, positions, x, d, hq=d)  # head h holds the basis vector e_h
    e = (np.float32(2.0) * np.arange(half, dtype=np.float32)) / np.float32(d)
    inv = np.float32(1.0) / np.power(np.float64(5e6), e.astype(np.float64)).astype(np.float32)
    ang = (positions[:, None].astype(np.float32) * inv[None, :]).astype(np.float32)
    c = np.cos(ang.astype(np.float64)).astype(np.float32)
    s = np.sin(ang.astype(np.float64)).astype(np.float32)
    for r in range(positions.size):
        m = got[r]  # m[h] = rotation of e_h
        want = np.zeros((d, d), np.float32)
        for i in range(half):
            want[i, i], want[i, i + half] = c[r, i], s[r, i]
            want[i + half, i], want[i + half, i + half] = -s[r, i], c[r, i]
        assert np.array_equal(m, want), f"position {positions[r]}"


@pytest.mark.parametrize("d", [64, 128])
def test_rope_preserves_pair_norms(O, d):
    half = d // 2
    rng = np.random.default_rng(5 + d)
    positions = rng.integers(0, 131072, 64).astype(np.uint32)
    x = rng.standard_normal((64, 2, d)).astype(np.float32)
    got = _rope_all(O, positions, x, d, hq=2).astype(np.float64)
    x64 = x.astype(np.float64)
    n0 = np.hypot(x64[..., :half], x64[..., half:])
    n1 = np.hypot(got[..., :half], got[..., half:])
    # f32 cos/sin (cos^2 + sin^2 = 1 within ~2^-23), two rounded products and an fma
    assert np.all(np.abs(n1 - n0) <= 8 * 2.0 ** -24 * n0 + 1e-37)


@pytest.mark.parametrize("d", [64, 128])
def test_rope_scores_depend_on_relative_position(O, d):
    """<R(q, m), R(k, n)> = <R(q, m + s), R(k, n + s)> (f64 dot products of the f32 results).
    Positions stay small so the f32 angles keep a phase error well under 1e-6."""
    rng = np.random.default_rng(9 + d)
    q = rng.standard_normal((1, 1, d)).astype(np.float32)
    k = rng.standard_normal((1, 1, d)).astype(np.float32)
    scale = float(np.linalg.norm(q) * np.linalg.norm(k))
    for m, n in [(0, 0), (3, 0), (0, 5), (17, 9), (31, 32)]:
        base = None
        for shift in (0, 1, 8, 21):
            rq = _rope_all(O, [m + shift], q, d)[0, 0].astype(np.float64)
            rk = _rope_all(O, [n + shift], k, d)[0, 0].astype(np.float64)
            dot = float(rq @ rk)
            if base is None:
                base = dot
                if m == n:  # same position: the rotation cancels
                    assert abs(dot - float(q[0, 0].astype(np.float64) @ k[0, 0].astype(np.float64))) <= 1e-5 * scale
            assert abs(dot - base) <= 1e-5 * scale, (m, n, shift)
