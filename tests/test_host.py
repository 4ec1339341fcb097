"""CPU tests of the product library: exports and host packing (no GPU calls)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "lia_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lia_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(lia):
    lib = lia.lib()
    names = _declared_symbols()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_bindings_cover_header(lia):
    assert set(_declared_symbols()) <= set(lia.EXPORTS)


def _random_batch(rng, max_sequences=8, page=16, context=1024, pool_pages=400):
    n_seq = int(rng.integers(1, max_sequences + 1))
    perm = rng.permutation(pool_pages)
    tables, rows, at = [], [], 0
    for s in range(n_seq):
        ctx = int(rng.integers(1, context))
        q = int(rng.integers(1, min(ctx, 40) + 1))
        n = -(-ctx // page)
        tables.append([int(x) for x in perm[at:at + n]])
        at += n
        rows += [(int(rng.integers(0, 1000)), p, s) for p in range(ctx - q, ctx)]
    return tables, rows


def test_pack_rows_matches_oracle_random(lia, O):
    rng = np.random.default_rng(11)
    for trial in range(60):
        tables, rows = _random_batch(rng)
        if rng.random() < 0.3:  # interleave two sequences' rows: two groups per sequence
            rows = sorted(rows, key=lambda r: (r[1] % 3, r[2], r[1]))
        outputs = sorted(set(int(x) for x in rng.integers(0, len(rows), size=min(4, len(rows)))))
        lim_o = O.PagingLimits(8, 1024, 16, 400, 1000, 4096)
        lim_p = lia.PagingLimits(8, 1024, 16, 400, 1000, 4096)
        st, ref = O.pack_rows(lim_o, rows, tables, outputs)
        try:
            got = lia.pack_rows(lim_p, rows, tables, outputs)
            gst = 0
        except lia.LiaError as e:
            gst = e.status
        assert gst == st, trial
        if st == 0:
            for key in ("positions", "sequences", "flat", "groups", "cu_seqlens", "slot_mapping"):
                assert np.array_equal(np.asarray(got[key]), np.asarray(ref[key])), key
            for key in ("stride", "maximum", "decoding", "span", "parts"):
                assert got[key] == ref[key], key


@pytest.mark.parametrize("case,expected", [
    ("rows0", -1), ("outcount", -2), ("outrow", -3), ("tables", -4), ("tablelen", -5),
    ("pagerange", -6), ("token", -7), ("position", -8), ("missingtable", -9),
    ("missingpage", -10), ("duplicate", -11), ("nonconsecutive", -12)])
def test_pack_rows_error_order(lia, case, expected):
    lim = lia.PagingLimits(4, 256, 32, 32, 1000, 64)
    tables = [[1, 2], [3]]
    rows = [(1, 0, 0), (1, 1, 0)]
    outputs = []
    if case == "rows0":
        rows = []
    elif case == "outcount":
        outputs = [0] * 5
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
    with pytest.raises(lia.LiaError) as e:
        lia.pack_rows(lim, rows, tables, outputs)
    assert e.value.status == expected


def test_decode_span_parts_match_oracle(lia, O):
    for tokens in list(range(1, 300, 7)) + [2047, 2048, 2049, 8191, 8192, 8193, 32768, 131072]:
        s = lia.decode_span(tokens)
        assert s == O.decode_span(tokens)
        assert lia.decode_parts(tokens, s) == O.decode_parts(tokens, s)


def test_workload_shapes(wl):
    b = wl.config2(seed=0)
    assert b.n_seqs == 8 and b.n_rows == 8
    assert np.all((b.ctx >= 1024) & (b.ctx <= 32768))
    slots = b.slot_mapping()
    assert len(set(slots.tolist())) == len(slots)
    b3 = wl.config3(seed=0)
    assert b3.n_rows == 512 + 1024 + 2048 + 5
    b4 = wl.config4(seed=0)
    assert set(np.unique(b4.q_len)) <= {2, 3, 4}
    b1 = wl.config1()
    assert list(b1.ctx) == [17, 64, 200, 511]
    used = np.concatenate(b1.tables)
    assert len(np.unique(used)) == len(used) == 2 + 4 + 13 + 32


def test_partial_append_validates_before_launch(lia):
    """The fused-append entry point rejects FP8 pools, missing rows and unaligned rows
    before it touches the device."""
    F16, FP8 = 1, 3
    ws = (C.c_uint8 * 4096)()
    fake = C.c_void_p(0x10000)
    odd = C.c_void_p(0x10008)

    def call(kv, new_k, slots):
        cfg = lia.AttentionConfig(16, 2, 128, 16, 64, 8, 2, kv, 2, 0.088, 4, 4, 128)
        return lia.lib().lia_attention_partial_append(
            C.byref(cfg), 2, 2, fake, slots, fake, new_k, fake, fake, fake, C.cast(ws, C.c_void_p),
            4096, fake, None)

    assert call(FP8, fake, fake) == -23
    assert call(F16, None, fake) == -20
    assert call(F16, fake, None) == -20
    assert call(F16, odd, fake) == -21
