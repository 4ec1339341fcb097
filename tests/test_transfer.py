"""CPU tests of KV page transfer: payload geometry, the reference's validation order
(src/inference/paging_transfer.rs:37-74) through the C ABI with no GPU call, and the oracle's
wire layout pinned by the reference's own upload test."""
import ctypes as C

import numpy as np
import pytest

MINICPM5_PAGE_BYTES = 42 * 2 * 32 * 256 * 2   # src/inference/paging_transfer.rs:4


def _layout(lia, hkv=2, d=128, page=32, pool=3, dtype=1):
    return lia.KVLayout(hkv, d, page, pool, dtype)


def test_page_bytes_match_reference_constant(lia):
    L = _layout(lia)
    assert lia.lib().lia_kv_page_bytes(C.byref(L), 42) == MINICPM5_PAGE_BYTES
    fp8 = _layout(lia, dtype=lia.FP8)
    # FP8: one byte per element plus [layer][plane][hkv] f32 scales
    assert lia.lib().lia_kv_page_bytes(C.byref(fp8), 42) == MINICPM5_PAGE_BYTES // 2 + 42 * 2 * 2 * 4
    total = lia.lib().lia_kv_transfer_bytes(C.byref(L), 42)
    header = total - 16 * MINICPM5_PAGE_BYTES
    assert header >= (4 * 42 + 16) * 8 and header % 256 == 0
    assert lia.lib().lia_kv_page_bytes(C.byref(L), 0) == 0
    assert lia.lib().lia_kv_page_bytes(C.byref(L), lia.MAX_LAYERS + 1) == 0
    assert lia.lib().lia_kv_page_bytes(C.byref(_layout(lia, dtype=lia.F32)), 1) == 0


def _call(lia, fn, pages, pool=3, planes=None):
    L = _layout(lia, pool=pool)
    if planes is None:
        planes = lia.KVPlanes()
        planes.n_layers = 42          # null plane addresses: rejected only after the page checks
    staging = C.create_string_buffer(lia.lib().lia_kv_transfer_bytes(C.byref(L), 42))
    ids = (C.c_uint32 * max(len(pages), 1))(*pages)
    payload = C.create_string_buffer(16)
    ptrs = (C.c_void_p * max(len(pages), 1))(*([C.addressof(payload)] * len(pages)))
    return getattr(lia.lib(), fn)(C.byref(L), C.byref(planes), len(pages), ids, ptrs, staging,
                                  C.c_void_p(1), None)


@pytest.mark.parametrize("fn", ["lia_kv_write_pages", "lia_kv_read_pages"])
def test_transfer_validation_order(lia, fn):
    assert _call(lia, fn, []) == -13                      # invalid KV transfer window
    assert _call(lia, fn, list(range(17)), pool=32) == -13
    assert _call(lia, fn, [3]) == -6                      # KV page outside physical pool
    assert _call(lia, fn, [1, 1]) == -14                  # duplicate KV transfer destination
    assert _call(lia, fn, [1, 1, 9]) == -14               # per page: range, then duplicate
    assert _call(lia, fn, [1, 9, 1]) == -6
    assert _call(lia, fn, [2, 0]) == -20                  # geometry valid, planes missing
    assert _call(lia, fn, list(range(16)), pool=16) == -20


def test_oracle_layout_matches_reference_upload_test(O):
    """The reference's pinned-upload test (src/inference/paging_upload.rs:110-150): payloads
    (index*17+31) and (index*29+71) written to pages 2 and 0 of 42 layers of 3-page f16
    planes; every element at layer l, plane p, column c of page q equals the little-endian
    u16 at (2l+p)*16384 + 2c of that page's payload, and page 1 stays zero."""
    idx = np.arange(MINICPM5_PAGE_BYTES, dtype=np.int64)
    a = ((idx * 17 + 31) % 256).astype(np.uint8).tobytes()
    b = ((idx * 29 + 71) % 256).astype(np.uint8).tobytes()
    k = [np.zeros((3 * 32, 2, 128), np.uint16) for _ in range(42)]
    v = [np.zeros((3 * 32, 2, 128), np.uint16) for _ in range(42)]
    O.kv_page_store(k, v, 2, 32, a)
    O.kv_page_store(k, v, 0, 32, b)
    for layer in range(42):
        for plane, buf in enumerate((k[layer], v[layer])):
            flat = buf.reshape(-1)
            assert not flat[8192:16384].any(), "untargeted KV page changed"
            for physical, expected in ((0, b), (2, a)):
                base = (layer * 2 + plane) * 16384
                want = np.frombuffer(expected[base:base + 16384], "<u2")
                assert np.array_equal(flat[physical * 8192:(physical + 1) * 8192], want)
    assert O.kv_page_payload(k, v, 2, 32) == a
    assert O.kv_page_payload(k, v, 0, 32) == b


def test_oracle_fp8_payload_round_trip(O):
    rng = np.random.default_rng(0)
    k = [rng.integers(0, 256, (5 * 16, 4, 64), dtype=np.uint8) for _ in range(3)]
    v = [rng.integers(0, 256, (5 * 16, 4, 64), dtype=np.uint8) for _ in range(3)]
    ks = [rng.random(5 * 4, dtype=np.float32) for _ in range(3)]
    vs = [rng.random(5 * 4, dtype=np.float32) for _ in range(3)]
    p = O.kv_page_payload(k, v, 3, 16, ks, vs, hkv=4)
    assert len(p) == 3 * 2 * (16 * 4 * 64 + 4 * 4)
    # scales sit after every plane, layer-major then K before V
    tail = np.frombuffer(p[3 * 2 * 16 * 4 * 64:], np.float32).reshape(3, 2, 4)
    assert np.array_equal(tail[1, 1], vs[1][12:16])
    k2 = [np.zeros_like(x) for x in k]
    v2 = [np.zeros_like(x) for x in v]
    ks2 = [np.zeros_like(x) for x in ks]
    vs2 = [np.zeros_like(x) for x in vs]
    O.kv_page_store(k2, v2, 0, 16, p, ks2, vs2, hkv=4)
    assert O.kv_page_payload(k2, v2, 0, 16, ks2, vs2, hkv=4) == p
    assert not k2[0][16:].any() and not ks2[2][4:].any()
