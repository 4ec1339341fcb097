"""GPU tests of KV page transfer (and of the host page manager over it) through the C ABI: bit-exact against the oracle's wire
layout (oracle.kv_page_payload / kv_page_store) and the reference's own transfer tests
(src/inference/paging_upload.rs:110-150, tests/minicpm5.rs:98-110)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MINICPM5_PAGE_BYTES = 42 * 2 * 32 * 256 * 2


def _host(planes):
    return [p.view(torch.int16).cpu().numpy().view(np.uint16) for p in planes]


def test_pinned_upload_preserves_every_plane_and_noncontiguous_page(lia, O):
    """The reference's upload test: 42 layers, 3-page f16 planes, pages 2 and 0 written with
    two byte patterns, page 1 untouched."""
    print("[case] upload 42 layers pages (2, 0)", flush=True)
    L = lia.KVLayout(2, 128, 32, 3, lia.F16)
    k = [torch.zeros((96, 2, 128), dtype=torch.uint16, device="cuda") for _ in range(42)]
    v = [torch.zeros((96, 2, 128), dtype=torch.uint16, device="cuda") for _ in range(42)]
    t = lia.KVTransfer(L, k, v)
    assert t.page_bytes == MINICPM5_PAGE_BYTES
    idx = np.arange(MINICPM5_PAGE_BYTES, dtype=np.int64)
    a = ((idx * 17 + 31) % 256).astype(np.uint8).tobytes()
    b = ((idx * 29 + 71) % 256).astype(np.uint8).tobytes()
    t.write_kv_pages([(2, a), (0, b)])
    hk, hv = _host(k), _host(v)
    ek = [np.zeros((96, 2, 128), np.uint16) for _ in range(42)]
    ev = [np.zeros((96, 2, 128), np.uint16) for _ in range(42)]
    O.kv_page_store(ek, ev, 2, 32, a)
    O.kv_page_store(ek, ev, 0, 32, b)
    for layer in range(42):
        assert np.array_equal(hk[layer], ek[layer]), layer
        assert np.array_equal(hv[layer], ev[layer]), layer
        assert not hk[layer][32:64].any() and not hv[layer][32:64].any()
    assert t.read_kv_pages([0, 2]) == [b, a]


def test_engine_window_transfer_round_trip(lia, O):
    """tests/minicpm5.rs:98-110: saved = read(3); write [(1, saved), (0, saved)]; a duplicate
    destination fails; both pages read back bit-identical."""
    print("[case] engine window transfer", flush=True)
    e = lia.Engine(layers=42, pool_tokens=8 * 32)
    e.configure_paging(2, 128)
    g = torch.Generator(device="cuda").manual_seed(1)
    for planes in (e.k, e.v):
        for p in planes:
            p.view(torch.int16).copy_(torch.randint(-32768, 32768, p.shape, generator=g,
                                                    device="cuda", dtype=torch.int16))
    saved = e.read_kv_page(3)
    assert saved == O.kv_page_payload(_host(e.k), _host(e.v), 3, 32)
    before = [p.view(torch.int16).clone() for p in e.k]
    e.write_kv_pages([(1, saved), (0, saved)])
    with pytest.raises(lia.LiaError) as err:
        e.write_kv_pages([(1, saved), (1, saved)])
    assert err.value.status == -14
    with pytest.raises(lia.LiaError):
        e.write_kv_pages([(8, saved)])
    with pytest.raises(lia.LiaError):
        e.write_kv_page(0, saved[:-2])
    assert e.read_kv_page(0) == saved
    assert e.read_kv_page(1) == saved
    for layer in range(42):  # pages outside the window are untouched
        assert torch.equal(e.k[layer].view(torch.int16)[64:], before[layer][64:])


@pytest.mark.parametrize("kv", [2, 3])   # BF16, FP8 (with page scales)
def test_full_window_read_write_matches_oracle(lia, O, kv):
    print(f"[case] 16-page window kv={kv}", flush=True)
    layers, hkv, d, page, pool = 5, 4, 64, 16, 40
    rng = np.random.default_rng(kv)
    store = np.uint8 if kv == 3 else np.uint16
    hi = 256 if kv == 3 else 65536
    nk = [rng.integers(0, hi, (pool * page, hkv, d)).astype(store) for _ in range(layers)]
    nv = [rng.integers(0, hi, (pool * page, hkv, d)).astype(store) for _ in range(layers)]
    fp8 = kv == 3
    nks = [rng.random(pool * hkv, dtype=np.float32) for _ in range(layers)] if fp8 else None
    nvs = [rng.random(pool * hkv, dtype=np.float32) for _ in range(layers)] if fp8 else None
    dev = lambda xs: [torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x)
                      .cuda() for x in xs] if xs is not None else None
    k, v, ks, vs = dev(nk), dev(nv), dev(nks), dev(nvs)
    t = lia.KVTransfer(lia.KVLayout(hkv, d, page, pool, kv), k, v, ks, vs)
    src = list(rng.permutation(pool)[:16])
    got = t.read_kv_pages(src)
    want = [O.kv_page_payload(nk, nv, p, page, nks, nvs, hkv=hkv) for p in src]
    assert got == want
    reused = [bytearray(t.page_bytes) for _ in src]
    assert t.read_kv_pages(src, out=reused) is not None and reused == want
    dst = list(rng.permutation(pool)[:16])
    t.write_kv_pages(list(zip(dst, got)))
    for p, payload in zip(dst, got):
        O.kv_page_store(nk, nv, p, page, payload, nks, nvs, hkv=hkv)
    for layer in range(layers):
        assert np.array_equal(k[layer].cpu().numpy().view(store), nk[layer]), layer
        assert np.array_equal(v[layer].cpu().numpy().view(store), nv[layer]), layer
        if fp8:
            assert np.array_equal(ks[layer].cpu().numpy(), nks[layer])
            assert np.array_equal(vs[layer].cpu().numpy(), nvs[layer])


def test_page_cache_evicts_and_restores_through_device_pool(lia, O):
    """The host page manager with its page I/O on the device pool (page_cache.rs:275-287
    eviction reads a page, attach restores through write_kv_pages): evicted payloads are the
    pool's bytes, and a restored prefix is bit-identical after the pool was cleared."""
    print("[case] page cache over the device pool", flush=True)
    layers, pool_pages = 3, 8
    L = lia.KVLayout(2, 128, 32, pool_pages, lia.F16)
    k = [torch.randint(-32768, 32768, (pool_pages * 32, 2, 128), dtype=torch.int16,
                       device="cuda") for _ in range(layers)]
    v = [torch.randint(-32768, 32768, (pool_pages * 32, 2, 128), dtype=torch.int16,
                       device="cuda") for _ in range(layers)]
    t = lia.KVTransfer(L, k, v)
    store = {}
    ns = bytes(range(32))
    cache = lia.PageCache(ns, pool_pages, 32, store=store, transfer=t)
    prompt = list(range(1000, 1097))                 # 3 full pages + 1 token
    seq, cached = cache.attach(prompt)
    assert cached == 0
    for pos in range(len(prompt)):
        assert cache.ensure_position(seq, pos)
    pages = seq.pages
    want = t.read_kv_pages(pages[:3])
    assert want[0] == O.kv_page_payload([x.cpu().numpy() for x in k],
                                        [x.cpu().numpy() for x in v], pages[0], 32)
    cache.seal(seq, prompt, len(prompt))
    cache.release(seq)
    cache.evict_idle()
    key, keys = ns, []
    for b in range(3):
        key = lia.prefix_key(key, prompt[32 * b:32 * (b + 1)])
        keys.append(key)
    assert [store[x] for x in keys] == [bytes(w) for w in want]
    for x in k + v:
        x.zero_()
    seq, cached = cache.attach(prompt)
    assert cached == 96 and cache.gpu_hits == 0
    assert t.read_kv_pages(seq.pages) == [bytes(w) for w in want]
    cache.release(seq)
