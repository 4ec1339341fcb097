"""CPU tests of the host page manager (lia_page_cache_*, lia_prefix_key, lia_schedule_rows):
keys against SHA-256, a randomized differential run against the oracle restatement
(oracle/page_cache.py) with brute-force invariants after every operation, and one scenario
per rule of src/inference/page_cache.rs."""
import hashlib

import numpy as np
import pytest

from oracle import page_cache as OP


def _sha(parent, tokens):
    return hashlib.sha256(b"lia-kv-prefix-v1" + bytes(parent) + len(tokens).to_bytes(8, "little")
                          + b"".join(int(t).to_bytes(4, "little") for t in tokens)).digest()


@pytest.mark.parametrize("n", [0, 1, 13, 32, 100, 1000])
def test_prefix_key_is_sha256_of_reference_bytes(lia, n):
    rng = np.random.default_rng(n)
    parent = rng.integers(0, 256, 32, dtype=np.uint8).tobytes()
    tokens = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    want = _sha(parent, tokens)
    assert OP.prefix_key(parent, tokens) == want
    assert lia.prefix_key(parent, tokens) == want
    # chained keys differ with the parent and with the count
    assert lia.prefix_key(want, tokens) != want


def _payload(tag, page_bytes=16):
    return bytes([(tag * 37 + i) % 256 for i in range(page_bytes)])


class Pair:
    """The product cache and the oracle driven with the same operations."""

    def __init__(self, lia, pages, P, ns=b"\x07" * 32):
        self.lia, self.P = lia, P
        self.store_c, self.store_o = {}, {}
        self.pool_c, self.pool_o = {}, {}
        self.c = lia.PageCache(ns, pages, P, store=self.store_c, pool=self.pool_c, page_bytes=16)
        self.o = OP.PageCache(ns, pages, P, store=self.store_o, pool=self.pool_o)
        self.seqs = {}          # id -> (product Sequence, oracle Sequence, tokens, computed)
        self.next = 0

    def check(self):
        c, o = self.c, self.o
        assert c.available_pages() == o.available_pages()
        assert (c.gpu_hits, c.evictions) == (o.gpu_hits, o.evictions)
        assert self.store_c == self.store_o
        for sid, (sc, so, _, _) in self.seqs.items():
            assert sc.pages == so.pages, sid
        # oracle invariants: users = pages held by live sequences; prefixes = keyed pages
        held = np.zeros(len(o.users), int)
        for _, so, _, _ in self.seqs.values():
            for p in so.pages:
                held[p] += 1
        assert list(held) == o.users
        assert {k: p for p, k in enumerate(o.key) if k is not None} == o.prefixes
        assert o.available_pages() == sum(1 for u in o.users if u == 0)

    def attach(self, tokens):
        sc, cc = self.c.attach(tokens)
        so, co = self.o.attach(tokens)
        assert cc == co
        sid = self.next
        self.next += 1
        self.seqs[sid] = [sc, so, list(tokens), co]
        return sid

    def step(self, sid, n):
        sc, so, tokens, computed = self.seqs[sid]
        end = min(computed + n, len(tokens))
        done = computed
        for pos in range(computed, end):
            a = self.c.ensure_position(sc, pos)
            b = self.o.ensure_position(so, pos)
            assert a == b
            if not a:
                break
            done += 1
        for p in sc.pages[len(so.keys):]:
            self.pool_c.setdefault(p, _payload(p))
        for p in so.pages[len(so.keys):]:
            self.pool_o.setdefault(p, _payload(p))
        self.c.seal(sc, tokens, done)
        self.o.seal(so, tokens, done)
        self.seqs[sid][3] = done

    def release(self, sid):
        sc, so, _, _ = self.seqs.pop(sid)
        self.c.release(sc)
        self.o.release(so)

    def evict_idle(self):
        self.c.evict_idle()
        self.o.evict_idle()


@pytest.mark.parametrize("seed", range(6))
def test_differential_against_oracle(lia, seed):
    rng = np.random.default_rng(seed)
    P = 4
    pair = Pair(lia, pages=int(rng.integers(6, 40)), P=P)
    # a few shared prompt families so prefixes collide, restore and get evicted
    families = [list(rng.integers(0, 50, 60)) for _ in range(3)]
    for _ in range(300):
        op = rng.random()
        if op < 0.3 and len(pair.seqs) < 6:
            f = families[int(rng.integers(0, 3))]
            n = int(rng.integers(1, 60))
            tail = list(rng.integers(0, 50, int(rng.integers(0, 9))))
            tokens = f[:n] + tail
            assert pair.c.can_fit(tokens) == pair.o.can_fit(tokens)
            pair.attach(tokens)
        elif op < 0.75 and pair.seqs:
            sid = list(pair.seqs)[int(rng.integers(0, len(pair.seqs)))]
            pair.step(sid, int(rng.integers(1, 12)))
        elif op < 0.95 and pair.seqs:
            sid = list(pair.seqs)[int(rng.integers(0, len(pair.seqs)))]
            pair.release(sid)
        else:
            pair.evict_idle()
        pair.check()
    for sid in list(pair.seqs):
        pair.release(sid)
    pair.check()
    assert pair.c.available_pages() == len(pair.o.users)


def _sealed(lia, cache, tokens, pool):
    """A request that computed every token and sealed its full pages, then released."""
    seq, _ = cache.attach(tokens)
    for pos in range(len(tokens)):
        assert cache.ensure_position(seq, pos)
    for p in seq.pages:
        pool.setdefault(p, _payload(p))
    cache.seal(seq, tokens, len(tokens))
    pages = seq.pages
    cache.release(seq)
    return pages


def test_full_prefix_hit_keeps_last_token_uncached(lia):
    """page_cache.rs:54-55: the final token is never served from cache, so a prompt of
    exactly k pages reuses k - 1 of them."""
    pool = {}
    cache = lia.PageCache(b"\0" * 32, 16, 32, pool=pool, page_bytes=16)
    tokens = list(range(96))
    first = _sealed(lia, cache, tokens, pool)
    seq, cached = cache.attach(tokens)
    assert cached == 64 and seq.pages == first[:2] and cache.gpu_hits == 2
    seq2, cached2 = cache.attach(tokens + [7])
    assert cached2 == 96 and seq2.pages == first
    assert cache.available_pages() == 16 - 3


def test_retain_before_allocate_protects_later_pages(lia):
    """page_cache.rs:65-66: restoring an early hole must not evict a later resident page of
    the same prefix.  The prompt's first page lives in the store only; its pages 1 and 2 are
    the least recently used idle pages of a pool with no unkeyed page left, so the restore
    must take the next idle page (page 3) instead."""
    store, pool = {}, {}
    P, ns = 4, b"\1" * 32
    cache = lia.PageCache(ns, 5, P, store=store, pool=pool, page_bytes=16)
    prompt = list(range(100, 113))                   # 3 full pages + 1 token
    assert _sealed(lia, cache, prompt, pool) == [0, 1, 2, 3]
    other, _ = cache.attach(list(range(200, 209)))   # 9 tokens: pages 3, 4 and LRU page 0
    for pos in range(9):
        assert cache.ensure_position(other, pos)
    assert other.pages == [3, 4, 0] and cache.evictions == 1
    key0 = OP.prefix_key(ns, prompt[:P])
    assert store[key0] == _payload(0)
    cache.seal(other, list(range(200, 209)), 9)      # pages 3, 4 keyed, newer than 1, 2
    cache.release(other)
    hold, _ = cache.attach([7])
    assert cache.ensure_position(hold, 0) and hold.pages == [0]
    seq, cached = cache.attach(prompt)
    assert cached == 12 and seq.pages == [3, 1, 2]
    assert cache.evictions == 2 and cache.gpu_hits == 2
    assert pool[3] == _payload(0)                    # the restored payload


def test_restore_windows_of_sixteen_and_store_miss(lia):
    """page_cache.rs:77-140: restores go to the pool in windows of at most 16 pages; a store
    miss ends the cached prefix there."""
    store, pool = {}, {}
    P, ns = 2, b"\2" * 32
    cache = lia.PageCache(ns, 48, P, store=store, pool=pool, page_bytes=16)
    prompt = list(range(81))                         # 40 full pages + 1 token
    _sealed(lia, cache, prompt, pool)
    cache.evict_idle()
    assert len(store) == 40 and cache.available_pages() == 48
    fresh = lia.PageCache(ns, 48, P, store=store, pool={}, page_bytes=16)
    calls = []
    inner = fresh._write

    def counting(ctx, n, pages, payloads):
        calls.append(n)
        return inner(ctx, n, pages, payloads)
    fresh._write = counting
    seq, cached = fresh.attach(prompt)
    assert cached == 80 and calls == [16, 16, 8]
    key = ns
    for b, p in enumerate(seq.pages):
        key = OP.prefix_key(key, prompt[b * P:(b + 1) * P])
        assert fresh.pool[p] == store[key]
    key1 = OP.prefix_key(OP.prefix_key(ns, prompt[:2]), prompt[2:4])
    del store[key1]
    third = lia.PageCache(ns, 48, P, store=store, pool={}, page_bytes=16)
    seq3, cached3 = third.attach(prompt)
    assert cached3 == 2 and len(seq3.pages) == 1


def test_allocation_order_and_pressure(lia):
    """page_cache.rs:250-273: lowest idle unkeyed page first, then the least recently used
    idle keyed page; ensure_position refuses when the pool cannot hold the request."""
    pool = {}
    cache = lia.PageCache(b"\3" * 32, 4, 4, pool=pool, page_bytes=16)
    s, _ = cache.attach([1] * 3)
    assert cache.ensure_position(s, 5) and s.pages == [0, 1]
    assert not cache.ensure_position(s, 4 * 4)       # needs 3 more, 2 idle
    assert cache.ensure_position(s, 15) and s.pages == [0, 1, 2, 3]
    assert cache.available_pages() == 0
    t, _ = cache.attach([2] * 3)
    assert not cache.ensure_position(t, 0)
    cache.seal(s, [1] * 16, 16)                      # all four pages keyed
    cache.release(s)
    # seal touched blocks 0..3 in order, so page 0 is the least recently used keyed page
    assert cache.ensure_position(t, 0) and t.pages == [0]
    assert cache.evictions == 1
    o = OP.PageCache(b"\3" * 32, 4, 4, pool={})
    so, _ = o.attach([1] * 3)
    assert o.ensure_position(so, 15)
    to, _ = o.attach([2] * 3)
    o.seal(so, [1] * 16, 16)
    o.release(so)
    assert o.ensure_position(to, 0) and to.pages == [0]


def test_seal_shares_an_existing_prefix_page(lia):
    """page_cache.rs:218-224: two requests computing the same block end up on one page."""
    pool = {}
    cache = lia.PageCache(b"\4" * 32, 8, 4, pool=pool, page_bytes=16)
    a, _ = cache.attach([5] * 9)
    b, _ = cache.attach([5] * 9)
    for s in (a, b):
        for pos in range(9):
            assert cache.ensure_position(s, pos)
    assert a.pages[:2] != b.pages[:2]
    cache.seal(a, [5] * 9, 9)
    before = cache.available_pages()
    cache.seal(b, [5] * 9, 9)
    assert b.pages[:2] == a.pages[:2]
    assert cache.available_pages() == before + 2


def test_error_statuses(lia):
    with pytest.raises(lia.LiaError) as e:
        lia.PageCache(b"\0" * 32, 0, 32)
    assert e.value.status == -19
    cache = lia.PageCache(b"\0" * 32, 4, 4, pool={}, page_bytes=16)
    s, _ = cache.attach([1, 2, 3])
    with pytest.raises(lia.LiaError) as e:
        cache.seal(s, [1, 2, 3], 4)                  # computed beyond the tokens
    assert e.value.status == -15
    with pytest.raises(lia.LiaError) as e:
        cache.seal(s, [1, 2, 3, 4, 5], 5)            # computed beyond the pages
    assert e.value.status == -15


def test_failing_store_callback_releases_the_sequence(lia):
    class Broken(dict):
        def get(self, key):
            raise IOError("disk gone")
    pool = {}
    store = {}
    cache = lia.PageCache(b"\5" * 32, 8, 4, store=store, pool=pool, page_bytes=16)
    _sealed(lia, cache, list(range(9)), pool)
    cache.evict_idle()
    broken = lia.PageCache(b"\5" * 32, 8, 4, store=Broken(store), pool={}, page_bytes=16)
    with pytest.raises(lia.LiaError) as e:
        broken.attach(list(range(9)))
    assert e.value.status == -24
    assert broken.available_pages() == 8


def test_schedule_rows_matches_oracle(lia):
    """schedule.rs:5-60 on a mix of a long prefill, decodes, a closed stream and an empty
    slot, with a pool too small for everything."""
    P = 4
    rng = np.random.default_rng(3)
    ns = b"\6" * 32
    c = lia.PageCache(ns, 12, P, pool={}, page_bytes=16)
    o = OP.PageCache(ns, 12, P, pool={})
    prompts = [list(rng.integers(0, 99, n)) for n in (30, 3, 5, 7)]
    reqs_c, reqs_o = [], []
    for i, t in enumerate(prompts):
        sc, _ = c.attach(t)
        so, _ = o.attach(t)
        computed = 0 if i == 0 else len(t) - 1
        for pos in range(computed):
            assert c.ensure_position(sc, pos) == o.ensure_position(so, pos)
        reqs_c.append(dict(tokens=t, computed=computed, sequence=sc, closed=(i == 2)))
        reqs_o.append(dict(tokens=t, computed=computed, sequence=so, closed=(i == 2)))
    reqs_c.insert(1, None)
    reqs_o.insert(1, None)
    for batch in (16, 3):
        got = c.schedule_rows(reqs_c, batch)
        want = OP.schedule_rows(o, reqs_o, batch)
        assert got == tuple(want)
        assert reqs_c[3].get("done") and reqs_o[3].get("done")
        for rc, ro in zip(reqs_c, reqs_o):
            if rc is not None:
                assert rc["sequence"].pages == ro["sequence"].pages
        for slot, computed, _ in got[2]:
            reqs_c[slot]["computed"] = computed
            reqs_o[slot]["computed"] = computed
    assert c.available_pages() == o.available_pages()
