"""Seeded synthetic ragged batches for the benchmark configurations.

A batch is described on the host (numpy): per-sequence key counts and new-token counts,
block tables drawn from a seeded permutation of the pool's pages, and the packed
per-row metadata.  K/V/Q values are N(0,1) rounded to the storage type; large pools are
filled on the GPU with a seeded torch generator.
"""
import math
from dataclasses import dataclass, field

import numpy as np

F32, F16, BF16, FP8 = 0, 1, 2, 3


@dataclass
class Geometry:
    hq: int = 16
    hkv: int = 2
    d: int = 128
    page_size: int = 16
    kv_dtype: int = BF16
    q_dtype: int = BF16
    out_dtype: int = BF16

    @property
    def scale(self):
        return 1.0 / math.sqrt(self.d)


@dataclass
class Batch:
    geom: Geometry
    ctx: np.ndarray        # keys per sequence after this step (cached + new)
    q_len: np.ndarray      # new query rows per sequence
    pool_pages: int
    tables: list           # per sequence page list
    stride: int
    name: str = ""
    layers: int = 1
    notes: list = field(default_factory=list)
    shared: dict = field(default_factory=dict)  # sequence -> (donor, prefix pages shared)

    @property
    def n_seqs(self):
        return len(self.ctx)

    @property
    def cached(self):
        return self.ctx - self.q_len

    @property
    def n_rows(self):
        return int(self.q_len.sum())

    def cu_seqlens(self):
        return np.concatenate([[0], np.cumsum(self.q_len)]).astype(np.uint32)

    def positions(self):
        return np.concatenate([np.arange(c - q, c) for c, q in zip(self.ctx, self.q_len)]).astype(np.uint32)

    def sequences(self):
        return np.repeat(np.arange(self.n_seqs), self.q_len).astype(np.uint32)

    def flat_table(self):
        flat = np.full(self.n_seqs * self.stride, 0xFFFFFFFF, dtype=np.uint32)
        for s, t in enumerate(self.tables):
            flat[s * self.stride:s * self.stride + len(t)] = t
        return flat

    def slot_mapping(self):
        P = self.geom.page_size
        pos, seq = self.positions(), self.sequences()
        flat = self.flat_table()
        return (flat[seq * self.stride + pos // P] * P + pos % P).astype(np.uint32)

    def kv_bytes(self):
        """Algorithmic K+V bytes read by one attention pass (each sequence's keys read once;
        a shared prefix page is attended by each sequence that holds it)."""
        eb = 1 if self.geom.kv_dtype == FP8 else 2
        return int(self.ctx.sum()) * self.geom.hkv * self.geom.d * 2 * eb

    def algorithmic_bytes(self):
        """Decode roofline bytes per layer: K/V of every attended key + Q + O + block
        table (+ FP8 scales)."""
        g = self.geom
        qb = 4 if g.q_dtype == F32 else 2
        ob = 4 if g.out_dtype == F32 else 2
        pages = int(sum(-(-int(c) // g.page_size) for c in self.ctx))
        extra = pages * g.hkv * 2 * 4 if g.kv_dtype == FP8 else 0
        return self.kv_bytes() + self.n_rows * g.hq * g.d * (qb + ob) + pages * 4 + extra

    def flops(self):
        """4 * H_q * d * sum over rows of attended keys."""
        g = self.geom
        keys = int((self.positions().astype(np.int64) + 1).sum())
        return 4 * g.hq * g.d * keys


def _tables(rng, ctx, page_size, pool_pages, shared=None):
    """Block tables from a seeded permutation of the pool's pages.  `shared` maps a
    sequence to (donor sequence, n prefix pages) for prefix-cache hits."""
    need = [-(-int(c) // page_size) for c in ctx]
    perm = rng.permutation(pool_pages).astype(np.uint32)
    tables, at = [], 0
    for s, n in enumerate(need):
        if shared and s in shared:
            donor, k = shared[s]
            own = perm[at:at + n - k]
            at += n - k
            tables.append(np.concatenate([tables[donor][:k], own]).astype(np.uint32))
        else:
            tables.append(perm[at:at + n].copy())
            at += n
    if at > pool_pages:
        raise ValueError("pool too small for the batch")
    return tables


def config1(seed=0):
    """CPU plumbing: 4 sequences, ctx {17, 64, 200, 511}, one new token each, GQA 8/2,
    head_dim 64, page 16, pool of 256 pages."""
    g = Geometry(hq=8, hkv=2, d=64, page_size=16)
    ctx = np.array([17, 64, 200, 511], dtype=np.int64)
    q = np.ones(4, dtype=np.int64)
    rng = np.random.default_rng(seed)
    pool = 256
    return Batch(g, ctx, q, pool, _tables(rng, ctx, 16, pool), stride=-(-511 // 16) + 1,
                 name="cfg1_plumbing")


def config2(seed=0, layers=40):
    """Ragged bf16 decode, batch 8, contexts U[1024, 32768], GQA 16/2, d 128, page 16."""
    g = Geometry()
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1024, 32768, size=8, endpoint=True).astype(np.int64)
    q = np.ones(8, dtype=np.int64)
    pages = int(sum(-(-int(c) // 16) for c in ctx))
    pool = max(65536 // 16, pages)
    b = Batch(g, ctx, q, pool, _tables(rng, ctx, 16, pool), stride=32768 // 16,
              name="cfg2_decode_b8", layers=layers)
    if pool > 65536 // 16:
        b.notes.append(f"pool sized to {pool * 16} tokens (> 65536) to hold sum(ctx)={int(ctx.sum())}")
    return b


def config3(seed=0):
    """Mixed chunked prefill + decode: chunks (new, cached) = (512, 0), (1024, 4096),
    (2048, 8192) plus 5 decode sequences with ctx U[2048, 16384].  Prefix-cache hits share
    pages by reference count: the 4096-token cached prefix of the second chunk (256 full,
    immutable pages) is also the first 4096 tokens of the third chunk's prefix and of every
    decode sequence whose cached keys cover it, so those tables start with the same 256
    physical pages (src/inference/page_cache.rs:48-157 attaches a prefix hit that way)."""
    g = Geometry()
    rng = np.random.default_rng(seed)
    dec = rng.integers(2048, 16384, size=5, endpoint=True)
    ctx = np.array([512, 4096 + 1024, 8192 + 2048, *dec], dtype=np.int64)
    q = np.array([512, 1024, 2048, 1, 1, 1, 1, 1], dtype=np.int64)
    cached = ctx - q
    shared_pages = 4096 // 16
    shared = {s: (1, shared_pages) for s in range(2, 8) if cached[s] >= 4096}
    pages = int(sum(-(-int(c) // 16) for c in ctx)) - shared_pages * len(shared)
    pool = pages + 64
    b = Batch(g, ctx, q, pool, _tables(rng, ctx, 16, pool, shared=shared),
              stride=-(-int(ctx.max()) // 16), name="cfg3_mixed")
    b.notes.append(f"sequences {sorted(shared)} share sequence 1's first {shared_pages} pages")
    b.shared = shared
    return b


def config4(seed=0):
    """MTP verify: 32 sequences with 1 + k rows, k ~ U{1,2,3}, ctx U[512, 16384]."""
    g = Geometry()
    rng = np.random.default_rng(seed)
    k = rng.integers(1, 3, size=32, endpoint=True)
    ctx = rng.integers(512, 16384, size=32, endpoint=True).astype(np.int64)
    q = (1 + k).astype(np.int64)
    pages = int(sum(-(-int(c) // 16) for c in ctx))
    pool = pages + 64
    return Batch(g, ctx, q, pool, _tables(rng, ctx, 16, pool), stride=-(-16384 // 16),
                 name="cfg4_mtp")


def config5(seed=0):
    """FP8 KV decode: 64 sequences, ctx log-uniform [1k, 128k], e4m3 K/V with a
    per-page per-head scale."""
    g = Geometry(kv_dtype=FP8)
    rng = np.random.default_rng(seed)
    ctx = np.exp(rng.uniform(np.log(1024), np.log(131072), size=64)).astype(np.int64)
    q = np.ones(64, dtype=np.int64)
    pages = int(sum(-(-int(c) // 16) for c in ctx))
    pool = pages + 64
    return Batch(g, ctx, q, pool, _tables(rng, ctx, 16, pool), stride=131072 // 16,
                 name="cfg5_fp8_decode")


def custom(ctx, q_len, geom=None, seed=0, pool_slack=8, stride=None):
    g = geom or Geometry()
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, dtype=np.int64)
    q = np.asarray(q_len, dtype=np.int64)
    pages = int(sum(-(-int(c) // g.page_size) for c in ctx))
    pool = pages + pool_slack
    st = stride or -(-int(ctx.max()) // g.page_size)
    return Batch(g, ctx, q, pool, _tables(rng, ctx, g.page_size, pool), stride=st)
