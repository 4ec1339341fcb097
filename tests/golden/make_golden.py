"""Writes the golden fixtures of this directory from the CPU oracle (oracle/lia_oracle.c).

    python tests/golden/make_golden.py

Every input is a closed form or a seeded numpy draw, so the fixtures hold only what the
oracle computed plus SHA-256 digests of the inputs they were computed from:

- cfg1.npz: the CPU plumbing case (4 sequences, ctx 17/64/200/511, GQA 8/2, head_dim 64,
  page 16, bf16 K/V/Q, seed 0): the packing of its rows (paging.rs:118-201), the float64
  softmax of the stored K/V (llama_attention.rs:253-284) and the scalar split-K path in f32
  (kernels/llama.rs:63-159 + 201-290, span 32).
- reference_attention.npz: the float64 attention of the reference's known-answer inputs
  (llama_attention.rs:212-252: value(), reversed tables, 17 rows up to 16,385 keys).
- reference_merge.npz: the merge of the reference's merge vectors (llama_merge.rs:91-108)
  for 1, 2, 3, 4, 8 and 16 parts, guard rows included.
- reference_rotary.npz: the fused RoPE + append of the reference's fixture
  (llama_position.rs:128-152): rotated queries (f32 bits) and the five appended K/V rows.

tests/test_golden.py checks that the oracle still reproduces these files; the GPU tests in
tests/test_gpu_golden.py check the HIP library against them without running the oracle."""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

F32, F16, BF16, FP8 = 0, 1, 2, 3


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def cfg1_inputs(O, wl):
    """The seeded bf16 inputs of config 1 (same draws as tests/gpu_data.Case, seed 0)."""
    b = wl.config1(seed=0)
    g = b.geom
    rng = np.random.default_rng(1000)
    tokens = b.pool_pages * g.page_size
    kf = rng.standard_normal((tokens, g.hkv, g.d), dtype=np.float32)
    vf = rng.standard_normal((tokens, g.hkv, g.d), dtype=np.float32)
    qf = rng.standard_normal((b.n_rows, g.hq, g.d), dtype=np.float32)
    kc = O.from_f32(kf, BF16).reshape(-1)
    vc = O.from_f32(vf, BF16).reshape(-1)
    q_store = O.from_f32(qf, BF16)
    return b, kc, vc, q_store


def make_cfg1(O, wl):
    b, kc, vc, q_store = cfg1_inputs(O, wl)
    g = b.geom
    P = g.page_size
    context = int(b.stride * P)
    rows = [(0, int(p), int(s)) for p, s in zip(b.positions(), b.sequences())]
    lim = O.PagingLimits(b.n_seqs, context, P, b.pool_pages, 1, b.n_rows)
    st, packed = O.pack_rows(lim, rows, [t.tolist() for t in b.tables])
    assert st == 0, st
    geo = O.geom(g.hq, g.hkv, g.d, P, b.stride, BF16, g.scale)
    q32 = O.to_f32(q_store, BF16)
    f64 = O.attention_f64(geo, packed["positions"], packed["sequences"], packed["flat"], q32, kc, vc)
    f32 = O.paged_attention_f32(geo, packed["positions"], packed["sequences"], packed["flat"], q32,
                                kc, vc, span=32)
    return dict(inputs_sha256=np.array(digest(kc, vc, q_store)),
                ctx=b.ctx.astype(np.uint32), q_len=b.q_len.astype(np.uint32),
                cached=b.cached.astype(np.uint32), stride=np.uint32(b.stride),
                pool_pages=np.uint32(b.pool_pages),
                tables=np.concatenate([np.asarray(t, np.uint32) for t in b.tables]),
                table_lens=np.array([len(t) for t in b.tables], np.uint32),
                positions=packed["positions"], sequences=packed["sequences"], flat=packed["flat"],
                cu_seqlens=packed["cu_seqlens"], slot_mapping=packed["slot_mapping"],
                out_f64=f64, out_split_f32=f32)


def make_reference_attention(O):
    from test_oracle import _reference_vectors
    stride, pos, seq, tables, keys, vals, q, _ = _reference_vectors()
    kc = keys.astype(np.float16).view(np.uint16)
    vc = vals.astype(np.float16).view(np.uint16)
    g = O.geom(16, 2, 128, 32, stride, F16, 1.0 / np.sqrt(128.0))
    f64 = O.attention_f64(g, pos, seq, tables, q, kc, vc)
    return dict(inputs_sha256=np.array(digest(kc, vc, q, tables)), positions=pos, sequences=seq,
                out_f32=f64.astype(np.float32))


def merge_partial(parts):
    """llama_merge.rs:91-108: 48 (query, head) groups of `parts` records of 130 floats."""
    partial = np.zeros((3 * 16 * parts, 130), np.float32)
    for group in range(48):
        for p in range(parts):
            at = group * parts + p
            partial[at, :128] = ((group * 7 + p * 13 + np.arange(128) * 17) % 59) / 32.0 - 1.0
            valid = p == 0 or (group + p) % 3 != 0
            partial[at, 128] = (group % 7 + p) / 8.0 if valid else -np.inf
            partial[at, 129] = 0.25 + p / 16.0 if valid else 0.0
    return partial


MERGE_PARTS = (1, 2, 3, 4, 8, 16)


def make_reference_merge(O):
    d = {}
    for parts in MERGE_PARTS:
        out = np.full((9, 16, 128), 7.0, np.float32)  # guard rows around query_start 5
        O.merge(16, 128, 5, 3, parts, merge_partial(parts), out)
        d[f"out_parts{parts}"] = out
    return d


def rotary_inputs():
    """llama_position.rs:132-152."""
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
    slots = np.array([int(tables[s * 4096 + p // 32]) * 32 + int(p) % 32
                      for p, s in zip(positions, sequences)], np.uint32)
    return positions, sequences, tables, combined, slots


def make_reference_rotary(O):
    positions, sequences, tables, combined, slots = rotary_inputs()
    coeffs = O.coefficients(positions)
    query = np.zeros(5 * 2048, np.float32)
    keys = np.zeros(8 * 32 * 256, np.uint16)
    values = np.zeros_like(keys)
    O.rotary_cache(5, 4096, 32, positions, sequences, tables, coeffs, combined, query, keys, values)
    return dict(inputs_sha256=np.array(digest(combined, tables)), slots=slots,
                query_bits=query.view(np.uint32),
                k_rows=keys.reshape(-1, 256)[slots], v_rows=values.reshape(-1, 256)[slots])


def build_all():
    from oracle import oracle as O
    from conftest import load_package
    load_package()
    import lia_rs_amd.workloads as wl
    return {"cfg1.npz": make_cfg1(O, wl),
            "reference_attention.npz": make_reference_attention(O),
            "reference_merge.npz": make_reference_merge(O),
            "reference_rotary.npz": make_reference_rotary(O)}


def main():
    for name, arrays in build_all().items():
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
