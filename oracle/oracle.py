"""ctypes/numpy front end of the CPU oracle (oracle/lia_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the checker
and by bench.py's cpu_baseline leg.  The product path never imports this module.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblia_oracle.so")

F32, F16, BF16, FP8 = 0, 1, 2, 3
NP_STORAGE = {F32: np.float32, F16: np.uint16, BF16: np.uint16, FP8: np.uint8}

STATUS = {
    0: "ok", -1: "invalid packed row count", -2: "invalid output row count",
    -3: "output row outside packed input", -4: "too many sequence tables",
    -5: "sequence table exceeds context", -6: "physical page outside KV pool",
    -7: "invalid packed token", -8: "packed position exceeds context",
    -9: "missing sequence table", -10: "missing physical KV page",
    -11: "duplicate physical KV write",
    -12: "packed positions must be consecutive within each request",
}


class PagingLimits(C.Structure):
    _fields_ = [("max_sequences", C.c_uint32), ("context", C.c_uint32),
                ("page_size", C.c_uint32), ("pool_pages", C.c_uint32),
                ("vocabulary", C.c_uint32), ("prefill_batch", C.c_uint32)]


class PackInfo(C.Structure):
    _fields_ = [("stride", C.c_uint32), ("maximum", C.c_uint32), ("decoding", C.c_uint32),
                ("span", C.c_uint32), ("parts", C.c_uint32), ("n_groups", C.c_uint32)]


class KVLayout(C.Structure):
    _fields_ = [("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("page_size", C.c_uint32), ("pool_pages", C.c_uint32), ("dtype", C.c_int32)]


class Geom(C.Structure):
    _fields_ = [("hq", C.c_uint32), ("hkv", C.c_uint32), ("d", C.c_uint32),
                ("page_size", C.c_uint32), ("stride", C.c_uint32), ("kv_dtype", C.c_int32),
                ("scale", C.c_double)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _b  # noqa: F401  (package-relative when imported as oracle)
        _lib = C.CDLL(LIB_PATH)
        _lib.lo_f32_to_f16.restype = C.c_uint16
        _lib.lo_f32_to_f16.argtypes = [C.c_float]
        _lib.lo_f32_to_bf16.restype = C.c_uint16
        _lib.lo_f32_to_bf16.argtypes = [C.c_float]
        _lib.lo_f32_to_e4m3.restype = C.c_uint8
        _lib.lo_f32_to_e4m3.argtypes = [C.c_float]
        _lib.lo_f16_to_f32.restype = C.c_float
        _lib.lo_f16_to_f32.argtypes = [C.c_uint16]
        _lib.lo_bf16_to_f32.restype = C.c_float
        _lib.lo_bf16_to_f32.argtypes = [C.c_uint16]
        _lib.lo_e4m3_to_f32.restype = C.c_float
        _lib.lo_e4m3_to_f32.argtypes = [C.c_uint8]
        _lib.lo_decode_span.restype = C.c_uint32
        _lib.lo_decode_span.argtypes = [C.c_uint32]
        _lib.lo_decode_parts.restype = C.c_uint32
        _lib.lo_decode_parts.argtypes = [C.c_uint32, C.c_uint32]
        _lib.lo_convert.argtypes = [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_size_t]
        _lib.lo_pack_rows.restype = C.c_int
    return _lib


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def u32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


# ---------------------------------------------------------------- conversions

def convert(x, src, dst):
    x = np.ascontiguousarray(x, dtype=NP_STORAGE[src])
    out = np.empty(x.shape, dtype=NP_STORAGE[dst])
    lib().lo_convert(ptr(x), src, ptr(out), dst, x.size)
    return out


def to_f32(x, dtype):
    return convert(x, dtype, F32)


def from_f32(x, dtype):
    return convert(np.asarray(x, dtype=np.float32), F32, dtype)


# ---------------------------------------------------------------- packing

def pack_rows(limits, rows, tables, outputs=()):
    """Restates Engine::run_paged's host packing (src/inference/paging.rs:118-201).
    rows: sequence of (token, position, sequence).  Returns (status, dict)."""
    n = len(rows)
    rows_a = u32(np.array(rows, dtype=np.uint32).reshape(n, 3) if n else np.zeros((0, 3)))
    lens = u32([len(t) for t in tables])
    data = u32(np.concatenate([np.asarray(t, dtype=np.uint32) for t in tables]) if tables and sum(map(len, tables)) else np.zeros(1))
    outs = u32(outputs if len(outputs) else np.zeros(1))
    stride = (limits.context + limits.page_size - 1) // limits.page_size
    cap = max(n, 1)
    positions = np.zeros(cap, np.uint32)
    sequences = np.zeros(cap, np.uint32)
    flat = np.zeros(max(limits.max_sequences * stride, 1), np.uint32)
    groups = np.zeros((cap, 3), np.uint32)
    cu = np.zeros(cap + 1, np.uint32)
    slots = np.zeros(cap, np.uint32)
    info = PackInfo()
    st = lib().lo_pack_rows(C.byref(limits), ptr(rows_a), n, ptr(data), ptr(lens), len(tables),
                            ptr(outs), len(outputs), ptr(positions), ptr(sequences), ptr(flat),
                            ptr(groups), ptr(cu), ptr(slots), C.byref(info))
    if st != 0:
        return st, None
    g = info.n_groups
    return 0, dict(positions=positions[:n], sequences=sequences[:n], flat=flat,
                   groups=groups[:g].copy(), cu_seqlens=cu[:g + 1].copy(), slot_mapping=slots[:n],
                   stride=info.stride, maximum=info.maximum, decoding=bool(info.decoding),
                   span=info.span, parts=info.parts)


def decode_span(tokens):
    return lib().lo_decode_span(tokens)


def decode_parts(tokens, span):
    return lib().lo_decode_parts(tokens, span)


# ---------------------------------------------------------------- KV append

def kv_append(layout, positions, sequences, pages, stride, k, v, kc, vc, src_dtype=F32,
              slot_mapping=None, k_scales=None, v_scales=None):
    """llama_cache_paged (src/gpu/kernels/llama.rs:162-183), in place on kc/vc."""
    rows = k.shape[0]
    k = np.ascontiguousarray(k, dtype=NP_STORAGE[src_dtype])
    v = np.ascontiguousarray(v, dtype=NP_STORAGE[src_dtype])
    positions, sequences, pages = u32(positions), u32(sequences), u32(pages)
    sm = u32(slot_mapping) if slot_mapping is not None else None
    lib().lo_kv_append(C.byref(layout), rows, ptr(positions), ptr(sequences), ptr(pages),
                       C.c_uint32(stride), ptr(sm), src_dtype, ptr(k), ptr(v), ptr(kc), ptr(vc),
                       ptr(k_scales), ptr(v_scales))


def kv_quantize_pages(layout, page_ids, k, v, kc, vc, k_scales, v_scales, src_dtype=F32):
    page_ids = u32(page_ids)
    k = np.ascontiguousarray(k, dtype=NP_STORAGE[src_dtype])
    v = np.ascontiguousarray(v, dtype=NP_STORAGE[src_dtype])
    lib().lo_kv_quantize_pages(C.byref(layout), len(page_ids), ptr(page_ids), src_dtype, ptr(k),
                               ptr(v), ptr(kc), ptr(vc), ptr(k_scales), ptr(v_scales))


# ---------------------------------------------------------------- attention

def geom(hq, hkv, d, page_size, stride, kv_dtype, scale=None):
    return Geom(hq, hkv, d, page_size, stride, kv_dtype,
                float(scale if scale is not None else 1.0 / np.sqrt(d)))


def attention_f64(g, positions, sequences, pages, q, kc, vc, k_scales=None, v_scales=None):
    """f64 softmax attention on the stored K/V (src/gpu/llama_attention.rs:253-284)."""
    positions, sequences, pages = u32(positions), u32(sequences), u32(pages)
    q = np.ascontiguousarray(q, dtype=np.float32)
    rows = positions.size
    out = np.zeros((rows, g.hq, g.d), np.float64)
    lib().lo_attention_f64(C.byref(g), rows, ptr(positions), ptr(sequences), ptr(pages), ptr(q),
                           ptr(kc), ptr(vc), ptr(k_scales), ptr(v_scales), ptr(out))
    return out


def attention_partial(g, query_start, queries, parts, span, positions, sequences, pages, q, kc, vc,
                      k_scales=None, v_scales=None):
    """llama_attention_partial (src/gpu/kernels/llama.rs:63-159), reference record format."""
    positions, sequences, pages = u32(positions), u32(sequences), u32(pages)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros((queries * g.hq * parts, g.d + 2), np.float32)
    lib().lo_attention_partial(C.byref(g), query_start, queries, parts, span, ptr(positions),
                               ptr(sequences), ptr(pages), ptr(q), ptr(kc), ptr(vc),
                               ptr(k_scales), ptr(v_scales), ptr(out))
    return out


def merge(hq, d, query_start, queries, parts, partial, out):
    """llama_attention_merge (src/gpu/kernels/llama.rs:201-290), in place on out."""
    partial = np.ascontiguousarray(partial, dtype=np.float32)
    lib().lo_merge(hq, d, query_start, queries, parts, ptr(partial), ptr(out))


def baseline_lib(path):
    """The oracle built by build.build_baseline (-O3 -march=native) for timing on this host."""
    b = C.CDLL(path)
    b.lo_omp_threads.restype = C.c_int
    return b


def paged_attention_f32(g, positions, sequences, pages, q, kc, vc, span=256, k_scales=None,
                        v_scales=None, lib_=None):
    """Split-K scalar attention + merge over every row (the CPU baseline); lib_ selects a
    build of the oracle other than the checker's (baseline_lib)."""
    positions, sequences, pages = u32(positions), u32(sequences), u32(pages)
    q = np.ascontiguousarray(q, dtype=np.float32)
    rows = positions.size
    maxparts = int((positions.max() + span) // span) if rows else 1
    work = np.zeros(rows * g.hq * maxparts * (g.d + 2), np.float32)
    out = np.zeros((rows, g.hq, g.d), np.float32)
    (lib_ or lib()).lo_paged_attention_f32(C.byref(g), rows, span, ptr(positions), ptr(sequences), ptr(pages),
                                 ptr(q), ptr(kc), ptr(vc), ptr(k_scales), ptr(v_scales), ptr(work),
                                 C.c_size_t(work.size), ptr(out))
    return out


# ---------------------------------------------------------------- RoPE / gather

def coefficients(positions, base=5e6):
    positions = u32(positions)
    out = np.zeros(positions.size * 128, np.float32)
    lib().lo_coefficients(positions.size, C.c_float(base), ptr(positions), ptr(out))
    return out


def rope_coefficients(positions, head_dim, base=5e6):
    positions = u32(positions)
    out = np.zeros(positions.size * head_dim, np.float32)
    lib().lo_rope_coefficients(positions.size, head_dim, C.c_float(base), ptr(positions), ptr(out))
    return out


def rope_kv_append(layout, hq, positions, sequences, pages, stride, coeffs, combined, query,
                   query_dtype, kc, vc, slot_mapping=None, k_scales=None, v_scales=None):
    """Generalised rotary_cache (llama_position.rs:49-118), in place on query/kc/vc."""
    positions, sequences, pages = u32(positions), u32(sequences), u32(pages)
    sm = u32(slot_mapping) if slot_mapping is not None else None
    coeffs = np.ascontiguousarray(coeffs, dtype=np.float32)
    combined = np.ascontiguousarray(combined, dtype=np.float32)
    rows = positions.size
    lib().lo_rope_kv_append(C.byref(layout), hq, rows, ptr(positions), ptr(sequences), ptr(pages),
                            C.c_uint32(stride), ptr(sm), ptr(coeffs), ptr(combined), ptr(query),
                            query_dtype, ptr(kc), ptr(vc), ptr(k_scales), ptr(v_scales))


def rope(heads, positions, x, base=5e6):
    positions = u32(positions)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    lib().lo_rope(heads, C.c_float(base), x.size, ptr(positions), ptr(x), ptr(out))
    return out


def rotary_cache(rows, stride, page_size, positions, sequences, pages, coeffs, combined, query,
                 keys, values):
    positions, sequences, pages = u32(positions), u32(sequences), u32(pages)
    coeffs = np.ascontiguousarray(coeffs, dtype=np.float32)
    combined = np.ascontiguousarray(combined, dtype=np.float32)
    lib().lo_rotary_cache(rows, stride, page_size, ptr(positions), ptr(sequences), ptr(pages),
                          ptr(coeffs), ptr(combined), ptr(query), ptr(keys), ptr(values))


def gather(indices, x, width):
    indices = u32(indices)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(indices.size * width, np.float32)
    lib().lo_gather(indices.size, width, ptr(indices), ptr(x), ptr(out))
    return out


def kv_page_payload(k_planes, v_planes, page, page_size, k_scales=None, v_scales=None, hkv=0):
    """Wire payload of one physical page (transfer_kv_pages_raw, src/inference/
    paging_transfer.rs:80-99): for layer l and plane p (K=0, V=1) the bytes
    [page * page_size, (page + 1) * page_size) token rows of that plane land at
    (2 * l + p) * plane_bytes.  FP8 pools append the page's [layer][plane][hkv] f32 scales
    (no counterpart in the reference, which has no FP8 pool).  Planes are numpy arrays of
    [pool_tokens][hkv][d] storage elements."""
    parts = []
    for k, v in zip(k_planes, v_planes):
        for plane in (k, v):
            parts.append(np.ascontiguousarray(plane[page * page_size:(page + 1) * page_size])
                         .view(np.uint8).reshape(-1))
    if k_scales is not None:
        for ks, vs in zip(k_scales, v_scales):
            for s in (ks, vs):
                parts.append(np.ascontiguousarray(s[page * hkv:(page + 1) * hkv], np.float32)
                             .view(np.uint8))
    return np.concatenate(parts).tobytes()


def kv_page_store(k_planes, v_planes, page, page_size, payload, k_scales=None, v_scales=None,
                  hkv=0):
    """Inverse of kv_page_payload: writes one payload into the planes in place (the upload
    direction of the same copies, paging_transfer.rs:94-97)."""
    raw = np.frombuffer(payload, np.uint8)
    at = 0
    for k, v in zip(k_planes, v_planes):
        for plane in (k, v):
            rows = plane[page * page_size:(page + 1) * page_size]
            n = rows.nbytes
            rows[...] = raw[at:at + n].view(plane.dtype).reshape(rows.shape)
            at += n
    if k_scales is not None:
        for ks, vs in zip(k_scales, v_scales):
            for s in (ks, vs):
                s[page * hkv:(page + 1) * hkv] = raw[at:at + 4 * hkv].view(np.float32)
                at += 4 * hkv
    assert at == raw.size, "payload extent"
