"""Host side of the MI355X paged continuous-batching attention path.

A thin ctypes layer over liblia_hip.so (the C ABI declared in include/lia_hip.h) plus a
small engine object that mirrors the reference engine's paged entry points
(src/inference/paging.rs: Engine::configure_paging, the packing half of
Engine::run_paged; src/inference/llama.rs: the attention half of
llama_attention_selected).  PyTorch is used only for device memory and streams.

Importing this module requires the built library: there is no fallback path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblia_hip.so")

F32, F16, BF16, FP8 = 0, 1, 2, 3
NONE = 0xFFFFFFFF

ERRORS = {
    -1: "invalid packed row count", -2: "invalid output row count",
    -3: "output row outside packed input", -4: "too many sequence tables",
    -5: "sequence table exceeds context", -6: "physical page outside KV pool",
    -7: "invalid packed token", -8: "packed position exceeds context",
    -9: "missing sequence table", -10: "missing physical KV page",
    -11: "duplicate physical KV write",
    -12: "packed positions must be consecutive within each request",
    -13: "invalid KV transfer window", -14: "duplicate KV transfer destination",
    -15: "invalid computed prefix extent", -16: "attempted to overwrite immutable KV page",
    -17: "KV page reference underflow", -18: "cannot evict an active KV page",
    -24: "page store callback failed",
    -25: "invalid sampling settings", -26: "invalid sampling logits",
    -27: "empty sampling distribution", -28: "duplicate sampling candidate",
    -29: "invalid nucleus normalizer, mass or candidates",
    -19: "invalid paging configuration", -20: "invalid argument", -21: "unaligned buffer",
    -22: "workspace exhausted", -23: "unsupported geometry", -30: "HIP runtime error",
}


class LiaError(RuntimeError):
    def __init__(self, status, where=""):
        self.status = status
        super().__init__(f"{where}: {ERRORS.get(status, 'status %d' % status)} ({status})")


class PagedRow(C.Structure):
    """PagedRow (src/inference/paging.rs:7-11)."""
    _fields_ = [("token", C.c_uint32), ("position", C.c_uint32), ("sequence", C.c_uint32)]


class Group(C.Structure):
    """Query group (src/inference/llama_plan.rs:2-6)."""
    _fields_ = [("start", C.c_uint32), ("count", C.c_uint32), ("maximum", C.c_uint32)]


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


MAX_LAYERS = 128


class KVPlanes(C.Structure):
    """Per-layer plane addresses of one KV pool (lia_kv_planes)."""
    _fields_ = [("n_layers", C.c_uint32), ("k", C.c_void_p * MAX_LAYERS),
                ("v", C.c_void_p * MAX_LAYERS), ("k_scales", C.c_void_p * MAX_LAYERS),
                ("v_scales", C.c_void_p * MAX_LAYERS)]


LOAD_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_uint8), C.POINTER(C.c_void_p))
PUT_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_uint8), C.c_void_p)
READ_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_void_p)
WRITE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32),
                       C.POINTER(C.c_void_p))


class PageIO(C.Structure):
    _fields_ = [("ctx", C.c_void_p), ("page_bytes", C.c_size_t), ("load", LOAD_FN),
                ("put", PUT_FN), ("read_page", READ_FN), ("write_pages", WRITE_FN)]


class Request(C.Structure):
    """One active slot of the paged runtime (lia_request)."""
    _fields_ = [("tokens", C.c_void_p), ("n_tokens", C.c_size_t), ("computed", C.c_size_t),
                ("sequence", C.c_void_p), ("active", C.c_int32), ("closed", C.c_int32),
                ("done", C.c_int32), ("reserved", C.c_int32)]


class Update(C.Structure):
    _fields_ = [("slot", C.c_uint32), ("computed", C.c_uint64), ("output", C.c_uint32)]


class AttentionConfig(C.Structure):
    _fields_ = [("num_q_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("page_size", C.c_uint32),
                ("pool_pages", C.c_uint32), ("stride", C.c_uint32), ("q_dtype", C.c_int32),
                ("kv_dtype", C.c_int32), ("out_dtype", C.c_int32), ("scale", C.c_float),
                ("max_seqs", C.c_uint32), ("max_rows", C.c_uint32),
                ("max_context", C.c_uint32)]


EXPORTS = {
    # name: (restype, argtypes)
    "lia_pack_rows": (C.c_int, [C.POINTER(PagingLimits), C.POINTER(PagedRow), C.c_uint32,
                                C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.c_void_p, C.POINTER(PackInfo)]),
    "lia_decode_span": (C.c_uint32, [C.c_uint32]),
    "lia_decode_parts": (C.c_uint32, [C.c_uint32, C.c_uint32]),
    "lia_pack_device": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                  C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.c_void_p]),
    "lia_pack_plan_device": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_size_t, C.c_void_p]),
    "lia_kv_append": (C.c_int, [C.POINTER(KVLayout), C.c_uint32, C.c_void_p, C.c_void_p,
                                C.c_void_p, C.c_uint32, C.c_void_p, C.c_int32, C.c_void_p,
                                C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.c_void_p]),
    "lia_kv_quantize_pages": (C.c_int, [C.POINTER(KVLayout), C.c_uint32, C.c_void_p, C.c_int32,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_void_p, C.c_void_p]),
    "lia_attention_workspace_bytes": (C.c_size_t, [C.POINTER(AttentionConfig)]),
    "lia_paged_attention": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                      C.c_void_p]),
    "lia_gather_rows": (C.c_int, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.c_void_p]),
    "lia_rope_coefficients": (C.c_int, [C.c_uint32, C.c_uint32, C.c_float, C.c_void_p,
                                        C.c_void_p, C.c_void_p]),
    "lia_rope_kv_append": (C.c_int, [C.POINTER(KVLayout), C.c_uint32, C.c_uint32, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_void_p]),
    "lia_attention_plan": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_size_t, C.c_void_p]),
    "lia_attention_partial_append": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32,
                                               C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]),
    "lia_attention_partial_append_fp8": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32,
                                                   C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                                   C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                                   C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                                   C.c_void_p, C.c_void_p]),
    "lia_attention_partial": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                        C.c_void_p, C.c_void_p]),
    "lia_attention_merge": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32,
                                      C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]),
    "lia_hbm_read": (C.c_int, [C.c_void_p, C.c_size_t, C.c_uint32, C.c_void_p, C.c_void_p]),
    "lia_paged_read": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p]),
    "lia_paged_read_sink_words": (C.c_size_t, [C.POINTER(AttentionConfig)]),
    "lia_kv_page_bytes": (C.c_size_t, [C.POINTER(KVLayout), C.c_uint32]),
    "lia_kv_transfer_bytes": (C.c_size_t, [C.POINTER(KVLayout), C.c_uint32]),
    "lia_kv_write_pages": (C.c_int, [C.POINTER(KVLayout), C.POINTER(KVPlanes), C.c_uint32,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "lia_kv_read_pages": (C.c_int, [C.POINTER(KVLayout), C.POINTER(KVPlanes), C.c_uint32,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "lia_prefix_key": (C.c_int, [C.c_char_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "lia_page_cache_create": (C.c_int, [C.c_char_p, C.c_uint32, C.c_uint32, C.POINTER(PageIO),
                                        C.POINTER(C.c_void_p)]),
    "lia_page_cache_destroy": (None, [C.c_void_p]),
    "lia_page_cache_attach": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t,
                                        C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
    "lia_page_cache_can_fit": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "lia_page_cache_available": (C.c_size_t, [C.c_void_p]),
    "lia_page_cache_ensure_position": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "lia_page_cache_seal": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t,
                                      C.c_size_t]),
    "lia_page_cache_release": (C.c_int, [C.c_void_p, C.c_void_p]),
    "lia_page_cache_evict_idle": (C.c_int, [C.c_void_p]),
    "lia_page_cache_stats": (None, [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "lia_sequence_pages": (C.c_uint32, [C.c_void_p, C.POINTER(C.POINTER(C.c_uint32))]),
    "lia_schedule_rows": (C.c_int, [C.c_void_p, C.c_uint32, C.POINTER(Request), C.c_uint32,
                                    C.POINTER(PagedRow), C.c_uint32, C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                    C.POINTER(Update), C.POINTER(C.c_uint32)]),
    "lia_sampler_create": (C.c_int, [C.c_double, C.c_uint32, C.c_double, C.c_uint64, C.c_int32,
                                     C.POINTER(C.c_void_p)]),
    "lia_sampler_destroy": (None, [C.c_void_p]),
    "lia_sampler_set_position": (None, [C.c_void_p, C.c_uint64]),
    "lia_sampler_distribution": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
                                           C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32)]),
    "lia_sampler_draw": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
                                   C.POINTER(C.c_uint32)]),
    "lia_nucleus_workspace_bytes": (C.c_size_t, [C.c_uint32, C.c_uint32]),
    "lia_nucleus_host_bytes": (C.c_size_t, [C.c_uint32, C.c_uint32]),
    "lia_nucleus_candidates": (C.c_int, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_void_p, C.c_void_p]),
    "lia_sample_host": (C.c_int, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(C.c_uint64)]),
    "lia_sample_paged": (C.c_int, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p,
                                   C.POINTER(C.c_uint64), C.c_void_p]),
    "lia_paged_attention_static": (C.c_int, [C.POINTER(AttentionConfig), C.c_uint32, C.c_uint32,
                                             C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                             C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                             C.c_void_p, C.c_void_p, C.c_void_p]),
    "lia_static_workspace_bytes": (C.c_size_t, []),
    "lia_device_cus": (C.c_uint32, []),
    "lia_init": (C.c_int, [C.c_int]),
}

_lib = None


def lib():
    """Load liblia_hip.so.  Raises if it has not been built: there is no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               "`python lia.rs_amd/build.py` (no CPU fallback exists)")
        _lib = C.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _check(status, where):
    if status != 0:
        raise LiaError(status, where)


def _dptr(t):
    """Device (or host) address of a torch tensor, None for None."""
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def torch_dtype_code(dt):
    import torch
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
            torch.uint8: FP8}[dt]


# ------------------------------------------------------------------ host packing

def pack_rows(limits, rows, tables, outputs=()):
    """Engine::run_paged host packing (src/inference/paging.rs:118-201).

    rows: iterable of (token, position, sequence); tables: list of page lists.
    Returns a dict of numpy arrays, raising LiaError with the reference's message on the
    first failing check."""
    rows = list(rows)
    n = len(rows)
    row_arr = (PagedRow * max(n, 1))(*[PagedRow(*r) for r in rows])
    lens = np.ascontiguousarray([len(t) for t in tables] or [0], dtype=np.uint32)
    data = np.ascontiguousarray(
        np.concatenate([np.asarray(t, dtype=np.uint32) for t in tables])
        if tables and sum(map(len, tables)) else np.zeros(1, np.uint32), dtype=np.uint32)
    outs = np.ascontiguousarray(list(outputs) or [0], dtype=np.uint32)
    stride = (limits.context + limits.page_size - 1) // limits.page_size
    cap = max(n, 1)
    positions = np.zeros(cap, np.uint32)
    sequences = np.zeros(cap, np.uint32)
    flat = np.zeros(max(limits.max_sequences * stride, 1), np.uint32)
    groups = (Group * cap)()
    cu = np.zeros(cap + 1, np.uint32)
    slots = np.zeros(cap, np.uint32)
    info = PackInfo()
    st = lib().lia_pack_rows(C.byref(limits), row_arr, n, data.ctypes.data, lens.ctypes.data,
                             len(tables), outs.ctypes.data, len(outputs), positions.ctypes.data,
                             sequences.ctypes.data, flat.ctypes.data, C.addressof(groups),
                             cu.ctypes.data, slots.ctypes.data, C.byref(info))
    _check(st, "pack_rows")
    g = info.n_groups
    return dict(positions=positions[:n], sequences=sequences[:n], flat=flat,
                groups=np.array([[groups[i].start, groups[i].count, groups[i].maximum]
                                 for i in range(g)], dtype=np.uint32).reshape(g, 3),
                cu_seqlens=cu[:g + 1].copy(), slot_mapping=slots[:n], stride=info.stride,
                maximum=info.maximum, decoding=bool(info.decoding), span=info.span,
                parts=info.parts)


def decode_span(tokens):
    return lib().lia_decode_span(tokens)


def decode_parts(tokens, span):
    return lib().lia_decode_parts(tokens, span)


# ------------------------------------------------------------------ device entry points

def pack_device(seq_slots, q_lens, cached, pages, stride, page_size, pool_pages, context,
                max_rows, cu_seqlens, positions, sequences, slot_mapping, status, stream=None):
    """Device packing (lia_pack_device); all arrays are int32/uint32 cuda tensors."""
    st = lib().lia_pack_device(seq_slots.numel(), _dptr(seq_slots), _dptr(q_lens), _dptr(cached),
                               _dptr(pages), stride, page_size, pool_pages, context, max_rows,
                               _dptr(cu_seqlens), _dptr(positions), _dptr(sequences),
                               _dptr(slot_mapping), _dptr(status), _stream(stream))
    _check(st, "pack_device")


def pack_plan_device(config, seq_slots, q_lens, cached, pages, n_rows, context, cu_seqlens,
                     positions, sequences, slot_mapping, status, workspace, stream=None):
    """Device packing and the attention plan in two launches (lia_pack_plan_device)."""
    st = lib().lia_pack_plan_device(C.byref(config), seq_slots.numel(), n_rows, _dptr(seq_slots),
                                    _dptr(q_lens), _dptr(cached), _dptr(pages), context,
                                    _dptr(cu_seqlens), _dptr(positions), _dptr(sequences),
                                    _dptr(slot_mapping), _dptr(status), _dptr(workspace),
                                    workspace.numel() * workspace.element_size(), _stream(stream))
    _check(st, "pack_plan_device")


def kv_append(layout, k, v, kc, vc, positions=None, sequences=None, pages=None, stride=0,
              slot_mapping=None, k_scales=None, v_scales=None, stream=None):
    """KV append scatter (lia_kv_append, semantics of llama_cache_paged)."""
    rows = k.shape[0]
    st = lib().lia_kv_append(C.byref(layout), rows, _dptr(positions), _dptr(sequences),
                             _dptr(pages), stride, _dptr(slot_mapping), torch_dtype_code(k.dtype),
                             _dptr(k), _dptr(v), _dptr(kc), _dptr(vc), _dptr(k_scales),
                             _dptr(v_scales), _stream(stream))
    _check(st, "kv_append")


def kv_quantize_pages(layout, page_ids, k, v, kc, vc, k_scales, v_scales, stream=None):
    st = lib().lia_kv_quantize_pages(C.byref(layout), page_ids.numel(), _dptr(page_ids),
                                     torch_dtype_code(k.dtype), _dptr(k), _dptr(v), _dptr(kc),
                                     _dptr(vc), _dptr(k_scales), _dptr(v_scales), _stream(stream))
    _check(st, "kv_quantize_pages")


def rope_coefficients(positions, head_dim, out, base=5e6, stream=None):
    """RoPE table [rows][head_dim/2][2] (lia_rope_coefficients)."""
    st = lib().lia_rope_coefficients(positions.numel(), head_dim, C.c_float(base), _dptr(positions),
                                     _dptr(out), _stream(stream))
    _check(st, "rope_coefficients")


def rope_kv_append(layout, num_q_heads, coefficients, combined, query, kc, vc, slot_mapping=None,
                   positions=None, sequences=None, pages=None, stride=0, k_scales=None,
                   v_scales=None, stream=None):
    """Fused RoPE + KV append (lia_rope_kv_append); combined rows are q | k | v heads in f32."""
    st = lib().lia_rope_kv_append(C.byref(layout), num_q_heads, combined.shape[0],
                                  _dptr(positions), _dptr(sequences), _dptr(pages), stride,
                                  _dptr(slot_mapping), _dptr(coefficients), _dptr(combined),
                                  _dptr(query), torch_dtype_code(query.dtype), _dptr(kc), _dptr(vc),
                                  _dptr(k_scales), _dptr(v_scales), _stream(stream))
    _check(st, "rope_kv_append")


def gather_rows(indices, src, dst, stream=None):
    """dst[i] = src[indices[i]] over rows of 32-bit words (lia_gather_rows)."""
    width = src[0].numel() * src.element_size() // 4
    st = lib().lia_gather_rows(indices.numel(), width, _dptr(indices), _dptr(src), _dptr(dst),
                               _stream(stream))
    _check(st, "gather_rows")


class KVTransfer:
    """Stream-ordered page transfers of one KV pool in the reference's page wire format
    (Engine::read_kv_page / write_kv_page / write_kv_pages, src/inference/paging_transfer.rs:
    26-58): a payload is one physical page of every layer and plane, layer-major, plus the
    page's f32 scales for FP8 pools.  Owns a pinned host and a device staging buffer."""

    def __init__(self, layout, k, v, k_scales=None, v_scales=None):
        import torch
        if not 1 <= len(k) <= MAX_LAYERS or len(v) != len(k):
            raise LiaError(-20, "KVTransfer: one K and one V plane per layer")
        self.layout = layout
        self.planes = KVPlanes()
        self.planes.n_layers = len(k)
        for i in range(len(k)):
            self.planes.k[i], self.planes.v[i] = k[i].data_ptr(), v[i].data_ptr()
            if k_scales is not None:
                self.planes.k_scales[i] = k_scales[i].data_ptr()
                self.planes.v_scales[i] = v_scales[i].data_ptr()
        self._keep = (k, v, k_scales, v_scales)
        self.page_bytes = lib().lia_kv_page_bytes(C.byref(layout), len(k))
        total = lib().lia_kv_transfer_bytes(C.byref(layout), len(k))
        if self.page_bytes == 0 or total == 0:
            raise LiaError(-20, "KVTransfer: invalid pool geometry")
        self.host = torch.empty(total, dtype=torch.uint8, pin_memory=True)
        self.device = torch.empty(total, dtype=torch.uint8, device=k[0].device)

    def _ids(self, pages):
        return (C.c_uint32 * max(len(pages), 1))(*pages)

    def read_kv_pages(self, pages, stream=None, out=None):
        """Payloads (bytearray) of up to 16 distinct physical pages; `out` may supply
        writable buffers of page_bytes each to fill instead of new ones."""
        n = len(pages)
        bufs = list(out) if out is not None else [bytearray(self.page_bytes) for _ in range(n)]
        if len(bufs) != n:
            raise LiaError(-20, "read_kv_pages: one output buffer per page")
        views = [(C.c_char * self.page_bytes).from_buffer(b) for b in bufs]
        ptrs = (C.c_void_p * max(n, 1))(*[C.addressof(x) for x in views])
        st = lib().lia_kv_read_pages(C.byref(self.layout), C.byref(self.planes), n,
                                     self._ids(pages), ptrs, _dptr(self.host),
                                     _dptr(self.device), _stream(stream))
        del views
        _check(st, "read_kv_pages")
        return bufs

    def read_kv_page(self, page, stream=None):
        return self.read_kv_pages([page], stream)[0]

    def write_kv_pages(self, pages, stream=None):
        """pages: [(physical page, payload bytes)], 1 to 16 distinct destinations."""
        for _, payload in pages:
            if len(payload) != self.page_bytes:
                raise LiaError(-20, "write_kv_pages: invalid saved KV page extent")
        n = len(pages)
        held = [p if isinstance(p, bytes) else bytes(p) for _, p in pages]
        ptrs = (C.c_void_p * max(n, 1))(*[C.cast(C.c_char_p(b), C.c_void_p).value
                                          for b in held])
        st = lib().lia_kv_write_pages(C.byref(self.layout), C.byref(self.planes), n,
                                      self._ids([p for p, _ in pages]), ptrs, _dptr(self.host),
                                      _dptr(self.device), _stream(stream))
        _check(st, "write_kv_pages")

    def write_kv_page(self, page, payload, stream=None):
        self.write_kv_pages([(page, payload)], stream)


def prefix_key(parent, tokens):
    """Key::prefix (src/prefix_cache.rs:61-70) through lia_prefix_key."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = C.create_string_buffer(32)
    _check(lib().lia_prefix_key(bytes(parent), t.ctypes.data, t.size, out), "prefix_key")
    return out.raw


class Sequence:
    """A sequence's pages in the cache (page_cache::Sequence); `pages` is its block-table row."""

    def __init__(self, handle):
        self.handle = handle

    @property
    def pages(self):
        p = C.POINTER(C.c_uint32)()
        n = lib().lia_sequence_pages(self.handle, C.byref(p))
        return [p[i] for i in range(n)]


class PageCache:
    """Host page manager (PageCache, src/inference/page_cache.rs:18-304) over liblia_hip.
    `store` is a dict-like key -> payload (the RAM/SSD tiers; None drops evicted pages);
    the KV pool is either a KVTransfer (device planes) or, for host-only use, a dict
    page -> payload of `page_bytes` bytes."""

    def __init__(self, namespace, pages, page_size=32, store=None, transfer=None, pool=None,
                 page_bytes=None):
        self.store, self.transfer, self.pool = store, transfer, pool
        self.page_bytes = transfer.page_bytes if transfer is not None else (page_bytes or 0)
        self._held = []
        io = PageIO()
        io.ctx = None
        io.page_bytes = self.page_bytes
        # dispatch through the instance so a subclass or a test can wrap a callback
        self._callbacks = (LOAD_FN(lambda *a: self._load(*a)), PUT_FN(lambda *a: self._put(*a)),
                           READ_FN(lambda *a: self._read(*a)),
                           WRITE_FN(lambda *a: self._write(*a)))
        if store is not None:
            io.load, io.put = self._callbacks[0], self._callbacks[1]
        io.read_page, io.write_pages = self._callbacks[2], self._callbacks[3]
        self._io = io
        h = C.c_void_p()
        _check(lib().lia_page_cache_create(bytes(namespace), pages, page_size, C.byref(io),
                                           C.byref(h)), "PageCache")
        self.handle = h
        self._destroy = lib().lia_page_cache_destroy

    def __del__(self):
        if getattr(self, "handle", None):
            self._destroy(self.handle)
            self.handle = None

    # callbacks: 0 ok, a negative lia status, or 1 (-> LIA_E_STORE) on a Python error
    @staticmethod
    def _status(e):
        return e.status if isinstance(e, LiaError) else 1

    def _load(self, ctx, key, payload):
        try:
            data = self.store.get(C.string_at(key, 32))
            if data is None:
                return 0
            buf = C.create_string_buffer(bytes(data), len(data))
            self._held.append(buf)
            payload[0] = C.addressof(buf)
            return 1
        except Exception as e:  # noqa: BLE001 - a positive return means "hit" here
            return e.status if isinstance(e, LiaError) else -24

    def _put(self, ctx, key, payload):
        try:
            self.store[C.string_at(key, 32)] = C.string_at(payload, self.page_bytes)
            return 0
        except Exception as e:  # noqa: BLE001
            return self._status(e)

    def _read(self, ctx, page, dst):
        try:
            data = (self.transfer.read_kv_page(page) if self.transfer is not None
                    else self.pool[page])
            C.memmove(dst, bytes(data), self.page_bytes)
            return 0
        except Exception as e:  # noqa: BLE001
            return self._status(e)

    def _write(self, ctx, n, pages, payloads):
        try:
            items = [(pages[i], C.string_at(payloads[i], self.page_bytes)) for i in range(n)]
            if self.transfer is not None:
                self.transfer.write_kv_pages(items)
            else:
                for p, d in items:
                    self.pool[p] = d
            self._held.clear()
            return 0
        except Exception as e:  # noqa: BLE001
            return self._status(e)

    @staticmethod
    def _tokens(tokens):
        return np.ascontiguousarray(tokens, dtype=np.uint32)

    def attach(self, tokens):
        t = self._tokens(tokens)
        h, cached = C.c_void_p(), C.c_size_t()
        st = lib().lia_page_cache_attach(self.handle, t.ctypes.data, t.size, C.byref(h),
                                         C.byref(cached))
        self._held.clear()
        _check(st, "attach")
        return Sequence(h), cached.value

    def can_fit(self, tokens):
        t = self._tokens(tokens)
        return lib().lia_page_cache_can_fit(self.handle, t.ctypes.data, t.size) == 1

    def available_pages(self):
        return lib().lia_page_cache_available(self.handle)

    def ensure_position(self, sequence, position):
        st = lib().lia_page_cache_ensure_position(self.handle, sequence.handle, position)
        if st < 0:
            _check(st, "ensure_position")
        return st == 1

    def seal(self, sequence, tokens, computed):
        t = self._tokens(tokens)
        _check(lib().lia_page_cache_seal(self.handle, sequence.handle, t.ctypes.data, t.size,
                                         computed), "seal")

    def release(self, sequence):
        st = lib().lia_page_cache_release(self.handle, sequence.handle)
        sequence.handle = None
        _check(st, "release")

    def evict_idle(self):
        _check(lib().lia_page_cache_evict_idle(self.handle), "evict_idle")

    @property
    def gpu_hits(self):
        a, b = C.c_uint64(), C.c_uint64()
        lib().lia_page_cache_stats(self.handle, C.byref(a), C.byref(b))
        return a.value

    @property
    def evictions(self):
        a, b = C.c_uint64(), C.c_uint64()
        lib().lia_page_cache_stats(self.handle, C.byref(a), C.byref(b))
        return b.value

    def schedule_rows(self, requests, prefill_batch):
        """Runtime::step row construction (src/server/paged/schedule.rs:5-60).  requests: one
        dict per slot (tokens, computed, sequence, closed) or None.  Returns (rows as
        [(token, position, slot)], output row indices, updates [(slot, computed, output)])."""
        n = len(requests)
        arr = (Request * max(n, 1))()
        keep = []
        for i, r in enumerate(requests):
            if r is None:
                continue
            t = self._tokens(r["tokens"])
            keep.append(t)
            arr[i] = Request(t.ctypes.data, t.size, r["computed"], r["sequence"].handle, 1,
                             int(bool(r.get("closed"))), 0, 0)
        active = sum(r is not None for r in requests)
        cap = max(prefill_batch, active, 1)
        rows = (PagedRow * cap)()
        outs = (C.c_uint32 * cap)()
        ups = (Update * max(n, 1))()
        nr, no, nu = C.c_uint32(), C.c_uint32(), C.c_uint32()
        _check(lib().lia_schedule_rows(self.handle, n, arr, prefill_batch, rows, cap,
                                       C.byref(nr), outs, C.byref(no), ups, C.byref(nu)),
               "schedule_rows")
        for i, r in enumerate(requests):
            if r is not None and arr[i].done:
                r["done"] = True
        return ([(rows[i].token, rows[i].position, rows[i].sequence) for i in range(nr.value)],
                [outs[i] for i in range(no.value)],
                [(ups[i].slot, ups[i].computed, bool(ups[i].output)) for i in range(nu.value)])


class Sampler:
    """Sampling (src/sampling.rs:19-190) held by the library: temperature, top_k (0 = none,
    else 1..20), top_p, the seed's MT19937 stream, or position-keyed Gumbel draws."""

    def __init__(self, temperature, top_k, top_p, seed, position_keyed=False):
        h = C.c_void_p()
        _check(lib().lia_sampler_create(temperature, top_k, top_p, seed, int(position_keyed),
                                        C.byref(h)), "Sampler")
        self.handle = h
        self._destroy = lib().lia_sampler_destroy   # still reachable at interpreter exit
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p

    def __del__(self):
        if getattr(self, "handle", None):
            self._destroy(self.handle)
            self.handle = None

    def set_position(self, position):
        lib().lia_sampler_set_position(self.handle, position)

    def distribution(self, candidates):
        """[(id, logit)] -> [(id, probability)] (Sampling::distribution)."""
        ids = np.array([c[0] for c in candidates], np.uint32)
        vals = np.array([c[1] for c in candidates], np.float32)
        n = len(ids)
        oi = np.zeros(max(n, 1), np.uint32)
        op = np.zeros(max(n, 1), np.float64)
        k = C.c_uint32()
        _check(lib().lia_sampler_distribution(self.handle, n, ids.ctypes.data, vals.ctypes.data,
                                              oi.ctypes.data, op.ctypes.data, C.byref(k)),
               "distribution")
        return [(int(oi[i]), float(op[i])) for i in range(k.value)]

    def draw(self, entries):
        ids = np.array([e[0] for e in entries], np.uint32)
        ps = np.array([e[1] for e in entries], np.float64)
        t = C.c_uint32()
        _check(lib().lia_sampler_draw(self.handle, len(ids), ids.ctypes.data, ps.ctypes.data,
                                      C.byref(t)), "draw")
        return t.value


def _sampler_array(samplers):
    arr = (C.c_void_p * max(len(samplers), 1))()
    for i, s in enumerate(samplers):
        arr[i] = s.handle.value if s is not None else None
    return arr


def sample_host(vocab, samplers, positions, candidates, normalizers, logits=None):
    """Host tail of forward_paged_sampled on host candidate records (lia_sample_host)."""
    n = len(samplers)
    pos = np.ascontiguousarray(positions, np.uint32)
    cand = np.ascontiguousarray(candidates, np.uint64)
    norm = np.ascontiguousarray(normalizers, np.float64)
    lg = None if logits is None else np.ascontiguousarray(logits, np.float32)
    tokens = np.zeros(max(n, 1), np.uint32)
    fb = C.c_uint64()
    _check(lib().lia_sample_host(vocab, n, _sampler_array(samplers), pos.ctypes.data,
                                 cand.ctypes.data, norm.ctypes.data,
                                 None if lg is None else lg.ctypes.data, tokens.ctypes.data,
                                 C.byref(fb)), "sample_host")
    return [int(t) for t in tokens[:n]], fb.value


def nucleus_candidates(temperatures, logits, candidates, normalizers, stream=None):
    """llama_nucleus_candidates on device tensors (lia_nucleus_candidates)."""
    rows, vocab = logits.shape
    _check(lib().lia_nucleus_candidates(vocab, rows, _dptr(temperatures), _dptr(logits),
                                        _dptr(candidates), _dptr(normalizers), _stream(stream)),
           "nucleus_candidates")


class PagedSampler:
    """Sparse sampling of a step's output rows (Engine::forward_paged_sampled's tail,
    src/inference/paged_sampling.rs:7-76) with its device workspace and host buffer."""

    def __init__(self, vocab, max_rows, device="cuda"):
        import torch
        self.vocab, self.max_rows = vocab, max_rows
        self.ws_bytes = lib().lia_nucleus_workspace_bytes(vocab, max_rows)
        self.host_bytes = lib().lia_nucleus_host_bytes(vocab, max_rows)
        self.workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)
        self.host = torch.empty(self.host_bytes, dtype=torch.uint8, pin_memory=True)
        self.fallbacks = 0

    def sample(self, logits, samplers, positions, stream=None):
        """logits: device f32 [rows][vocab]; samplers: Sampler or None (greedy) per row."""
        n = len(samplers)
        if logits.shape[0] != n or n > self.max_rows or logits.shape[1] != self.vocab:
            raise LiaError(-20, "sample: logits do not match the sampler rows")
        pos = np.ascontiguousarray(positions, np.uint32)
        tokens = np.zeros(max(n, 1), np.uint32)
        fb = C.c_uint64()
        _check(lib().lia_sample_paged(self.vocab, n, _sampler_array(samplers), pos.ctypes.data,
                                      _dptr(logits), _dptr(self.workspace), self.ws_bytes,
                                      _dptr(self.host), self.host_bytes, tokens.ctypes.data,
                                      C.byref(fb), _stream(stream)), "sample_paged")
        self.fallbacks += fb.value
        return [int(t) for t in tokens[:n]]


def workspace_bytes(config):
    return lib().lia_attention_workspace_bytes(C.byref(config))


def paged_attention(config, n_seqs, cu_seqlens, positions, sequences, pages, q, kc, vc, out,
                    workspace, k_scales=None, v_scales=None, stream=None):
    """Ragged paged attention (lia_paged_attention)."""
    st = lib().lia_paged_attention(C.byref(config), n_seqs, q.shape[0], _dptr(cu_seqlens),
                                   _dptr(positions), _dptr(sequences), _dptr(pages), _dptr(q),
                                   _dptr(kc), _dptr(vc), _dptr(k_scales), _dptr(v_scales),
                                   _dptr(workspace), workspace.numel() * workspace.element_size(),
                                   _dptr(out), _stream(stream))
    _check(st, "paged_attention")


def paged_attention_static(config, n_seqs, cu_seqlens, positions, sequences, pages, q, kc, vc,
                           out, k_scales=None, v_scales=None, stream=None):
    """lia_paged_attention with the library's static device workspace (allocates nothing)."""
    st = lib().lia_paged_attention_static(C.byref(config), n_seqs, q.shape[0], _dptr(cu_seqlens),
                                          _dptr(positions), _dptr(sequences), _dptr(pages),
                                          _dptr(q), _dptr(kc), _dptr(vc), _dptr(k_scales),
                                          _dptr(v_scales), _dptr(out), _stream(stream))
    _check(st, "paged_attention_static")


def attention_plan(config, n_seqs, n_rows, cu_seqlens, positions, sequences, workspace,
                   pages=None, stream=None):
    """Stage 1: the step's work list (shared by every layer of the step).  With `pages`
    the plan also records the first table entries of every workgroup's range."""
    st = lib().lia_attention_plan(C.byref(config), n_seqs, n_rows, _dptr(cu_seqlens),
                                  _dptr(positions), _dptr(sequences), _dptr(pages),
                                  _dptr(workspace),
                                  workspace.numel() * workspace.element_size(), _stream(stream))
    _check(st, "attention_plan")


def attention_partial(config, n_seqs, pages, q, kc, vc, out, workspace, k_scales=None,
                      v_scales=None, stream=None):
    """Stage 2: the split attention kernel over the planned work list."""
    st = lib().lia_attention_partial(C.byref(config), n_seqs, q.shape[0], _dptr(pages), _dptr(q),
                                     _dptr(kc), _dptr(vc), _dptr(k_scales), _dptr(v_scales),
                                     _dptr(workspace),
                                     workspace.numel() * workspace.element_size(), _dptr(out),
                                     _stream(stream))
    _check(st, "attention_partial")


def attention_partial_append(config, n_seqs, pages, slot_mapping, q, new_k, new_v, kc, vc, out,
                             workspace, stream=None):
    """Stage 2 with this step's KV append fused in (lia_attention_partial_append): new_k /
    new_v are the step's rows in the pool dtype."""
    st = lib().lia_attention_partial_append(C.byref(config), n_seqs, q.shape[0], _dptr(pages),
                                            _dptr(slot_mapping), _dptr(q), _dptr(new_k),
                                            _dptr(new_v), _dptr(kc), _dptr(vc), _dptr(workspace),
                                            workspace.numel() * workspace.element_size(),
                                            _dptr(out), _stream(stream))
    _check(st, "attention_partial_append")


def attention_partial_append_fp8(config, n_seqs, pages, slot_mapping, q, new_k, new_v, kc, vc,
                                 k_scales, v_scales, out, workspace, stream=None):
    """Stage 2 with this step's KV append fused in, FP8 pools (lia_attention_partial_append_fp8):
    new_k / new_v are the step's bf16 rows, quantised with their pages' scales."""
    st = lib().lia_attention_partial_append_fp8(
        C.byref(config), n_seqs, q.shape[0], _dptr(pages), _dptr(slot_mapping), _dptr(q),
        _dptr(new_k), _dptr(new_v), _dptr(kc), _dptr(vc), _dptr(k_scales), _dptr(v_scales),
        _dptr(workspace), workspace.numel() * workspace.element_size(), _dptr(out), _stream(stream))
    _check(st, "attention_partial_append_fp8")


def hbm_read(src, workgroups, sink, nbytes=None, stream=None):
    """Read-only HBM stream over a device tensor (lia_hbm_read): the contiguous-read ceiling."""
    nbytes = src.numel() * src.element_size() if nbytes is None else nbytes
    st = lib().lia_hbm_read(_dptr(src), nbytes, workgroups, _dptr(sink), _stream(stream))
    _check(st, "hbm_read")


def paged_read_sink_words(config):
    """Words of the sink paged_read needs (lia_paged_read_sink_words)."""
    return lib().lia_paged_read_sink_words(C.byref(config))


def paged_read(config, n_seqs, pages, q, kc, vc, sink, workspace, k_scales=None, v_scales=None,
               stream=None):
    """The decode kernel's loads over the planned work list without the attention arithmetic
    (lia_paged_read): the ceiling of its own access pattern.  sink: int32 device tensor of at
    least paged_read_sink_words(config) words."""
    st = lib().lia_paged_read(C.byref(config), n_seqs, q.shape[0], _dptr(pages), _dptr(q), _dptr(kc),
                              _dptr(vc), _dptr(k_scales), _dptr(v_scales), _dptr(workspace),
                              workspace.numel() * workspace.element_size(), _dptr(sink), sink.numel(),
                              _stream(stream))
    _check(st, "paged_read")


def attention_merge(config, n_seqs, n_rows, out, workspace, stream=None):
    """Stage 3: combine the split records into out."""
    st = lib().lia_attention_merge(C.byref(config), n_seqs, n_rows, _dptr(workspace),
                                   workspace.numel() * workspace.element_size(), _dptr(out),
                                   _stream(stream))
    _check(st, "attention_merge")


# ------------------------------------------------------------------ engine mirror

class Engine:
    """Paged KV pool + metadata of one engine, mirroring the reference Engine's paged
    surface (src/inference/paging.rs:30-261, src/inference/llama.rs:79-299) for the
    attention path only: the model's projections are outside this path, so
    `attention()` takes the per-layer q/k/v rows directly."""

    def __init__(self, num_q_heads=16, num_kv_heads=2, head_dim=128, pool_tokens=65536,
                 layers=1, page_size=32, kv_dtype=F16, q_dtype=F32, out_dtype=F32,
                 vocabulary=130560, prefill_batch=512, scale=None, device="cuda"):
        import torch
        if pool_tokens % page_size:
            raise LiaError(-19, "Engine: physical KV pool must contain complete pages")
        self.hq, self.hkv, self.d = num_q_heads, num_kv_heads, head_dim
        self.page_size, self.pool_pages = page_size, pool_tokens // page_size
        self.layers, self.kv_dtype = layers, kv_dtype
        self.q_dtype, self.out_dtype = q_dtype, out_dtype
        self.vocabulary, self.prefill_batch = vocabulary, prefill_batch
        self.scale = float(scale if scale is not None else 1.0 / np.sqrt(head_dim))
        self.device = device
        storage = torch.uint8 if kv_dtype == FP8 else torch.uint16
        shape = (pool_tokens, num_kv_heads, head_dim)
        self.k = [torch.zeros(shape, dtype=storage, device=device) for _ in range(layers)]
        self.v = [torch.zeros(shape, dtype=storage, device=device) for _ in range(layers)]
        if kv_dtype == FP8:
            self.k_scales = [torch.ones(self.pool_pages * num_kv_heads, dtype=torch.float32,
                                        device=device) for _ in range(layers)]
            self.v_scales = [torch.ones_like(self.k_scales[0]) for _ in range(layers)]
        else:
            self.k_scales = self.v_scales = [None] * layers
        self.paging = None

    def configure_paging(self, maximum_sequences, context):
        """Engine::configure_paging (src/inference/paging.rs:30-93)."""
        import torch
        if self.paging is not None:
            raise LiaError(-19, "paging must be configured before execution")
        if not 1 <= maximum_sequences <= 64:
            raise LiaError(-19, "invalid sequence count")
        if not 1 <= context <= 131072:
            raise LiaError(-19, "invalid per-request context")
        stride = -(-context // self.page_size)
        rows = self.prefill_batch
        dev = self.device
        self.limits = PagingLimits(maximum_sequences, context, self.page_size, self.pool_pages,
                                   self.vocabulary, rows)
        self.config = AttentionConfig(self.hq, self.hkv, self.d, self.page_size, self.pool_pages,
                                      stride, self.q_dtype, self.kv_dtype, self.out_dtype,
                                      self.scale, maximum_sequences, rows, context)
        self.paging = dict(
            stride=stride,
            positions=torch.zeros(rows, dtype=torch.int32, device=dev),
            sequences=torch.zeros(rows, dtype=torch.int32, device=dev),
            slot_mapping=torch.zeros(rows, dtype=torch.int32, device=dev),
            pages=torch.zeros(maximum_sequences * stride, dtype=torch.int32, device=dev),
            cu_seqlens=torch.zeros(rows + 1, dtype=torch.int32, device=dev),
            workspace=torch.zeros(workspace_bytes(self.config), dtype=torch.uint8, device=dev),
            n_seqs=0, n_rows=0)
        torch.cuda.synchronize()

    def stage(self, rows, tables, outputs=()):
        """Host packing + metadata upload of Engine::run_paged (paging.rs:118-237)."""
        import torch
        if self.paging is None:
            raise LiaError(-19, "paging is not configured")
        packed = pack_rows(self.limits, rows, tables, outputs)
        w = self.paging
        n = len(packed["positions"])
        ng = len(packed["cu_seqlens"]) - 1
        as_i32 = lambda a: torch.from_numpy(a.view(np.int32))
        w["positions"][:n].copy_(as_i32(packed["positions"]))
        w["sequences"][:n].copy_(as_i32(packed["sequences"]))
        w["slot_mapping"][:n].copy_(as_i32(packed["slot_mapping"]))
        w["pages"].copy_(as_i32(packed["flat"]))
        w["cu_seqlens"][:ng + 1].copy_(as_i32(packed["cu_seqlens"]))
        w["n_seqs"], w["n_rows"] = ng, n
        torch.cuda.current_stream().synchronize()
        return packed

    def attention(self, layer, q, k, v, out=None):
        """Append this step's K/V rows to layer's pool and attend (llama.rs:203-288)."""
        import torch
        w = self.paging
        n = w["n_rows"]
        if q.shape[0] != n or k.shape[0] != n:
            raise LiaError(-20, "attention: row count differs from the staged batch")
        layout = KVLayout(self.hkv, self.d, self.page_size, self.pool_pages, self.kv_dtype)
        kv_append(layout, k.reshape(n, -1), v.reshape(n, -1), self.k[layer], self.v[layer],
                  slot_mapping=w["slot_mapping"], k_scales=self.k_scales[layer],
                  v_scales=self.v_scales[layer])
        if out is None:
            odt = torch.float32 if self.out_dtype == F32 else torch.bfloat16
            out = torch.empty((n, self.hq, self.d), dtype=odt, device=q.device)
        paged_attention(self.config, w["n_seqs"], w["cu_seqlens"], w["positions"],
                        w["sequences"], w["pages"], q, self.k[layer], self.v[layer], out,
                        w["workspace"], self.k_scales[layer], self.v_scales[layer])
        return out

    def _transfer(self):
        if self.paging is None:
            raise LiaError(-19, "KV pages require configured paging")
        if getattr(self, "_kv_transfer", None) is None:
            layout = KVLayout(self.hkv, self.d, self.page_size, self.pool_pages, self.kv_dtype)
            fp8 = self.kv_dtype == FP8
            self._kv_transfer = KVTransfer(layout, self.k, self.v,
                                           self.k_scales if fp8 else None,
                                           self.v_scales if fp8 else None)
        return self._kv_transfer

    def read_kv_page(self, page):
        """Engine::read_kv_page (src/inference/paging_transfer.rs:26-31)."""
        return self._transfer().read_kv_page(page)

    def write_kv_page(self, page, payload):
        """Engine::write_kv_page (src/inference/paging_transfer.rs:33-35)."""
        self._transfer().write_kv_page(page, payload)

    def write_kv_pages(self, pages):
        """Engine::write_kv_pages (src/inference/paging_transfer.rs:37-58)."""
        self._transfer().write_kv_pages(pages)
