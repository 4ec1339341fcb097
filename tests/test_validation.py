"""Launch validation of the attention entry points, on the CPU.

The reference validates every launch before it touches the device
(gpu::llama_attention::partial / merge, src/gpu/llama_attention.rs:36-91, 163-170): bad
extents, unaligned buffers and an exhausted workspace are errors, never launches.  Each
case below starts from a configuration and arguments that pass, breaks exactly one thing and
expects the status the C ABI documents; no case reaches a kernel launch, so no device
pointer is dereferenced (the addresses are placeholders).
"""
import ctypes as C

import pytest

F32, F16, BF16, FP8 = 0, 1, 2, 3
OK, E_ARG, E_ALIGN, E_WORKSPACE, E_UNSUPPORTED = 0, -20, -21, -22, -23

A = 0x100000          # a 256-byte aligned placeholder address
ODD16 = 0x100008      # 8-byte but not 16-byte aligned
ODD256 = 0x100080     # 16-byte but not 256-byte aligned


def _cfg(lia, **kw):
    base = dict(num_q_heads=16, num_kv_heads=2, head_dim=128, page_size=16, pool_pages=64,
                stride=8, q_dtype=BF16, kv_dtype=BF16, out_dtype=BF16, scale=0.088,
                max_seqs=4, max_rows=8, max_context=128)
    base.update(kw)
    return lia.AttentionConfig(**base)


def _args(lia, cfg, **kw):
    a = dict(n_seqs=2, n_rows=2, cu=A, positions=A, sequences=A, pages=A, q=A, kc=A, vc=A,
             ks=None, vs=None, ws=A, ws_bytes=lia.workspace_bytes(cfg), out=A)
    a.update(kw)
    return a


def _paged(lia, cfg, a):
    p = lambda x: None if x is None else C.c_void_p(x)
    return lia.lib().lia_paged_attention(
        None if cfg is None else C.byref(cfg), a["n_seqs"], a["n_rows"], p(a["cu"]),
        p(a["positions"]), p(a["sequences"]), p(a["pages"]), p(a["q"]), p(a["kc"]), p(a["vc"]),
        p(a["ks"]), p(a["vs"]), p(a["ws"]), a["ws_bytes"], p(a["out"]), None)


def _plan(lia, cfg, a):
    p = lambda x: None if x is None else C.c_void_p(x)
    return lia.lib().lia_attention_plan(C.byref(cfg), a["n_seqs"], a["n_rows"], p(a["cu"]),
                                        p(a["positions"]), p(a["sequences"]), p(a["pages"]),
                                        p(a["ws"]), a["ws_bytes"], None)


def _partial(lia, cfg, a):
    p = lambda x: None if x is None else C.c_void_p(x)
    return lia.lib().lia_attention_partial(C.byref(cfg), a["n_seqs"], a["n_rows"], p(a["pages"]),
                                           p(a["q"]), p(a["kc"]), p(a["vc"]), p(a["ks"]),
                                           p(a["vs"]), p(a["ws"]), a["ws_bytes"], p(a["out"]), None)


def _merge(lia, cfg, a):
    p = lambda x: None if x is None else C.c_void_p(x)
    return lia.lib().lia_attention_merge(C.byref(cfg), a["n_seqs"], a["n_rows"], p(a["ws"]),
                                         a["ws_bytes"], p(a["out"]), None)


GEOMETRY = [
    ("num_kv_heads", 0, E_ARG),          # no KV heads
    ("num_q_heads", 0, E_ARG),
    ("num_q_heads", 15, E_ARG),          # not a multiple of the KV heads
    ("num_q_heads", 66, E_UNSUPPORTED),  # a GQA group of 33
    ("head_dim", 96, E_UNSUPPORTED),
    ("head_dim", 256, E_UNSUPPORTED),
    ("page_size", 8, E_UNSUPPORTED),
    ("page_size", 48, E_UNSUPPORTED),
    ("q_dtype", F16, E_UNSUPPORTED),
    ("out_dtype", F16, E_UNSUPPORTED),
    ("kv_dtype", F32, E_UNSUPPORTED),
    ("stride", 0, E_ARG),
    ("max_seqs", 0, E_ARG),
    ("max_rows", 0, E_ARG),
]


@pytest.mark.parametrize("field,value,expect", GEOMETRY)
@pytest.mark.parametrize("entry", ["paged", "plan", "partial", "merge"])
def test_geometry_is_validated(lia, field, value, expect, entry):
    cfg = _cfg(lia)
    a = _args(lia, cfg)
    setattr(cfg, field, value)
    fn = {"paged": _paged, "plan": _plan, "partial": _partial, "merge": _merge}[entry]
    assert fn(lia, cfg, a) == expect


def test_null_config(lia):
    cfg = _cfg(lia)
    assert _paged(lia, None, _args(lia, cfg)) == E_ARG


@pytest.mark.parametrize("change,expect", [
    (dict(n_seqs=0), E_ARG),             # an empty batch
    (dict(n_seqs=5), E_ARG),             # more sequences than configured
    (dict(n_rows=0), E_ARG),
    (dict(n_rows=9), E_ARG),             # more rows than configured
    (dict(cu=None), E_ARG),
    (dict(positions=None), E_ARG),
    (dict(sequences=None), E_ARG),
    (dict(pages=None), E_ARG),
    (dict(q=None), E_ARG),
    (dict(kc=None), E_ARG),
    (dict(vc=None), E_ARG),
    (dict(ws=None), E_ARG),
    (dict(out=None), E_ARG),
    (dict(out=ODD16), E_ALIGN),          # outputs 16-byte aligned (the reference: 8)
    (dict(q=ODD16), E_ALIGN),            # q / k / v 16-byte aligned, as the reference
    (dict(kc=ODD16), E_ALIGN),
    (dict(vc=ODD16), E_ALIGN),
    (dict(ws=ODD256), E_ALIGN),
    (dict(ws_bytes=1), E_WORKSPACE),     # "GQA partial workspace exhausted"
])
def test_paged_attention_arguments(lia, change, expect):
    cfg = _cfg(lia)
    a = _args(lia, cfg, **change)
    assert _paged(lia, cfg, a) == expect


def test_workspace_exhausted_by_one_byte(lia):
    cfg = _cfg(lia)
    need = lia.workspace_bytes(cfg)
    assert need > 0
    a = _args(lia, cfg, ws_bytes=need - 1)
    for fn in (_paged, _plan, _partial, _merge):
        assert fn(lia, cfg, a) == E_WORKSPACE


def test_fp8_pool_needs_scales(lia):
    cfg = _cfg(lia, kv_dtype=FP8)
    assert _paged(lia, cfg, _args(lia, cfg)) == E_ARG
    assert _paged(lia, cfg, _args(lia, cfg, ks=A)) == E_ARG
    assert _partial(lia, cfg, _args(lia, cfg, vs=A)) == E_ARG


def test_32_bit_ranges(lia):
    """q and the FP8 scale arrays are read through 32-bit buffer ranges."""
    cfg = _cfg(lia, max_rows=1 << 17)  # 2^17 rows x 16 heads x 128 dims x 4 B = 2^30: in range
    assert _paged(lia, cfg, _args(lia, cfg, ws_bytes=1)) == E_WORKSPACE  # the next check
    cfg = _cfg(lia, max_rows=1 << 18)
    assert _paged(lia, cfg, _args(lia, cfg)) == E_UNSUPPORTED
    cfg = _cfg(lia, pool_pages=1 << 28)
    assert _paged(lia, cfg, _args(lia, cfg)) == E_UNSUPPORTED


@pytest.mark.parametrize("entry,change", [
    ("plan", dict(sequences=None)),
    ("plan", dict(cu=None)),
    ("plan", dict(positions=None)),
    ("partial", dict(pages=None)),
    ("partial", dict(q=None)),
    ("partial", dict(out=None)),
    ("merge", dict(out=None)),
    ("merge", dict(ws=None)),
])
def test_stage_entry_points_check_what_they_read(lia, entry, change):
    cfg = _cfg(lia)
    fn = {"plan": _plan, "partial": _partial, "merge": _merge}[entry]
    assert fn(lia, cfg, _args(lia, cfg, **change)) == E_ARG


def test_stage_entry_points_ignore_what_they_do_not_read(lia):
    """The plan reads no q / K / V / out; the merge reads no metadata: null pointers there are
    not errors (these calls then fail only at the workspace check we force)."""
    cfg = _cfg(lia)
    a = _args(lia, cfg, q=None, kc=None, vc=None, out=None, ws_bytes=1)
    assert _plan(lia, cfg, a) == E_WORKSPACE
    a = _args(lia, cfg, cu=None, positions=None, sequences=None, pages=None, q=None, ws_bytes=1)
    assert _merge(lia, cfg, a) == E_WORKSPACE


@pytest.mark.parametrize("scale", [0.0, -0.088, float("inf"), float("nan")])
def test_scale_must_be_positive_and_finite(lia, scale):
    """The kernels take maxima of raw scores and scale them afterwards, which needs a
    positive scale (the reference's is 1/sqrt(head_dim))."""
    cfg = _cfg(lia, scale=scale)
    assert _paged(lia, cfg, _args(lia, cfg)) == E_ARG


def test_fp8_partial_append_validates_both_launches_first(lia):
    """lia_attention_partial_append_fp8 checks the append's and the attention's arguments
    before it issues either launch."""
    def call(cfg, new_k=A, ws_bytes=None, ks=A):
        p = lambda x: None if x is None else C.c_void_p(x)
        return lia.lib().lia_attention_partial_append_fp8(
            C.byref(cfg), 2, 2, p(A), p(A), p(A), p(new_k), p(A), p(A), p(A), p(ks), p(A), p(A),
            lia.workspace_bytes(cfg) if ws_bytes is None else ws_bytes, p(A), None)
    assert call(_cfg(lia, kv_dtype=BF16)) == E_UNSUPPORTED
    fp8 = _cfg(lia, kv_dtype=FP8)
    assert call(fp8, new_k=None) == E_ARG
    assert call(fp8, new_k=ODD16) == E_ALIGN
    assert call(fp8, ks=None) == E_ARG
    assert call(fp8, ws_bytes=1) == E_WORKSPACE


def _read(lia, cfg, a, sink=A, sink_words=None):
    p = lambda x: None if x is None else C.c_void_p(x)
    words = lia.lib().lia_paged_read_sink_words(C.byref(cfg)) if sink_words is None else sink_words
    return lia.lib().lia_paged_read(C.byref(cfg), a["n_seqs"], a["n_rows"], p(a["pages"]), p(a["q"]),
                                    p(a["kc"]), p(a["vc"]), p(a["ks"]), p(a["vs"]), p(a["ws"]),
                                    a["ws_bytes"], p(sink), words, None)


def test_paged_read_sink_words(lia):
    cfg = _cfg(lia)
    # one word per wave (head_dim / 64 waves) of every workgroup the plan may use
    assert lia.lib().lia_paged_read_sink_words(C.byref(cfg)) > 0
    assert lia.lib().lia_paged_read_sink_words(C.byref(cfg)) % 2 == 0
    assert lia.lib().lia_paged_read_sink_words(C.byref(_cfg(lia, num_kv_heads=0))) == 0


@pytest.mark.parametrize("case,expect", [
    ("fp8", E_ARG),                  # an FP8 pool without its scales
    ("prefill", E_UNSUPPORTED),      # a batch the prefill kernel serves
    ("no_sink", E_ARG),
    ("short_sink", E_ARG),
    ("odd_sink", E_ALIGN),
    ("no_q", E_ARG),
    ("no_pages", E_ARG),
    ("workspace", E_WORKSPACE),
    ("rows", E_ARG),
])
def test_paged_read_validation(lia, case, expect):
    """lia_paged_read checks its arguments like lia_attention_partial, plus its sink."""
    cfg = _cfg(lia, kv_dtype=FP8) if case == "fp8" else _cfg(lia, max_rows=4096, max_seqs=4)
    a = _args(lia, cfg)
    sink, words = A, None
    if case == "prefill":
        a.update(n_seqs=1, n_rows=2048)
    elif case == "no_sink":
        sink = None
    elif case == "short_sink":
        words = lia.lib().lia_paged_read_sink_words(C.byref(cfg)) - 1
    elif case == "odd_sink":
        sink = A + 2
    elif case == "no_q":
        a.update(q=None)
    elif case == "no_pages":
        a.update(pages=None)
    elif case == "workspace":
        a.update(ws_bytes=a["ws_bytes"] - 1)
    elif case == "rows":
        a.update(n_rows=0)
    assert _read(lia, cfg, a, sink, words) == expect
