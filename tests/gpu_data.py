"""Materialise a workloads.Batch for a GPU parity test: host copies for the oracle and
device tensors for the HIP library, from the same seeded values."""
import numpy as np
import torch

from oracle import oracle as O

F32, F16, BF16, FP8 = 0, 1, 2, 3
TORCH_STORAGE = {F32: torch.float32, F16: torch.int16, BF16: torch.int16, FP8: torch.uint8}


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def u32_dev(a):
    return to_dev(np.asarray(a, dtype=np.uint32).view(np.int32))


class Case:
    def __init__(self, batch, seed=0, fill="normal", v_scale=1.0):
        g = batch.geom
        self.batch, self.g = batch, g
        rng = np.random.default_rng(seed + 1000)
        P = g.page_size
        tokens = batch.pool_pages * P
        if fill == "fp8_codes":
            # FP8 pools drawn as codes: every finite e4m3fn byte (0x7F / 0xFF are NaN) with
            # per-(page, head) scales, no float pool to quantise (the 64-sequence pool of
            # config 5 holds 430M values per plane)
            assert g.kv_dtype == FP8
            n = tokens * g.hkv * g.d

            def draw():  # uniform over the 254 finite codes: 0..0x7E, 0x80..0xFE
                c = rng.integers(0, 254, n, dtype=np.uint8)
                c += c >= 0x7F
                return c

            self.kc = draw()
            self.vc = draw()
            self.k_scales = rng.uniform(0.002, 0.01, batch.pool_pages * g.hkv).astype(np.float32)
            self.v_scales = rng.uniform(0.002, 0.01, batch.pool_pages * g.hkv).astype(np.float32)
            self._finish(batch, rng)
            return
        kf = rng.standard_normal((tokens, g.hkv, g.d), dtype=np.float32)
        vf = rng.standard_normal((tokens, g.hkv, g.d), dtype=np.float32)
        if fill == "uniform":
            kf = rng.uniform(-1, 1, kf.shape).astype(np.float32)
            vf = rng.uniform(-1, 1, vf.shape).astype(np.float32)
        if v_scale != 1.0:
            vf *= np.float32(v_scale)
        self.k_scales = self.v_scales = None
        if g.kv_dtype == FP8:
            layout = O.KVLayout(g.hkv, g.d, P, batch.pool_pages, FP8)
            self.kc = np.zeros(tokens * g.hkv * g.d, np.uint8)
            self.vc = np.zeros_like(self.kc)
            self.k_scales = np.zeros(batch.pool_pages * g.hkv, np.float32)
            self.v_scales = np.zeros_like(self.k_scales)
            O.kv_quantize_pages(layout, np.arange(batch.pool_pages), kf, vf, self.kc, self.vc,
                                self.k_scales, self.v_scales)
        else:
            self.kc = O.from_f32(kf, g.kv_dtype).reshape(-1)
            self.vc = O.from_f32(vf, g.kv_dtype).reshape(-1)
        self._finish(batch, rng)

    def _finish(self, batch, rng):
        g = self.g
        qf = rng.standard_normal((batch.n_rows, g.hq, g.d), dtype=np.float32)
        if g.q_dtype == BF16:
            self.q_store = O.from_f32(qf, BF16)
            self.q32 = O.to_f32(self.q_store, BF16)
        else:
            self.q_store = qf
            self.q32 = qf
        self.positions = batch.positions()
        self.sequences = batch.sequences()
        self.cu = batch.cu_seqlens()
        self.flat = batch.flat_table()

    def oracle_geom(self):
        g = self.g
        return O.geom(g.hq, g.hkv, g.d, g.page_size, self.batch.stride, g.kv_dtype, g.scale)

    def f64(self):
        return O.attention_f64(self.oracle_geom(), self.positions, self.sequences, self.flat,
                               self.q32, self.kc, self.vc, self.k_scales, self.v_scales)

    def device(self):
        g = self.g
        d = dict(
            kc=to_dev(self.kc, torch.uint8 if g.kv_dtype == FP8 else torch.int16),
            vc=to_dev(self.vc, torch.uint8 if g.kv_dtype == FP8 else torch.int16),
            q=to_dev(self.q_store, torch.bfloat16 if g.q_dtype == BF16 else None),
            positions=u32_dev(self.positions), sequences=u32_dev(self.sequences),
            cu=u32_dev(self.cu), pages=u32_dev(self.flat),
            k_scales=to_dev(self.k_scales) if self.k_scales is not None else None,
            v_scales=to_dev(self.v_scales) if self.v_scales is not None else None)
        return d

    def config(self, lia, max_rows=None):
        g = self.g
        b = self.batch
        return lia.AttentionConfig(g.hq, g.hkv, g.d, g.page_size, b.pool_pages, b.stride,
                                   g.q_dtype, g.kv_dtype, g.out_dtype, g.scale, b.n_seqs,
                                   max_rows or max(b.n_rows, 1), int(b.ctx.max()))

    def run(self, lia, dev=None, max_rows=None):
        dev = dev or self.device()
        cfg = self.config(lia, max_rows)
        ws = dirty_workspace(lia, cfg)
        odt = torch.float32 if self.g.out_dtype == F32 else torch.bfloat16
        out = torch.full((self.batch.n_rows, self.g.hq, self.g.d), float("nan"), dtype=odt,
                         device="cuda")
        lia.paged_attention(cfg, self.batch.n_seqs, dev["cu"], dev["positions"], dev["sequences"],
                            dev["pages"], dev["q"], dev["kc"], dev["vc"], out, ws,
                            dev["k_scales"], dev["v_scales"])
        torch.cuda.synchronize()
        self.last_ws = ws  # the plan's header (units, blocks, ranges, overflow) is its first 16 bytes
        return out.float().cpu().numpy()


def dirty_workspace(lia, cfg):
    """A workspace for `cfg` filled with 0x7E bytes.  The workspace holds no required initial
    state, so every test starts it dirty: a split record the merge read without the kernel
    writing it (m and l 8.4e37 as floats) would outweigh every written one and show in the
    output."""
    return torch.full((lia.workspace_bytes(cfg),), 0x7E, dtype=torch.uint8, device="cuda")


def errors(got, ref):
    diff = np.abs(got.astype(np.float64) - ref)
    return float(np.nanmax(diff)) if diff.size else 0.0, float(np.nanmean(diff)) if diff.size else 0.0
