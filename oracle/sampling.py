"""CPU oracle of sparse paged sampling - test infrastructure only, never product code.

Restates, in plain Python (f64 through `math`, f32 steps rounded explicitly, logf/fmaf from
the C library as the reference's f32::ln / mul_add use it):
- llama_nucleus_candidates (src/gpu/kernels/llama_nucleus.rs:18-117): per row and part of
  1024 vocabulary entries, the 21 largest entries by the total-order key of their f32 bits
  (ties: larger id first), the part's maximum and the f64 mass sum exp((x - max) / T);
- Workspace::read (src/gpu/nucleus.rs:78-144): the per-row reduction of those records;
- Sampling::{new, distribution, draw} (src/sampling.rs:33-190), MT19937 + its two-word
  double (src/sampling/random.rs), the position-keyed Gumbel draw (src/sampling/gumbel.rs),
  distribution_logits / checked_nucleus / select_nucleus (src/sampling/nucleus.rs:9-124);
- the per-row sampling of Engine::forward_paged_sampled (src/inference/paged_sampling.rs:7-76).

Pinned by the reference's own tests (tests/test_sampling.py): the published MT19937 vector
and its doubles (random.rs:52-71), every case of sampling.rs:192-313 and nucleus.rs:127-181,
the Gumbel categorical-mass test (gumbel.rs:98-110) and the GPU candidates test's expected
sparse / fallback pattern (nucleus.rs:183-231).
"""
import ctypes
import math
import struct

import numpy as np

SLOTS = 21          # src/gpu/nucleus.rs:4
PART = 1024
_libm = ctypes.CDLL("libm.so.6")
_libm.logf.restype = ctypes.c_float
_libm.logf.argtypes = [ctypes.c_float]
_libm.fmaf.restype = ctypes.c_float
_libm.fmaf.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def total_key(value):
    """f32::total_cmp as an integer key (llama_nucleus.rs:80-81)."""
    bits = f32_bits(value)
    signed = bits - (1 << 32) if bits >> 31 else bits
    return signed ^ (0x7FFFFFFF if signed < 0 else 0)


class Error(Exception):
    pass


# ------------------------------------------------------------------ random.rs

class Random:
    """MT19937 (src/sampling/random.rs:2-53)."""

    def __init__(self, seed):
        w = [0] * 624
        w[0] = seed & 0xFFFFFFFF
        for i in range(1, 624):
            w[i] = (1812433253 * (w[i - 1] ^ (w[i - 1] >> 30)) + i) & 0xFFFFFFFF
        self.words, self.index = w, 624

    def next(self):
        w = self.words
        if self.index == 624:
            for i in range(624):
                mixed = (w[i] & 0x80000000) | (w[(i + 1) % 624] & 0x7FFFFFFF)
                w[i] = w[(i + 397) % 624] ^ (mixed >> 1) ^ (0x9908B0DF if mixed & 1 else 0)
            self.index = 0
        v = w[self.index]
        self.index += 1
        v ^= v >> 11
        v ^= (v << 7) & 0x9D2C5680
        v ^= (v << 15) & 0xEFC60000
        return v ^ (v >> 18)

    def uniform_f32(self):
        return min(f32(self.next() / 4294967296.0), f32(struct.unpack(
            "<f", struct.pack("<I", f32_bits(1.0) - 1))[0]))

    def uniform(self):
        low = float(self.next())
        high = float(self.next())
        return min((low + high * 4294967296.0) / 18446744073709551616.0,
                   struct.unpack("<d", struct.pack("<Q", struct.unpack("<Q", struct.pack(
                       "<d", 1.0))[0] - 1))[0])


# ------------------------------------------------------------------ gumbel.rs

def _rotl(x, r):
    return ((x << r) | (x >> (32 - r))) & 0xFFFFFFFF


def gumbel_hash(seed, position, token):
    """MurmurHash3 mixing of (seed lo, seed hi, position lo, token) (gumbel.rs:4-22)."""
    h = 0
    for word in (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF, position & 0xFFFFFFFF, token):
        k = _rotl((word * 0xCC9E2D51) & 0xFFFFFFFF, 15) * 0x1B873593 & 0xFFFFFFFF
        h = (_rotl(h ^ k, 13) * 5 + 0xE6546B64) & 0xFFFFFFFF
    h ^= 16
    h ^= h >> 16
    h = h * 0x85EBCA6B & 0xFFFFFFFF
    h ^= h >> 13
    h = h * 0xC2B2AE35 & 0xFFFFFFFF
    return h ^ (h >> 16)


def gumbel_uniform(word):
    a = f32(f32(float(word >> 16)) * f32(1.0 / 65536.0))
    b = f32(f32(float(word & 65535) + 0.5) * f32(1.0 / 4294967296.0))
    return f32(a + b)


def gumbel_noise(u):
    """-ln(-ln(1-u)) with the series for small u (gumbel.rs:28-40)."""
    if u < 0.25:
        poly = f32(1.0 / 8.0)
        for d in range(7, 0, -1):
            poly = _libm.fmaf(u, poly, float(np.float32(1.0) / np.float32(d)))
        neg = f32(u * poly)
    else:
        neg = f32(-_libm.logf(max(f32(1.0 - u), f32(1.0 / 16777216.0))))
    return f32(-_libm.logf(neg))


def gumbel_draw(entries, seed, position):
    best = None
    for token, p in entries:
        score = f32(f32(math.log(p)) + gumbel_noise(gumbel_uniform(gumbel_hash(seed, position,
                                                                                  token))))
        # max_by(total_cmp(score) then reverse id): larger score, then smaller id
        key = (total_key(score), -token)
        if best is None or key > best[0]:
            best = (key, token)
    return best[1]


# ------------------------------------------------------------------ sampling.rs / nucleus.rs

def _order_key(c):
    """Sort key of the reference's `order` (descending total order of value, then id)."""
    return (-total_key(c[1]), -c[0])


class Sampling:
    def __init__(self, temperature, top_k, top_p, seed, position_keyed=False):
        if not (math.isfinite(temperature) and temperature > 0.0):
            raise Error("temperature must be finite and positive")
        if top_k > 20:
            raise Error("sampling top_k must be 0 (unrestricted) or 1..=20")
        if not (math.isfinite(top_p) and 0.0 < top_p <= 1.0):
            raise Error("top_p must be in (0,1]")
        self.temperature, self.top_k, self.top_p, self.seed = temperature, top_k, top_p, seed
        self.random = Random(seed & 0xFFFFFFFF)
        self.position = 0 if position_keyed else None

    def set_position(self, position):
        if self.position is not None:
            self.position = position

    def distribution(self, candidates):
        """sampling.rs:82-128."""
        cands = list(candidates)
        if any(math.isnan(x) or x == math.inf for _, x in cands):
            raise Error("invalid sampling logits")
        cands = [c for c in cands if c[1] != -math.inf]
        cands.sort(key=_order_key)
        if self.top_k != 0 and len(cands) > self.top_k:
            cands = cands[:self.top_k]
        if not cands:
            raise Error("empty sampling distribution")
        mx = float(cands[0][1])
        if len({i for i, _ in cands}) != len(cands):
            raise Error("duplicate sampling candidate")
        entries = [(i, math.exp((float(x) - mx) / self.temperature)) for i, x in cands]
        total = 0.0
        for _, p in entries:
            total += p
        mass, keep = 0.0, len(entries)
        for i, (_, w) in enumerate(entries):
            mass += w
            if mass >= self.top_p * total:
                keep = i + 1
                break
        entries = entries[:keep]
        total = 0.0
        for _, p in entries:
            total += p
        return [(i, p / total) for i, p in entries]

    def _weight(self, v, maximum):
        return math.exp((float(v) - maximum) / self.temperature)

    def select_nucleus(self, candidates, maximum, total):
        """nucleus.rs:96-124; sorts the retained prefix of `candidates` in place."""
        if not candidates:
            raise Error("empty nucleus candidate list")
        target = self.top_p * total
        count = min(len(candidates), 128)
        while True:
            if count < len(candidates):
                candidates.sort(key=_order_key)      # same prefix as a partial selection
            mass = 0.0
            for _, v in candidates[:count]:
                mass += self._weight(v, maximum)
            if mass >= target or count == len(candidates):
                break
            count = min(count * 2, len(candidates))
        head = sorted(candidates[:count], key=_order_key)
        candidates[:count] = head
        mass, entries = 0.0, []
        for i, v in head:
            w = self._weight(v, maximum)
            mass += w
            entries.append((i, w))
            if mass >= target:
                break
        if not (math.isfinite(mass) and mass > 0.0):
            raise Error("invalid nucleus mass")
        return [(i, p / mass) for i, p in entries]

    def distribution_logits(self, logits):
        """nucleus.rs:9-46."""
        if self.top_k != 0 or self.top_p == 1.0:
            return self.distribution(enumerate(float(x) for x in logits))
        vals = [float(x) for x in np.asarray(logits, np.float32)]
        if any(math.isnan(v) or v == math.inf for v in vals):
            raise Error("invalid sampling logits")
        cands = [(i, v) for i, v in enumerate(vals) if v != -math.inf]
        if not cands:
            raise Error("empty sampling distribution")
        maximum = float(max(cands, key=lambda c: total_key(c[1]))[1])
        total = 0.0
        for _, v in cands:
            total += self._weight(v, maximum)
        return self.select_nucleus(cands, maximum, total)

    def checked_nucleus(self, candidates, maximum, total, omitted):
        """nucleus.rs:49-93: None when the sparse candidates cannot prove the cutoff."""
        if not (math.isfinite(total) and total > 0.0 and math.isfinite(maximum)):
            raise Error("invalid full-vocabulary normalizer")
        if self.top_p == 1.0:
            return None
        cands = list(candidates)
        entries = self.select_nucleus(cands, maximum, total)
        if not entries:
            return None
        keep = len(entries)
        last = entries[-1][0]
        if cands[keep - 1][0] != last:
            raise Error("inconsistent nucleus candidate order")
        if not total_key(cands[keep - 1][1]) > total_key(omitted):
            return None
        target = self.top_p * total
        through = 0.0
        for _, v in cands[:keep]:
            through += self._weight(v, maximum)
        before = through - self._weight(cands[keep - 1][1], maximum)
        uncertainty = abs(total) * 1e-10
        if before >= target - uncertainty or through <= target + uncertainty:
            return None
        return entries

    def draw(self, entries):
        """sampling.rs:134-146."""
        if self.position is not None:
            position = self.position
            self.position = (position + 1) & 0xFFFFFFFFFFFFFFFF
            return gumbel_draw(entries, self.seed, position)
        if len(entries) == 1:
            return entries[0][0]
        sample = self.random.uniform()
        cumulative = 0.0
        for i, p in entries:
            cumulative += p
            if sample < cumulative:
                return i
        return entries[-1][0]


# ------------------------------------------------------------------ llama_nucleus.rs / nucleus.rs

def nucleus_candidates(logits, temperatures):
    """(candidates u64 [rows][parts][21], normalizers f64 [rows][parts][2]) as the kernel
    writes them.  logits: f32 [rows][vocab]."""
    logits = np.asarray(logits, np.float32)
    rows, vocab = logits.shape
    parts = -(-vocab // PART)
    cand = np.zeros((rows, parts, SLOTS), np.uint64)
    norm = np.zeros((rows, parts, 2), np.float64)
    for r in range(rows):
        t = float(temperatures[r])
        for p in range(parts):
            vals = logits[r, p * PART:(p + 1) * PART]
            ids = list(range(p * PART, p * PART + len(vals)))
            fv = [float(x) for x in vals]
            finite_or_neg = [x for x in fv if not math.isnan(x)]
            mx = max(finite_or_neg) if finite_or_neg else -math.inf
            invalid = any(math.isnan(x) or x == math.inf for x in fv)
            s = math.nan if invalid else 0.0
            if t > 0.0 and math.isfinite(mx):
                for x in fv:
                    if math.isfinite(x):
                        s += math.exp((x - mx) / t)
            norm[r, p] = (mx, s)
            order = sorted(zip(fv, ids), key=lambda c: (total_key(c[0]), c[1]), reverse=True)
            for rank in range(SLOTS):
                if rank < len(order):
                    v, i = order[rank]
                    word = (i << 32) | f32_bits(v)
                else:
                    word = (0xFFFFFFFF << 32) | f32_bits(-math.inf)
                cand[r, p, rank] = word
    return cand, norm


def read_rows(cand, norm, temperatures, vocab):
    """Workspace::read's reduction (nucleus.rs:103-143) -> [(candidates, max, total, omitted)]."""
    rows, parts, _ = cand.shape
    out = []
    for r in range(rows):
        ns = norm[r]
        if not all(math.isfinite(x) for x in ns[:, 1]):
            raise Error("invalid sampler logits or normalizer")
        maximum = max((float(x) for x in ns[:, 0]), key=lambda v: (v != v, v)) if parts else -math.inf
        t = float(temperatures[r])
        total = 0.0
        if t > 0.0:
            for m, s in ns:
                if s > 0.0:
                    total += s * math.exp((m - maximum) / t)
        selected, omitted = [], -math.inf
        for p in range(parts):
            for rank, word in enumerate(cand[r, p]):
                word = int(word)
                i, v = word >> 32, struct.unpack("<f", struct.pack("<I", word & 0xFFFFFFFF))[0]
                if i == 0xFFFFFFFF or not math.isfinite(v):
                    continue
                if i >= vocab:
                    raise Error("sampler candidate ID outside vocabulary")
                if rank < SLOTS - 1:
                    selected.append((i, v))
                else:
                    omitted = max(omitted, v)
        out.append((selected, maximum, total, omitted))
    return out


def sample_rows(logits, samplers, positions):
    """The per-row tail of forward_paged_sampled (paged_sampling.rs:7-76): tokens and the
    number of full-row fallbacks.  samplers: Sampling or None (greedy) per output row."""
    temps = [(s.temperature if s.top_k == 0 else 0.0) if s is not None else 0.0
             for s in samplers]
    for s, pos in zip(samplers, positions):
        if s is not None:
            s.set_position(pos)
    logits = np.asarray(logits, np.float32)
    cand, norm = nucleus_candidates(logits, temps)
    rows = read_rows(cand, norm, temps, logits.shape[1])
    tokens, fallbacks = [], 0
    for i, ((c, mx, total, omitted), s) in enumerate(zip(rows, samplers)):
        if s is not None:
            if s.top_k != 0:
                d = s.distribution(c)
            else:
                d = s.checked_nucleus(c, mx, total, omitted)
                if d is None:
                    fallbacks += 1
                    d = s.distribution_logits(logits[i])
            tokens.append(s.draw(d))
        else:
            if not c:
                raise Error("empty greedy vocabulary")
            tokens.append(max(c, key=lambda e: (total_key(e[1]), e[0]))[0])
    return tokens, fallbacks
