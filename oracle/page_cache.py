"""CPU oracle of the host page manager - test infrastructure only, never product code.

A direct restatement of src/inference/page_cache.rs:48-304 (PageCache), the key chain of
src/prefix_cache.rs:61-70 (Key::prefix) and the row construction of
src/server/paged/schedule.rs:5-60, with the reference's linear scans kept as they are (the
product library indexes its pool instead).  The page store and the KV pool are plain dicts
here: `store` maps key -> payload bytes and `pool` maps page -> payload bytes.

Pinned by: Key::prefix against hashlib's SHA-256 of the byte string the reference hashes
(tests/test_page_cache.py), brute-force invariants after every operation (reference counts
equal the pages held by live sequences, the prefix map is exactly the keyed pages, idle
counts), and hand-built scenarios for each rule the reference states in its comments
(retain-before-allocate, immutable pages, LRU victim choice, restore windows of 16).
"""
import hashlib

PREFIX_TAG = b"lia-kv-prefix-v1"   # src/prefix_cache.rs:63


def prefix_key(parent, tokens):
    """Key::prefix (src/prefix_cache.rs:61-70)."""
    h = hashlib.sha256()
    h.update(PREFIX_TAG)
    h.update(bytes(parent))
    h.update(len(tokens).to_bytes(8, "little"))
    for t in tokens:
        h.update(int(t).to_bytes(4, "little"))
    return h.digest()


class Error(Exception):
    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


class Sequence:
    def __init__(self):
        self.pages = []
        self.keys = []


class PageCache:
    """PageCache (src/inference/page_cache.rs:18-27)."""

    def __init__(self, namespace, pages, page_size=32, store=None, pool=None):
        if pages <= 0:
            raise Error(-19, "empty KV page pool")            # page_cache.rs:30
        self.namespace = bytes(namespace)
        self.page_size = page_size
        self.key = [None] * pages
        self.users = [0] * pages
        self.age = [0] * pages
        self.prefixes = {}
        self.clock = 0
        self.store = store            # None: every lookup misses, evictions are dropped
        self.pool = pool              # page -> payload (stands for the engine's KV pool)
        self.gpu_hits = 0
        self.evictions = 0

    def _keys(self, tokens):
        count = max(len(tokens) - 1, 0) // self.page_size   # page_cache.rs:55
        parent, keys = self.namespace, []
        for b in range(count):
            parent = prefix_key(parent, tokens[b * self.page_size:(b + 1) * self.page_size])
            keys.append(parent)
        return keys

    def attach(self, tokens):
        """page_cache.rs:48-157 -> (sequence, cached tokens)."""
        seq = Sequence()
        keys = self._keys(tokens)
        retained = []
        for k in keys:                                        # page_cache.rs:67-75
            page = self.prefixes.get(k)
            if page is not None:
                self.users[page] += 1
            retained.append(page)
        try:
            for w0 in range(0, len(keys), 16):                # page_cache.rs:77
                window = keys[w0:w0 + 16]
                staged = [None] * len(window)
                for i, k in enumerate(window):
                    if retained[w0 + i] is None and self.store is not None:
                        staged[i] = self.store.get(k)
                restored, stop = [], False
                for i, k in enumerate(window):
                    if retained[w0 + i] is not None:
                        page = retained[w0 + i]
                        retained[w0 + i] = None
                        self.gpu_hits += 1
                    else:
                        if staged[i] is None:                 # page_cache.rs:97-101
                            stop = True
                            break
                        page = self._allocate()
                        if page is None:
                            stop = True
                            break
                        restored.append((page, k, staged[i]))
                    self._touch(page)
                    seq.pages.append(page)
                    seq.keys.append(k)
                if restored:                                  # page_cache.rs:111-140
                    for page, _, data in restored:
                        self.pool[page] = data
                    for page, k, _ in restored:
                        self.key[page] = k
                        self.prefixes[k] = page
                if stop:
                    break
        finally:
            for page in retained:                             # page_cache.rs:148-150
                if page is not None:
                    self._release_page(page)
        return seq, len(seq.pages) * self.page_size

    def available_pages(self):
        return sum(1 for u in self.users if u == 0)

    def can_fit(self, tokens):
        """page_cache.rs:163-180."""
        shared = sum(1 for k in self._keys(tokens)
                     if k in self.prefixes and self.users[self.prefixes[k]] > 0)
        return -(-len(tokens) // self.page_size) <= self.available_pages() + shared

    def ensure_position(self, seq, position):
        """page_cache.rs:183-206."""
        additional = max(position // self.page_size + 1 - len(seq.pages), 0)
        if additional == 0:
            return True
        if additional > self.available_pages():
            return False
        while len(seq.pages) <= position // self.page_size:
            page = self._allocate()
            if page is None:
                return False
            seq.pages.append(page)
        return True

    def seal(self, seq, tokens, computed):
        """page_cache.rs:208-237."""
        P = self.page_size
        if computed > len(tokens) or -(-computed // P) > len(seq.pages):
            raise Error(-15, "invalid computed prefix extent")
        while len(seq.keys) < computed // P:
            block = len(seq.keys)
            parent = seq.keys[-1] if seq.keys else self.namespace
            k = prefix_key(parent, tokens[block * P:(block + 1) * P])
            current = seq.pages[block]
            shared = self.prefixes.get(k)
            if shared is not None:
                if shared != current:
                    self._release_page(current)
                    self.users[shared] += 1
                    seq.pages[block] = shared
            else:
                if self.key[current] is not None:
                    raise Error(-16, "attempted to overwrite immutable KV page")
                self.key[current] = k
                self.prefixes[k] = current
            self._touch(seq.pages[block])
            seq.keys.append(k)

    def release(self, seq):
        for page in seq.pages:
            self._release_page(page)

    def _release_page(self, page):
        if self.users[page] == 0:
            raise Error(-17, "KV page reference underflow")
        self.users[page] -= 1

    def evict_idle(self):
        for page in range(len(self.users)):
            if self.users[page] == 0 and self.key[page] is not None:
                self._evict(page)

    def _allocate(self):
        """page_cache.rs:250-273: first idle unkeyed page, else the idle page of least age."""
        free = next((i for i in range(len(self.users))
                     if self.users[i] == 0 and self.key[i] is None), None)
        if free is None:
            idle = [i for i in range(len(self.users)) if self.users[i] == 0]
            if not idle:
                return None
            free = min(idle, key=lambda i: self.age[i])
        if self.key[free] is not None:
            self._evict(free)
        self.users[free] = 1
        self._touch(free)
        return free

    def _evict(self, page):
        if self.users[page]:
            raise Error(-18, "cannot evict an active KV page")
        k = self.key[page]
        if k is not None:
            if self.store is not None:
                self.store[k] = self.pool.get(page)
            del self.prefixes[k]
            self.key[page] = None
            self.evictions += 1

    def _touch(self, page):
        self.clock += 1
        self.age[page] = self.clock


def schedule_rows(cache, requests, prefill_batch):
    """Runtime::step row construction (src/server/paged/schedule.rs:5-60).  requests: list of
    dicts (tokens, computed, sequence, closed) or None per slot.  Returns rows
    [(token, position, slot)], output row indices, updates [(slot, computed, output)]."""
    count = sum(1 for r in requests if r is not None)
    rows, outputs, updates = [], [], []
    if count == 0:
        return rows, outputs, updates
    allowance = max(prefill_batch // count, 1)
    for slot, r in enumerate(requests):
        if r is None:
            continue
        if r.get("closed"):
            r["done"] = True
            continue
        end = min(r["computed"] + allowance, len(r["tokens"]))
        computed = r["computed"]
        for position in range(r["computed"], end):
            if not cache.ensure_position(r["sequence"], position):
                break
            rows.append((r["tokens"][position], position, slot))
            computed += 1
        if computed > r["computed"]:
            output = computed == len(r["tokens"])
            if output:
                outputs.append(len(rows) - 1)
            updates.append((slot, computed, output))
    return rows, outputs, updates
