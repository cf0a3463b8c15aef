"""The prefix cache (vk_radix_*) on the CPU.

1. The reference's own RadixCache tests (radix_cache.rs:272-391) restated,
   run against the C ABI and against the Python restatement oracle/radix_ref.py.
2. Differential: random insert / lookup / evict / capacity sequences give the
   same results from the C++ cache and the restatement.
3. Pages: a cache bound to a block manager releases replaced and evicted
   handles; cache_sequence aliases the cached prefix's pages (reference counts),
   copies a shared partial page on write, and frees everything on release.
"""
import numpy as np
import pytest

import velokv
from radix_ref import RadixRef


class Adapter:
    """One interface over both implementations; handles are (block_id, token_len)."""

    def __init__(self, impl, cap=None):
        self.impl = impl
        self.c = velokv.RadixCache(None, cap) if impl == "c" else RadixRef(cap)
        self.lens = {}

    def insert(self, tokens, handle):
        if self.impl == "c":
            self.lens[handle[0]] = handle[1]
            old = self.c.insert(tokens, handle[0])
            return None if old is None else (old, self.lens[old])
        return self.c.insert(tokens, handle)

    def lookup(self, tokens):
        if self.impl == "c":
            r = self.c.lookup(tokens)
            return r.matched_tokens, (None if r.handle is None else (r.handle, self.lens[r.handle]))
        return self.c.lookup(tokens)

    def evict(self, n):
        if self.impl == "c":
            return [(h, self.lens[h]) for h in self.c.evict_coldest(n)]
        return self.c.evict_coldest(n)

    def len(self):
        return len(self.c)

    def resident(self):
        return self.c.resident_tokens() if self.impl == "c" else self.c.resident

    def set_cap(self, cap):
        self.c.set_capacity_tokens(cap)


IMPLS = ["c", "ref"]


def h(i, n):
    return (i, n)


@pytest.mark.parametrize("impl", IMPLS)
def test_returns_empty_lookup_on_miss(impl):
    c = Adapter(impl)
    assert c.lookup([1, 2, 3]) == (0, None)


@pytest.mark.parametrize("impl", IMPLS)
def test_reuses_longest_cached_prefix(impl):
    c = Adapter(impl)
    c.insert([10, 20], h(1, 2))
    c.insert([10, 20, 30, 40], h(2, 4))
    assert c.lookup([10, 20, 30, 40, 50]) == (4, h(2, 4))


@pytest.mark.parametrize("impl", IMPLS)
def test_splits_edge_when_new_prefix_is_shorter_than_existing_path(impl):
    c = Adapter(impl)
    c.insert([1, 2, 3, 4], h(7, 4))
    c.insert([1, 2], h(8, 2))
    assert c.lookup([1, 2, 9]) == (2, h(8, 2))
    assert c.lookup([1, 2, 3, 4, 5]) == (4, h(7, 4))


@pytest.mark.parametrize("impl", IMPLS)
def test_splits_edge_when_paths_diverge_mid_edge(impl):
    c = Adapter(impl)
    c.insert([1, 2, 3, 4], h(11, 4))
    c.insert([1, 2, 8, 9], h(12, 4))
    assert c.lookup([1, 2, 3, 4]) == (4, h(11, 4))
    assert c.lookup([1, 2, 8, 9]) == (4, h(12, 4))
    assert c.lookup([1, 2, 0]) == (0, None)


@pytest.mark.parametrize("impl", IMPLS)
def test_replaces_existing_handle_for_same_prefix(impl):
    c = Adapter(impl)
    c.insert([4, 5, 6], h(1, 3))
    assert c.insert([4, 5, 6], h(2, 3)) == h(1, 3)
    assert c.lookup([4, 5, 6, 7]) == (3, h(2, 3))
    assert c.len() == 1


@pytest.mark.parametrize("impl", IMPLS)
def test_evicts_oldest_prefixes_when_capacity_is_exceeded(impl):
    c = Adapter(impl, cap=5)
    c.insert([1, 2], h(1, 2))
    c.insert([3, 4], h(2, 2))
    c.insert([5, 6], h(3, 2))
    assert c.resident() == 4
    assert c.lookup([1, 2])[1] is None
    assert c.lookup([3, 4])[1] == h(2, 2)
    assert c.lookup([5, 6])[1] == h(3, 2)
    if impl == "c":
        assert c.c.capacity_tokens() == 5


@pytest.mark.parametrize("impl", IMPLS)
def test_cache_is_empty_and_len(impl):
    c = Adapter(impl)
    assert c.len() == 0
    c.insert([1], h(1, 1))
    assert c.len() == 1


@pytest.mark.parametrize("impl", IMPLS)
def test_capacity_updates(impl):
    c = Adapter(impl)
    c.insert([1, 2, 3], h(1, 3))
    assert c.resident() == 3
    c.set_cap(1)
    assert c.resident() == 0
    assert c.len() == 0


@pytest.mark.parametrize("seed", range(6))
def test_differential_random_operations(seed):
    rng = np.random.default_rng(seed)
    cap = [None, 40, 120][seed % 3]
    a, b = Adapter("c", cap), Adapter("ref", cap)
    nxt = 1
    for step in range(400):
        op = rng.integers(0, 10)
        toks = rng.integers(0, 4, rng.integers(0, 12)).tolist()  # small alphabet: shared prefixes, splits
        if op < 4:
            hd = (nxt, len(toks))
            nxt += 1
            assert a.insert(toks, hd) == b.insert(toks, hd), step
        elif op < 8:
            assert a.lookup(toks) == b.lookup(toks), step
        elif op == 8:
            n = int(rng.integers(0, 20))
            assert a.evict(n) == b.evict(n), step
        else:
            c2 = [None, int(rng.integers(0, 80))][int(rng.integers(0, 2))]
            a.set_cap(c2)
            b.set_cap(c2)
        assert a.len() == b.len() and a.resident() == b.resident(), step


# ---- pages ------------------------------------------------------------------------

def test_bound_cache_releases_replaced_and_evicted_handles():
    bm = velokv.BlockManager(16, 64)
    rc = velokv.RadixCache(bm)
    bm.allocate(1, 40)   # 3 pages
    bm.allocate(2, 40)
    rc.insert(list(range(40)), 1)
    assert bm.free_pages() == 64 - 6
    assert rc.insert(list(range(40)), 2) == 1   # replaced: handle 1's pages go back
    assert bm.free_pages() == 64 - 3
    with pytest.raises(velokv.VkError):
        bm.release(1)                            # already released by the cache
    assert rc.evict_coldest(1) == [2]
    assert bm.free_pages() == 64
    bm.allocate(3, 16)
    rc.insert(list(range(16)), 3)
    rc.close()                                   # destroy releases what the cache holds
    assert bm.free_pages() == 64


def test_cache_sequence_aliases_prefix_pages_and_copies_the_partial_page():
    bs = 16
    bm = velokv.BlockManager(bs, 1000)
    rc = velokv.RadixCache(bm)
    prefix = list(range(100, 100 + 4 * bs + 5))  # 69 tokens: 4 full pages + 5 in a fifth
    a = rc.cache_sequence(prefix + [1, 2, 3], seq_handle=10, cache_handle=11)
    assert a.matched_tokens == 0 and a.cow is None
    assert len(a.pages) == 5
    # a second prompt that extends the cached 72-token prompt (handle 11)
    b = rc.cache_sequence(prefix + [1, 2, 3] + [9] * 30, seq_handle=20, cache_handle=21)
    assert b.matched_tokens == 72
    assert b.pages[:4] == a.pages[:4]           # full pages aliased
    assert b.cow is not None and b.cow[0] == a.pages[4] and b.pages[4] == b.cow[1] != a.pages[4]
    for pg in a.pages[:4]:
        assert bm.refcount(pg) == 4             # seq 10, cache 11, seq 20, cache 21
    # a lookup now finds the longer prompt
    assert rc.lookup(prefix + [1, 2, 3] + [9] * 30 + [5]).matched_tokens == 102
    # the same prompt again: full hit, nothing new cached, pages aliased
    c = rc.cache_sequence(prefix + [1, 2, 3], seq_handle=30, cache_handle=31)
    assert c.matched_tokens == 72 and c.pages == a.pages and c.cow is None
    assert len(rc) == 2
    # release the sequences, then evict the cache: every page comes back
    for hd in (10, 20, 30):
        bm.release(hd)
    assert bm.free_pages() < 1000
    rc.evict_coldest(10 ** 6)
    assert bm.free_pages() == 1000


def test_configuration4_page_budget():
    """256 prompts sharing a 4096-token prefix with unique suffixes U[0, 512]:
    aliasing stores the prefix once (the reference allocates every prompt's
    pages, engine.rs:478-484)."""
    bs, S = 16, 256
    rng = np.random.default_rng(4)
    suffix = rng.integers(0, 513, S)
    prefix = list(range(4096))
    bm = velokv.BlockManager(bs, 200000)
    rc = velokv.RadixCache(bm)
    rc.cache_sequence(prefix, seq_handle=1 << 40, cache_handle=(1 << 40) + 1)
    bm.release(1 << 40)
    reference_pages = 4096 // bs  # the prefix prompt itself
    cows = 0
    for s in range(S):
        toks = prefix + [100000 + s * 1000 + t for t in range(int(suffix[s]))]
        r = rc.cache_sequence(toks, seq_handle=2 * s, cache_handle=2 * s + 1)
        assert r.matched_tokens == 4096
        cows += r.cow is not None
        reference_pages += -(-len(toks) // bs)
    used = 200000 - bm.free_pages()
    own = sum(-(-(4096 + int(x)) // bs) - 4096 // bs for x in suffix)
    assert used == 4096 // bs + own and cows == 0  # the prefix ends on a page boundary
    assert reference_pages > 15 * used
