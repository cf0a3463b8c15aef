"""Pure-Python restatement of the reference's RadixCache (radix_cache.rs:28-264).

TEST INFRASTRUCTURE ONLY: the checker for the C++ prefix cache
(velo-core_amd/csrc/velokv_radix.cpp) in tests/; nothing in the product imports it.
Handles are (block_id, token_len) tuples as KvCacheHandle (radix_cache.rs:6-9).
Pinned by the reference's own unit tests (radix_cache.rs:272-391), restated in
tests/test_radix.py against this class and the C ABI alike.
"""
from __future__ import annotations


class _Node:
    __slots__ = ("edge", "children", "handle", "tick", "hits")

    def __init__(self, edge=(), tick=0, hits=0):
        self.edge = list(edge)
        self.children = {}   # BTreeMap<TokenId, NodeId>
        self.handle = None
        self.tick = tick
        self.hits = hits


def _common(a, b):
    n = 0
    for x, y in zip(a, b):
        if x != y:
            break
        n += 1
    return n


class RadixRef:
    def __init__(self, capacity_tokens=None):      # new / with_capacity_tokens (58-71)
        self.nodes = [_Node()]
        self.capacity = capacity_tokens
        self.resident = 0
        self.clock = 1

    def insert(self, tokens, handle):               # insert (73-99)
        assert len(tokens) == handle[1]
        self.clock += 1
        self.nodes[0].tick = self.clock
        self.nodes[0].hits += 1
        leaf = self._insert_from(0, list(tokens))
        replaced = self.nodes[leaf].handle
        self.nodes[leaf].handle = handle
        self.nodes[leaf].tick = self.clock
        self.nodes[leaf].hits += 1
        if replaced is not None:
            self.resident -= replaced[1]
        self.resident += handle[1]
        self._evict_to_capacity()
        return replaced

    def lookup(self, tokens):                       # lookup (101-140)
        self.clock += 1
        tick = self.clock
        node, cursor = 0, 0
        best = (0, self.nodes[0].handle) if self.nodes[0].handle is not None else None
        self.nodes[0].tick = tick
        self.nodes[0].hits += 1
        while cursor < len(tokens):
            child = self.nodes[node].children.get(tokens[cursor])
            if child is None:
                break
            m = _common(tokens[cursor:], self.nodes[child].edge)
            if m < len(self.nodes[child].edge):
                break
            cursor += m
            node = child
            self.nodes[node].tick = tick
            self.nodes[node].hits += 1
            if self.nodes[node].handle is not None:
                best = (cursor, self.nodes[node].handle)
        return best if best is not None else (0, None)

    def __len__(self):                              # len (142-144)
        return sum(1 for n in self.nodes if n.handle is not None)

    def set_capacity_tokens(self, cap):             # set_capacity_tokens (150-153)
        self.capacity = cap
        self._evict_to_capacity()

    def evict_coldest(self, tokens_to_evict):       # evict_coldest (163-187)
        order = sorted(((n.tick, i) for i, n in enumerate(self.nodes) if n.handle is not None),
                       key=lambda t: t[0])
        evicted, freed = [], 0
        for _, i in order:
            if freed >= tokens_to_evict:
                break
            h = self.nodes[i].handle
            self.nodes[i].handle = None
            self.resident -= h[1]
            freed += h[1]
            evicted.append(h)
        return evicted

    def _insert_from(self, parent, tokens):         # insert_from (189-221)
        while tokens:
            child = self.nodes[parent].children.get(tokens[0])
            if child is None:
                self.nodes.append(_Node(tokens, self.clock, 0))
                self.nodes[parent].children[tokens[0]] = len(self.nodes) - 1
                return len(self.nodes) - 1
            common = _common(tokens, self.nodes[child].edge)
            if common == len(self.nodes[child].edge):
                parent, tokens = child, tokens[common:]
                continue
            split = self._split_child(parent, child, common)
            if common == len(tokens):
                return split
            parent, tokens = split, tokens[common:]
        return parent

    def _split_child(self, parent, child, at):      # split_child (223-242)
        old_first = self.nodes[child].edge[0]
        prefix, suffix = self.nodes[child].edge[:at], self.nodes[child].edge[at:]
        self.nodes[child].edge = suffix
        s = _Node(prefix, self.clock, self.nodes[child].hits)
        s.children = {suffix[0]: child}
        self.nodes.append(s)
        self.nodes[parent].children[old_first] = len(self.nodes) - 1
        return len(self.nodes) - 1

    def _evict_to_capacity(self):                   # evict_to_capacity (250-262)
        if self.capacity is None or self.resident <= self.capacity:
            return
        self.evict_coldest(self.resident - self.capacity)
