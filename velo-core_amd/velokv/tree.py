"""Draft-tree topology for tree-verify attention.

SpeculativeTree mirrors speculative.rs:48-130 (new, add_child, get_path,
find_best_path). ancestor_mask() gives the per-node visibility rows that
vk_tree_verify takes: bit j of row i is set when node j is node i or one of its
ancestors (the bitmask form of forward_tree's ancestors_map, metal/model.rs:615-632).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._capi import check, lib


@dataclass
class TreeNode:
    token: int
    parent: int | None


@dataclass
class TreeVerifyResult:
    """Target-model token per tree node (speculative.rs:36-40)."""
    expected: list[int]


@dataclass
class SpeculativeTree:
    nodes: list[TreeNode] = field(default_factory=list)

    @classmethod
    def new(cls, token: int) -> "SpeculativeTree":
        return cls([TreeNode(token, None)])

    def add_child(self, parent_idx: int, token: int) -> int:
        if not 0 <= parent_idx < len(self.nodes):
            raise IndexError(f"parent {parent_idx} out of range")
        self.nodes.append(TreeNode(token, parent_idx))
        return len(self.nodes) - 1

    def get_path(self, node_idx: int) -> list[int]:
        path = []
        cur: int | None = node_idx
        while cur is not None:
            path.append(self.nodes[cur].token)
            cur = self.nodes[cur].parent
        return path[::-1]

    def find_best_path(self, verified: TreeVerifyResult) -> tuple[list[int], int | None]:
        """Longest root path whose every token matches the target's prediction at
        its parent; ties go to the later node. Returns (path, the target's token
        after the path's last node, if any)."""
        n = len(self.nodes)
        valid = [False] * n
        valid[0] = True
        for i in range(1, n):
            p = self.nodes[i].parent
            if p is not None and valid[p] and self.nodes[i].token == verified.expected[p]:
                valid[i] = True
        best: list[int] = []
        rejected = None
        for i in range(n):
            if valid[i]:
                path = self.get_path(i)
                if len(path) >= len(best):
                    best = path
                    rejected = verified.expected[i] if i < len(verified.expected) else None
        return best, rejected

    def path_nodes(self, node_idx: int) -> list[int]:
        """Node indices from the root to node_idx (get_path, speculative.rs:81-94, as node indices)."""
        path = []
        cur: int | None = node_idx
        while cur is not None:
            path.append(cur)
            cur = self.nodes[cur].parent
        return path[::-1]

    def best_path_nodes(self, verified: TreeVerifyResult) -> list[int]:
        """Node indices of find_best_path's path (speculative.rs:97-128): the rows vk_tree_commit moves to
        context_len + 0, 1, ... (root first)."""
        n = len(self.nodes)
        valid = [False] * n
        valid[0] = True
        for i in range(1, n):
            p = self.nodes[i].parent
            if p is not None and valid[p] and self.nodes[i].token == verified.expected[p]:
                valid[i] = True
        best: list[int] = []
        for i in range(n):
            if valid[i]:
                path = self.path_nodes(i)
                if len(path) >= len(best):
                    best = path
        return best

    def parents(self) -> np.ndarray:
        return np.array([-1 if nd.parent is None else nd.parent for nd in self.nodes], dtype=np.int32)

    def ancestor_mask(self) -> np.ndarray:
        """uint32 [n_nodes] visibility rows (vk_tree_mask)."""
        par = np.ascontiguousarray(self.parents())
        out = np.zeros(len(par), dtype=np.uint32)
        check(lib().vk_tree_mask(par.ctypes.data_as(C.POINTER(C.c_int32)), len(par),
                                 out.ctypes.data_as(C.POINTER(C.c_uint32))))
        return out


def branching_tree(branching: list[int], n_nodes: int | None = None, token0: int = 0) -> SpeculativeTree:
    """Breadth-first tree with the given branching per level (e.g. [2, 2, 2]),
    truncated to n_nodes nodes when given. Tokens are token0, token0+1, ..."""
    t = SpeculativeTree.new(token0)
    level = [0]
    tok = token0 + 1
    for b in branching:
        nxt = []
        for p in level:
            for _ in range(b):
                if n_nodes is not None and len(t.nodes) >= n_nodes:
                    return t
                nxt.append(t.add_child(p, tok))
                tok += 1
        level = nxt
    return t
