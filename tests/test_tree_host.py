"""Host side of tree verify, no GPU: the draft-tree topology
(speculative.rs:48-130) and the ancestor bitmask vk_tree_mask builds
(forward_tree's ancestors_map, metal/model.rs:615-632, as bits)."""
import ctypes as C

import numpy as np
import pytest

import velokv
from velokv import SpeculativeTree, TreeVerifyResult, branching_tree
from velokv import _capi


def brute_mask(parents):
    """Ancestors-or-self by walking parent links (independent of vk_tree_mask's
    parent-before-child recurrence)."""
    out = []
    for i in range(len(parents)):
        m, c = 0, i
        while c != -1:
            m |= 1 << c
            c = parents[c]
        out.append(m)
    return np.array(out, np.uint32)


def test_root_and_chain():
    t = SpeculativeTree.new(7)
    assert list(t.ancestor_mask()) == [1]
    for i in range(31):
        t.add_child(i, 100 + i)
    m = t.ancestor_mask()
    assert len(m) == 32
    assert all(int(m[i]) == (1 << (i + 1)) - 1 for i in range(32))


def test_222_tree_masks():
    t = branching_tree([2, 2, 2])
    assert len(t.nodes) == 15
    par = t.parents()
    assert list(par[:7]) == [-1, 0, 0, 1, 1, 2, 2]
    assert np.array_equal(t.ancestor_mask(), brute_mask(list(par)))
    # the 8-node draft tree: root, two children, four grandchildren, one great-grandchild
    t8 = branching_tree([2, 2, 2], 8)
    assert [bin(int(x)).count("1") for x in t8.ancestor_mask()] == [1, 2, 2, 3, 3, 3, 3, 4]


@pytest.mark.parametrize("seed", range(5))
def test_random_trees_match_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 33))
    par = [-1] + [int(rng.integers(0, i)) for i in range(1, n)]
    t = SpeculativeTree.new(0)
    for i in range(1, n):
        t.add_child(par[i], i)
    assert np.array_equal(t.ancestor_mask(), brute_mask(par))


def test_mask_rejects_bad_trees():
    lib = _capi.lib()
    out = (C.c_uint32 * 40)()
    for par in ([0, 0], [-1, 1], [-1, 0, 5], list(range(-1, 32))):
        arr = (C.c_int32 * len(par))(*par)
        assert lib.vk_tree_mask(arr, len(par), out) == velokv.ERR_BAD_ARG
    assert lib.vk_tree_mask(None, 1, out) == velokv.ERR_BAD_ARG


def test_get_path_and_find_best_path():
    # root 10 -> (11 -> 13, 12 -> 14)
    t = SpeculativeTree.new(10)
    a = t.add_child(0, 11)
    b = t.add_child(0, 12)
    c = t.add_child(a, 13)
    d = t.add_child(b, 14)
    assert t.get_path(c) == [10, 11, 13] and t.get_path(d) == [10, 12, 14]
    # target agrees with 12 after the root and with 14 after 12; rejects 13 after 11
    res = TreeVerifyResult(expected=[12, 99, 14, 0, 55])
    path, nxt = t.find_best_path(res)
    assert path == [10, 12, 14] and nxt == 55
    # nothing accepted: the root alone, and the target's token after it
    path, nxt = t.find_best_path(TreeVerifyResult(expected=[1, 2, 3, 4, 5]))
    assert path == [10] and nxt == 1
    # ties go to the later node (>= in speculative.rs:121)
    path, _ = t.find_best_path(TreeVerifyResult(expected=[11, 13, 14, 0, 0]))
    assert path == [10, 11, 13]
    path, _ = t.find_best_path(TreeVerifyResult(expected=[12, 13, 14, 0, 0]))
    assert path == [10, 12, 14]


def test_tree_workspace_query_validates_without_gpu():
    lib = _capi.lib()
    n = C.c_uint64()
    assert lib.vk_tree_verify_workspace(None, None, C.byref(n)) == velokv.ERR_BAD_ARG
