"""Configuration 4 at full batch, as bench.py --workload tree runs it: 256
sequences whose 4096-token prefix is cached once in the radix cache and aliased
into every prompt's table (vk_radix_cache_sequence), suffixes U[0, 512], the
partial last prompt page of every sequence copied on write, 8 draft tokens
appended, an 8-node 2-2-2 tree verified with the shared prefix declared
(shared_blocks = 256), then the accepted path of every sequence committed
(vk_tree_commit). At this size the planner cuts the prefix into one chunk of
256 pages and the 256 x 8 x 4 query rows of each KV head into 32 row tiles.

Checked against the oracle on one layer:
  - the pool bytes after the appends and copies, then after the commit, bit
    for bit (the oracle performs the same appends, copies and commits);
  - the verify outputs of 8 sampled sequences within the north-star
    tolerance (the oracle's vko_tree_verify restricted to their table rows).
Tree semantics as vk_tree_verify defines them (node j at context_len + j, a
node sees its ancestors and itself); kernels.metal:512-599 is the reference's
tree kernel.
"""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD
from test_gpu_append_copy import assert_layer_equal
from test_gpu_tree import check, tree_q
from velokv import synth

pytestmark = pytest.mark.gpu


def radix_tables(S, prefix, suffix, N):
    """Tables as bench.run_tree builds them: (tables, fill_tables, COW pairs,
    n_blocks), pages scattered over the pool by a seeded permutation."""
    committed = prefix + suffix
    total = committed + N
    stride = int(-(-int(total.max()) // BS))
    budget = -(-prefix // BS) + int(sum(-(-int(t) // BS) + 1 for t in total))
    bm = velokv.BlockManager(BS, budget)
    rc = velokv.RadixCache(bm)
    prefix_tokens = list(range(prefix))
    rc.cache_sequence(prefix_tokens, seq_handle=1 << 40, cache_handle=(1 << 40) + 1)
    bm.release(1 << 40)
    tables = np.zeros((S, stride), np.int32)
    fill_tables = np.zeros((S, stride), np.int32)
    pairs = []
    for s in range(S):
        toks = prefix_tokens + [10 ** 6 + s * 1000 + t for t in range(int(suffix[s]))]
        rc.cache_sequence(toks, seq_handle=2 * s, cache_handle=2 * s + 1)
        pages = bm.extend(2 * s, int(total[s]))
        fill_tables[s, :len(pages)] = pages
        c = int(committed[s])
        if c % BS:
            cw = bm.cow(2 * s, c // BS)
            if cw is not None:
                pairs.append(cw)
            pages = bm.materialize_span(2 * s)
        tables[s, :len(pages)] = pages
    n_blocks = int(max(tables.max(), fill_tables.max(), max((max(p) for p in pairs), default=0))) + 1
    perm = synth.rng(5).permutation(n_blocks).astype(np.int32)
    pairs = perm[np.array(pairs, np.int64)] if pairs else np.zeros((0, 2), np.int32)
    return perm[tables], perm[fill_tables], pairs.astype(np.int32), n_blocks


def test_config4_full_batch(ctx):
    print("config4 full batch: radix tables, COW, drafts, verify, commit", flush=True)
    S, N, Hkv, G, prefix = 256, 8, 8, 4, 4096
    H = Hkv * G
    kv = O.I8_BLK
    suffix = synth.rng(4).integers(0, 513, S).astype(np.int32)
    committed = prefix + suffix
    tables, fill_tables, pairs, n_blocks = radix_tables(S, prefix, suffix, N)
    shared = prefix // BS
    assert np.all(tables[:, :shared] == tables[0, :shared])
    assert len(pairs) > 200  # nearly every sequence copies its partial prompt page
    pool = velokv.Pool(ctx, 1, n_blocks, BS, Hkv, HD, kv)
    ref = O.Layer(n_blocks, Hkv, BS, HD, kv)
    row = Hkv * HD
    try:
        # prefix once through sequence 0's row, then every suffix (as the bench fills it)
        rows = np.concatenate([np.zeros(prefix, np.int64)] + [np.full(int(x), i) for i, x in enumerate(suffix)])
        pos = np.concatenate([np.arange(prefix)] + [np.arange(prefix, int(c)) for c in committed])
        sl = synth.slots_for_positions(fill_tables, pos, BS, rows)
        k = synth.normals_f16(len(pos) * row, 4001, row, 8.0).reshape(-1, Hkv, HD)
        v = synth.normals_f16(len(pos) * row, 4002, row, 8.0).reshape(-1, Hkv, HD)
        ctx.append(pool, 0, ctx.upload(k), ctx.upload(v), velokv.DT_F16, ctx.upload(sl), len(sl))
        O.append(ref, k, v, sl)
        ctx.copy_blocks(pool, pairs)
        O.copy_blocks(ref, pairs)
        dpos = (committed[:, None] + np.arange(N)[None, :]).reshape(-1)
        dsl = synth.slots_for_positions(tables, dpos, BS, np.repeat(np.arange(S), N))
        dk = synth.normals_f16(S * N * row, 4003, row, 8.0).reshape(-1, Hkv, HD)
        dv = synth.normals_f16(S * N * row, 4004, row, 8.0).reshape(-1, Hkv, HD)
        ctx.append(pool, 0, ctx.upload(dk), ctx.upload(dv), velokv.DT_F16, ctx.upload(dsl), len(dsl))
        O.append(ref, dk, dv, dsl)
        ctx.sync()
        assert_layer_equal(pool, 0, ref)

        stride = tables.shape[1]
        pl = ctx.tree_plan(pool, S, N, H, int(committed.max()), bt_stride=stride, shared_blocks=shared)
        assert pl["prefix_chunks"] == 1 and pl["prefix_row_tiles"] == 32, pl
        assert pl["prefix_kernel"] == "vk_tree_pfx_kv3_g4_q1" and pl["kernel"] == "vk_tree_kv3_g4_r2_q1", pl
        assert not pl["merge_launch"], pl
        q = tree_q(S, N, H, 4005)
        tree = velokv.branching_tree([2, 2, 2, 2, 2], N)
        mask = np.tile(tree.ancestor_mask(), (S, 1))
        out = ctx.alloc(S * N * H * HD * 4)
        ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask),
                        S, N, H, int(committed.max()), block_tables=ctx.upload(tables), bt_stride=stride,
                        shared_blocks=shared)
        ctx.sync()
        got = out.download((S, N, H, HD), np.float32)
        sample = sorted({0, 37, 100, 128, 199, 255, int(np.argmax(committed)), int(np.argmin(committed))})
        expect = O.tree_verify(ref, q[sample], tables[sample], committed[sample], mask[sample])
        check(got[sample], expect, "config 4 full batch, sampled sequences")

        # accepted path of every sequence: root to node s % N (what find_best_path
        # returns when the target agrees along that branch), committed in place
        acc_rows = [tree.path_nodes(s % N) for s in range(S)]
        acc = np.full((S, 32), -1, np.int32)
        n_acc = np.array([len(a) for a in acc_rows], np.int32)
        for s, a in enumerate(acc_rows):
            acc[s, :len(a)] = a
        status = ctx.alloc(4 * S)
        ctx.tree_commit(pool, ctx.upload(tables), stride, ctx.upload(committed), ctx.upload(acc), 32,
                        ctx.upload(n_acc), S, status=status)
        ctx.sync()
        assert np.all(status.download((S,), np.int32) == velokv.COMMIT_OK)
        for s in range(S):
            assert O.tree_commit(ref, tables[s], int(committed[s]), acc_rows[s]) == 0
        assert_layer_equal(pool, 0, ref)
    finally:
        pool.close()
