"""GPU flow of prefix sharing through the radix cache: prompts that share a
75-token prefix get their page lists from vk_radix_cache_sequence (the prefix's
full pages aliased, its partial last page copied on write), append their own
suffixes, and decode over the aliased pages. The GPU pool must equal the
oracle's byte for byte after the same copies and appends, and the decode must
match within the north-star tolerance."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, tol_check
from test_gpu_append_copy import assert_layer_equal
from velokv import synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_radix_prefix_sharing_flow(ctx, kv):
    print(f"radix flow kv={kv}", flush=True)
    Hkv, H, n_blocks = 2, 8, 128
    row = Hkv * HD
    rng = np.random.default_rng(7)
    prefix = list(range(1000, 1075))
    suffix_lens = [0, 1, 5, 20, 40, 53]
    bm = velokv.BlockManager(BS, n_blocks)
    rc = velokv.RadixCache(bm)
    pool = velokv.Pool(ctx, 1, n_blocks, BS, Hkv, HD, kv)
    ref = O.Layer(n_blocks, Hkv, BS, HD, kv)

    def append(pages, pos0, k, v):
        n = k.shape[0]
        if n == 0:
            return
        bt = np.asarray(pages, np.int32)[None, :]
        sl = synth.slots_for_positions(bt, np.arange(pos0, pos0 + n), BS, np.zeros(n, np.int64))
        ctx.append(pool, 0, ctx.upload(k), ctx.upload(v), velokv.DT_F16, ctx.upload(sl), n)
        O.append(ref, k, v, sl)

    kp = synth.normals_f16(75 * row, 1, row, 8.0).reshape(75, Hkv, HD)
    vp = synth.normals_f16(75 * row, 2, row, 8.0).reshape(75, Hkv, HD)
    first = rc.cache_sequence(prefix, seq_handle=1000, cache_handle=1001)
    append(first.pages, 0, kp, vp)
    bm.release(1000)  # the cache keeps the prefix (handle 1001)

    tables, lens, own = [], [], []
    for s, n in enumerate(suffix_lens):
        toks = prefix + [int(t) for t in rng.integers(0, 50000, n)] + [9000 + s]
        r = rc.cache_sequence(toks, seq_handle=2 * s, cache_handle=2 * s + 1)
        assert r.matched_tokens == 75
        assert r.pages[:4] == first.pages[:4]
        assert r.cow is not None  # 75 = 4 pages + 11 tokens: the fifth page is copied
        ctx.copy_blocks(pool, [r.cow])
        O.copy_blocks(ref, [r.cow])
        m = len(toks) - 75
        ks = synth.normals_f16(m * row, 10 + 2 * s, row, 8.0).reshape(m, Hkv, HD)
        vs = synth.normals_f16(m * row, 11 + 2 * s, row, 8.0).reshape(m, Hkv, HD)
        append(r.pages, 75, ks, vs)
        tables.append(r.pages)
        lens.append(len(toks))
        own.append(r.pages[4:])
    ctx.sync()
    assert_layer_equal(pool, 0, ref)
    # the prefix pages are shared by every sequence, the copied and fresh ones are not
    for pg in first.pages[:4]:
        assert bm.refcount(pg) == 1 + 2 * len(suffix_lens)
    flat = [p for o in own for p in o]
    assert len(flat) == len(set(flat)) and not set(flat) & set(first.pages)

    S = len(suffix_lens)
    stride = max(len(t) for t in tables)
    bt = np.zeros((S, stride), np.int32)
    for s, t in enumerate(tables):
        bt[s, :len(t)] = t
    cl = np.asarray(lens, np.int32)
    q = synth.normals_f16(S * H * HD, 99).reshape(S, H, HD)
    out = ctx.alloc(q.size * 4)
    ctx.paged_decode(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(cl), S, H, int(cl.max()),
                     block_tables=ctx.upload(bt), bt_stride=stride)
    ctx.sync()
    got = out.download(q.shape, np.float32)
    ok, err, nbad = tol_check(got, O.paged_decode(ref, q, bt, cl))
    assert ok, (err, nbad)
    # releasing every sequence and then the cache returns every page
    for s in range(S):
        bm.release(2 * s)
    rc.evict_coldest(10 ** 9)
    assert bm.free_pages() == n_blocks
