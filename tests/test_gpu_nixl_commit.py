"""GPU parity of the NIXL wire records (vk_nixl_pack / vk_nixl_unpack) and of the
accepted-path commit of a draft tree (vk_tree_commit): wire bytes, statuses and
pool bytes must equal the oracle's bit for bit."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD
from velokv import synth

pytestmark = pytest.mark.gpu

KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]


def random_pool(ctx, kv, n_layer, n_blocks, n_kv_heads, seed):
    """A pool and its oracle mirror filled with random bytes (every layer)."""
    pool = velokv.Pool(ctx, n_layer, n_blocks, BS, n_kv_heads, HD, kv)
    rng = synth.rng(seed)
    layers = []
    for l in range(n_layer):
        L = O.Layer(n_blocks, n_kv_heads, BS, HD, kv)
        for key in ("k", "v", "ks", "vs"):
            a = getattr(L, key)
            if a is not None:
                a[:] = rng.integers(0, 256, a.size, dtype=np.uint8)
        pool.upload_layer(l, {"k": L.k, "v": L.v, "ks": L.ks, "vs": L.vs})
        layers.append(L)
    ctx.sync()
    return pool, layers


def assert_pool_equal(pool, layers, layer0=0):
    for i, ref in enumerate(layers):
        got = pool.download_layer(layer0 + i)
        for key in ("k", "v", "ks", "vs"):
            r = getattr(ref, key)
            if r is None:
                continue
            if not np.array_equal(got[key], r):
                bad = np.nonzero(got[key] != r)[0]
                raise AssertionError(f"layer {layer0 + i} {key}: {len(bad)} bytes differ, first at {bad[:8]}")


def run_pack(ctx, pool, items, pages, wire_bytes, layer0=0, n_layers=None, fill=0xEE):
    wire = ctx.upload(np.full(wire_bytes, fill, np.uint8))
    pg = ctx.upload(np.asarray(pages, np.int32)) if len(pages) else ctx.alloc(4)
    status = ctx.upload(np.full(max(1, len(items)), -7, np.int32))
    ctx.nixl_pack(pool, items, pg, len(pages), wire, wire_bytes, status, layer0=layer0, n_layers=n_layers)
    ctx.sync()
    return wire.download((wire_bytes,), np.uint8), list(status.download((max(1, len(items)),), np.int32)[:len(items)])


def run_unpack(ctx, pool, items, pages, wire_host, layer0=0, n_layers=None):
    wire = ctx.upload(np.ascontiguousarray(wire_host, np.uint8))
    pg = ctx.upload(np.asarray(pages, np.int32)) if len(pages) else ctx.alloc(4)
    status = ctx.upload(np.full(max(1, len(items)), -7, np.int32))
    ctx.nixl_unpack(pool, items, pg, len(pages), wire, wire_host.size, status, layer0=layer0, n_layers=n_layers)
    ctx.sync()
    return list(status.download((max(1, len(items)),), np.int32)[:len(items)])


def layout(token_lens, pool, n_layers):
    """items (block_id, token_len, first_page, wire_offset) packed back to back at
    16-aligned offsets with a gap, and the total wire size."""
    items, off, fp = [], 0, 0
    for i, tl in enumerate(token_lens):
        items.append((1000 + 7 * i, tl, fp, off))
        fp += (tl + BS - 1) // BS
        off += 16 + pool.nixl_payload_bytes(tl, n_layers)
        off = (off + 15) // 16 * 16 + 32
    return items, off + 64, fp


@pytest.mark.parametrize("kv", KV_ALL)
def test_nixl_pack_bit_exact(ctx, kv):
    print(f"nixl pack kv={kv}", flush=True)
    pool, layers = random_pool(ctx, kv, 3, 48, 2, seed=31 + kv)
    token_lens = [40, 0, 1, 15, 16, 17, 100]
    items, wire_bytes, n_pages = layout(token_lens, pool, 3)
    pages = synth.rng(5).permutation(48)[:n_pages].astype(np.int32)
    got, st = run_pack(ctx, pool, items, pages, wire_bytes)
    ref = np.full(wire_bytes, 0xEE, np.uint8)
    ref_st = O.nixl_pack(layers, items, pages, ref)
    assert st == ref_st == [velokv.NIXL_OK] * len(items)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_nixl_pack_layer_subrange(ctx, kv):
    print(f"nixl pack layer subrange kv={kv}", flush=True)
    pool, layers = random_pool(ctx, kv, 4, 32, 8, seed=41)
    items, wire_bytes, n_pages = layout([33, 64], pool, 2)
    pages = np.arange(n_pages, dtype=np.int32)[::-1].copy()
    got, st = run_pack(ctx, pool, items, pages, wire_bytes, layer0=1, n_layers=2)
    ref = np.full(wire_bytes, 0xEE, np.uint8)
    assert O.nixl_pack(layers[1:3], items, pages, ref) == st
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("kv", KV_ALL)
def test_nixl_unpack_into_other_pages(ctx, kv):
    print(f"nixl unpack kv={kv}", flush=True)
    src_pool, src_layers = random_pool(ctx, kv, 2, 40, 2, seed=51)
    dst_pool, dst_layers = random_pool(ctx, kv, 2, 40, 2, seed=52)
    items, wire_bytes, n_pages = layout([50, 0, 16, 7], src_pool, 2)
    src_pages = synth.rng(6).permutation(40)[:n_pages].astype(np.int32)
    dst_pages = synth.rng(7).permutation(40)[:n_pages].astype(np.int32)
    wire, st = run_pack(ctx, src_pool, items, src_pages, wire_bytes)
    assert st == [velokv.NIXL_OK] * len(items)
    st = run_unpack(ctx, dst_pool, items, dst_pages, wire)
    ref_st = O.nixl_unpack(dst_layers, items, dst_pages, wire)
    assert st == ref_st == [velokv.NIXL_OK] * len(items)
    assert_pool_equal(dst_pool, dst_layers)
    # and packing the destination pages again gives the same wire
    wire2, _ = run_pack(ctx, dst_pool, items, dst_pages, wire_bytes)
    assert np.array_equal(wire2, wire)


def test_nixl_many_records_span_launches(ctx):
    """More records than one launch carries (80), with empty records in between."""
    print("nixl many records", flush=True)
    pool, layers = random_pool(ctx, O.I8_BLK, 2, 400, 2, seed=61)
    token_lens = [(i * 37) % 70 for i in range(200)]
    items, wire_bytes, n_pages = layout(token_lens, pool, 2)
    pages = synth.rng(8).integers(0, 400, n_pages).astype(np.int32)  # repeats are fine for pack
    got, st = run_pack(ctx, pool, items, pages, wire_bytes)
    ref = np.full(wire_bytes, 0xEE, np.uint8)
    assert st == O.nixl_pack(layers, items, pages, ref)
    assert np.array_equal(got, ref)


def test_nixl_statuses_and_no_partial_writes(ctx):
    print("nixl statuses", flush=True)
    kv = O.I8_BLK
    src_pool, src_layers = random_pool(ctx, kv, 1, 16, 2, seed=71)
    items, wire_bytes, n_pages = layout([20, 16], src_pool, 1)
    pages = np.array([3, 4, 9], np.int32)
    wire, st = run_pack(ctx, src_pool, items, pages, wire_bytes)
    assert st == [velokv.NIXL_OK] * 2
    dst_pool, dst_layers = random_pool(ctx, kv, 1, 16, 2, seed=72)
    rec1 = items[1][3]
    cases = [
        # (items, pages, wire) -> expected status list
        ([items[0], (items[1][0], 16, 2, wire_bytes)], pages, wire),           # short header (0 bytes left)
        ([items[0], items[1]], pages, wire[:rec1 + 16 + 100]),                  # truncated payload
        ([items[0], (items[1][0] + 1, 16, 2, rec1)], pages, wire),              # handle mismatch
        ([(items[0][0], 21, 0, 0), items[1]], pages, wire),                     # token_len mismatch
        ([items[0], items[1]], np.array([1, 2, 77], np.int32), wire),           # page outside the pool
    ]
    for its, pg, w in cases:
        st = run_unpack(ctx, dst_pool, its, pg, w)
        ref_st = O.nixl_unpack(dst_layers, its, pg, w)
        assert st == ref_st, (st, ref_st)
        assert_pool_equal(dst_pool, dst_layers)
    assert [s for its, pg, w in cases for s in O.nixl_unpack(dst_layers, its, pg, w)] == [
        0, 1, 0, 2, 0, 3, 3, 0, 0, 5]
    # a record packed for 1 layer read back as 2 layers: byte_len mismatch
    two_pool, two_layers = random_pool(ctx, kv, 2, 16, 2, seed=73)
    st = run_unpack(ctx, two_pool, items[:1], pages, wire, n_layers=2)
    assert st == [velokv.NIXL_LENGTH_MISMATCH]
    assert_pool_equal(two_pool, two_layers)
    # pack with a page outside the pool: that record is skipped
    got, st = run_pack(ctx, src_pool, items, np.array([3, 99, 9], np.int32), wire_bytes)
    assert st == [velokv.NIXL_BAD_PAGE, velokv.NIXL_OK]
    assert np.all(got[:items[1][3]] == 0xEE)


def test_nixl_host_errors(ctx):
    pool, _ = random_pool(ctx, O.I8_BLK, 2, 16, 2, seed=81)
    wb = 1 << 18
    wire = ctx.alloc(wb)
    pg = ctx.upload(np.arange(8, dtype=np.int32))
    st = ctx.alloc(64)
    n = pool.nixl_payload_bytes(32, 2)
    assert n % 16 == 0 and 2 * (16 + n) < wb
    for items, n_pages, layer0, nl in (
        ([(1, 32, 0, 8)], 8, 0, 2),                          # misaligned offset
        ([(1, 32, 0, 0), (2, 32, 2, n)], 8, 0, 2),           # overlapping records
        ([(1, 32, 0, wb - 16)], 8, 0, 2),                    # record past the wire
        ([(1, 32, 7, 0)], 8, 0, 2),                          # pages past the array
        ([(1, 32, 0, 0)], 8, 1, 2),                          # layer range past the pool
    ):
        with pytest.raises(velokv.VkError) as e:
            ctx.nixl_pack(pool, items, pg, n_pages, wire, wb, st, layer0=layer0, n_layers=nl)
        assert "overlap" in str(e.value) or items != [(1, 32, 0, 0), (2, 32, 2, n)]
        assert e.value.code == velokv.ERR_BAD_ARG


# ---- accepted-path commit ------------------------------------------------------

def commit_case(ctx, kv, ctxs, n_nodes, n_layer, seed, spread=True):
    """S sequences with committed contexts ctxs and n_nodes tree tokens each,
    appended in every layer on the GPU and in the oracle."""
    S = len(ctxs)
    tot = [c + n_nodes for c in ctxs]
    pages = [(t + BS - 1) // BS for t in tot]
    n_blocks = 2 * sum(pages) + 8
    bt = synth.scatter_block_tables(n_blocks, pages, seed)
    pool = velokv.Pool(ctx, n_layer, n_blocks, BS, 2, HD, kv)
    layers = []
    row = 2 * HD
    for l in range(n_layer):
        L = O.Layer(n_blocks, 2, BS, HD, kv)
        ks, vs, sl = [], [], []
        for s in range(S):
            k = synth.normals_f16(tot[s] * row, seed * 97 + 10 * l + 2 * s, row, 8.0).reshape(tot[s], 2, HD)
            v = synth.normals_f16(tot[s] * row, seed * 97 + 10 * l + 2 * s + 1, row, 8.0).reshape(tot[s], 2, HD)
            if spread:
                k[ctxs[s]:] = (k[ctxs[s]:].astype(np.float32) * (1 + (s % 5))).astype(np.float16)
                v[ctxs[s]:] = (v[ctxs[s]:].astype(np.float32) * (1 + (s % 3))).astype(np.float16)
            ks.append(k)
            vs.append(v)
            sl.append(synth.slots_for_positions(bt, np.arange(tot[s]), BS, np.full(tot[s], s)))
        kk, vv, sm = np.concatenate(ks), np.concatenate(vs), np.concatenate(sl)
        O.append(L, kk, vv, sm)
        ctx.append(pool, l, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sm), len(sm))
        layers.append(L)
    ctx.sync()
    return pool, layers, bt


def run_commit(ctx, pool, layers, bt, ctxs, accepts, stride=32, layer0=0, n_layers=None, n_accept=None):
    """Commit on the GPU and in the oracle; returns the GPU's per-sequence status."""
    S = len(ctxs)
    acc = np.full((S, stride), -1, np.int32)
    na = np.zeros(S, np.int32)
    for s, a in enumerate(accepts):
        acc[s, :len(a)] = a
        na[s] = len(a)
    if n_accept is not None:
        na = np.asarray(n_accept, np.int32)
    status = ctx.upload(np.full(S, -7, np.int32))
    ctx.tree_commit(pool, ctx.upload(bt), bt.shape[1], ctx.upload(np.asarray(ctxs, np.int32)), ctx.upload(acc),
                    stride, ctx.upload(na), S, layer0=layer0, n_layers=n_layers, status=status)
    ctx.sync()
    n_layers = len(layers) - layer0 if n_layers is None else n_layers
    for L in layers[layer0:layer0 + n_layers]:
        for s, a in enumerate(accepts):
            if n_accept is None or n_accept[s] == len(a):
                O.tree_commit(L, bt[s], ctxs[s], a)
    return status.download((S,), np.int32)


@pytest.mark.parametrize("kv", KV_ALL)
def test_tree_commit_bit_exact(ctx, kv):
    print(f"tree commit kv={kv}", flush=True)
    ctxs = [0, 1, 14, 15, 16, 17, 31, 32, 33, 100, 255, 8]
    pool, layers, bt = commit_case(ctx, kv, ctxs, 8, 2, seed=91)
    rng = synth.rng(92)
    accepts = []
    for s in range(len(ctxs)):
        n = int(rng.integers(1, 9))
        accepts.append(sorted(rng.choice(8, n, replace=False).tolist()))
    accepts[0] = [0, 1, 2]        # already in place
    accepts[1] = [3]              # one node, moved
    accepts[2] = [1, 2, 3, 4, 5, 6, 7]
    accepts[3] = [0, 2, 4, 6]     # crosses a block boundary
    st = run_commit(ctx, pool, layers, bt, ctxs, accepts)
    assert_pool_equal(pool, layers)
    assert np.all(st == velokv.COMMIT_OK), st


def test_tree_commit_invalid_rows_and_layer_range(ctx):
    print("tree commit invalid rows", flush=True)
    kv = O.I8_BLK
    ctxs = [20, 40, 60, 80, 100]
    pool, layers, bt = commit_case(ctx, kv, ctxs, 8, 3, seed=93)
    accepts = [[0, 3, 3], [2, 1], [0, 40], [], [0, 2, 5]]  # three rejected rows, one empty, one good
    st = run_commit(ctx, pool, layers, bt, ctxs, accepts, layer0=1, n_layers=1)
    assert_pool_equal(pool, layers)
    assert st.tolist() == [velokv.COMMIT_BAD_ROW] * 3 + [velokv.COMMIT_OK] * 2, st


def test_tree_commit_status_past_table_bad_page_and_counts(ctx):
    """Each rejection reason is reported per sequence and leaves the pool
    untouched: a path past the block-table row, a page id outside the pool, a
    negative n_accept, an n_accept above 32 and a negative context."""
    print("tree commit statuses", flush=True)
    kv = O.I8_BLK
    ctxs = [20, 40, 60, 80, 100, 30]
    pool, layers, bt = commit_case(ctx, kv, ctxs, 8, 1, seed=96)
    bt = bt.copy()
    ctxs[0] = bt.shape[1] * BS - 3          # accepted node 5 lands past the row
    bt[1, (40 + 2) // BS] = pool.n_blocks + 5   # the destination page of sequence 1 is outside the pool
    accepts = [[0, 5], [0, 2], [1], [1], [1], [0, 1, 3]]
    na = [2, 2, -1, 33, 1, 3]
    ctxs[4] = -4
    # the GPU pool's table rows are the caller's; the oracle sees the same rejected rows untouched
    status = run_commit(ctx, pool, layers, bt, ctxs, accepts, n_accept=na)
    assert_pool_equal(pool, layers)
    assert status.tolist() == [velokv.COMMIT_PAST_TABLE, velokv.COMMIT_BAD_PAGE, velokv.COMMIT_BAD_ROW,
                               velokv.COMMIT_BAD_ROW, velokv.COMMIT_BAD_ROW, velokv.COMMIT_OK], status


def test_tree_commit_then_decode_matches_oracle(ctx):
    """The config-4 step: after commit, decode over context + accepted tokens."""
    print("tree commit then decode", flush=True)
    from cases import tol_check
    kv = O.I8_BLK
    ctxs = [45, 64, 130]
    pool, layers, bt = commit_case(ctx, kv, ctxs, 8, 1, seed=94)
    accepts = [[0, 1, 4], [1, 3, 7], [0, 2, 5, 6]]
    run_commit(ctx, pool, layers, bt, ctxs, accepts)
    lens = np.array([c + len(a) for c, a in zip(ctxs, accepts)], np.int32)
    q = synth.normals_f16(len(ctxs) * 8 * HD, 95).reshape(len(ctxs), 8, HD)
    out = ctx.alloc(q.size * 4)
    ctx.paged_decode(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(lens), len(ctxs), 8, int(lens.max()),
                     block_tables=ctx.upload(bt), bt_stride=bt.shape[1])
    ctx.sync()
    got = out.download(q.shape, np.float32)
    ref = O.paged_decode(layers[0], q, bt, lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, (err, nbad)
    assert_pool_equal(pool, layers)
