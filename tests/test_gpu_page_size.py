"""GPU parity for pages of 32, 48, 64 and 256 tokens (the reference takes any
paged_block_size > 0, paged_attention.rs:103-106, metal/runtime.rs:152-155,
and indexes the cache with it at kernels.metal:472, 637-640, 770-774).

The kernels work on 16-token tiles; a page of 16 k tokens is k tiles back
to back (48 tokens: 3 tiles, the page and the tile in it found by division), so a flat slot page * page_tokens + offset is also tile * 16 + offset
% 16 and the pool bytes equal those of a 16-token pool whose tables list the
pages' tiles. The checks therefore compare against the oracle on the expanded
16-token tables (bit-exact pool bytes, decode and tree verify within the
north-star tolerance), and for fp16 / fp32 KV also against the oracle run
directly with the page size (which pins the expansion itself)."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, Case, oracle_layer, tol_check
from test_gpu_append_copy import assert_layer_equal
from velokv import synth

pytestmark = pytest.mark.gpu

KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]


def page_case(kv, lens, page, n_kv_heads=2, n_heads=8, seed=1, outlier_scale=8.0, n_pages=None):
    """A Case whose block_tables are 16-token tile tables expanded from random
    page tables; returns (case, page tables, number of pages)."""
    k = page // BS
    lens = np.asarray(lens, np.int32)
    pages = [(int(L) + page - 1) // page for L in lens]
    n_pages = n_pages if n_pages is not None else max(2 * sum(pages), 8)
    pt = synth.scatter_block_tables(n_pages, pages, seed)
    bt16 = (pt[:, :, None].astype(np.int64) * k + np.arange(k)[None, None, :]).reshape(pt.shape[0], -1)
    bt16 = np.where(np.repeat(pt, k, axis=1) < 0, -1, bt16).astype(np.int32)
    c = Case(kv, n_pages * k, n_kv_heads, n_heads, lens, bt16)
    row = n_kv_heads * HD
    for s, L in enumerate(lens):
        L = int(L)
        c.k.append(synth.normals_f16(L * row, seed * 1000 + 2 * s, row, outlier_scale).reshape(L, n_kv_heads, HD))
        c.v.append(synth.normals_f16(L * row, seed * 1000 + 2 * s + 1, row, outlier_scale).reshape(L, n_kv_heads, HD))
    c.q = synth.normals_f16(c.S * n_heads * HD, seed * 1000 + 999).reshape(c.S, n_heads, HD)
    return c, pt, n_pages


def page_pool(ctx, case, page, n_pages, n_layer=1, with_last=True):
    pool = velokv.Pool(ctx, n_layer, n_pages, page, case.n_kv_heads, HD, case.kv_type)
    sl, kk, vv = case.prefill_slots()   # flat slots are the same in tiles and pages
    if len(sl):
        ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    if with_last:
        sl, kk, vv = case.last_slots()
        ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    ctx.sync()
    return pool


def page_oracle(case, pt, page, n_pages):
    """The oracle run with the page size itself (fp16 / fp32 KV)."""
    L = O.Layer(n_pages, case.n_kv_heads, page, HD, case.kv_type)
    for part in (case.prefill_slots(), case.last_slots()):
        sl, kk, vv = part
        if len(sl):
            O.append(L, kk, vv, sl)
    return L


@pytest.mark.parametrize("kv", KV_ALL)
@pytest.mark.parametrize("page", [32, 48, 64, 256])
def test_page_append_bit_exact(ctx, kv, page):
    print(f"page append kv={kv} page={page}", flush=True)
    case, pt, n_pages = page_case(kv, [1, 15, 16, 17, 31, 33, 100, 257, 600], page, seed=1300 + page)
    pool = page_pool(ctx, case, page, n_pages)
    assert pool.n_blocks == n_pages
    assert_layer_equal(pool, 0, oracle_layer(case))


SCHEDS = {"split": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0), "split-p48": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 48),
          "stream": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0), "valu": (velokv.DECODE_VALU, velokv.SCHED_SPLIT, 0),
          "auto": (velokv.DECODE_AUTO, velokv.SCHED_AUTO, 0)}


@pytest.mark.parametrize("kv", KV_ALL)
@pytest.mark.parametrize("page", [32, 48, 64, 256])
@pytest.mark.parametrize("sched", list(SCHEDS))
def test_page_decode(ctx, kv, page, sched):
    print(f"page decode kv={kv} page={page} sched={sched}", flush=True)
    kind, sc, P = SCHEDS[sched]
    lens = [1, 16, 17, page - 1, page, page + 1, 700, 2100]
    case, pt, n_pages = page_case(kv, lens, page, seed=1310 + page)
    pool = page_pool(ctx, case, page, n_pages)
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sc)
    try:
        out = ctx.alloc(case.S * case.n_heads * HD * 4)
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S,
                         case.n_heads, int(case.ctx_lens.max()), block_tables=ctx.upload(pt), bt_stride=pt.shape[1],
                         partition_tokens=P)
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    got = out.download((case.S, case.n_heads, HD), np.float32)
    ref = O.paged_decode(oracle_layer(case), case.q, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"
    if kv in (O.F16, O.F32):
        ref_p = O.paged_decode(page_oracle(case, pt, page, n_pages), case.q, pt, case.ctx_lens)
        ok, err, nbad = tol_check(got, ref_p)
        assert ok, f"vs the oracle at page {page}: max err {err:.3g}, {nbad} out of tolerance"


@pytest.mark.parametrize("kv", [O.F32, O.I8_BLK])
def test_page_workgroup_split_and_append_decode(ctx, kv):
    """A batch that fills the GPU (64 x 8 pairs) takes the workgroup split over
    32-token pages, through vk_append_decode (slots derived from page tables)."""
    print(f"page workgroup split kv={kv}", flush=True)
    page = 32
    lens = list(synth.rng(1320).integers(2, 500, 64))
    case, pt, n_pages = page_case(kv, lens, page, n_kv_heads=8, n_heads=32, seed=1321)
    pool = page_pool(ctx, case, page, n_pages, with_last=False)
    sl, kk, vv = case.last_slots()
    out = ctx.alloc(case.S * case.n_heads * HD * 4)
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=pt.shape[1])
        assert pl["kernel"].startswith(f"vk_decode_wg_kv{kv}_g4"), pl
        ctx.append_decode(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(case.q), velokv.DT_F16,
                          out, ctx.upload(case.ctx_lens), case.S, case.n_heads, int(case.ctx_lens.max()),
                          block_tables=ctx.upload(pt), bt_stride=pt.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    ref_layer = oracle_layer(case)
    assert_layer_equal(pool, 0, ref_layer)
    got = out.download((case.S, case.n_heads, HD), np.float32)
    ok, err, nbad = tol_check(got, O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens))
    assert ok, (err, nbad)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_BLK])
@pytest.mark.parametrize("page,shared", [(32, 0), (32, 3), (48, 0), (48, 3), (64, 2)])
def test_page_tree_verify(ctx, kv, page, shared):
    """Tree verify over page tables, with the shared-prefix pass over the first
    `shared` pages of every row (fp16 / I8_BLK) or without."""
    print(f"page tree kv={kv} page={page} shared={shared}", flush=True)
    N, G, Hkv = 8, 4, 2
    committed = np.array([shared * page + 5, shared * page + 40, shared * page + 130, max(1, shared * page)], np.int32)
    case, pt, n_pages = page_case(kv, committed + N, page, n_kv_heads=Hkv, n_heads=Hkv * G, seed=1330 + page)
    if shared:
        # every row shares sequence 0's first pages: copy its prefix tokens into the others
        for s in range(1, case.S):
            case.k[s][:shared * page] = case.k[0][:shared * page]
            case.v[s][:shared * page] = case.v[0][:shared * page]
    pool = page_pool(ctx, case, page, n_pages)
    ref_layer = oracle_layer(case)
    pt_v, bt_v = pt.copy(), case.block_tables.copy()
    if shared:
        pt_v[1:, :shared] = pt_v[0, :shared]
        k = page // BS
        bt_v[1:, :shared * k] = bt_v[0, :shared * k]
    q = synth.normals_f16(case.S * N * case.n_heads * HD, 1331).reshape(case.S, N, case.n_heads, HD)
    mask = np.tile(velokv.branching_tree([2, 2, 2], N).ancestor_mask(), (case.S, 1)).astype(np.uint32)
    out = ctx.alloc(q.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask), case.S, N,
                    case.n_heads, int(committed.max()), block_tables=ctx.upload(pt_v), bt_stride=pt_v.shape[1],
                    shared_blocks=shared)
    ctx.sync()
    got = out.download(q.shape, np.float32)
    ref = O.tree_verify(ref_layer, q, bt_v, committed, mask)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"


def test_page_slot_mapping_and_bad_pages(ctx):
    """vk_slot_mapping over 64-token pages equals page * 64 + pos % 64; a page id
    outside the pool maps to -1; a decode reading one reports misuse."""
    print("page slot mapping", flush=True)
    page = 64
    case, pt, n_pages = page_case(O.I8_BLK, [70, 200, 5], page, seed=1340)
    pool = page_pool(ctx, case, page, n_pages)
    rows = np.array([0, 0, 1, 1, 2, 1], np.int32)
    pos = np.array([0, 69, 63, 64, 4, 199], np.int32)
    sm = ctx.slot_mapping(pool, ctx.upload(pos), block_tables=ctx.upload(pt), bt_stride=pt.shape[1],
                          seq_rows=ctx.upload(rows))
    ctx.sync()
    got = sm.download((len(pos),), np.int64)
    want = pt[rows, pos // page].astype(np.int64) * page + pos % page
    assert np.array_equal(got, want), (got, want)
    bad = pt.copy()
    bad[1, 199 // page] = n_pages + 3  # the page of row 1's position 199
    sm = ctx.slot_mapping(pool, ctx.upload(pos), block_tables=ctx.upload(bad), bt_stride=bad.shape[1],
                          seq_rows=ctx.upload(rows))
    ctx.sync()
    assert sm.download((len(pos),), np.int64)[5] == -1
    out = ctx.alloc(case.S * case.n_heads * HD * 4)
    ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                     int(case.ctx_lens.max()), block_tables=ctx.upload(bad), bt_stride=bad.shape[1])
    with pytest.raises(velokv.VkError) as e:
        ctx.sync()
    assert e.value.code == velokv.ERR_BAD_ARG
    ctx.sync()


@pytest.mark.parametrize("kv", [O.F16, O.I8_REF, O.I8_BLK])
def test_page_copy_blocks_moves_whole_pages(ctx, kv):
    print(f"page copy kv={kv}", flush=True)
    page, k = 32, 2
    case, pt, n_pages = page_case(kv, [100, 60], page, seed=1350)
    pool = page_pool(ctx, case, page, n_pages)
    ref = oracle_layer(case)
    free = [p for p in range(n_pages) if p not in set(pt[pt >= 0].ravel().tolist())]
    pairs = [(int(pt[0, 1]), free[0]), (int(pt[1, 0]), free[1])]
    ctx.copy_blocks(pool, pairs)
    ctx.sync()
    # the oracle's copy over the pages' tiles
    O.copy_blocks(ref, [(s * k + i, d * k + i) for s, d in pairs for i in range(k)])
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("page", [32, 48])
@pytest.mark.parametrize("kv", [O.F32, O.I8_BLK])
def test_page_tree_commit(ctx, kv, page):
    """Accepted-path commit over 32- and 48-token pages equals the oracle's
    commit on the expanded tile tables."""
    print(f"page commit kv={kv} page={page}", flush=True)
    N = 8
    ctxs = np.array([0, 14, 30, 31, 32, 60, 100], np.int32)
    case, pt, n_pages = page_case(kv, ctxs + N, page, seed=1360)
    pool = page_pool(ctx, case, page, n_pages)
    ref = oracle_layer(case)
    accepts = [[0, 2, 5], [1, 3], [0, 1, 2, 3, 4, 5, 6, 7], [2, 4, 6], [7], [0, 3, 6], [1, 2]]
    stride = 32
    acc = np.full((case.S, stride), -1, np.int32)
    na = np.zeros(case.S, np.int32)
    for s, a in enumerate(accepts):
        acc[s, :len(a)] = a
        na[s] = len(a)
    status = ctx.upload(np.full(case.S, -7, np.int32))
    ctx.tree_commit(pool, ctx.upload(pt), pt.shape[1], ctx.upload(ctxs), ctx.upload(acc), stride, ctx.upload(na),
                    case.S, status=status)
    ctx.sync()
    assert np.all(status.download((case.S,), np.int32) == velokv.COMMIT_OK)
    for s, a in enumerate(accepts):
        O.tree_commit(ref, case.block_tables[s], int(ctxs[s]), a)
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("page", [32, 48])
@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_page_nixl_round_trip(ctx, kv, page):
    """NIXL records over 32- and 48-token pages: the payload of a (page, layer)
    unit is the page's K codes (its tiles back to back), V codes, then the
    scales; pack then unpack into other pages restores the bytes exactly."""
    print(f"page nixl kv={kv} page={page}", flush=True)
    k, n_layer = page // BS, 2
    case, pt, n_pages = page_case(kv, [70, 33], page, seed=1370)
    pool = velokv.Pool(ctx, n_layer, n_pages, page, case.n_kv_heads, HD, kv)
    sl, kk, vv = case.prefill_slots()
    for l in range(n_layer):
        ctx.append(pool, l, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    ctx.sync()
    before = [pool.download_layer(l) for l in range(n_layer)]
    items, off, pages = [], 0, []
    for s, tl in enumerate([69, 32]):
        np_ = (tl + page - 1) // page
        items.append((500 + s, tl, len(pages), off))
        pages += pt[s, :np_].tolist()
        off = (off + 16 + pool.nixl_payload_bytes(tl) + 15) // 16 * 16
    assert pool.nixl_payload_bytes(69) == -(-69 // page) * pool.nixl_payload_bytes(32)  # whole pages
    wire = ctx.upload(np.zeros(off, np.uint8))
    status = ctx.upload(np.full(2, -7, np.int32))
    ctx.nixl_pack(pool, items, ctx.upload(np.asarray(pages, np.int32)), len(pages), wire, off, status)
    ctx.sync()
    assert status.download((2,), np.int32).tolist() == [0, 0]
    w = wire.download((off,), np.uint8)
    # expected payload of record 0, page 0, layer 0: the page's K codes region
    tb = HD * BS * {O.F32: 4, O.F16: 2}.get(kv, 1) * case.n_kv_heads  # one tile, every head
    p0 = pages[0]
    assert np.array_equal(w[16:16 + k * tb], before[0]["k"][p0 * k * tb:(p0 + 1) * k * tb])
    assert np.array_equal(w[16 + k * tb:16 + 2 * k * tb], before[0]["v"][p0 * k * tb:(p0 + 1) * k * tb])
    # unpack into fresh pages of a second pool and compare those pages' bytes
    pool2 = velokv.Pool(ctx, n_layer, n_pages, page, case.n_kv_heads, HD, kv)
    dst = list(range(n_pages - len(pages), n_pages))
    status2 = ctx.upload(np.full(2, -7, np.int32))
    ctx.nixl_unpack(pool2, items, ctx.upload(np.asarray(dst, np.int32)), len(dst), ctx.upload(w), off, status2)
    ctx.sync()
    assert status2.download((2,), np.int32).tolist() == [0, 0]
    for l in range(n_layer):
        after = pool2.download_layer(l)
        for key in ("k", "v"):
            for sp, dp in zip(pages, dst):
                assert np.array_equal(after[key][dp * k * tb:(dp + 1) * k * tb],
                                      before[l][key][sp * k * tb:(sp + 1) * k * tb]), (l, key, sp, dp)
        if before[l]["ks"] is not None:
            sb = before[l]["ks"].size // (n_pages * k)  # scale bytes of one tile, every head
            for key in ("ks", "vs"):
                for sp, dp in zip(pages, dst):
                    assert np.array_equal(after[key][dp * k * sb:(dp + 1) * k * sb],
                                          before[l][key][sp * k * sb:(sp + 1) * k * sb]), (l, key, sp, dp)


def test_page_size_limits(ctx):
    for bad in (8, 24, 40, 272, 512):
        with pytest.raises(velokv.VkError) as e:
            velokv.Pool(ctx, 1, 8, bad, 2, HD, O.F16)
        assert e.value.code == velokv.ERR_UNSUPPORTED, bad
    with pytest.raises(velokv.VkError) as e:
        velokv.Pool(ctx, 1, 8, 0, 2, HD, O.F16)
    assert e.value.code == velokv.ERR_INVALID_BLOCK_SIZE
