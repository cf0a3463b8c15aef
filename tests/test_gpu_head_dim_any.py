"""GPU parity for head_dims other than 64 and 128 (the reference's kernels take
any head_dim up to 128, kernels.metal:464). A pool of head_dim hd (a multiple of
8) holds the tiles of the next width T (64 dims for hd <= 64, else 128) with the
dims past hd held as zeros; callers pass hd-long K, V, q and out rows and the
softmax scale defaults to 1/sqrt(hd).

The pool bytes must equal the oracle's layer at T over the same rows zero-padded
(bit for bit, every KV type), and attention must equal the oracle's over that
layer with the 1/sqrt(hd) scale (within the north-star tolerance). That padded
oracle is pinned on the CPU against the reference-kernel restatements at hd
itself and a numpy closed form of the int8 block rule (tests/test_oracle.py).
hd = 80 and 40 leave a lane group's last 8-dim chunks of q past the row (the
per-chunk q masks); hd = 40 and 8 run the 64-dim pieces; hd = 72 is the
narrowest head on 128-dim tiles."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, make_case, tol_check
from test_gpu_append_copy import assert_layer_equal
from velokv import synth

pytestmark = pytest.mark.gpu

KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]
HDS = [96, 80, 40]
HDS_EDGE = [72, 8]  # the narrowest head on 128-dim tiles, the narrowest head overall


def tile_w(hd):
    return 64 if hd <= 64 else 128


def pad(x, T):
    p = np.zeros(x.shape[:-1] + (T,), np.float32)
    p[..., :x.shape[-1]] = x
    return p


def hd_case(kv, lens, hd, n_kv_heads=2, n_heads=8, seed=1, outlier_scale=8.0):
    """make_case with hd-dim K, V and q (the 128-dim case's first hd dims)."""
    c = make_case(kv, lens, n_kv_heads=n_kv_heads, n_heads=n_heads, seed=seed, outlier_scale=outlier_scale)
    c.k = [np.ascontiguousarray(k[..., :hd]) for k in c.k]
    c.v = [np.ascontiguousarray(v[..., :hd]) for v in c.v]
    c.q = np.ascontiguousarray(c.q[..., :hd])
    return c


def gpu_pool(ctx, case, hd, with_last=True):
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, case.n_kv_heads, hd, case.kv_type)
    parts = [case.prefill_slots()] + ([case.last_slots()] if with_last else [])
    for sl, kk, vv in parts:
        if len(sl):
            ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    ctx.sync()
    return pool


def oracle_padded(case, hd, with_last=True):
    """The oracle's layer at the tile width over the case's rows zero-padded."""
    T = tile_w(hd)
    L = O.Layer(case.n_blocks, case.n_kv_heads, BS, T, case.kv_type)
    parts = [case.prefill_slots()] + ([case.last_slots()] if with_last else [])
    for sl, kk, vv in parts:
        if len(sl):
            O.append(L, pad(kk.astype(np.float32), T), pad(vv.astype(np.float32), T), sl)
    return L


def oracle_decode(layer, q, hd, bt, lens):
    ref = O.paged_decode(layer, pad(q.astype(np.float32), layer.head_dim), bt, lens, scale=1.0 / np.sqrt(hd))
    assert not np.any(ref[..., hd:])
    return ref[..., :hd]


@pytest.mark.parametrize("hd", HDS + HDS_EDGE)
@pytest.mark.parametrize("kv", KV_ALL)
def test_append_bit_exact(ctx, kv, hd):
    print(f"hd{hd} append kv={kv}", flush=True)
    case = hd_case(kv, [1, 15, 16, 17, 33, 200, 257], hd, seed=1500 + hd)
    pool = gpu_pool(ctx, case, hd)
    ref = oracle_padded(case, hd)
    esz = {O.F32: 4, O.F16: 2}.get(kv, 1)
    assert pool.download_layer(0)["k"].size == case.n_blocks * case.n_kv_heads * BS * tile_w(hd) * esz
    assert_layer_equal(pool, 0, ref)


SCHEDS = {"split": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0), "split-p64": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 64),
          "stream": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0), "auto": (velokv.DECODE_AUTO, velokv.SCHED_AUTO, 0)}


@pytest.mark.parametrize("qd", [np.float16, np.float32])
@pytest.mark.parametrize("sched", list(SCHEDS))
@pytest.mark.parametrize("hd", HDS + HDS_EDGE)
@pytest.mark.parametrize("kv", KV_ALL)
def test_decode(ctx, kv, hd, sched, qd):
    print(f"hd{hd} decode kv={kv} sched={sched} q={np.dtype(qd).name}", flush=True)
    kind, sc, P = SCHEDS[sched]
    case = hd_case(kv, [1, 16, 17, 255, 700, 2100], hd, seed=1510 + kv + hd)
    pool = gpu_pool(ctx, case, hd)
    q = case.q.astype(qd)
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sc)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()),
                             bt_stride=case.block_tables.shape[1], partition_tokens=P, q_dtype=qdt)
        # 64-dim tiles of every pool run the 64-dim pieces
        assert ("_d64" in pl["kernel"]) == (tile_w(hd) == 64), pl
        out = ctx.alloc(case.S * case.n_heads * hd * 4)
        ctx.paged_decode(pool, 0, ctx.upload(q), qdt, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                         int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1], partition_tokens=P)
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    got = out.download((case.S, case.n_heads, hd), np.float32)
    ref = oracle_decode(oracle_padded(case, hd), q, hd, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance ({pl['kernel']})"


@pytest.mark.parametrize("hd", [96, 40])
@pytest.mark.parametrize("kv", [O.F32, O.I8_BLK])
def test_workgroup_split_and_append_decode(ctx, kv, hd):
    """vk_append_decode under the workgroup split: over int8 block pools the
    decode launch appends the new hd-long rows itself (the tile's dims past hd
    get zero codes)."""
    print(f"hd{hd} append+decode kv={kv}", flush=True)
    lens = list(synth.rng(1520 + hd).integers(2, 500, 64))
    case = hd_case(kv, lens, hd, n_kv_heads=8, n_heads=32, seed=1521 + hd)
    pool = gpu_pool(ctx, case, hd, with_last=False)
    sl, kk, vv = case.last_slots()
    out = ctx.alloc(case.S * case.n_heads * hd * 4)
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1])
        assert "_wg_" in pl["kernel"], pl
        ctx.append_decode(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(case.q),
                          velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                          int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                          bt_stride=case.block_tables.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    ref_layer = oracle_padded(case, hd)
    assert_layer_equal(pool, 0, ref_layer)
    got = out.download((case.S, case.n_heads, hd), np.float32)
    ok, err, nbad = tol_check(got, oracle_decode(ref_layer, case.q, hd, case.block_tables, case.ctx_lens))
    assert ok, (err, nbad)


@pytest.mark.parametrize("shared", [0, 8])
@pytest.mark.parametrize("hd", [96, 40])
@pytest.mark.parametrize("kv", KV_ALL)
def test_tree_verify(ctx, kv, hd, shared):
    print(f"hd{hd} tree kv={kv} shared={shared}", flush=True)
    N, G, Hkv = 8, 4, 2
    committed = np.array([shared * BS + 3, shared * BS + 60, shared * BS + 200, shared * BS], np.int32)
    case = hd_case(kv, committed + N, hd, n_kv_heads=Hkv, n_heads=Hkv * G, seed=1530 + kv + hd)
    if shared:
        for s in range(1, case.S):
            case.k[s][:shared * BS] = case.k[0][:shared * BS]
            case.v[s][:shared * BS] = case.v[0][:shared * BS]
    pool = gpu_pool(ctx, case, hd)
    bt = case.block_tables.copy()
    if shared:
        bt[1:, :shared] = bt[0, :shared]
    q = synth.normals_f16(case.S * N * case.n_heads * hd, 1531).reshape(case.S, N, case.n_heads, hd)
    mask = np.tile(velokv.branching_tree([2, 2, 2], N).ancestor_mask(), (case.S, 1)).astype(np.uint32)
    out = ctx.alloc(q.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask), case.S, N,
                    case.n_heads, int(committed.max()), block_tables=ctx.upload(bt), bt_stride=bt.shape[1],
                    shared_blocks=shared)
    ctx.sync()
    got = out.download(q.shape, np.float32)
    layer = oracle_padded(case, hd)
    ref = O.tree_verify(layer, pad(q.astype(np.float32), layer.head_dim), bt, committed, mask, scale=1.0 / np.sqrt(hd))
    assert not np.any(ref[..., hd:])
    ok, err, nbad = tol_check(got, ref[..., :hd])
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"


@pytest.mark.parametrize("style", [O.ROPE_INTERLEAVED, O.ROPE_HALF])
@pytest.mark.parametrize("hd", [96, 40, 8])
@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_append_rope_bit_exact(ctx, kv, hd, style):
    """RoPE over hd-dim rows (pairs (2i, 2i+1) or (i, i + hd/2), the angles of an
    hd-dim table) fused into the append: pool bytes and rotated q bit for bit."""
    print(f"hd{hd} rope kv={kv} style={style}", flush=True)
    case = hd_case(kv, [1, 17, 100, 257], hd, n_kv_heads=2, n_heads=8, seed=1540 + hd)
    rows = np.concatenate([np.full(int(L), s) for s, L in enumerate(case.ctx_lens)])
    cpos = np.concatenate([np.arange(int(L)) for L in case.ctx_lens])
    sl = synth.slots_for_positions(case.block_tables, cpos, BS, rows)
    kk = np.concatenate([case.k[s] for s in range(case.S)])
    vv = np.concatenate([case.v[s] for s in range(case.S)])
    pos = (cpos + 5).astype(np.int32)
    n_pos = int(pos.max()) + 1
    table = velokv.rope_table(n_pos, hd, 500000.0)
    q = synth.normals_f16(len(sl) * 8 * hd, 1541).reshape(len(sl), 8, hd)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 2, hd, kv)
    dq = ctx.upload(q)
    ctx.append_rope(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(pos), ctx.upload(sl), len(sl),
                    ctx.upload(table), n_pos, style, q=dq, q_dtype=velokv.DT_F16, n_heads=8)
    ctx.sync()
    T = tile_w(hd)
    kr = O.rope_apply(kk, pos, style, table)          # fp32, hd dims
    ref = O.Layer(case.n_blocks, 2, BS, T, kv)
    O.append(ref, pad(kr, T), pad(vv.astype(np.float32), T), sl)
    assert_layer_equal(pool, 0, ref)
    qr = O.rope_apply(q, pos, style, table).astype(np.float16)
    assert np.array_equal(dq.download(q.shape, np.float16).view(np.uint16), qr.view(np.uint16))


@pytest.mark.parametrize("hd", [96, 40])
@pytest.mark.parametrize("kv", [O.F32, O.I8_BLK])
def test_tree_commit(ctx, kv, hd):
    print(f"hd{hd} commit kv={kv}", flush=True)
    N = 8
    ctxs = np.array([0, 14, 31, 33, 100], np.int32)
    case = hd_case(kv, ctxs + N, hd, seed=1550 + hd)
    pool = gpu_pool(ctx, case, hd)
    ref = oracle_padded(case, hd)
    accepts = [[0, 2, 5], [1, 3], [0, 1, 2, 3, 4, 5, 6, 7], [2, 4, 6], [7]]
    acc = np.full((case.S, 32), -1, np.int32)
    na = np.array([len(a) for a in accepts], np.int32)
    for s, a in enumerate(accepts):
        acc[s, :len(a)] = a
    ctx.tree_commit(pool, ctx.upload(case.block_tables), case.block_tables.shape[1], ctx.upload(ctxs),
                    ctx.upload(acc), 32, ctx.upload(na), case.S)
    ctx.sync()
    for s, a in enumerate(accepts):
        O.tree_commit(ref, case.block_tables[s], int(ctxs[s]), a)
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("in_dt", [np.float16, np.float32])
@pytest.mark.parametrize("hd", [64, 96, 40])
@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
def test_stream_k_folds_the_append(ctx, kv, hd, in_dt):
    """vk_append_decode under stream-K over int8 block and fp16 pools of head_dim
    64 (the 64-dim stream-K pieces, lanes 32-63 storing nothing), 96 and 40 (new
    rows shorter than the tile): the piece that ends at a context's last token
    appends the hd-long new rows in the decode launch. fp32 new rows (scaled so
    they are not fp16 values) are rounded by the fold as the append kernels
    round them; half the rows are 3x larger, so int8 block scales grow and the
    earlier codes are requantized. Pool bytes bit for bit, outputs within the
    tolerance."""
    print(f"hd{hd} stream-K fold kv={kv} in={np.dtype(in_dt).name}", flush=True)
    lens = synth.rng(1530 + hd).integers(1, 1500, 40)
    lens[:6] = [1, 16, 17, 32, 33, 48]
    case = hd_case(kv, lens, hd, n_kv_heads=8, n_heads=32, seed=1531 + hd)
    pool = gpu_pool(ctx, case, hd, with_last=False)
    sl, kk, vv = case.last_slots()
    kk, vv = kk.astype(np.float32), vv.astype(np.float32)
    kk[::2] *= 3
    vv[::2] *= 3
    if in_dt == np.float32:
        kk, vv = kk * np.float32(1.37), vv * np.float32(0.61)
    else:
        kk, vv = kk.astype(np.float16), vv.astype(np.float16)
    out = ctx.alloc(case.S * case.n_heads * hd * 4)
    ctx.set_decode_kernel(velokv.DECODE_MFMA)
    ctx.set_decode_schedule(velokv.SCHED_STREAM)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1])
        assert pl["schedule"] == velokv.SCHED_STREAM and "_sk_" in pl["kernel"], pl
        assert ("_d64" in pl["kernel"]) == (hd <= 64), pl
        ctx.append_decode(pool, 0, ctx.upload(kk), ctx.upload(vv),
                          velokv.DT_F32 if in_dt == np.float32 else velokv.DT_F16, ctx.upload(case.q),
                          velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                          int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                          bt_stride=case.block_tables.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    T = tile_w(hd)
    ref_layer = oracle_padded(case, hd, with_last=False)
    O.append(ref_layer, pad(kk.astype(np.float32), T), pad(vv.astype(np.float32), T), sl)
    assert_layer_equal(pool, 0, ref_layer)
    got = out.download((case.S, case.n_heads, hd), np.float32)
    ok, err, nbad = tol_check(got, oracle_decode(ref_layer, case.q, hd, case.block_tables, case.ctx_lens))
    assert ok, (err, nbad)
