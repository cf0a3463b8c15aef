"""GPU parity for head_dim 64 (the reference's kernels take any head_dim up to
128, kernels.metal:464; the byte formula of model_loader.rs:129-140 scales with
it). A head_dim-64 pool stores 64-dim tiles (16 tokens x 64 dims, the layouts of
the 128-dim tiles at D = 64), so it holds and reads its own bytes only.

The pool bytes must equal the oracle's layer built at head_dim 64 (bit for bit,
every KV type) and attention must equal the oracle's at head_dim 64 (within the
north-star tolerance). The oracle at 64 dims is pinned on the CPU against the
oracle at 128 dims over zero-padded rows (tests/test_oracle.py)."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, make_case, tol_check
from test_gpu_append_copy import assert_layer_equal
from velokv import synth

pytestmark = pytest.mark.gpu

D = 64
KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]


def hd64_case(kv, lens, n_kv_heads=2, n_heads=8, seed=1, outlier_scale=8.0):
    """make_case with 64-dim K, V and q (the 128-dim case's first 64 dims)."""
    c = make_case(kv, lens, n_kv_heads=n_kv_heads, n_heads=n_heads, seed=seed, outlier_scale=outlier_scale)
    c.k = [np.ascontiguousarray(k[..., :D]) for k in c.k]
    c.v = [np.ascontiguousarray(v[..., :D]) for v in c.v]
    c.q = np.ascontiguousarray(c.q[..., :D])
    return c


def hd64_pool(ctx, case, with_last=True):
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, case.n_kv_heads, D, case.kv_type)
    parts = [case.prefill_slots()] + ([case.last_slots()] if with_last else [])
    for sl, kk, vv in parts:
        if len(sl):
            ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    ctx.sync()
    return pool


def oracle64(case, with_last=True):
    """The oracle's layer at head_dim 64 with the case's tokens."""
    L = O.Layer(case.n_blocks, case.n_kv_heads, BS, D, case.kv_type)
    parts = [case.prefill_slots()] + ([case.last_slots()] if with_last else [])
    for sl, kk, vv in parts:
        if len(sl):
            O.append(L, kk, vv, sl)
    return L


@pytest.mark.parametrize("kv", KV_ALL)
def test_hd64_append_bit_exact(ctx, kv):
    print(f"hd64 append kv={kv}", flush=True)
    case = hd64_case(kv, [1, 15, 16, 17, 33, 200, 257], seed=1400)
    pool = hd64_pool(ctx, case)
    ref = oracle64(case)
    # 16 tokens x 64 dims per (page, head): the reference's byte formula at D = 64
    esz = {O.F32: 4, O.F16: 2}.get(kv, 1)
    assert pool.download_layer(0)["k"].size == ref.k.size == case.n_blocks * case.n_kv_heads * BS * D * esz
    assert_layer_equal(pool, 0, ref)


SCHEDS = {"split": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0), "split-p64": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 64),
          "stream": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0), "auto": (velokv.DECODE_AUTO, velokv.SCHED_AUTO, 0),
          "valu-request": (velokv.DECODE_VALU, velokv.SCHED_SPLIT, 0)}


@pytest.mark.parametrize("kv", KV_ALL)
@pytest.mark.parametrize("sched", list(SCHEDS))
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_hd64_decode(ctx, kv, sched, qd):
    print(f"hd64 decode kv={kv} sched={sched} q={np.dtype(qd).name}", flush=True)
    kind, sc, P = SCHEDS[sched]
    case = hd64_case(kv, [1, 16, 17, 255, 700, 2100], seed=1410 + kv)
    pool = hd64_pool(ctx, case)
    q64 = np.ascontiguousarray(case.q[..., :D]).astype(qd)
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sc)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()),
                             bt_stride=case.block_tables.shape[1], partition_tokens=P, q_dtype=qdt)
        assert "mfma" in pl["kernel"] or "_sk_" in pl["kernel"] or "_wg_" in pl["kernel"], pl  # no VALU at 64
        # every pool type runs the 64-dim pieces (half the products per block of a 128-dim piece)
        assert pl["kernel"].endswith("_d64" + ("_q0" if qd == np.float32 else "")), pl
        out = ctx.alloc(case.S * case.n_heads * D * 4)
        ctx.paged_decode(pool, 0, ctx.upload(q64), qdt, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                         int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1], partition_tokens=P)
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    got = out.download((case.S, case.n_heads, D), np.float32)
    ref = O.paged_decode(oracle64(case), q64, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance ({pl['kernel']})"


@pytest.mark.parametrize("kv", [O.F32, O.I8_BLK])
def test_hd64_workgroup_split_and_append_decode(ctx, kv):
    print(f"hd64 workgroup split kv={kv}", flush=True)
    lens = list(synth.rng(1420).integers(2, 500, 64))
    case = hd64_case(kv, lens, n_kv_heads=8, n_heads=32, seed=1421)
    pool = hd64_pool(ctx, case, with_last=False)
    sl, kk, vv = case.last_slots()
    q64 = np.ascontiguousarray(case.q[..., :D])
    out = ctx.alloc(case.S * case.n_heads * D * 4)
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1])
        assert pl["kernel"] == f"vk_decode_wg_kv{kv}_gx_d64", pl
        ctx.append_decode(pool, 0, ctx.upload(np.ascontiguousarray(kk[..., :D])),
                          ctx.upload(np.ascontiguousarray(vv[..., :D])), velokv.DT_F16, ctx.upload(q64),
                          velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                          int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                          bt_stride=case.block_tables.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    ref_layer = oracle64(case)
    assert_layer_equal(pool, 0, ref_layer)
    got = out.download((case.S, case.n_heads, D), np.float32)
    ref = O.paged_decode(ref_layer, q64, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, (err, nbad)


@pytest.mark.parametrize("G,qd", [(4, np.float16), (1, np.float16), (4, np.float32), (5, np.float16)])
@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
@pytest.mark.parametrize("shared", [0, 8])
def test_hd64_tree_verify(ctx, kv, shared, G, qd):
    """Tree verify over 64-dim tiles on the 64-dim tree kernels (one or two row
    tiles, fp16 or fp32 q, any group size, every pool type)."""
    print(f"hd64 tree kv={kv} shared={shared} G={G} q={np.dtype(qd).name}", flush=True)
    N, Hkv = 8, 2
    committed = np.array([shared * BS + 3, shared * BS + 60, shared * BS + 200, shared * BS], np.int32)
    case = hd64_case(kv, committed + N, n_kv_heads=Hkv, n_heads=Hkv * G, seed=1430 + kv)
    if shared:
        for s in range(1, case.S):
            case.k[s][:shared * BS] = case.k[0][:shared * BS]
            case.v[s][:shared * BS] = case.v[0][:shared * BS]
    pool = hd64_pool(ctx, case)
    bt = case.block_tables.copy()
    if shared:
        bt[1:, :shared] = bt[0, :shared]
    q64 = synth.normals_f16(case.S * N * case.n_heads * D, 1431).reshape(case.S, N, case.n_heads, D).astype(qd)
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    mask = np.tile(velokv.branching_tree([2, 2, 2], N).ancestor_mask(), (case.S, 1)).astype(np.uint32)
    pl = ctx.tree_plan(pool, case.S, N, case.n_heads, int(committed.max()), bt_stride=bt.shape[1],
                       q_dtype=qdt, shared_blocks=shared)
    assert "_gx_d64_" in pl["kernel"], pl
    if shared and kv in (O.F16, O.I8_BLK):  # the shared-prefix pass, built for 64 dims
        assert "_gx_d64_" in pl["prefix_kernel"], pl
    out = ctx.alloc(q64.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q64), qdt, out, ctx.upload(committed), ctx.upload(mask), case.S, N,
                    case.n_heads, int(committed.max()), block_tables=ctx.upload(bt), bt_stride=bt.shape[1],
                    shared_blocks=shared)
    ctx.sync()
    got = out.download(q64.shape, np.float32)
    ref = O.tree_verify(oracle64(case), q64, bt, committed, mask)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"


@pytest.mark.parametrize("G,N", [(1, 1), (3, 5), (16, 2), (40, 32), (2, 24)])
@pytest.mark.parametrize("kv", KV_ALL)
def test_hd64_tree_row_tiles_and_random_masks(ctx, kv, G, N):
    """The 64-dim tree kernels over row tiles of 1 to 1280 rows (one or two
    16-row tiles per wave, several row groups) with random per-sequence masks,
    rows that see no tree node and, at context 0, nothing at all."""
    print(f"hd64 tree tiles kv={kv} G={G} N={N}", flush=True)
    Hkv = 2
    committed = np.array([0, 3, 33, 250], np.int32)
    case = hd64_case(kv, committed + N, n_kv_heads=Hkv, n_heads=Hkv * G, seed=1440 + 7 * G + N)
    pool = hd64_pool(ctx, case)
    q64 = synth.normals_f16(case.S * N * case.n_heads * D, 1441 + N).reshape(case.S, N, case.n_heads, D)
    rng = np.random.default_rng(G * 100 + N)
    full = (1 << N) - 1 if N < 32 else 0xFFFFFFFF
    mask = rng.integers(0, 1 << 32, size=(case.S, N), dtype=np.uint64).astype(np.uint32) & np.uint32(full)
    mask[0, 0] = 0  # context 0 and no visible node: output zeros
    bt = case.block_tables
    pl = ctx.tree_plan(pool, case.S, N, case.n_heads, int(committed.max()), bt_stride=bt.shape[1])
    assert "_gx_d64_" in pl["kernel"], pl
    out = ctx.alloc(q64.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q64), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask), case.S, N,
                    case.n_heads, int(committed.max()), block_tables=ctx.upload(bt), bt_stride=bt.shape[1])
    ctx.sync()
    got = out.download(q64.shape, np.float32)
    ref = O.tree_verify(oracle64(case), q64, bt, committed, mask)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"
    assert np.all(got[0, 0] == 0.0)


@pytest.mark.parametrize("style", [O.ROPE_INTERLEAVED, O.ROPE_HALF])
@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_hd64_append_rope_bit_exact(ctx, kv, style):
    """RoPE over 64-dim rows (pairs (2i, 2i+1) or (i, i + 32), angles of a 64-dim
    table) fused into the append: pool bytes and rotated q bit for bit."""
    print(f"hd64 rope kv={kv} style={style}", flush=True)
    case = hd64_case(kv, [1, 17, 100, 257], n_kv_heads=2, n_heads=8, seed=1440)
    rows = np.concatenate([np.full(int(L), s) for s, L in enumerate(case.ctx_lens)])
    cpos = np.concatenate([np.arange(int(L)) for L in case.ctx_lens])
    sl = synth.slots_for_positions(case.block_tables, cpos, BS, rows)
    kk = np.concatenate([case.k[s][..., :D] for s in range(case.S)])
    vv = np.concatenate([case.v[s][..., :D] for s in range(case.S)])
    pos = (cpos + 5).astype(np.int32)
    n_pos = int(pos.max()) + 1
    table = velokv.rope_table(n_pos, D, 500000.0)
    q = synth.normals_f16(len(sl) * 8 * D, 1441).reshape(len(sl), 8, D)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 2, D, kv)
    dq = ctx.upload(q)
    ctx.append_rope(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(pos), ctx.upload(sl), len(sl),
                    ctx.upload(table), n_pos, style, q=dq, q_dtype=velokv.DT_F16, n_heads=8)
    ctx.sync()
    kr = O.rope_apply(kk, pos, style, table)          # fp32, 64 dims
    ref = O.Layer(case.n_blocks, 2, BS, D, kv)
    O.append(ref, kr, vv.astype(np.float32), sl)
    assert_layer_equal(pool, 0, ref)
    qr = O.rope_apply(q, pos, style, table).astype(np.float16)
    assert np.array_equal(dq.download(q.shape, np.float16).view(np.uint16), qr.view(np.uint16))


@pytest.mark.parametrize("kv", [O.F32, O.I8_BLK])
def test_hd64_tree_commit(ctx, kv):
    print(f"hd64 commit kv={kv}", flush=True)
    N = 8
    ctxs = np.array([0, 14, 31, 33, 100], np.int32)
    case = hd64_case(kv, ctxs + N, seed=1450)
    pool = hd64_pool(ctx, case)
    ref = oracle64(case)
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


def test_hd64_limits(ctx):
    # head_dim takes multiples of 8 up to 128 (64- or 128-dim tiles)
    for bad in (100, 36, 136, 256):
        with pytest.raises(velokv.VkError) as e:
            velokv.Pool(ctx, 1, 8, BS, 2, bad, O.F16)
        assert e.value.code == velokv.ERR_UNSUPPORTED, bad


@pytest.mark.parametrize("kv", KV_ALL)
@pytest.mark.parametrize("G", [3, 8, 16])
@pytest.mark.parametrize("sched", ["split", "stream", "auto"])
def test_hd64_pieces_group_sizes_and_long_units(ctx, kv, G, sched):
    """The 64-dim pieces at runtime group sizes (rows padded to one 16-row tile)
    over units that fill all four block-id windows: contexts of 4095-4097 tokens
    with 4096-token partitions (split), a ragged batch (stream-K) and a uniform
    batch under AUTO (the workgroup split for int8 pools)."""
    print(f"hd64 pieces kv={kv} G={G} sched={sched}", flush=True)
    kind, sc, P = {"split": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 4096),
                   "stream": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0),
                   "auto": (velokv.DECODE_AUTO, velokv.SCHED_AUTO, 0)}[sched]
    lens = {"split": [4095, 4096, 4097, 1, 300], "stream": [4095, 33, 1000, 2500, 17, 4000],
            "auto": [3000] * 6}[sched]
    Hkv = 2
    case = hd64_case(kv, lens, n_kv_heads=Hkv, n_heads=G * Hkv, seed=1450 + 7 * G + kv)
    pool = hd64_pool(ctx, case)
    q64 = np.ascontiguousarray(case.q[..., :D]).astype(np.float16)
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sc)
    try:
        sum_len = int(sum(lens))
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1],
                             partition_tokens=P, sum_context_len=sum_len)
        assert pl["kernel"].endswith("_gx_d64"), pl
        out = ctx.alloc(case.S * case.n_heads * D * 4)
        ctx.paged_decode(pool, 0, ctx.upload(q64), velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S,
                         case.n_heads, int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1], partition_tokens=P, sum_context_len=sum_len)
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    got = out.download((case.S, case.n_heads, D), np.float32)
    ref = O.paged_decode(oracle64(case), q64, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance ({pl['kernel']})"


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_BLK])
@pytest.mark.parametrize("G", [3, 8])
def test_hd64_workgroup_split_group_sizes(ctx, kv, G):
    """The 64-dim workgroup split over fp32, fp16 and int8 pools at runtime group sizes."""
    print(f"hd64 workgroup split kv={kv} G={G}", flush=True)
    lens = list(synth.rng(1470 + G).integers(2, 400, 64))
    case = hd64_case(kv, lens, n_kv_heads=8, n_heads=8 * G, seed=1471 + G)
    pool = hd64_pool(ctx, case)
    q64 = np.ascontiguousarray(case.q[..., :D])
    out = ctx.alloc(case.S * case.n_heads * D * 4)
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1])
        assert pl["kernel"] == f"vk_decode_wg_kv{kv}_gx_d64", pl
        ctx.paged_decode(pool, 0, ctx.upload(q64), velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S, case.n_heads,
                         int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    got = out.download((case.S, case.n_heads, D), np.float32)
    ref = O.paged_decode(oracle64(case), q64, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, (err, nbad)
