"""GPU parity of vk_append_rope_decode: per sequence, the new K row rotated at
position context_len - 1 and appended there with the new V row, q rotated at
the same position (the caller's q rows left as they are), then decode over the
rotated q. metal/model.rs:399-471 runs rope, kv_update and attention per layer;
kernels.metal:103-131 is the reference's rotation.

Checked against the oracle's fused RoPE append at those positions (the same
table) followed by its decode: pool bytes bit for bit, outputs within the
north-star tolerance; and against the two-call path on a second pool
(vk_append_rope writing the rotated q, then vk_paged_decode under the same
schedule): pool bytes bit for bit, and under stream-K, where both calls cut the
contexts into the same pieces and round the rotated q the same way, outputs bit
for bit. The folding kernels rotate inside the decode launch; plans that do
not fold (fixed partitions, fp32 and int8-ref pools, heads narrower than the
tile) rotate in the append launch into the workspace, which the workspace query
shows."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import assert_layer_equal, gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu

STYLES = [O.ROPE_INTERLEAVED, O.ROPE_HALF]


def dt_of(a):
    return velokv.DT_F32 if a.dtype == np.float32 else velokv.DT_F16


def fused(ctx, case, style, qd, sched, n_pos=None, in_dt=np.float16):
    """The one call on a pool holding every token but the last; returns (plan,
    pool, out, table, n_pos, workspace bytes beyond the decode's own under the
    same schedule)."""
    S, H = case.S, case.n_heads
    pool = gpu_pool(ctx, case, with_last=False, in_dtype=in_dt)
    sl, kk, vv = case.last_slots()
    n_pos = n_pos or int(case.ctx_lens.max())
    table = velokv.rope_table(n_pos, HD, 500000.0)
    q = case.q.astype(qd)
    dq = ctx.upload(q)
    out = ctx.alloc(S * H * HD * 4)
    stride = case.block_tables.shape[1]
    L = int(case.ctx_lens.max())
    ctx.set_decode_schedule(sched)
    try:
        pl = ctx.decode_plan(pool, S, H, L, bt_stride=stride, q_dtype=dt_of(q), sum_context_len=int(case.ctx_lens.sum()))
        ws = ctx.append_rope_decode_workspace_bytes(pool, S, H, L, bt_stride=stride, q_dtype=dt_of(q),
                                                    sum_context_len=int(case.ctx_lens.sum()))
        ws -= ctx.decode_workspace_bytes(pool, S, H, L, bt_stride=stride, q_dtype=dt_of(q),
                                         sum_context_len=int(case.ctx_lens.sum()))
        ctx.append_rope_decode(pool, 0, ctx.upload(kk.astype(in_dt)), ctx.upload(vv.astype(in_dt)),
                               dt_of(kk.astype(in_dt)), ctx.upload(table), n_pos, style, dq, dt_of(q), out,
                               ctx.upload(case.ctx_lens), S, H, L, block_tables=ctx.upload(case.block_tables),
                               bt_stride=stride, sum_context_len=int(case.ctx_lens.sum()))
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    q_after = dq.download(q.shape, qd)
    assert np.array_equal(q_after.view(np.uint8), q.view(np.uint8)), "the caller's q rows changed"
    return pl, pool, out.download((S, H, HD), np.float32), table, n_pos, ws


def two_call(ctx, case, style, qd, sched, table, n_pos, in_dt=np.float16):
    S, H = case.S, case.n_heads
    pool = gpu_pool(ctx, case, with_last=False, in_dtype=in_dt)
    sl, kk, vv = case.last_slots()
    pos = (case.ctx_lens - 1).astype(np.int32)
    dq = ctx.upload(case.q.astype(qd))
    ctx.append_rope(pool, 0, ctx.upload(kk.astype(in_dt)), ctx.upload(vv.astype(in_dt)), dt_of(kk.astype(in_dt)),
                    ctx.upload(pos), ctx.upload(sl), len(sl), ctx.upload(table), n_pos, style, q=dq,
                    q_dtype=dt_of(case.q.astype(qd)), n_heads=H)
    out = ctx.alloc(S * H * HD * 4)
    ctx.set_decode_schedule(sched)
    try:
        ctx.paged_decode(pool, 0, dq, dt_of(case.q.astype(qd)), out, ctx.upload(case.ctx_lens), S, H,
                         int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1], sum_context_len=int(case.ctx_lens.sum()))
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    ctx.sync()
    return pool, out.download((S, H, HD), np.float32)


def check(ctx, case, style, qd, sched, pl, pool, got, table, n_pos, in_dt=np.float16, same_pieces=False):
    sl, kk, vv = case.last_slots()
    pos = (case.ctx_lens - 1).astype(np.int64)
    ref = O.Layer(case.n_blocks, case.n_kv_heads, BS, HD, case.kv_type)
    psl, pk, pv = case.prefill_slots()
    if len(psl):
        O.append(ref, pk.astype(in_dt), pv.astype(in_dt), psl)
    qr = O.append_rope(ref, kk.astype(in_dt), vv.astype(in_dt), sl, pos, style, table, q=case.q.astype(qd))
    assert_layer_equal(pool, 0, ref)
    pool2, got2 = two_call(ctx, case, style, qd, sched, table, n_pos, in_dt)
    a, b = pool.download_layer(0), pool2.download_layer(0)
    for key in ("k", "v", "ks", "vs"):
        assert (a[key] is None and b[key] is None) or np.array_equal(a[key], b[key]), key
    if same_pieces:
        assert np.array_equal(got, got2), "fused call and RoPE append + decode differ"
    want = O.paged_decode(ref, qr, case.block_tables, case.ctx_lens)
    for g, what in ((got, "append_rope_decode"), (got2, "append_rope + decode")):
        ok, err, nbad = tol_check(g, want)
        assert ok, f"{what}: max err {err:.3g}, {nbad} out of tolerance"


@pytest.mark.parametrize("qd", [np.float16, np.float32])
@pytest.mark.parametrize("style", STYLES)
def test_workgroup_split_rotates_in_the_decode(ctx, style, qd):
    """64 sequences x 8 KV heads over an int8 block pool: the workgroup split's
    folding wave rotates and appends the new K row, every wave rotates q. New
    tokens at every block offset and at position 0 (L = 1)."""
    print(f"append_rope_decode wg style={style} q={np.dtype(qd).name}", flush=True)
    r = synth.rng(1701)
    lens = r.integers(1, 700, 64)
    lens[:6] = [1, 16, 17, 32, 33, 48]
    lens[6:22] = 200 + np.arange(16)
    case = make_case(O.I8_BLK, lens, seed=1702, outlier_scale=8.0)
    pl, pool, got, table, n_pos, ws = fused(ctx, case, style, qd, velokv.SCHED_SPLIT)
    assert pl["schedule"] == velokv.SCHED_WORKGROUP, pl
    assert ws == 0, "the RoPE should fold into the decode kernel"
    check(ctx, case, style, qd, velokv.SCHED_SPLIT, pl, pool, got, table, n_pos)


@pytest.mark.parametrize("style", STYLES)
@pytest.mark.parametrize("G", [4, 3])
@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
def test_stream_k_rotates_in_the_decode(ctx, kv, G, style):
    """A ragged batch under stream-K over int8 block and fp16 pools (group sizes
    4 and 3, the _gx kernels): the piece that ends at a context's last token
    rotates and appends; every piece rotates q. Half the new rows are 3x larger
    (int8 block scales grow, the earlier codes are requantized). Outputs equal
    the two-call path's bit for bit."""
    print(f"append_rope_decode stream-K kv={kv} G={G} style={style}", flush=True)
    r = synth.rng(1710 + G)
    lens = r.integers(1, 3000, 64)
    lens[:6] = [1, 16, 17, 32, 33, 48]
    lens[6:22] = 1200 + np.arange(16)
    case = make_case(kv, lens, n_kv_heads=8, n_heads=8 * G, seed=1711 + G, outlier_scale=8.0)
    for s_ in range(0, case.S, 2):
        case.k[s_][-1] = (case.k[s_][-1].astype(np.float32) * 3).astype(np.float16)
        case.v[s_][-1] = (case.v[s_][-1].astype(np.float32) * 3).astype(np.float16)
    pl, pool, got, table, n_pos, ws = fused(ctx, case, style, np.float16, velokv.SCHED_STREAM)
    assert pl["schedule"] == velokv.SCHED_STREAM and "_sk_" in pl["kernel"], pl
    assert ws == 0
    check(ctx, case, style, np.float16, velokv.SCHED_STREAM, pl, pool, got, table, n_pos, same_pieces=True)


def test_stream_k_fp32_q_and_inputs(ctx):
    """fp32 q (rotated in fp32, then split into fp16 hi + lo) and fp32 new rows."""
    print("append_rope_decode stream-K fp32", flush=True)
    lens = synth.rng(1720).integers(1, 2000, 48)
    lens[:4] = [1, 2, 16, 17]
    case = make_case(O.I8_BLK, lens, n_kv_heads=8, n_heads=32, seed=1721, outlier_scale=8.0)
    case.k = [(k.astype(np.float32) * np.float32(1.37)) for k in case.k]
    case.v = [(v.astype(np.float32) * np.float32(0.61)) for v in case.v]
    pl, pool, got, table, n_pos, ws = fused(ctx, case, O.ROPE_HALF, np.float32, velokv.SCHED_STREAM,
                                            in_dt=np.float32)
    assert pl["schedule"] == velokv.SCHED_STREAM, pl
    check(ctx, case, O.ROPE_HALF, np.float32, velokv.SCHED_STREAM, pl, pool, got, table, n_pos, in_dt=np.float32,
          same_pieces=True)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_plans_that_do_not_fold(ctx, kv):
    """Fixed partitions over a small ragged batch (and fp32 / int8-ref pools
    under any plan): the RoPE append rotates the new K row into the pool and q
    into the workspace, then the decode reads the rotated q there."""
    print(f"append_rope_decode unfolded kv={kv}", flush=True)
    case = make_case(kv, [1, 17, 300, 64, 1000], seed=1730, outlier_scale=8.0)
    pl, pool, got, table, n_pos, ws = fused(ctx, case, O.ROPE_INTERLEAVED, np.float16, velokv.SCHED_SPLIT)
    assert pl["schedule"] == velokv.SCHED_SPLIT, pl
    assert ws == -(-case.S * case.n_heads * HD * 2 // 256) * 256  # the rotated q rows
    check(ctx, case, O.ROPE_INTERLEAVED, np.float16, velokv.SCHED_SPLIT, pl, pool, got, table, n_pos,
          same_pieces=True)


@pytest.mark.parametrize("sched", [velokv.SCHED_SPLIT, velokv.SCHED_STREAM])
def test_positions_outside_the_table(ctx, sched):
    """A table shorter than some contexts: those sequences append nothing (as
    the RoPE append skips a position outside the table) and attend with q as
    it is, over the workgroup split and stream-K."""
    print(f"append_rope_decode short table sched={sched}", flush=True)
    lens = synth.rng(1740).integers(1, 700, 64)
    lens[:4] = [1, 300, 301, 699]
    case = make_case(O.I8_BLK, lens, seed=1741, outlier_scale=8.0)
    pl, pool, got, table, n_pos, ws = fused(ctx, case, O.ROPE_HALF, np.float16, sched, n_pos=300)
    assert pl["schedule"] == (velokv.SCHED_WORKGROUP if sched == velokv.SCHED_SPLIT else velokv.SCHED_STREAM), pl
    check(ctx, case, O.ROPE_HALF, np.float16, sched, pl, pool, got, table, n_pos,
          same_pieces=sched == velokv.SCHED_STREAM)


def test_rejects_bad_arguments(ctx):
    case = make_case(O.I8_BLK, [5], seed=1750)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, O.I8_BLK)
    buf = ctx.alloc(1 << 20)
    for style, n_pos, in_dt in ((0, 16, velokv.DT_F16), (3, 16, velokv.DT_F16), (O.ROPE_HALF, 0, velokv.DT_F16),
                                (O.ROPE_HALF, 16, 7)):
        with pytest.raises(velokv.VkError) as e:
            ctx.append_rope_decode(pool, 0, buf, buf, in_dt, buf, n_pos, style, buf, velokv.DT_F16, buf, buf, 1,
                                   32, 5, block_tables=buf, bt_stride=1)
        assert e.value.code == velokv.ERR_BAD_ARG
    with pytest.raises(velokv.VkError) as e:  # the table is read in 16-byte chunks
        ctx.append_rope_decode(pool, 0, buf, buf, velokv.DT_F16, buf.ptr + 8, 16, O.ROPE_HALF, buf, velokv.DT_F16,
                               buf, buf, 1, 32, 5, block_tables=buf, bt_stride=1)
    assert e.value.code == velokv.ERR_BAD_ARG and "aligned" in str(e.value)
