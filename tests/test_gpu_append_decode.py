"""GPU parity of vk_append_decode (the new token of every sequence appended at
position context_len - 1, then decode; metal/model.rs:399-471 runs kv_update then
the attention kernel per layer): the append kernel with the slots derived from
the block table in the kernel, then the decode, over every schedule.
Each case is checked three ways: pool bytes bit for bit against the oracle's
append of the same tokens and against vk_append + vk_paged_decode (same
schedule) on a second pool, and outputs within the north-star tolerance of the
oracle's decode. Under stream-K the two calls cut the contexts into the same
pieces, so their outputs are also compared bit for bit; under the workgroup
split the folding wave's range is kFoldBlocks shorter, so outputs agree to fp32
rounding of a different split (checked within the tolerance)."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import assert_layer_equal, gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu


def one_call_step(ctx, pool, case, qd=np.float16, in_dt=np.float16, block_tables=None, seq_rows=None, bt_stride=None):
    """vk_append_decode of every sequence's last token; returns (plan, output).
    Fixed-partition planning (VK_SCHED_SPLIT), whose workgroup split takes a batch
    of 64 x 8 pairs; AUTO would send these ragged test batches to stream-K."""
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        return _one_call_step(ctx, pool, case, qd, in_dt, block_tables, seq_rows, bt_stride)
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)


def _one_call_step(ctx, pool, case, qd, in_dt, block_tables, seq_rows, bt_stride):
    S, H = case.S, case.n_heads
    sl, kk, vv = case.last_slots()
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    bt = case.block_tables if block_tables is None or block_tables is False else block_tables
    stride = bt.shape[1] if bt_stride is None else bt_stride
    pl = ctx.decode_plan(pool, S, H, int(case.ctx_lens.max()), bt_stride=stride, q_dtype=qdt,
                         sum_context_len=int(case.ctx_lens.sum()))
    out = ctx.alloc(S * H * HD * 4)
    ctx.append_decode(pool, 0, ctx.upload(kk.astype(in_dt)), ctx.upload(vv.astype(in_dt)),
                      velokv.DT_F32 if in_dt == np.float32 else velokv.DT_F16, ctx.upload(case.q.astype(qd)), qdt, out,
                      ctx.upload(case.ctx_lens), S, H, int(case.ctx_lens.max()),
                      block_tables=None if block_tables is False else ctx.upload(bt), bt_stride=stride,
                      seq_rows=ctx.upload(seq_rows) if seq_rows is not None else None,
                      sum_context_len=int(case.ctx_lens.sum()))
    ctx.sync()
    return pl, out.download((S, H, HD), np.float32)


def two_call_step(ctx, case, qd=np.float16, in_dt=np.float16, sched=velokv.SCHED_SPLIT):
    pool = gpu_pool(ctx, case, with_last=False, in_dtype=in_dt)
    sl, kk, vv = case.last_slots()
    ctx.append(pool, 0, ctx.upload(kk.astype(in_dt)), ctx.upload(vv.astype(in_dt)),
               velokv.DT_F32 if in_dt == np.float32 else velokv.DT_F16, ctx.upload(sl), len(sl))
    out = ctx.alloc(case.S * case.n_heads * HD * 4)
    ctx.set_decode_schedule(sched)
    try:
        ctx.paged_decode(pool, 0, ctx.upload(case.q.astype(qd)), velokv.DT_F32 if qd == np.float32 else velokv.DT_F16,
                         out, ctx.upload(case.ctx_lens), case.S, case.n_heads, int(case.ctx_lens.max()),
                         block_tables=ctx.upload(case.block_tables), bt_stride=case.block_tables.shape[1],
                         sum_context_len=int(case.ctx_lens.sum()))
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    ctx.sync()
    return pool, out.download((case.S, case.n_heads, HD), np.float32)


def check_all(ctx, case, pool, got, qd, in_dt=np.float16, sched=velokv.SCHED_SPLIT, same_pieces=False):
    ref_layer = oracle_layer_in(case, in_dt)
    assert_layer_equal(pool, 0, ref_layer)
    pool2, got2 = two_call_step(ctx, case, qd, in_dt, sched)
    a, b = pool.download_layer(0), pool2.download_layer(0)
    for key in ("k", "v", "ks", "vs"):
        assert (a[key] is None and b[key] is None) or np.array_equal(a[key], b[key]), key
    if same_pieces:
        assert np.array_equal(got, got2), "folded call and append + decode differ"
    ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
    for g, what in ((got, "append_decode"), (got2, "append + decode")):
        ok, err, nbad = tol_check(g, ref)
        assert ok, f"{what}: max err {err:.3g}, {nbad} out of tolerance"


def oracle_layer_in(case, in_dt):
    if in_dt == np.float16:
        return oracle_layer(case)
    L = O.Layer(case.n_blocks, case.n_kv_heads, BS, HD, case.kv_type)
    sl, kk, vv = case.prefill_slots()
    if len(sl):
        O.append(L, kk.astype(in_dt), vv.astype(in_dt), sl)
    sl, kk, vv = case.last_slots()
    O.append(L, kk.astype(in_dt), vv.astype(in_dt), sl)
    return L


@pytest.mark.parametrize("qd", [np.float16, np.float32])
@pytest.mark.parametrize("in_dt", [np.float16, np.float32])
def test_int8_workgroup_split(ctx, qd, in_dt):
    """64 sequences x 8 KV heads: the append, then the workgroup split.
    The new tokens land at every block offset (0 starts a fresh scale, 15 ends
    a block), including the first token of a context (L = 1) and outliers."""
    print(f"append_decode wg q={np.dtype(qd).name} in={np.dtype(in_dt).name}", flush=True)
    r = synth.rng(951)
    lens = r.integers(1, 700, 64)
    lens[:6] = [1, 16, 17, 32, 33, 48]
    lens[6:22] = 200 + np.arange(16)  # every offset of a block
    case = make_case(O.I8_BLK, lens, seed=952, outlier_scale=8.0)
    if in_dt == np.float32:
        case.k = [(k.astype(np.float32) * np.float32(1.37)) for k in case.k]
        case.v = [(v.astype(np.float32) * np.float32(0.61)) for v in case.v]
    pool = gpu_pool(ctx, case, with_last=False, in_dtype=in_dt)
    pl, got = one_call_step(ctx, pool, case, qd, in_dt)
    assert pl["schedule"] == velokv.SCHED_WORKGROUP, pl
    check_all(ctx, case, pool, got, qd, in_dt)


@pytest.mark.parametrize("qd", [np.float16, np.float32])
@pytest.mark.parametrize("G", [4, 3])
@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
def test_stream_k_folds_the_append(ctx, kv, G, qd):
    """A ragged batch under stream-K over int8 block and fp16 pools: the piece
    that ends at a context's last token appends the new token in the decode
    launch. New tokens at every block offset, first tokens of a context (L = 1),
    and (even sequences) new rows 3x larger, so that an int8 block scale grows
    and the earlier codes are requantized."""
    print(f"append_decode stream-K kv={kv} G={G} q={np.dtype(qd).name}", flush=True)
    r = synth.rng(960 + G)
    lens = r.integers(1, 3000, 64)
    lens[:6] = [1, 16, 17, 32, 33, 48]
    lens[6:22] = 1200 + np.arange(16)  # every offset of a block
    case = make_case(kv, lens, n_kv_heads=8, n_heads=8 * G, seed=961 + G, outlier_scale=8.0)
    for s_ in range(0, case.S, 2):
        case.k[s_][-1] = (case.k[s_][-1].astype(np.float32) * 3).astype(np.float16)
        case.v[s_][-1] = (case.v[s_][-1].astype(np.float32) * 3).astype(np.float16)
    pool = gpu_pool(ctx, case, with_last=False)
    ctx.set_decode_schedule(velokv.SCHED_STREAM)
    try:
        pl, got = _one_call_step(ctx, pool, case, qd, np.float16, None, None, None)
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    assert pl["schedule"] == velokv.SCHED_STREAM and "_sk_" in pl["kernel"], pl
    check_all(ctx, case, pool, got, qd, sched=velokv.SCHED_STREAM, same_pieces=True)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_small_ragged_batches(ctx, kv):
    """Small ragged batches (fixed partitions or stream-K) over every KV type."""
    print(f"append_decode small kv={kv}", flush=True)
    lens = [1, 17, 300, 64, 1000]
    case = make_case(kv, lens, seed=953, outlier_scale=8.0)
    pool = gpu_pool(ctx, case, with_last=False)
    pl, got = one_call_step(ctx, pool, case)
    check_all(ctx, case, pool, got, np.float16)


def test_slot_table_rows_empty_context_and_bad_page(ctx):
    """seq_rows into the pool's slot table; a context of 0 appends nothing and
    attends to nothing; a page id outside the pool stores nothing and is
    reported (VK_MISUSE_PAGE_OUT_OF_POOL) by the next sync."""
    print("append_decode slot table / empty / bad page", flush=True)
    lens = list(synth.rng(954).integers(2, 300, 64))
    case = make_case(O.I8_BLK, lens, seed=955)
    stride = case.block_tables.shape[1]
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, O.I8_BLK, max_slots=80, max_pages_per_slot=stride)
    sl, kk, vv = case.prefill_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    rows = np.arange(64, dtype=np.int32) + 10
    for s in range(64):
        pool.bind_slot(int(rows[s]), case.block_tables[s, :-(-int(case.ctx_lens[s]) // BS)])
    pl, got = one_call_step(ctx, pool, case, block_tables=False, seq_rows=rows, bt_stride=stride)
    assert pl["schedule"] == velokv.SCHED_WORKGROUP, pl
    ref_layer = oracle_layer(case)
    assert_layer_equal(pool, 0, ref_layer)
    ok, err, nbad = tol_check(got, O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens))
    assert ok, (err, nbad)
    # context 0 for sequence 3: nothing appended, zero output
    before = pool.download_layer(0)
    case.ctx_lens = case.ctx_lens.copy()
    case.ctx_lens[3] = 0
    _, got = one_call_step(ctx, pool, case, block_tables=False, seq_rows=rows, bt_stride=stride)
    assert not got[3].any()
    # the other sequences appended the same token at the same position again: the
    # append rule is idempotent there, so the whole layer is unchanged
    after = pool.download_layer(0)
    for key in ("k", "v", "ks", "vs"):
        assert np.array_equal(before[key], after[key]), key
    # a bad page in sequence 5's last block: nothing stored there, reported at sync
    bt = case.block_tables.copy()
    bt[5, (int(case.ctx_lens[5]) - 1) // BS] = case.n_blocks + 9
    out = ctx.alloc(64 * 32 * HD * 4)
    sl, kk, vv = case.last_slots()
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    ctx.append_decode(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(case.q), velokv.DT_F16, out,
                      ctx.upload(case.ctx_lens), 64, 32, int(case.ctx_lens.max()), block_tables=ctx.upload(bt),
                      bt_stride=stride, sum_context_len=int(case.ctx_lens.sum()))
    ctx.set_decode_schedule(velokv.SCHED_AUTO)
    with pytest.raises(velokv.VkError) as e:
        ctx.sync()
    assert "0x1" in str(e.value)


@pytest.mark.parametrize("shape", ["headline", "config5"])
def test_full_shape_fold_sampled(ctx, shape):
    """The folded call at the shapes the bench times, INT8, against the oracle on
    four sampled sequences (pool bytes of their blocks and outputs): 64 x 8192
    (the metric's shape, GQA 4, 4-wave workgroups of 128 blocks) and config 5's
    one-GPU share, 32 x 32768 with GQA 8 in a 65,536-block pool (8-wave
    workgroups of 256 blocks: the folding wave takes its last block from
    block-id window 3)."""
    print(f"append_decode full shape {shape}", flush=True)
    from test_gpu_fullshape import build_pool, oracle_sample, check_pool_bytes
    S, L, Hkv, H, n_blocks, kernel, waves = {
        "headline": (64, 8192, 8, 32, 40000, "vk_decode_wg_kv3_g4", 4),
        "config5": (32, 32768, 8, 64, 65536, "vk_decode_wg_kv3_g8", 8)}[shape]
    sample = [0, S // 3, 2 * S // 3, S - 1]
    lens_pre = np.full(S, L - 1, np.int32)
    pool, bt, inputs = build_pool(ctx, O.I8_BLK, lens_pre, Hkv, n_blocks, seed=58, sample=sample, outlier_scale=8.0)
    try:
        row = Hkv * HD
        kn = synth.normals_f16(S * row, 5801, row, 8.0).reshape(S, Hkv, HD)
        vn = synth.normals_f16(S * row, 5802, row, 8.0).reshape(S, Hkv, HD)
        bt_full = np.zeros((S, L // BS), np.int32)
        bt_full[:, :bt.shape[1]] = bt
        lens = np.full(S, L, np.int32)
        q = synth.normals_f16(S * H * HD, 5803).reshape(S, H, HD)
        out = ctx.alloc(S * H * HD * 4)
        pl = ctx.decode_plan(pool, S, H, L, bt_stride=bt_full.shape[1], sum_context_len=S * L)
        assert pl["kernel"] == kernel and pl["wg_waves"] == waves, pl
        assert pl["max_blocks_per_wave"] == L // BS // waves, pl
        ctx.append_decode(pool, 0, ctx.upload(kn), ctx.upload(vn), velokv.DT_F16, ctx.upload(q), velokv.DT_F16, out,
                          ctx.upload(lens), S, H, L, block_tables=ctx.upload(bt_full), bt_stride=bt_full.shape[1],
                          sum_context_len=S * L)
        ctx.sync()
        got = out.download((S, H, HD), np.float32)
        full = {s: (np.concatenate([inputs[s][0], kn[s][None]]), np.concatenate([inputs[s][1], vn[s][None]]))
                for s in sample}
        lay, cbt = oracle_sample(O.I8_BLK, Hkv, lens, full, sample)
        check_pool_bytes(pool, O.I8_BLK, Hkv, bt_full, lens, lay, cbt, sample)
        ref = O.paged_decode(lay, q[sample], cbt, lens[sample])
        ok, err, nbad = tol_check(got[sample], ref)
        assert ok, (err, nbad)
    finally:
        pool.close()
