"""GPU parity of paged decode attention against the oracle, within the north-star
tolerance (|err| <= 2e-3 + 1e-2 |ref|, fp32-accumulated oracle), for every KV
type, query dtype, GQA group size and split-K partition size."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from velokv import synth
from cases import BS, HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import gpu_pool

pytestmark = pytest.mark.gpu

KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]
IMPLS = [(velokv.DECODE_MFMA, velokv.SCHED_SPLIT), (velokv.DECODE_MFMA, velokv.SCHED_STREAM),
         (velokv.DECODE_VALU, velokv.SCHED_SPLIT)]


@pytest.fixture(params=IMPLS, ids=["mfma", "mfma-streamk", "valu"])
def impl(request, ctx):
    kind, sched = request.param
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sched)
    yield request.param
    ctx.set_decode_kernel(velokv.DECODE_AUTO)
    ctx.set_decode_schedule(velokv.SCHED_AUTO)


def run_decode(ctx, pool, case, q=None, q_dtype=np.float16, partition_tokens=0, layer=0, seq_rows=None,
               block_tables=None, n_seqs=None):
    q = case.q if q is None else q
    q = q.astype(q_dtype)
    S = q.shape[0] if n_seqs is None else n_seqs
    out = ctx.alloc(S * case.n_heads * HD * 4)
    bt = case.block_tables if block_tables is None else block_tables
    ctx.paged_decode(pool, layer, ctx.upload(q), velokv.DT_F16 if q_dtype == np.float16 else velokv.DT_F32, out,
                     ctx.upload(case.ctx_lens[:S]), S, case.n_heads, int(case.ctx_lens[:S].max()),
                     block_tables=ctx.upload(bt), bt_stride=bt.shape[1],
                     seq_rows=ctx.upload(seq_rows) if seq_rows is not None else None,
                     partition_tokens=partition_tokens)
    ctx.sync()
    return out.download((S, case.n_heads, HD), np.float32)


def check(got, ref, what):
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"{what}: max err {err:.3g}, {nbad} elements out of tolerance"
    return err


@pytest.mark.parametrize("kv", KV_ALL)
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_decode_config1(ctx, impl, kv, qd):
    print(f"decode config1 impl={impl} kv={kv} q={np.dtype(qd).name}", flush=True)
    case = make_case(kv, [512], n_blocks=64, seed=201)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    got = run_decode(ctx, pool, case, q_dtype=qd)
    ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
    check(got, ref, "config1")


@pytest.mark.parametrize("kv", KV_ALL)
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_decode_gqa_groups_ragged(ctx, impl, kv, G):
    print(f"decode gqa impl={impl} kv={kv} G={G}", flush=True)
    Hkv = 2 if G == 8 else 4
    lens = [1, 16, 17, 100, 255, 256, 257, 600]
    case = make_case(kv, lens, n_kv_heads=Hkv, n_heads=Hkv * G, seed=202 + G, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, Hkv, HD, kv)
    sl, kk, vv = case.prefill_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    sl, kk, vv = case.last_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    for qd in (np.float16, np.float32):
        got = run_decode(ctx, pool, case, q_dtype=qd)
        ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
        check(got, ref, f"G={G} q={np.dtype(qd).name}")


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
@pytest.mark.parametrize("P", [16, 256, 1024, 2048, 4096, 0])
def test_decode_split_k_partitions(ctx, impl, kv, P):
    print(f"decode split impl={impl} kv={kv} P={P}", flush=True)
    # 4095 / 4096 / 4097: a 256-block unit at P = 4096 (the last block-id window) and its edges
    lens = [3000, 1024, 2049, 777, 4095, 4096, 4097]
    case = make_case(kv, lens, seed=210, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    got = run_decode(ctx, pool, case, partition_tokens=P)
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    check(got, ref, f"P={P}")


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_decode_config2_3_shapes_reduced_batch(ctx, impl, kv):
    """Configs 2 / 3: L ~ U[1024, 8192], 40k-block pool, GQA 4 (8 of the 64 sequences)."""
    print(f"decode config2/3 impl={impl} kv={kv}", flush=True)
    r = np.random.default_rng(301)
    lens = r.integers(1024, 8193, 8)
    case = make_case(kv, lens, n_blocks=40000, seed=302, outlier_scale=8.0 if kv == O.I8_BLK else 1.0,
                     stride=512)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    got = run_decode(ctx, pool, case)
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    err = check(got, ref, "config2/3")
    print(f"  max abs err {err:.3g}")


def test_decode_seq_rows_and_pool_slot_table(ctx):
    """Rows chosen through seq_rows, and the pool's own slot table (bind_slot)."""
    print("decode seq_rows / slot table", flush=True)
    case = make_case(O.I8_BLK, [300, 45, 129], seed=303)
    ref_layer = oracle_layer(case)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, O.I8_BLK, max_slots=8,
                       max_pages_per_slot=case.block_tables.shape[1])
    sl, kk, vv = case.prefill_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    sl, kk, vv = case.last_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    slots = [5, 0, 7]
    for s, slot in enumerate(slots):
        n = -(-int(case.ctx_lens[s]) // BS)
        pool.bind_slot(slot, case.block_tables[s, :n])
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    out = ctx.alloc(3 * 32 * HD * 4)
    ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), 3, 32,
                     int(case.ctx_lens.max()), seq_rows=ctx.upload(np.array(slots, np.int32)))
    got = out.download((3, 32, HD), np.float32)
    check(got, ref, "slot table")


def test_decode_deterministic_and_block_permutation_invariant(ctx, impl):
    print(f"decode determinism impl={impl}", flush=True)
    case = make_case(O.I8_BLK, [700, 1500], seed=304)
    pool = gpu_pool(ctx, case)
    a = run_decode(ctx, pool, case)
    b = run_decode(ctx, pool, case)
    assert np.array_equal(a, b)
    # the same data under another physical block assignment gives the same bits
    case2 = make_case(O.I8_BLK, [700, 1500], seed=304)
    perm = np.random.default_rng(9).permutation(case2.n_blocks).astype(np.int32)
    case2.block_tables = perm[case2.block_tables]
    pool2 = gpu_pool(ctx, case2)
    c = run_decode(ctx, pool2, case2)
    assert np.array_equal(a, c)


def test_decode_empty_and_single_token(ctx, impl):
    print(f"decode empty / single impl={impl}", flush=True)
    case = make_case(O.F16, [1, 5], seed=305)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    got = run_decode(ctx, pool, case)
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    assert np.array_equal(got[0], ref[0])  # one token: out = v_0 exactly
    check(got, ref, "single")
    case.ctx_lens = np.array([0, 5], np.int32)
    got = run_decode(ctx, pool, case)
    assert not got[0].any()


def test_decode_rejects_bad_arguments(ctx):
    case = make_case(O.F16, [20], seed=306)
    pool = gpu_pool(ctx, case)
    with pytest.raises(velokv.VkError) as e:
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, ctx.alloc(32 * HD * 4),
                         ctx.upload(case.ctx_lens), 1, 264, 20, block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1])
    assert e.value.code == velokv.ERR_UNSUPPORTED  # 264 / 8 = 33 query heads per KV head: beyond 32
    with pytest.raises(velokv.VkError) as e:
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, ctx.alloc(32 * HD * 4),
                         ctx.upload(case.ctx_lens), 1, 28, 20, block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1])
    assert e.value.code == velokv.ERR_BAD_ARG  # 28 is not a multiple of 8 KV heads
    with pytest.raises(velokv.VkError) as e:
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, ctx.alloc(32 * HD * 4),
                         ctx.upload(case.ctx_lens), 1, 32, 10 ** 6, block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1])
    assert e.value.code == velokv.ERR_BAD_ARG
    with pytest.raises(velokv.VkError):
        ctx.paged_decode(pool, 5, ctx.upload(case.q), velokv.DT_F16, ctx.alloc(32 * HD * 4),
                         ctx.upload(case.ctx_lens), 1, 32, 20, block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1])


def test_decode_workspace_reuse_across_layouts(ctx, impl):
    """Split-K counters stay consistent when consecutive calls change the batch
    size and the partition layout, with the context's workspace and with a
    caller-owned one."""
    print(f"decode workspace reuse impl={impl}", flush=True)
    case = make_case(O.I8_BLK, [2000, 700, 1300, 64, 999, 3100], seed=307)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    own = ctx.alloc(1 << 25)
    for S, P in ((6, 16), (2, 256), (6, 1024), (3, 16), (6, 512), (1, 16), (6, 0)):
        for ws in (None, own):
            out = ctx.alloc(S * 32 * HD * 4)
            ctx.paged_decode(pool, 0, ctx.upload(case.q[:S]), velokv.DT_F16, out, ctx.upload(case.ctx_lens[:S]), S, 32,
                             int(case.ctx_lens[:S].max()), block_tables=ctx.upload(case.block_tables),
                             bt_stride=case.block_tables.shape[1], partition_tokens=P,
                             workspace=ws, workspace_bytes=(1 << 25) if ws is not None else 0)
            ctx.sync()
            check(out.download((S, 32, HD), np.float32), ref[:S], f"S={S} P={P} own_ws={ws is not None}")


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
@pytest.mark.parametrize("shape", ["mixed", "many_small", "wide"])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_decode_streamk_worker_boundaries(ctx, kv, shape, qd):
    """Stream-K ranges that split segments at arbitrary blocks, cross several
    sequences, skip empty contexts, and (many_small) leave fewer blocks than
    workers; more than 64 sequences exercise the chunked prefix scan."""
    print(f"decode stream-K kv={kv} shape={shape} q={np.dtype(qd).name}", flush=True)
    ctx.set_decode_kernel(velokv.DECODE_MFMA)
    ctx.set_decode_schedule(velokv.SCHED_STREAM)
    try:
        if shape == "mixed":
            lens = [0, 1, 0, 5, 16, 17, 4096, 3, 0, 2049, 100, 33, 0, 1500]
        elif shape == "many_small":
            lens = [(i * 7) % 20 for i in range(150)]
        else:
            lens = list(synth.rng(9).integers(0, 3000, 130))
        # fill every sequence with at least one token, then attend over the real lengths
        case = make_case(kv, [max(1, int(L)) for L in lens], n_kv_heads=2, n_heads=8, seed=401, outlier_scale=8.0)
        ref_layer = oracle_layer(case)
        pool = gpu_pool(ctx, case)
        case.ctx_lens = np.asarray(lens, np.int32)
        name = ctx.decode_kernel_name(pool, len(lens), 8, int(max(lens)), bt_stride=case.block_tables.shape[1],
                                      q_dtype=velokv.DT_F32 if qd == np.float32 else velokv.DT_F16)
        assert name.startswith(f"vk_decode_sk_kv{kv}_g4"), name
        got = run_decode(ctx, pool, case, q_dtype=qd)
        ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
        check(got, ref, f"stream-K {shape} q={np.dtype(qd).name}")
        assert np.all(got[np.asarray(lens) == 0] == 0.0)
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)


@pytest.mark.parametrize("kv", [O.F32, O.I8_REF, O.I8_BLK])
@pytest.mark.parametrize("S,G,nw", [(256, 4, 1), (128, 4, 2), (64, 4, 4), (32, 8, 8)])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_decode_workgroup_split(ctx, kv, S, G, nw, qd):
    """The workgroup-split kernel (one workgroup of nw waves per (sequence, KV
    head), partials combined in LDS) on ragged contexts, including empty and
    one-token ones and waves whose share is empty."""
    print(f"decode workgroup split kv={kv} S={S} G={G} nw={nw}", flush=True)
    Hkv = 8
    rng = synth.rng(300 + S)
    lens = rng.integers(0, 700, S)
    lens[:6] = [0, 1, 15, 16, 17, 33]
    case = make_case(kv, [max(1, int(L)) for L in lens], n_kv_heads=Hkv, n_heads=Hkv * G, seed=311 + S,
                     outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    case.ctx_lens = np.asarray(lens, np.int32)
    ctx.set_decode_kernel(velokv.DECODE_MFMA)
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
        name = ctx.decode_kernel_name(pool, S, Hkv * G, int(lens.max()), bt_stride=case.block_tables.shape[1],
                                      q_dtype=qdt)
        assert name == f"vk_decode_wg_kv{kv}_g{G}" + ("_q0" if qd == np.float32 else ""), name
        assert ctx.decode_workspace_bytes(pool, S, Hkv * G, int(lens.max()),
                                          bt_stride=case.block_tables.shape[1], q_dtype=qdt) == 0
        got = run_decode(ctx, pool, case, q_dtype=qd)
        ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
        check(got, ref, f"workgroup split S={S} G={G} q={np.dtype(qd).name}")
        assert np.all(got[lens == 0] == 0.0)
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)


def outlier_q(shape, seed, scale):
    """Queries with realistic magnitudes: N(0, 1) with four outlier channels
    scaled by `scale`, as fp32 values that fp16 does not hold exactly."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(shape).astype(np.float32)
    ch = rng.choice(shape[-1], 4, replace=False)
    q[..., ch] *= np.float32(scale)
    return q


@pytest.mark.parametrize("kv", [O.I8_BLK, O.I8_REF, O.F16])
@pytest.mark.parametrize("sched", [velokv.SCHED_SPLIT, velokv.SCHED_STREAM])
def test_decode_outlier_queries(ctx, sched, kv):
    """q with x10 and x30 outlier channels (|q| up to about 100), as fp16 and as
    fp32: the int8 kernels' biased products, sum_d q (1152 + c) - 1152 sum_d q,
    lose bits in proportion to sum_d |q|, and an fp32 q takes the hi + lo split.
    Outputs stay within the north-star tolerance of the oracle over the same q,
    on the workgroup split (int8) or split-K (fp16) and on stream-K. One pool
    and one oracle layer serve the four queries."""
    lens = synth.rng(451).integers(1, 3000, 64)
    lens[:4] = [1, 16, 17, 2999]
    case = make_case(kv, lens, n_kv_heads=8, n_heads=32, seed=452, outlier_scale=8.0 if kv != O.F16 else 1.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    for qd in (np.float16, np.float32):
        for scale in (10.0, 30.0):
            print(f"decode outlier q sched={sched} kv={kv} q={np.dtype(qd).name} x{scale}", flush=True)
            q = outlier_q(case.q.shape, 453, scale).astype(qd)
            ctx.set_decode_kernel(velokv.DECODE_MFMA)
            ctx.set_decode_schedule(sched)
            try:
                got = run_decode(ctx, pool, case, q=q, q_dtype=qd)
            finally:
                ctx.set_decode_kernel(velokv.DECODE_AUTO)
                ctx.set_decode_schedule(velokv.SCHED_AUTO)
            ref = O.paged_decode(ref_layer, q, case.block_tables, case.ctx_lens)
            err = check(got, ref, f"outlier q x{scale}")
            print(f"  max abs err {err:.3g}", flush=True)
