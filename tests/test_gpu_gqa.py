"""GPU parity for GQA group sizes other than 1, 2, 4, 8 (the reference maps any
integer ratio, kv_head = h / (H / Hkv), kernels.metal:456; llama_cpu.rs:260).
Such ratios run the "_gx" matrix-core kernels, which take the group size at run
time: decode on every schedule (fixed partitions, stream-K, workgroup split,
vk_append_decode) up to 16 query heads per KV head, fixed partitions with two
16-row tiles up to 32; tree verify (with and without the shared-prefix pass)
for any size. Oracle comparison within the north-star tolerance."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu

SCHEDS = {"split": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0), "split-p256": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 256),
          "stream": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0), "auto": (velokv.DECODE_AUTO, velokv.SCHED_AUTO, 0)}


def decode(ctx, pool, case, qd, kind, sched, P):
    S, H = case.S, case.n_heads
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sched)
    try:
        pl = ctx.decode_plan(pool, S, H, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1],
                             partition_tokens=P, q_dtype=qdt)
        out = ctx.alloc(S * H * HD * 4)
        ctx.paged_decode(pool, 0, ctx.upload(case.q.astype(qd)), qdt, out, ctx.upload(case.ctx_lens), S, H,
                         int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                         bt_stride=case.block_tables.shape[1], partition_tokens=P)
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    return pl, out.download((S, H, HD), np.float32)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
@pytest.mark.parametrize("G", [3, 5, 6, 7, 12, 16, 24, 32])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_decode_any_group_size(ctx, kv, G, qd):
    print(f"gqa decode kv={kv} G={G} q={np.dtype(qd).name}", flush=True)
    Hkv = 2
    lens = [1, 16, 17, 255, 700, 1500]
    case = make_case(kv, lens, n_kv_heads=Hkv, n_heads=Hkv * G, seed=960 + G, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
    for name, (kind, sched, P) in SCHEDS.items():
        if G > 16 and name == "stream":
            continue  # stream-K takes one 16-row tile; larger groups run fixed partitions
        pl, got = decode(ctx, pool, case, qd, kind, sched, P)
        assert "_gx" in pl["kernel"], pl
        ok, err, nbad = tol_check(got, ref)
        assert ok, f"{name}: max err {err:.3g}, {nbad} out of tolerance ({pl['kernel']})"


@pytest.mark.parametrize("G", [3, 6, 12])
def test_decode_any_group_workgroup_split_and_append_decode(ctx, G):
    """A batch that fills the GPU (64 x 8 pairs) takes the workgroup split,
    through vk_append_decode."""
    print(f"gqa workgroup split G={G}", flush=True)
    lens = list(synth.rng(970 + G).integers(2, 400, 64))
    case = make_case(O.I8_BLK, lens, n_kv_heads=8, n_heads=8 * G, seed=971 + G, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case, with_last=False)
    sl, kk, vv = case.last_slots()
    out = ctx.alloc(case.S * case.n_heads * HD * 4)
    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        pl = ctx.decode_plan(pool, case.S, case.n_heads, int(case.ctx_lens.max()), bt_stride=case.block_tables.shape[1])
        assert pl["kernel"] == "vk_decode_wg_kv3_gx", pl
        ctx.append_decode(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(case.q), velokv.DT_F16, out,
                          ctx.upload(case.ctx_lens), case.S, case.n_heads, int(case.ctx_lens.max()),
                          block_tables=ctx.upload(case.block_tables), bt_stride=case.block_tables.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    from test_gpu_append_copy import assert_layer_equal
    assert_layer_equal(pool, 0, ref_layer)
    got = out.download((case.S, case.n_heads, HD), np.float32)
    ok, err, nbad = tol_check(got, O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens))
    assert ok, (err, nbad)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
@pytest.mark.parametrize("G,N", [(3, 8), (6, 5), (16, 2), (12, 8), (40, 1)])
def test_tree_any_group_size(ctx, kv, G, N):
    print(f"gqa tree kv={kv} G={G} N={N}", flush=True)
    Hkv = 2
    committed = np.array([0, 5, 100, 333], np.int32)
    case = make_case(kv, committed + N, n_kv_heads=Hkv, n_heads=Hkv * G, seed=980 + G, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = synth.normals_f16(case.S * N * case.n_heads * HD, 981 + G).reshape(case.S, N, case.n_heads, HD)
    mask = (synth.rng(982 + G).integers(0, 2 ** N, (case.S, N)) | (1 << np.arange(N))).astype(np.uint32)
    out = ctx.alloc(q.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask), case.S, N,
                    case.n_heads, int(committed.max()), block_tables=ctx.upload(case.block_tables),
                    bt_stride=case.block_tables.shape[1])
    ctx.sync()
    got = out.download(q.shape, np.float32)
    ref = O.tree_verify(ref_layer, q, case.block_tables, committed, mask)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
@pytest.mark.parametrize("G", [3, 12])
def test_tree_shared_prefix_any_group_size(ctx, kv, G):
    """The shared-prefix pass with a runtime group size: 6 sequences whose
    tables share their first 8 pages."""
    print(f"gqa tree prefix kv={kv} G={G}", flush=True)
    Hkv, N, pre = 2, 4, 8
    committed = np.array([130, 140, 200, 129, 180, 300], np.int32)
    case = make_case(kv, committed + N, n_kv_heads=Hkv, n_heads=Hkv * G, seed=990 + G, outlier_scale=8.0)
    # sequences 1.. reuse sequence 0's first pages, whose data the oracle and the pool both hold
    bt = case.block_tables.copy()
    for s in range(1, case.S):
        case.k[s][:pre * BS] = case.k[0][:pre * BS]
        case.v[s][:pre * BS] = case.v[0][:pre * BS]
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    bt[1:, :pre] = bt[0, :pre]
    q = synth.normals_f16(case.S * N * case.n_heads * HD, 991 + G).reshape(case.S, N, case.n_heads, HD)
    mask = np.tile(velokv.branching_tree([2, 2], N).ancestor_mask(), (case.S, 1)).astype(np.uint32)
    out = ctx.alloc(q.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask), case.S, N,
                    case.n_heads, int(committed.max()), block_tables=ctx.upload(bt), bt_stride=bt.shape[1],
                    shared_blocks=pre)
    ctx.sync()
    got = out.download(q.shape, np.float32)
    ref = O.tree_verify(ref_layer, q, bt, committed, mask)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"


def test_group_size_limits(ctx):
    case = make_case(O.I8_BLK, [40], n_kv_heads=2, n_heads=66, seed=995)  # G = 33
    pool = gpu_pool(ctx, case)
    with pytest.raises(velokv.VkError) as e:
        ctx.decode_plan(pool, 1, 66, 40, bt_stride=case.block_tables.shape[1])
    assert e.value.code == velokv.ERR_UNSUPPORTED
    f32 = velokv.Pool(ctx, 1, 8, BS, 2, HD, O.F32)
    assert ctx.decode_plan(f32, 1, 6, 40, bt_stride=4)["kernel"].startswith("vk_decode_")  # G = 3 over fp32 KV
