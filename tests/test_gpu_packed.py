"""GPU parity of the packed workgroup split (vk_decode_pk_*: the (sequence, KV
head) pairs dealt longest first to one workgroup per resident slot in snake
order, split evenly over the workgroup's waves, split pairs combined in LDS)
against the oracle, within the north-star tolerance: many pairs per workgroup,
ties and empty contexts in the ranking, every GQA group, fp16 / INT8 KV, fp16 and
fp32 queries, and a batch with fewer pairs than workgroups.
kernels.metal:672-732, 440-501; llama_cpu.rs:251-284."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu


def run(ctx, pool, case, qd, sched=velokv.SCHED_AUTO):
    S, H = case.S, case.n_heads
    lens = case.ctx_lens
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    ctx.set_decode_schedule(sched)
    try:
        pl = ctx.decode_plan(pool, S, H, int(lens.max()), bt_stride=case.block_tables.shape[1], q_dtype=qdt)
        out = ctx.alloc(S * H * HD * 4)
        ctx.paged_decode(pool, 0, ctx.upload(case.q.astype(qd)), qdt, out, ctx.upload(lens), S, H, int(lens.max()),
                         block_tables=ctx.upload(case.block_tables), bt_stride=case.block_tables.shape[1])
        ctx.sync()
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    return pl, out.download((S, H, HD), np.float32)


@pytest.mark.parametrize("kv", [O.F16, O.I8_REF, O.I8_BLK])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_packed_many_pairs_per_workgroup(ctx, kv, G, qd):
    """256 sequences x 8 KV heads = 2048 pairs over the resident workgroups
    (about 8 per workgroup), contexts U[0, 300] with ties, zeros and the
    block-edge lengths."""
    print(f"packed many pairs kv={kv} G={G} q={np.dtype(qd).name}", flush=True)
    r = synth.rng(900 + G)
    lens = r.integers(0, 300, 256)
    lens[:8] = [0, 1, 15, 16, 17, 0, 299, 33]
    case = make_case(kv, [max(1, int(L)) for L in lens], n_kv_heads=8, n_heads=8 * G, seed=901 + G,
                     outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    case.ctx_lens = np.asarray(lens, np.int32)
    pl, got = run(ctx, pool, case, qd, sched=velokv.SCHED_PACKED)
    suffix = "_q0" if qd == np.float32 else ""
    assert pl["kernel"] == f"vk_decode_pk_kv{kv}_g{G}{suffix}", pl
    assert pl["schedule"] == velokv.SCHED_PACKED and not pl["merge_launch"] and pl["workspace_bytes"] == 0, pl
    assert 2048 // pl["n_workers"] >= 4, pl  # several pairs per workgroup
    ref = O.paged_decode(ref_layer, case.q.astype(qd), case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"
    assert np.all(got[lens == 0] == 0.0)


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_packed_forced_fewer_pairs_than_workgroups(ctx, kv):
    """VK_SCHED_PACKED with 5 sequences x 2 KV heads: one pair per workgroup,
    contexts that split a pair over all eight waves."""
    print(f"packed few pairs kv={kv}", flush=True)
    lens = [3000, 1, 4096, 700, 129]
    case = make_case(kv, lens, n_kv_heads=2, n_heads=8, seed=911, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    pl, got = run(ctx, pool, case, np.float16, sched=velokv.SCHED_PACKED)
    assert pl["schedule"] == velokv.SCHED_PACKED and pl["n_workers"] == 10, pl
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"


def test_packed_deterministic_and_equal_to_streamk_within_tolerance(ctx):
    print("packed determinism", flush=True)
    r = synth.rng(920)
    lens = r.integers(1, 2000, 64)
    case = make_case(O.I8_BLK, lens, seed=921, outlier_scale=8.0)
    pool = gpu_pool(ctx, case)
    _, a = run(ctx, pool, case, np.float16, sched=velokv.SCHED_PACKED)
    _, b = run(ctx, pool, case, np.float16, sched=velokv.SCHED_PACKED)
    assert np.array_equal(a, b)
    ctx.set_decode_kernel(velokv.DECODE_MFMA)
    try:
        pl, c = run(ctx, pool, case, np.float16, sched=velokv.SCHED_STREAM)
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
    assert pl["schedule"] == velokv.SCHED_STREAM
    ok, err, nbad = tol_check(a, c)
    assert ok, (err, nbad)
