"""vk_paged_decode_noalloc (the decode entry point that allocates nothing; its
split-K scratch is the library's fixed per-device array) against vk_paged_decode
through the C ABI: two calls in a row, the second with a smaller input, for the
stream-K schedule (ragged batches) and fixed split-K partitions, both of which
keep partials in the scratch; outputs must equal vk_paged_decode's bit for bit
(same kernels, same schedule) and the oracle's within the north-star tolerance.
Also: a caller workspace is refused, and a call whose scratch would exceed the
array is refused before anything is launched."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import gpu_pool

pytestmark = pytest.mark.gpu


def _run(ctx, pool, case, S, noalloc, P=0):
    out = ctx.alloc(S * case.n_heads * HD * 4)
    fn = ctx.paged_decode_noalloc if noalloc else ctx.paged_decode
    fn(pool, 0, ctx.upload(case.q[:S]), velokv.DT_F16, out, ctx.upload(case.ctx_lens[:S]), S, case.n_heads,
       int(case.ctx_lens[:S].max()), block_tables=ctx.upload(case.block_tables), bt_stride=case.block_tables.shape[1],
       partition_tokens=P)
    ctx.sync()
    return out.download((S, case.n_heads, HD), np.float32)


@pytest.mark.parametrize("kv", [velokv.KV_F16, velokv.KV_I8_BLK])
@pytest.mark.parametrize("sched,P", [(velokv.SCHED_STREAM, 0), (velokv.SCHED_SPLIT, 256)])
def test_noalloc_decode_equals_decode_two_calls(ctx, kv, sched, P):
    print(f"noalloc decode kv={kv} sched={sched} P={P}", flush=True)
    lens = [2000, 37, 1300, 4100, 16, 999, 2500, 3]
    case = make_case(kv, lens, seed=611, outlier_scale=8.0 if kv == velokv.KV_I8_BLK else 1.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    ref = O.paged_decode(ref_layer, case.q, case.block_tables, case.ctx_lens)
    ctx.set_decode_kernel(velokv.DECODE_MFMA)
    ctx.set_decode_schedule(sched)
    try:
        for S in (8, 3):  # the second call is smaller: the scratch keeps the first call's partials
            pl = ctx.decode_plan(pool, S, case.n_heads, int(case.ctx_lens[:S].max()),
                                 bt_stride=case.block_tables.shape[1], partition_tokens=P)
            assert 0 < pl["workspace_bytes"] <= velokv.NOALLOC_SCRATCH_BYTES, pl
            want = _run(ctx, pool, case, S, noalloc=False, P=P)
            got = _run(ctx, pool, case, S, noalloc=True, P=P)
            assert np.array_equal(got, want), f"S={S}: noalloc output differs from vk_paged_decode"
            ok, err, nbad = tol_check(got, ref[:S])
            assert ok, f"S={S}: max err {err:.3g}, {nbad} out of tolerance"
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)


def test_noalloc_refuses_workspace_and_oversized_calls(ctx):
    print("noalloc refusals", flush=True)
    case = make_case(velokv.KV_I8_BLK, [64], seed=612)
    pool = gpu_pool(ctx, case)
    # a caller workspace: the entry point takes its scratch from the library
    import ctypes as C
    from velokv import _capi
    buf = ctx.alloc(1 << 20)
    out = ctx.alloc(32 * HD * 4)
    a = _capi.DecodeArgs(0, C.c_void_p(ctx.upload(case.q).ptr), velokv.DT_F16, C.c_void_p(out.ptr),
                         C.c_void_p(ctx.upload(case.block_tables).ptr), case.block_tables.shape[1], None,
                         C.c_void_p(ctx.upload(case.ctx_lens).ptr), 1, 32, 64, 0.0, 0, C.c_void_p(buf.ptr), 1 << 20, 0)
    rc = _capi.lib().vk_paged_decode_noalloc(ctx.h, pool.h, C.byref(a), None)
    assert rc == velokv.ERR_BAD_ARG
    # 64 sequences x 8192 tokens in 16-token partitions: 512 MiB of partials
    big = velokv.Pool(ctx, 1, 64 * 512, 16, 8, HD, velokv.KV_I8_BLK)
    try:
        need = ctx.decode_plan(big, 64, 32, 8192, bt_stride=512, partition_tokens=16)["workspace_bytes"]
        assert need > velokv.NOALLOC_SCRATCH_BYTES
        bt = np.zeros((64, 512), np.int32)
        with pytest.raises(velokv.VkError) as e:
            ctx.paged_decode_noalloc(big, 0, ctx.alloc(64 * 32 * HD * 2), velokv.DT_F16, ctx.alloc(64 * 32 * HD * 4),
                                     ctx.upload(np.full(64, 8192, np.int32)), 64, 32, 8192,
                                     block_tables=ctx.upload(bt), bt_stride=512, partition_tokens=16)
        assert e.value.code == velokv.ERR_BAD_ARG and "scratch" in str(e.value)
    finally:
        big.close()
