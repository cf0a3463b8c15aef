"""GPU parity over fp32 KV pools (the reference's default KvCacheType::Fp32,
metal/runtime.rs:28; kernels.metal:440-501 reads fp32 K/V, llama_cpu.rs:251-284
computes in fp32): decode on every schedule (fixed partitions on the matrix
cores and on the VALU, stream-K, workgroup split), any GQA group size, and tree
verify, each against the oracle. With fp32 K, V and q the matrix-core kernels
(v_mfma_f32_16x16x4f32) keep every operand in fp32, so the bound here is far
tighter than the north-star tolerance: |err| <= 2e-5 + 2e-4 |ref|."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu

F32_TOL = dict(atol=2e-5, rtol=2e-4)

SCHEDS = {"split": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0),
          "split-p64": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 64),
          "stream": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0),
          "valu": (velokv.DECODE_VALU, velokv.SCHED_SPLIT, 0),
          "auto": (velokv.DECODE_AUTO, velokv.SCHED_AUTO, 0)}


def decode(ctx, pool, case, q, qdt, kind, sched, P):
    S, H = case.S, case.n_heads
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sched)
    try:
        bt = case.block_tables
        pl = ctx.decode_plan(pool, S, H, int(case.ctx_lens.max()), bt_stride=bt.shape[1], partition_tokens=P,
                             q_dtype=qdt)
        out = ctx.alloc(S * H * HD * 4)
        ctx.paged_decode(pool, 0, ctx.upload(q), qdt, out, ctx.upload(case.ctx_lens), S, H, int(case.ctx_lens.max()),
                         block_tables=ctx.upload(bt), bt_stride=bt.shape[1], partition_tokens=P)
        ctx.sync()
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    return pl, out.download((S, H, HD), np.float32)


def fp32_q(S, H, seed):
    return (synth.rng(seed).standard_normal((S, H, HD)) * 0.7).astype(np.float32)


@pytest.mark.parametrize("G", [1, 2, 4, 8, 3, 12, 32])
@pytest.mark.parametrize("sched", list(SCHEDS))
def test_fp32_decode_every_schedule(ctx, G, sched):
    print(f"fp32 KV decode G={G} sched={sched}", flush=True)
    kind, sc, P = SCHEDS[sched]
    if sched == "valu" and G not in (1, 2, 4, 8):
        pytest.skip("the VALU kernels take group sizes 1, 2, 4, 8")
    Hkv = 2
    lens = [1, 15, 16, 17, 255, 1000, 2500]
    case = make_case(O.F32, lens, n_kv_heads=Hkv, n_heads=Hkv * G, seed=1200 + G, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = fp32_q(case.S, case.n_heads, 1210 + G)
    pl, got = decode(ctx, pool, case, q, velokv.DT_F32, kind, sc, P)
    if kind != velokv.DECODE_VALU:
        assert "_kv0_" in pl["kernel"] and ("mfma" in pl["kernel"] or "_sk_" in pl["kernel"]), pl
    ref = O.paged_decode(ref_layer, q, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref, **F32_TOL)
    assert ok, f"{sched} ({pl['kernel']}): max err {err:.3g}, {nbad} out of the fp32 bound"


@pytest.mark.parametrize("S,G", [(64, 4), (32, 8), (128, 1)])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_fp32_decode_workgroup_split(ctx, S, G, qd):
    """Batches that fill the GPU take the workgroup split over fp32 KV."""
    print(f"fp32 KV workgroup split S={S} G={G}", flush=True)
    Hkv = 8
    lens = synth.rng(1220 + S).integers(0, 900, S)
    lens[:5] = [0, 1, 16, 17, 33]
    case = make_case(O.F32, [max(1, int(L)) for L in lens], n_kv_heads=Hkv, n_heads=Hkv * G, seed=1221 + S,
                     outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    case.ctx_lens = np.asarray(lens, np.int32)
    qdt = velokv.DT_F32 if qd == np.float32 else velokv.DT_F16
    q = fp32_q(S, case.n_heads, 1222 + S).astype(qd)
    pl, got = decode(ctx, pool, case, q, qdt, velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0)
    assert pl["kernel"].startswith(f"vk_decode_wg_kv0_g{G}"), pl
    assert pl["workspace_bytes"] == 0, pl
    ref = O.paged_decode(ref_layer, q, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, ref, **F32_TOL)
    assert ok, f"max err {err:.3g}, {nbad} out of the fp32 bound"
    assert np.all(got[lens == 0] == 0.0)


def test_fp32_matrix_cores_equal_fp32_valu(ctx):
    """The two fp32 kernel families agree to fp32 rounding."""
    print("fp32 KV mfma vs valu", flush=True)
    lens = list(synth.rng(1230).integers(1, 3000, 12))
    case = make_case(O.F32, lens, seed=1231, outlier_scale=8.0)
    pool = gpu_pool(ctx, case)
    q = fp32_q(case.S, case.n_heads, 1232)
    _, a = decode(ctx, pool, case, q, velokv.DT_F32, velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0)
    _, b = decode(ctx, pool, case, q, velokv.DT_F32, velokv.DECODE_VALU, velokv.SCHED_SPLIT, 0)
    ok, err, nbad = tol_check(a, b, **F32_TOL)
    assert ok, (err, nbad)


@pytest.mark.parametrize("G,N", [(4, 8), (1, 32), (8, 3), (4, 16), (6, 5)])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_fp32_tree_verify(ctx, G, N, qd):
    """Tree verify over an fp32 pool: one or two 16-row tiles per wave, random
    masks, a row that sees nothing at context 0."""
    print(f"fp32 KV tree G={G} N={N} q={np.dtype(qd).name}", flush=True)
    Hkv = 2
    committed = np.array([0, 7, 100, 1500], np.int32)
    case = make_case(O.F32, committed + N, n_kv_heads=Hkv, n_heads=Hkv * G, seed=1240 + G + N, outlier_scale=8.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = fp32_q(case.S * N, case.n_heads, 1241 + N).reshape(case.S, N, case.n_heads, HD).astype(qd)
    full = (1 << N) - 1 if N < 32 else 0xFFFFFFFF
    mask = synth.rng(1242 + N).integers(0, 1 << 32, size=(case.S, N), dtype=np.uint64).astype(np.uint32)
    mask = (mask & np.uint32(full)) | (np.uint32(1) << np.arange(N, dtype=np.uint32))
    mask[0, 0] = 0
    out = ctx.alloc(q.size * 4)
    ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F32 if qd == np.float32 else velokv.DT_F16, out,
                    ctx.upload(committed), ctx.upload(mask), case.S, N, case.n_heads, int(committed.max()),
                    block_tables=ctx.upload(case.block_tables), bt_stride=case.block_tables.shape[1])
    ctx.sync()
    got = out.download(q.shape, np.float32)
    ref = O.tree_verify(ref_layer, q, case.block_tables, committed, mask)
    ok, err, nbad = tol_check(got, ref, **F32_TOL)
    assert ok, f"max err {err:.3g}, {nbad} out of the fp32 bound"
    assert np.all(got[0, 0] == 0.0)
