"""GPU parity at the full shapes the measured kernels run (benchmark configurations 2, 3,
5 and the B=64 x 8k headline), on one layer of a full-size pool.

K/V are generated on the GPU (vk_fill_normal_f16), one sequence at a time, and
appended through vk_append; the exact fp16 inputs of a few sampled sequences are
downloaded and given to the oracle, which appends them into a compact layer of
its own and decodes those sequences. So each test checks, at full size:
  - the pool bytes (codes and scales) of the sampled sequences' blocks, bit for
    bit against the oracle's append of the same inputs;
  - the decode of the sampled sequences against the oracle, within the
    north-star tolerance, for every schedule the planner picks at that shape
    (AUTO) and the ones it can be forced to, with the plan asserted: the
    workgroup split of config 5 walks 256 blocks per wave (all four block-id
    windows), the headline 128.
kernels.metal:672-732 (paged_attention_flash_int8), 440-501, llama_cpu.rs:251-284.
"""
import numpy as np
import pytest

import pyoracle as O
import velokv
from velokv import synth
from cases import BS, HD, tol_check

pytestmark = pytest.mark.gpu


def build_pool(ctx, kv, lens, Hkv, n_blocks, seed, sample, outlier_scale):
    """One-layer pool holding len(lens) sequences; returns (pool, block tables,
    {s: (k, v)} fp16 inputs of the sampled sequences)."""
    pages = [-(-int(L) // BS) for L in lens]
    bt = synth.scatter_block_tables(n_blocks, pages, seed, stride=max(pages))
    pool = velokv.Pool(ctx, 1, n_blocks, BS, Hkv, HD, kv)
    row = Hkv * HD
    Lmax = int(max(lens))
    kbuf, vbuf = ctx.alloc(Lmax * row * 2), ctx.alloc(Lmax * row * 2)
    inputs = {}
    for s, L in enumerate(lens):
        L = int(L)
        ctx.fill_normal_f16(kbuf, L * row, seed * 7919 + 2 * s, row, outlier_scale)
        ctx.fill_normal_f16(vbuf, L * row, seed * 7919 + 2 * s + 1, row, outlier_scale)
        sl = synth.slots_for_positions(bt, np.arange(L), BS, np.full(L, s))
        ctx.append(pool, 0, kbuf, vbuf, velokv.DT_F16, ctx.upload(sl), L)
        if s in sample:
            inputs[s] = (kbuf.download((L, Hkv, HD), np.float16), vbuf.download((L, Hkv, HD), np.float16))
    ctx.sync()
    return pool, bt, inputs


def oracle_sample(kv, Hkv, lens, inputs, sample):
    """The oracle's own append of the sampled sequences into a compact layer
    (block j of sample i is block i * P + j)."""
    P = max(-(-int(lens[s]) // BS) for s in sample)
    lay = O.Layer(len(sample) * P, Hkv, BS, HD, kv)
    cbt = np.arange(len(sample) * P, dtype=np.int32).reshape(len(sample), P)
    for i, s in enumerate(sample):
        L = int(lens[s])
        k, v = inputs[s]
        O.append(lay, k, v, synth.slots_for_positions(cbt, np.arange(L), BS, np.full(L, i)))
    return lay, cbt


def check_pool_bytes(pool, kv, Hkv, bt, lens, lay, cbt, sample):
    got = pool.download_layer(0)
    esz = O.ESZ[kv]
    blk_bytes = Hkv * BS * HD * esz
    for key in ("k", "v", "ks", "vs"):
        ref = getattr(lay, key)
        if ref is None:
            continue
        per = blk_bytes if key in ("k", "v") else ref.size // lay.n_blocks
        g = got[key].reshape(-1, per)
        r = ref.reshape(-1, per)
        for i, s in enumerate(sample):
            n = -(-int(lens[s]) // BS)
            assert np.array_equal(g[bt[s, :n]], r[cbt[i, :n]]), f"{key} bytes of sequence {s} differ"


def decode(ctx, pool, q, lens, bt, H, qd, **kw):
    S = len(lens)
    out = ctx.alloc(S * H * HD * 4)
    ctx.paged_decode(pool, 0, ctx.upload(q.astype(qd)), velokv.DT_F32 if qd == np.float32 else velokv.DT_F16, out,
       ctx.upload(np.asarray(lens, np.int32)), S, H, int(max(lens)), block_tables=ctx.upload(bt),
       bt_stride=bt.shape[1], **kw)
    ctx.sync()
    return out.download((S, H, HD), np.float32)


def plan(ctx, pool, lens, H, bt, qd, **kw):
    return ctx.decode_plan(pool, len(lens), H, int(max(lens)), bt_stride=bt.shape[1],
                           q_dtype=velokv.DT_F32 if qd == np.float32 else velokv.DT_F16, **kw)


def with_schedule(ctx, kind, sched):
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sched)


def restore(ctx):
    ctx.set_decode_kernel(velokv.DECODE_AUTO)
    ctx.set_decode_schedule(velokv.SCHED_AUTO)


def run_variants(ctx, pool, bt, lens, H, q, lay, cbt, sample, variants):
    """variants: (label, kind, sched, partition_tokens, q dtype, expected kernel, check(plan))."""
    refs = {}
    for label, kind, sched, P, qd, want, pcheck in variants:
        print(f"  {label}", flush=True)
        with_schedule(ctx, kind, sched)
        try:
            kw = dict(partition_tokens=P, sum_context_len=int(np.sum(lens)))
            pl = plan(ctx, pool, lens, H, bt, qd, **kw)
            assert pl["kernel"] == want, (label, pl)
            pcheck(pl)
            got = decode(ctx, pool, q, lens, bt, H, qd, **kw)
        finally:
            restore(ctx)
        if qd not in refs:
            refs[qd] = O.paged_decode(lay, q[sample].astype(qd), cbt, np.asarray(lens)[sample])
        ok, err, nbad = tol_check(got[sample], refs[qd])
        assert ok, f"{label}: max err {err:.3g}, {nbad} elements out of tolerance"
        print(f"    max abs err {err:.3g} plan={pl}", flush=True)


MFMA, VALU = velokv.DECODE_MFMA, velokv.DECODE_VALU
AUTO_K, AUTO_S = velokv.DECODE_AUTO, velokv.SCHED_AUTO
SPLIT, STREAM, PACKED = velokv.SCHED_SPLIT, velokv.SCHED_STREAM, velokv.SCHED_PACKED


@pytest.fixture(scope="module")
def config5(ctx):
    """Config 5, one GPU's share: 32 sequences x 32768 tokens, 64 / 8 heads, INT8
    per-(block, head) scales, a 65,536-block pool (all of it used), seeded scatter."""
    print("config5: building a 65536-block INT8 layer (32 x 32768 tokens)", flush=True)
    S, L, Hkv = 32, 32768, 8
    lens = np.full(S, L, np.int32)
    sample = [0, 9, 22, 31]
    pool, bt, inputs = build_pool(ctx, O.I8_BLK, lens, Hkv, S * L // BS, seed=55, sample=sample, outlier_scale=8.0)
    lay, cbt = oracle_sample(O.I8_BLK, Hkv, lens, inputs, sample)
    yield pool, bt, lens, lay, cbt, sample
    pool.close()


def test_config5_pool_bytes_bit_exact(ctx, config5):
    pool, bt, lens, lay, cbt, sample = config5
    check_pool_bytes(pool, O.I8_BLK, 8, bt, lens, lay, cbt, sample)


def test_config5_decode_all_schedules(ctx, config5):
    pool, bt, lens, lay, cbt, sample = config5
    H = 64
    q = synth.normals_f16(len(lens) * H * HD, 5501).reshape(len(lens), H, HD)

    def wg256(pl):
        assert pl["schedule"] == velokv.SCHED_WORKGROUP and pl["wg_waves"] == 8 and pl["max_blocks_per_wave"] == 256
        assert not pl["merge_launch"] and pl["workspace_bytes"] == 0

    def sk_past_window_2(pl):
        assert pl["schedule"] == velokv.SCHED_STREAM and 192 < pl["max_blocks_per_wave"] <= 256, pl

    def split4096(pl):
        assert pl["partition_tokens"] == 4096 and pl["max_partitions"] == 8 and pl["max_blocks_per_wave"] == 256

    run_variants(ctx, pool, bt, lens, H, q, lay, cbt, sample, [
        ("AUTO fp16 q", AUTO_K, AUTO_S, 0, np.float16, "vk_decode_wg_kv3_g8", wg256),
        ("AUTO fp32 q", AUTO_K, AUTO_S, 0, np.float32, "vk_decode_wg_kv3_g8_q0", wg256),
        ("stream-K fp16 q", MFMA, STREAM, 0, np.float16, "vk_decode_sk_kv3_g8", sk_past_window_2),
        ("stream-K fp32 q", MFMA, STREAM, 0, np.float32, "vk_decode_sk_kv3_g8_q0", sk_past_window_2),
        ("split-K P=4096 MFMA", MFMA, SPLIT, 4096, np.float16, "vk_decode_mfma_kv3_g8", split4096),
        ("split-K P=4096 VALU", VALU, SPLIT, 4096, np.float16, "vk_decode_kv3_g8_q1", split4096),
    ])


@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
def test_headline_b64_ctx8k(ctx, kv):
    """The metric's workload: 64 sequences x 8192 tokens, 32 / 8 heads, AUTO
    (INT8: workgroup split, 4 waves of 128 blocks; fp16: dot2 split-K + merge)."""
    print(f"headline kv={kv}", flush=True)
    S, L, Hkv, H = 64, 8192, 8, 32
    lens = np.full(S, L, np.int32)
    sample = [0, 21, 42, 63]
    pool, bt, inputs = build_pool(ctx, kv, lens, Hkv, 40000, seed=56, sample=sample,
                                  outlier_scale=8.0 if kv == O.I8_BLK else 1.0)
    try:
        lay, cbt = oracle_sample(kv, Hkv, lens, inputs, sample)
        check_pool_bytes(pool, kv, Hkv, bt, lens, lay, cbt, sample)
        q = synth.normals_f16(S * H * HD, 5601).reshape(S, H, HD)
        if kv == O.I8_BLK:
            def wg128(pl):
                assert pl["schedule"] == velokv.SCHED_WORKGROUP and pl["wg_waves"] == 4
                assert pl["max_blocks_per_wave"] == 128
            variants = [("AUTO fp16 q", AUTO_K, AUTO_S, 0, np.float16, "vk_decode_wg_kv3_g4", wg128),
                        ("AUTO fp32 q", AUTO_K, AUTO_S, 0, np.float32, "vk_decode_wg_kv3_g4_q0", wg128)]
        else:
            def split(pl):
                assert pl["schedule"] == velokv.SCHED_SPLIT and pl["merge_launch"], pl
            variants = [("AUTO fp16 q", AUTO_K, AUTO_S, 0, np.float16, "vk_decode_kv1_g4_q1", split),
                        ("AUTO fp32 q", AUTO_K, AUTO_S, 0, np.float32, "vk_decode_mfma_kv1_g4_q0", split)]
        run_variants(ctx, pool, bt, lens, H, q, lay, cbt, sample, variants)
    finally:
        pool.close()


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_config2_3_full_batch_auto(ctx, kv):
    """Configs 2 (fp16) and 3 (INT8, 1 % outlier channels x8): 64 sequences with
    L ~ U[1024, 8192] in a 40k-block pool: AUTO (stream-K + merge at full batch)
    and the packed workgroup split."""
    print(f"config2/3 full batch kv={kv}", flush=True)
    r = synth.rng(303)
    lens = r.integers(1024, 8193, 64).astype(np.int32)
    lens[5], lens[17] = 8192, 1024
    sample = [5, 17, 40, 63]
    pool, bt, inputs = build_pool(ctx, kv, lens, 8, 40000, seed=57, sample=sample,
                                  outlier_scale=8.0 if kv == O.I8_BLK else 1.0)
    try:
        lay, cbt = oracle_sample(kv, 8, lens, inputs, sample)
        check_pool_bytes(pool, kv, 8, bt, lens, lay, cbt, sample)
        q = synth.normals_f16(64 * 32 * HD, 5701).reshape(64, 32, HD)

        def pk(pl):
            assert pl["schedule"] == velokv.SCHED_PACKED and not pl["merge_launch"], pl
            assert pl["workspace_bytes"] == 0 and pl["max_blocks_per_wave"] <= 256, pl

        def sk(pl):
            assert pl["schedule"] == velokv.SCHED_STREAM and pl["merge_launch"], pl
        run_variants(ctx, pool, bt, lens, 32, q, lay, cbt, sample, [
            ("AUTO fp16 q", AUTO_K, AUTO_S, 0, np.float16, f"vk_decode_sk_kv{kv}_g4", sk),
            ("AUTO fp32 q", AUTO_K, AUTO_S, 0, np.float32, f"vk_decode_sk_kv{kv}_g4_q0", sk),
            ("packed fp16 q", MFMA, PACKED, 0, np.float16, f"vk_decode_pk_kv{kv}_g4", pk),
            ("packed fp32 q", MFMA, PACKED, 0, np.float32, f"vk_decode_pk_kv{kv}_g4_q0", pk),
        ])
    finally:
        pool.close()
