"""GPU parity of the append (kv_update / kv_update_int8 and the per-block INT8
mode) and of the copy-on-write block copy: pool bytes must equal the oracle's
bit for bit."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer, ref_codes_closed_form
from velokv import synth

pytestmark = pytest.mark.gpu

KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]


def gpu_pool(ctx, case, n_layer=1, layer=0, in_dtype=np.float16, with_last=True):
    pool = velokv.Pool(ctx, n_layer, case.n_blocks, BS, case.n_kv_heads, HD, case.kv_type)
    sl, kk, vv = case.prefill_slots()
    if len(sl):
        ctx.append(pool, layer, ctx.upload(kk.astype(in_dtype)), ctx.upload(vv.astype(in_dtype)),
                   velokv.DT_F16 if in_dtype == np.float16 else velokv.DT_F32, ctx.upload(sl), len(sl))
    if with_last:
        sl, kk, vv = case.last_slots()
        ctx.append(pool, layer, ctx.upload(kk.astype(in_dtype)), ctx.upload(vv.astype(in_dtype)),
                   velokv.DT_F16 if in_dtype == np.float16 else velokv.DT_F32, ctx.upload(sl), len(sl))
    ctx.sync()
    return pool


def assert_layer_equal(pool, layer_idx, ref: O.Layer):
    got = pool.download_layer(layer_idx)
    for key in ("k", "v", "ks", "vs"):
        r = getattr(ref, key)
        if r is None:
            assert got[key] is None
            continue
        if not np.array_equal(got[key], r):
            bad = np.nonzero(got[key] != r)[0]
            raise AssertionError(f"{key}: {len(bad)} bytes differ, first at {bad[:8]}")


@pytest.mark.parametrize("kv", KV_ALL)
def test_append_bit_exact_config1(ctx, kv):
    print(f"append config1 kv={kv}", flush=True)
    # benchmark configuration 1: 32 blocks permuted within a 64-block pool, context 512
    case = make_case(kv, [512], n_blocks=64, seed=101)
    ref = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("kv", KV_ALL)
def test_append_bit_exact_ragged_batch_with_outliers(ctx, kv):
    print(f"append ragged kv={kv}", flush=True)
    lens = [1, 2, 15, 16, 17, 31, 33, 200, 257]
    case = make_case(kv, lens, seed=102, outlier_scale=8.0)
    ref = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("kv", [O.F32, O.I8_REF, O.I8_BLK, O.F16])
def test_append_fp32_input(ctx, kv):
    # the reference's kv_update / kv_update_int8 take fp32 K/V
    print(f"append fp32-in kv={kv}", flush=True)
    case = make_case(kv, [40, 70], seed=103)
    r = np.random.default_rng(5)
    case.k = [(r.standard_normal(k.shape) * 3).astype(np.float32) for k in case.k]
    case.v = [(r.standard_normal(v.shape) * 3).astype(np.float32) for v in case.v]
    ref = oracle_layer(case)
    pool = gpu_pool(ctx, case, in_dtype=np.float32)
    assert_layer_equal(pool, 0, ref)


def test_append_blk_token_by_token_equals_one_call(ctx):
    """Sequential semantics: one call with all tokens == one call per token."""
    print("append blk split", flush=True)
    case = make_case(O.I8_BLK, [77], seed=104, outlier_scale=8.0)
    pool_a = gpu_pool(ctx, case)
    pool_b = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, O.I8_BLK)
    sl = synth.slots_for_positions(case.block_tables, np.arange(77), BS, np.zeros(77, int))
    for t in range(77):
        ctx.append(pool_b, 0, ctx.upload(case.k[0][t:t + 1]), ctx.upload(case.v[0][t:t + 1]), velokv.DT_F16,
                   ctx.upload(sl[t:t + 1]), 1)
    ctx.sync()
    a, b = pool_a.download_layer(0), pool_b.download_layer(0)
    for key in ("k", "v", "ks", "vs"):
        assert np.array_equal(a[key], b[key])


@pytest.mark.parametrize("gap", [0, 5, 70, 130])
def test_append_blk_runs_with_padding_windows(ctx, gap):
    """Runs whose tokens are separated by `gap` padding slots (more than one
    64-slot window when gap >= 64), a run of a whole block (16 tokens in a row),
    and a run that restarts its block at offset 0 (positions 16..19 then 16..23,
    adjacent in the call: more than one 16-token chunk). Tokens of one block stay
    adjacent in the call, as vk_append requires."""
    print(f"append blk padding gap={gap}", flush=True)
    case = make_case(O.I8_BLK, [64], n_kv_heads=2, n_heads=8, seed=106, outlier_scale=8.0)
    bt = case.block_tables
    pos = list(range(0, 20)) + list(range(16, 24)) + list(range(32, 40)) + list(range(48, 64))
    rows = np.zeros(len(pos), np.int64)
    slots = synth.slots_for_positions(bt, np.array(pos), BS, rows)
    k = np.stack([case.k[0][p] for p in pos])
    v = np.stack([case.v[0][p] for p in pos])
    # interleave `gap` padding slots after every token
    n = len(pos) * (gap + 1)
    sl = np.full(n, -1, np.int64)
    kk = np.zeros((n, 2, HD), np.float16)
    vv = np.zeros((n, 2, HD), np.float16)
    sl[::gap + 1], kk[::gap + 1], vv[::gap + 1] = slots, k, v
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 2, HD, O.I8_BLK)
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), n)
    ctx.sync()
    ref = O.Layer(case.n_blocks, 2, BS, HD, O.I8_BLK)
    O.append(ref, kk, vv, sl)
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("kv", KV_ALL)
def test_append_large_call_windows(ctx, kv):
    """A call of ~9000 tokens over 8 KV heads, so that each workgroup covers a
    window of several tokens (36 here): runs of every length that start and end
    anywhere relative to the windows, sprinkled padding slots, and an existing
    partial block that a run continues (its stored scale applies)."""
    print(f"append large call kv={kv}", flush=True)
    rng = synth.rng(808)
    lens = rng.integers(1, 200, 80)
    case = make_case(kv, [int(L) + 16 for L in lens], n_kv_heads=8, n_heads=32, seed=808, outlier_scale=8.0)
    bt = case.block_tables
    # first call: a few tokens per sequence (partial blocks); second call: the rest
    first = np.minimum(lens, rng.integers(0, 9, len(lens)))
    ref = O.Layer(case.n_blocks, 8, BS, HD, kv)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, kv)
    for part in (0, 1):
        sl, kk, vv = [], [], []
        for s_, L in enumerate(lens):
            lo, hi = (0, int(first[s_])) if part == 0 else (int(first[s_]), int(L))
            if hi <= lo:
                continue
            pos = np.arange(lo, hi)
            sl.append(synth.slots_for_positions(bt, pos, BS, np.full(len(pos), s_)))
            kk.append(case.k[s_][lo:hi])
            vv.append(case.v[s_][lo:hi])
        sl, kk, vv = np.concatenate(sl), np.concatenate(kk), np.concatenate(vv)
        if part == 1:  # padding slots at random places (tokens of one block stay adjacent in the call)
            pad = rng.random(len(sl)) < 0.05
            sl = sl.copy()
            sl[pad] = -1
        O.append(ref, kk, vv, sl)
        ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
        ctx.sync()
    assert_layer_equal(pool, 0, ref)


def test_append_skips_negative_slots_and_layers_are_separate(ctx):
    print("append negative slots / layers", flush=True)
    case = make_case(O.I8_BLK, [20], seed=105)
    pool = velokv.Pool(ctx, 3, case.n_blocks, BS, 8, HD, O.I8_BLK)
    sl, kk, vv = case.prefill_slots()
    sl = sl.copy()
    sl[3] = -1
    ctx.append(pool, 1, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    ctx.sync()
    ref = O.Layer(case.n_blocks, 8, BS, HD, O.I8_BLK)
    O.append(ref, kk, vv, sl)
    assert_layer_equal(pool, 1, ref)
    for other in (0, 2):
        got = pool.download_layer(other)
        assert not got["k"].any() and not got["ks"].any()


@pytest.mark.parametrize("kv", [O.F16, O.I8_REF, O.I8_BLK])
def test_append_skips_slots_past_the_pool(ctx, kv):
    """A slot at or past n_blocks * block_size is padding, also in the middle
    of a block's run (the run continues across it)."""
    print(f"append slots past the pool kv={kv}", flush=True)
    case = make_case(kv, [40], seed=106, outlier_scale=8.0)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, kv)
    sl, kk, vv = case.prefill_slots()
    bad = sl.copy()
    end = case.n_blocks * BS
    bad[5], bad[6], bad[21] = end, end + 17, 2 ** 40
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(bad), len(bad))
    ctx.sync()
    ref = O.Layer(case.n_blocks, 8, BS, HD, kv)
    O.append(ref, kk, vv, bad)  # the oracle skips the same slots
    assert_layer_equal(pool, 0, ref)


@pytest.mark.parametrize("in_dt", [np.float32, np.float16])
def test_append_ref_codes_equal_truncating_closed_form(ctx, in_dt):
    """The GPU REF append against the numpy fp32 statement of kv_update_int8
    (truncating cast, kernels.metal:783-797) directly, not only through the
    oracle: 1024 tokens x 8 heads, one per slot of a 64-block pool in random
    order, row magnitudes spread so truncation and rounding differ often."""
    print(f"append REF closed form in={np.dtype(in_dt).name}", flush=True)
    r = np.random.default_rng(12)
    n_blocks, Hkv = 64, 8
    n_tok = n_blocks * BS
    k = (r.standard_normal((n_tok, Hkv, HD)) * r.uniform(0.01, 50, (n_tok, Hkv, 1))).astype(in_dt)
    v = (r.standard_normal((n_tok, Hkv, HD)) * r.uniform(0.01, 50, (n_tok, Hkv, 1))).astype(in_dt)
    k[::7, :, 3] *= 8
    slots = r.permutation(n_tok).astype(np.int64)
    pool = velokv.Pool(ctx, 1, n_blocks, BS, Hkv, HD, O.I8_REF)
    ctx.append(pool, 0, ctx.upload(k), ctx.upload(v), velokv.DT_F16 if in_dt == np.float16 else velokv.DT_F32,
               ctx.upload(slots), n_tok)
    ctx.sync()
    got = pool.download_layer(0)
    lay = O.Layer(n_blocks, Hkv, BS, HD, O.I8_REF)
    lay.k[:], lay.v[:], lay.ks[:], lay.vs[:] = got["k"], got["v"], got["ks"], got["vs"]
    for is_v, src, sc in ((0, k, got["ks"]), (1, v, got["vs"])):
        want_c, want_s = ref_codes_closed_form(src.astype(np.float32))
        scales = sc.view(np.float32).reshape(n_blocks, Hkv, BS)
        for blk in range(n_blocks):
            for h in range(Hkv):
                tile = lay.tile_codes(is_v, blk, h)  # [BS][HD] int8
                toks = np.nonzero(slots // BS == blk)[0]
                offs = slots[toks] % BS
                assert np.array_equal(tile[offs], want_c[toks, h]), f"codes is_v={is_v} blk={blk} h={h}"
                assert np.array_equal(scales[blk, h, offs], want_s[toks, h]), f"scales is_v={is_v} blk={blk}"


def test_slot_mapping_kernel(ctx):
    print("slot mapping", flush=True)
    case = make_case(O.F16, [50, 90, 3], seed=106)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 8, HD, O.F16)
    rows = np.array([0, 1, 1, 2, 0, 1], np.int32)
    pos = np.array([0, 89, 16, 2, 49, 31], np.int32)
    bt = ctx.upload(case.block_tables)
    out = ctx.slot_mapping(pool, ctx.upload(pos), block_tables=bt, bt_stride=case.block_tables.shape[1],
                           seq_rows=ctx.upload(rows))
    got = out.download((6,), np.int64)
    ref = synth.slots_for_positions(case.block_tables, pos, BS, rows)
    assert np.array_equal(got, ref)


def test_bind_slot_writes_table_rows(ctx):
    print("bind_slot", flush=True)
    pool = velokv.Pool(ctx, 1, 64, BS, 8, HD, O.F16, max_slots=4, max_pages_per_slot=10)
    pool.bind_slot(2, [5, 9, 1])
    pool.bind_slot(0, list(range(10)))
    ptr, stride = pool.block_table()
    tb = velokv.DeviceBuffer(ctx, 4 * 10 * 4, ptr=ptr, owned=False).download((4, 10), np.int32)
    assert stride == 10
    assert tb[2].tolist() == [5, 9, 1] + [0] * 7
    assert tb[0].tolist() == list(range(10))
    with pytest.raises(velokv.VkError) as e:
        pool.bind_slot(1, list(range(11)))
    assert e.value.code == velokv.ERR_TOO_MANY_PAGES
    with pytest.raises(velokv.VkError):
        pool.bind_slot(4, [1])
    with pytest.raises(velokv.VkError):
        pool.bind_slot(1, [64])


@pytest.mark.parametrize("kv", KV_ALL)
def test_copy_blocks_bit_exact_all_layers(ctx, kv):
    print(f"copy_blocks kv={kv}", flush=True)
    case = make_case(kv, [100, 60], seed=107, n_blocks=40)
    n_layer = 3
    pool = velokv.Pool(ctx, n_layer, case.n_blocks, BS, 8, HD, kv)
    refs = []
    sl, kk, vv = case.prefill_slots()
    for layer in range(n_layer):
        k = (kk.astype(np.float32) * (layer + 1)).astype(np.float16)
        ctx.append(pool, layer, ctx.upload(k), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
        r = O.Layer(case.n_blocks, 8, BS, HD, kv)
        O.append(r, k, vv, sl)
        refs.append(r)
    used = set(case.block_tables[0, :7].tolist()) | set(case.block_tables[1, :4].tolist())
    free = [b for b in range(case.n_blocks) if b not in used]
    pairs = np.array([[case.block_tables[0, 6], free[0]], [case.block_tables[1, 3], free[1]],
                      [case.block_tables[0, 0], free[2]]], np.int32)
    ctx.copy_blocks(pool, pairs)
    ctx.sync()
    for layer in range(n_layer):
        O.copy_blocks(refs[layer], pairs)
        assert_layer_equal(pool, layer, refs[layer])


def test_copy_blocks_rejects_bad_pairs(ctx):
    pool = velokv.Pool(ctx, 1, 8, BS, 8, HD, O.F16)
    for bad in ([[0, 8]], [[0, 1], [2, 1]], [[0, 1], [1, 2]], [[-1, 2]]):
        with pytest.raises(velokv.VkError) as e:
            ctx.copy_blocks(pool, bad)
        assert e.value.code == velokv.ERR_BAD_ARG
