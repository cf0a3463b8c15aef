"""GPU parity of the fused RoPE + append (vk_append_rope): pool bytes and the
rotated q must equal the oracle's bit for bit (same table, fp32 rotation with
every product and sum rounded separately)."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, tol_check
from test_gpu_append_copy import assert_layer_equal
from velokv import synth

pytestmark = pytest.mark.gpu

KV_ALL = [O.F32, O.F16, O.I8_REF, O.I8_BLK]
STYLES = [O.ROPE_INTERLEAVED, O.ROPE_HALF]


def run_case(ctx, kv, style, in_dtype, q_dtype, lens, seed, n_pos=None, bad_pos=()):
    case = make_case(kv, lens, n_kv_heads=4, n_heads=8, seed=seed, outlier_scale=8.0)
    # one call with every token of every sequence, sequence by sequence (the
    # tokens of one block stay adjacent, as vk_append requires)
    rows = np.concatenate([np.full(int(L), s) for s, L in enumerate(case.ctx_lens)])
    cpos = np.concatenate([np.arange(int(L)) for L in case.ctx_lens])
    sl = synth.slots_for_positions(case.block_tables, cpos, BS, rows)
    kk = np.concatenate([case.k[s] for s in range(case.S)]).astype(in_dtype)
    vv = np.concatenate([case.v[s] for s in range(case.S)]).astype(in_dtype)
    pos = (cpos + 3).astype(np.int32)  # positions need not equal cache slots (e.g. after a shared prefix)
    for i in bad_pos:
        pos[i] = -1 if i % 2 else 10 ** 6
    n_pos = n_pos or int(pos.max()) + 1
    table = velokv.rope_table(n_pos, HD, 500000.0)
    q = synth.normals_f16(len(sl) * 8 * HD, seed + 5).reshape(len(sl), 8, HD).astype(q_dtype)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, 4, HD, kv)
    dq = ctx.upload(q)
    ctx.append_rope(pool, 0, ctx.upload(kk), ctx.upload(vv),
                    velokv.DT_F16 if in_dtype == np.float16 else velokv.DT_F32, ctx.upload(pos), ctx.upload(sl),
                    len(sl), ctx.upload(table), n_pos, style, q=dq,
                    q_dtype=velokv.DT_F16 if q_dtype == np.float16 else velokv.DT_F32, n_heads=8)
    ctx.sync()
    ref = O.Layer(case.n_blocks, 4, BS, HD, kv)
    ref_q = O.append_rope(ref, kk, vv, sl, pos, style, table, q=q)
    got_q = dq.download(q.shape, q_dtype)
    return case, pool, ref, ref_q, got_q, rows


@pytest.mark.parametrize("style", STYLES)
@pytest.mark.parametrize("kv", KV_ALL)
def test_append_rope_bit_exact(ctx, kv, style):
    print(f"append rope kv={kv} style={style}", flush=True)
    case, pool, ref, ref_q, got_q, _ = run_case(ctx, kv, style, np.float16, np.float16, [1, 15, 16, 17, 100, 257],
                                                seed=201 + kv)
    assert_layer_equal(pool, 0, ref)
    assert np.array_equal(got_q.view(np.uint16), ref_q.view(np.uint16))


@pytest.mark.parametrize("style", STYLES)
def test_append_rope_fp32_inputs_and_q(ctx, style):
    print(f"append rope fp32 style={style}", flush=True)
    case, pool, ref, ref_q, got_q, _ = run_case(ctx, O.I8_BLK, style, np.float32, np.float32, [40, 70], seed=211)
    assert_layer_equal(pool, 0, ref)
    assert np.array_equal(got_q, ref_q)


def test_append_rope_positions_outside_the_table_are_skipped(ctx):
    print("append rope bad positions", flush=True)
    case, pool, ref, ref_q, got_q, _ = run_case(ctx, O.F16, O.ROPE_HALF, np.float16, np.float16, [30, 40], seed=221,
                                                bad_pos=(0, 5, 33, 69))
    assert_layer_equal(pool, 0, ref)
    assert np.array_equal(got_q.view(np.uint16), ref_q.view(np.uint16))


def test_append_rope_then_decode(ctx):
    """Attention over rotated keys: decode with a rotated q equals the oracle's."""
    print("append rope then decode", flush=True)
    kv = O.I8_BLK
    case, pool, ref, ref_q, got_q, rows = run_case(ctx, kv, O.ROPE_HALF, np.float16, np.float16, [64, 300, 129],
                                                   seed=231)
    last = np.cumsum(case.ctx_lens) - 1  # q rows of the last token of every sequence
    q = np.ascontiguousarray(got_q[last])
    out = ctx.alloc(q.size * 4)
    ctx.paged_decode(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S, 8,
                     int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                     bt_stride=case.block_tables.shape[1])
    ctx.sync()
    got = out.download(q.shape, np.float32)
    want = O.paged_decode(ref, q, case.block_tables, case.ctx_lens)
    ok, err, nbad = tol_check(got, want)
    assert ok, (err, nbad)


def test_append_rope_rejects_bad_arguments(ctx):
    pool = velokv.Pool(ctx, 1, 8, BS, 4, HD, O.F16)
    buf = ctx.alloc(1 << 16)
    for style, n_pos in ((0, 16), (3, 16), (O.ROPE_HALF, 0)):
        with pytest.raises(velokv.VkError) as e:
            ctx.append_rope(pool, 0, buf, buf, velokv.DT_F16, buf, buf, 1, buf, n_pos, style)
        assert e.value.code == velokv.ERR_BAD_ARG
    with pytest.raises(velokv.VkError) as e:  # the table is read in 16-byte chunks
        ctx.append_rope(pool, 0, buf, buf, velokv.DT_F16, buf, buf, 1, buf.ptr + 8, 16, O.ROPE_INTERLEAVED)
    assert e.value.code == velokv.ERR_BAD_ARG and "aligned" in str(e.value)
