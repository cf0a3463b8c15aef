"""Configuration-1 known answers committed under tests/golden/ (written by
tests/golden/make_golden.py): the oracle must keep reproducing them on the CPU,
and the HIP path must match them (bit-exact pool bytes, decode within the
north-star tolerance) on the GPU."""
import hashlib
import os

import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer, tol_check

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "config1.npz"), allow_pickle=False)
KV_NAMES = {O.F32: "f32", O.F16: "f16", O.I8_REF: "i8ref", O.I8_BLK: "i8blk"}
SEED = 101


def config1(kv):
    return make_case(kv, [512], n_blocks=64, seed=SEED)


def digest(arrays):
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def test_inputs_regenerate_bit_exactly():
    case = config1(O.F16)
    assert np.array_equal(case.block_tables, G["bt"])
    assert np.array_equal(case.ctx_lens, G["ctx_len"])
    assert np.array_equal(case.q, G["q"])
    assert hashlib.sha256(case.k[0].tobytes()).hexdigest() == str(G["k_sha256"])
    assert hashlib.sha256(case.v[0].tobytes()).hexdigest() == str(G["v_sha256"])


def test_f32_to_f16_vectors():
    bits = np.array([O.f32_to_f16(float(x)) for x in G["f32_in"]], dtype=np.uint16)
    assert np.array_equal(bits, G["f16_bits"])


@pytest.mark.parametrize("kv", list(KV_NAMES))
def test_oracle_reproduces_golden(kv):
    name = KV_NAMES[kv]
    case = config1(kv)
    layer = oracle_layer(case)
    assert digest([layer.k, layer.v, layer.ks, layer.vs]) == str(G[f"pool_sha256_{name}"])
    out = O.paged_decode(layer, case.q, case.block_tables, case.ctx_lens)
    assert np.array_equal(out, G[f"out_{name}"])


@pytest.mark.gpu
@pytest.mark.parametrize("kv", list(KV_NAMES))
def test_gpu_matches_golden(ctx, kv):
    print(f"golden config1 kv={kv}", flush=True)
    name = KV_NAMES[kv]
    case = config1(kv)
    pool = velokv.Pool(ctx, 1, case.n_blocks, BS, case.n_kv_heads, HD, kv)
    sl, kk, vv = case.prefill_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    sl, kk, vv = case.last_slots()
    ctx.append(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    ctx.sync()
    got = pool.download_layer(0)
    assert digest([got["k"], got["v"], got["ks"], got["vs"]]) == str(G[f"pool_sha256_{name}"])
    out = ctx.alloc(32 * HD * 4)
    ctx.paged_decode(pool, 0, ctx.upload(np.ascontiguousarray(G["q"])), velokv.DT_F16, out,
                     ctx.upload(G["ctx_len"]), 1, 32, 512, block_tables=ctx.upload(G["bt"]), bt_stride=G["bt"].shape[1])
    ctx.sync()
    ok, err, nbad = tol_check(out.download((1, 32, HD), np.float32), G[f"out_{name}"])
    assert ok, f"max err {err:.3g}, {nbad} out of tolerance"
