"""Pins of the CPU oracle (oracle/velokv_oracle.c) against known answers from the
reference's own tests, independent library routines (numpy float16, numpy
float64 attention), and invariants the mathematics fixes. CPU only."""
import numpy as np
import pytest

import pyoracle as O
from cases import BS, HD, make_case, oracle_layer, ref_codes_closed_form
from velokv import synth


# ---------------------------------------------------------------- fp16 ------

def test_f16_to_f32_reference_known_answers():
    # quant.rs:211-235 and 311-322
    assert O.f16_to_f32(0) == 0.0
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0xBC00) == -1.0
    assert O.f16_to_f32(0x0001) == 1.0 / (1 << 24)
    assert O.f16_to_f32(0x8001) == -(1.0 / (1 << 24))
    assert np.isinf(O.f16_to_f32(0x7C00)) and O.f16_to_f32(0x7C00) > 0
    assert np.isinf(O.f16_to_f32(0xFC00)) and O.f16_to_f32(0xFC00) < 0
    assert np.isnan(O.f16_to_f32(0x7C01))


def test_f16_to_f32_exhaustive_against_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _f16_all(xs):
    return np.array([O.f32_to_f16(float(x)) for x in xs], np.uint16)


def test_f32_to_f16_rne_against_numpy_wide_range():
    r = np.random.default_rng(7)
    x = (r.standard_normal(30000) * np.exp2(r.integers(-30, 18, 30000))).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504, 65519.996, 65520, 7e4, -7e4, 6.1035156e-05,
                                        5.9604645e-08, 2.9802322e-08, 2.98023259e-08, 1e-9, np.inf, -np.inf])])
    got = _f16_all(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_ties_to_even_at_every_midpoint_sample():
    # exact midpoints between adjacent fp16 values, normal and subnormal
    r = np.random.default_rng(8)
    lo = r.integers(0, 0x7BFF, 20000).astype(np.uint16)
    a = lo.view(np.float16).astype(np.float64)
    b = (lo + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((a + b) / 2).astype(np.float32)  # exact in fp32
    assert np.all(mid.astype(np.float64) == (a + b) / 2)
    got = _f16_all(mid)
    ref = mid.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    # ties go to the even neighbour
    assert np.all(got % 2 == 0)


def test_splitmix64_published_sequence():
    # SplitMix64 seeded with 0 (Steele, Lea & Flood): first outputs
    assert O.splitmix64(0) == 0xE220A8397B1DCDAF
    assert O.splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    assert O.splitmix64((2 * 0x9E3779B97F4A7C15) & (2**64 - 1)) == 0x06C45D188009454F
    # numpy restatement in velokv.synth agrees
    xs = np.array([0, 1, 12345, 2**63 + 5], np.uint64)
    assert [int(v) for v in synth.splitmix64(xs)] == [O.splitmix64(int(v)) for v in xs]


# ------------------------------------------------- reference INT8 (REF) -----

def _ref_quant_row(x):
    """Run the kernels.metal:753-802 restatement on one head row (reference layout)."""
    D = len(x)
    kc = np.zeros(D + 4, np.int8)
    vc = np.zeros(D + 4, np.int8)
    table = np.zeros(1, np.uint32)
    xx = np.ascontiguousarray(x, np.float32)
    O.ref_kv_update_int8(kc, vc, xx, xx, 0, table, 1, 1, 1, D, 0)
    return kc[:D].copy(), kc[D:].view(np.float32)[0]


def test_ref_int8_row_is_132_bytes_at_d128():
    # tests/kv_compression.rs:23-29: INT8 = head_dim + 4 = 132 bytes per head
    from velokv import KvCacheType, kv_bytes_per_token_per_head
    assert kv_bytes_per_token_per_head(128, KvCacheType.Int8) == 132
    assert kv_bytes_per_token_per_head(128, KvCacheType.Fp32) == 512
    L = O.Layer(2, 1, BS, HD, O.I8_REF)
    assert O.to_reference_layout(L, 0).size == 2 * BS * 1 * 132


def test_ref_int8_invariants():
    r = np.random.default_rng(3)
    for _ in range(200):
        x = (r.standard_normal(HD) * r.uniform(0.01, 50)).astype(np.float32)
        c, s = _ref_quant_row(x)
        amax = np.max(np.abs(x))
        assert np.all(np.abs(c.astype(int)) <= 127)
        assert s == np.float32(amax) / np.float32(127)
        # truncation: |x/s - c| < 1 and c has the sign of x (or is 0)
        ratio = x.astype(np.float64) * (127.0 / amax)
        assert np.all(np.abs(ratio - c) < 1.0 + 1e-5)
        assert np.all((c == 0) | (np.sign(c) == np.sign(x)))
        # the absmax element lands on 126 or 127 (fp32 rounding of 127/amax decides)
        i = int(np.argmax(np.abs(x)))
        assert abs(int(c[i])) in (126, 127)
        # odd symmetry and exact power-of-two scaling
        c2, s2 = _ref_quant_row(-x)
        assert np.array_equal(c2, -c) and s2 == s
        c3, s3 = _ref_quant_row(x * np.float32(4))
        assert np.array_equal(c3, c) and s3 == s * 4
    c, s = _ref_quant_row(np.zeros(HD, np.float32))
    assert s == 0.0 and not c.any()


def test_ref_int8_codes_equal_truncating_closed_form():
    """Over 10^4 random rows the REF quantizer's codes equal the numpy fp32
    closed form with truncation. The rows are drawn so that many products have
    fractional parts above 0.5 (where truncation and rounding differ) and so that
    the fp32 rounding of 127/amax sends some absmax elements to 126."""
    r = np.random.default_rng(11)
    n_rows = 10_000
    x = (r.standard_normal((n_rows, HD)) * r.uniform(0.01, 50, (n_rows, 1))).astype(np.float32)
    x[: n_rows // 10, 5] *= np.float32(8)  # outlier channel, as in config 3
    want_c, want_s = ref_codes_closed_form(x)
    got_c = np.empty((n_rows, HD), np.int8)
    got_s = np.empty(n_rows, np.float32)
    for i in range(n_rows):
        got_c[i], got_s[i] = _ref_quant_row(x[i])
    assert np.array_equal(got_c, want_c)
    assert np.array_equal(got_s, want_s)
    # the rows do separate truncation from round-to-nearest ...
    prod = (x * (np.float32(127) / np.max(np.abs(x), axis=1, keepdims=True)).astype(np.float32)).astype(np.float32)
    frac = np.abs(prod) - np.floor(np.abs(prod))
    assert int((frac > 0.5).sum()) > n_rows * HD // 4
    assert not np.array_equal(np.rint(prod).astype(np.int8), got_c)
    # ... and reach both absmax outcomes of the fp32 operation order
    imax = np.argmax(np.abs(x), axis=1)
    top = np.abs(got_c[np.arange(n_rows), imax].astype(int))
    assert (top == 126).any() and (top == 127).any()
    assert set(np.unique(top)) <= {126, 127}


def test_ref_layout_build_layout_agree_for_ref_int8():
    """Build-layout append then translate == reference-layout kv_update_int8."""
    n_blocks, Hkv = 6, 2
    table = np.array([4, 1, 5], np.uint32)  # slot 0's pages
    L = O.Layer(n_blocks, Hkv, BS, HD, O.I8_REF)
    kref = np.zeros(n_blocks * BS * Hkv * (HD + 4), np.int8)
    vref = np.zeros_like(kref)
    r = np.random.default_rng(4)
    for pos in range(40):
        k = (r.standard_normal((Hkv, HD)) * 3).astype(np.float32)
        v = (r.standard_normal((Hkv, HD)) * 3).astype(np.float32)
        O.ref_kv_update_int8(kref, vref, k, v, 0, table, 3, BS, Hkv, HD, pos)
        slot = int(table[pos // BS]) * BS + pos % BS
        O.append(L, k[None], v[None], [slot])
    assert np.array_equal(O.to_reference_layout(L, 0), kref.view(np.uint8))
    assert np.array_equal(O.to_reference_layout(L, 1), vref.view(np.uint8))


def test_ref_layout_build_layout_agree_for_f32():
    n_blocks, Hkv = 5, 2
    table = np.array([3, 0], np.uint32)
    L = O.Layer(n_blocks, Hkv, BS, HD, O.F32)
    kref = np.zeros(n_blocks * BS * Hkv * HD, np.float32)
    vref = np.zeros_like(kref)
    r = np.random.default_rng(5)
    for pos in range(25):
        k = r.standard_normal((Hkv, HD)).astype(np.float32)
        v = r.standard_normal((Hkv, HD)).astype(np.float32)
        O.ref_kv_update(kref, vref, k, v, 0, table, 2, BS, Hkv, HD, pos)
        O.append(L, k[None], v[None], [int(table[pos // BS]) * BS + pos % BS])
    assert np.array_equal(O.to_reference_layout(L, 0).view(np.float32), kref)
    assert np.array_equal(O.to_reference_layout(L, 1).view(np.float32), vref)


# ------------------------------------------- per-block INT8 (BLK) ---------

def _blk_block(tokens):
    """Append `tokens` ([n][D] fp32, one head) at offsets 0..n-1 of block 0."""
    L = O.Layer(1, 1, BS, HD, O.I8_BLK)
    for o, x in enumerate(tokens):
        O.append(L, np.asarray(x, np.float32)[None, None], np.asarray(x, np.float32)[None, None], [o])
    codes = L.tile_codes(0, 0, 0)
    scale = L.ks.view(np.float16)[0]
    return codes, scale, L


def test_blk_single_token_closed_form_via_numpy_float16():
    r = np.random.default_rng(11)
    for _ in range(300):
        x = (r.standard_normal(HD) * r.uniform(1e-3, 40)).astype(np.float32)
        codes, scale, _ = _blk_block([x])
        amax = np.float32(np.max(np.abs(x)))
        s = (amax / np.float32(127)).astype(np.float16)  # numpy's fp16 RNE
        assert scale.view(np.uint16) == s.view(np.uint16)
        c = codes[0].astype(int)
        assert np.all(np.abs(c) <= 127)
        # round-half-even dequantisation error is at most half a step
        err = np.abs(c * np.float64(s) - x)
        assert np.all(err <= np.float64(s) / 2 * (1 + 1e-6) + 1e-12) or np.any(np.abs(c) == 127)
        # absmax element maps to +-127 (fp16 scale is normal here)
        i = int(np.argmax(np.abs(x)))
        assert abs(c[i]) == 127
        # odd symmetry
        codes2, scale2, _ = _blk_block([-x])
        assert np.array_equal(codes2[0], -codes[0]) and scale2 == scale


def test_blk_zero_block_and_idempotence():
    codes, scale, _ = _blk_block([np.zeros(HD, np.float32)] * 3)
    assert scale == 0 and not codes[:3].any()
    r = np.random.default_rng(12)
    x = (r.standard_normal(HD) * 2).astype(np.float32)
    codes, scale, _ = _blk_block([x])
    deq = (codes[0].astype(np.float32) * np.float32(scale)).astype(np.float32)
    codes2, scale2, _ = _blk_block([deq])
    assert scale2 == scale and np.array_equal(codes2[0], codes[0])


def test_blk_decreasing_amax_never_requantizes():
    r = np.random.default_rng(13)
    base = r.standard_normal(HD).astype(np.float32)
    toks = [base * np.float32(8.0 / (1 + i)) for i in range(BS)]
    codes, scale, _ = _blk_block(toks)
    s0 = (np.float32(np.max(np.abs(toks[0]))) / np.float32(127)).astype(np.float16)
    assert scale == s0
    for i, x in enumerate(toks):
        ref = np.clip(np.rint(x / np.float32(s0)), -127, 127).astype(int)
        assert np.array_equal(codes[i].astype(int), ref)


def test_blk_increasing_amax_requantizes_existing_codes():
    r = np.random.default_rng(14)
    base = r.standard_normal(HD).astype(np.float32)
    toks = [base * np.float32(1 + i) for i in range(5)]
    codes, scale, _ = _blk_block(toks)
    s_last = (np.float32(np.max(np.abs(toks[-1]))) / np.float32(127)).astype(np.float16)
    assert scale == s_last
    # the last token is quantized directly at the final scale
    ref = np.clip(np.rint(toks[-1] / np.float32(s_last)), -127, 127).astype(int)
    assert np.array_equal(codes[4].astype(int), ref)
    # earlier tokens stay within one step of each requantisation: error <= (k/2) steps
    for i in range(4):
        err = np.abs(codes[i].astype(np.float64) * np.float64(s_last) - toks[i])
        assert np.all(err <= np.float64(s_last) * (0.5 * (4 - i) + 0.5) + 1e-9)
    # a single requantisation step: c' = rne(c * s_old / s_new) exactly
    c1, s1, _ = _blk_block(toks[:1])
    c2, s2, _ = _blk_block(toks[:2])
    step = np.clip(np.rint((c1[0].astype(np.float32) * np.float32(s1)) / np.float32(s2)), -127, 127)
    assert np.array_equal(c2[0].astype(np.float32), step)


def test_blk_offset_zero_resets_stale_block():
    r = np.random.default_rng(15)
    big = (r.standard_normal(HD) * 50).astype(np.float32)
    small = (r.standard_normal(HD) * 0.1).astype(np.float32)
    L = O.Layer(1, 1, BS, HD, O.I8_BLK)
    O.append(L, big[None, None], big[None, None], [0])
    O.append(L, small[None, None], small[None, None], [0])  # block reused: fresh scale
    s = (np.float32(np.max(np.abs(small))) / np.float32(127)).astype(np.float16)
    assert L.ks.view(np.float16)[0] == s


# -------------------------------------------------------- attention --------

def _np_attention_f64(case, layer):
    """Independent fp64 numpy attention over the oracle's dequantized pool."""
    S, H = case.S, case.n_heads
    G = H // case.n_kv_heads
    out = np.zeros((S, H, HD))
    for s in range(S):
        L = int(case.ctx_lens[s])
        for h in range(H):
            kvh = h // G
            K = np.array([[layer.elem(0, case.block_tables[s, t // BS], kvh, t % BS, d) for d in range(HD)]
                          for t in range(L)], np.float64)
            V = np.array([[layer.elem(1, case.block_tables[s, t // BS], kvh, t % BS, d) for d in range(HD)]
                          for t in range(L)], np.float64)
            sc = K @ case.q[s, h].astype(np.float64) / np.sqrt(HD)
            p = np.exp(sc - sc.max())
            out[s, h] = (p / p.sum()) @ V
    return out


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_decode_matches_numpy_f64_bruteforce(kv):
    case = make_case(kv, [37, 16], n_kv_heads=2, n_heads=4, seed=21)
    layer = oracle_layer(case)
    got = O.paged_decode(layer, case.q, case.block_tables, case.ctx_lens)
    ref = _np_attention_f64(case, layer)
    assert np.max(np.abs(got - ref)) < 2e-5
    got64 = O.paged_decode_f64(layer, case.q, case.block_tables, case.ctx_lens)
    assert np.max(np.abs(got64 - ref)) < 1e-9


def test_decode_matches_reference_kernel_restatements():
    """Paged two-pass oracle == online-softmax paged_attention_flash restatement
    (reference layout) == llama_cpu.rs attention on a contiguous cache."""
    Hkv, H = 8, 32
    case = make_case(O.F32, [100], n_kv_heads=Hkv, n_heads=H, n_blocks=16, seed=22)
    layer = oracle_layer(case)
    got = O.paged_decode(layer, case.q.astype(np.float32), case.block_tables, case.ctx_lens)[0]
    kref = O.to_reference_layout(layer, 0).view(np.float32)
    vref = O.to_reference_layout(layer, 1).view(np.float32)
    table = case.block_tables[0].astype(np.uint32)
    flash = O.ref_paged_attention_flash(case.q[0].astype(np.float32), kref, vref, False, HD, 99, 0, table,
                                        len(table), BS, Hkv, H)
    assert np.max(np.abs(flash - got)) < 1e-5
    kc = case.k[0].astype(np.float32)
    vc = case.v[0].astype(np.float32)
    cpu = O.ref_cpu_attention(case.q[0].astype(np.float32), kc, vc, H, Hkv, HD)
    assert np.max(np.abs(cpu - got)) < 1e-5


def test_decode_int8_ref_matches_flash_int8_restatement():
    Hkv, H = 4, 16
    case = make_case(O.I8_REF, [70], n_kv_heads=Hkv, n_heads=H, n_blocks=12, seed=23)
    layer = oracle_layer(case)
    got = O.paged_decode(layer, case.q, case.block_tables, case.ctx_lens)[0]
    kref = O.to_reference_layout(layer, 0)
    vref = O.to_reference_layout(layer, 1)
    table = case.block_tables[0].astype(np.uint32)
    flash = O.ref_paged_attention_flash(case.q[0].astype(np.float32), kref, vref, True, HD, 69, 0, table,
                                        len(table), BS, Hkv, H)
    assert np.max(np.abs(flash - got)) < 1e-5


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_decode_single_token_is_v0(kv):
    # tests/llama_parity.rs:59-82 compares at pos = 0, where attention is v_0
    case = make_case(kv, [1, 1], seed=24)
    layer = oracle_layer(case)
    got = O.paged_decode(layer, case.q, case.block_tables, case.ctx_lens)
    for s in range(2):
        for h in range(32):
            v0 = np.array([layer.elem(1, case.block_tables[s, 0], h // 4, 0, d) for d in range(HD)], np.float32)
            assert np.array_equal(got[s, h], v0)


def test_decode_invariants():
    case = make_case(O.F16, [53], seed=25)
    layer = oracle_layer(case)
    base = O.paged_decode(layer, case.q, case.block_tables, case.ctx_lens)
    # moving the blocks to other physical pages leaves the output bit-identical
    moved = O.Layer(case.n_blocks, 8, BS, HD, O.F16)
    perm = synth.rng(99).permutation(case.n_blocks).astype(np.int32)
    tile = BS * HD * 2 * 8
    for b in range(case.n_blocks):
        moved.k[perm[b] * tile:(perm[b] + 1) * tile] = layer.k[b * tile:(b + 1) * tile]
        moved.v[perm[b] * tile:(perm[b] + 1) * tile] = layer.v[b * tile:(b + 1) * tile]
    out2 = O.paged_decode(moved, case.q, perm[case.block_tables], case.ctx_lens)
    assert np.array_equal(out2, base)
    # identical queries in one GQA group give identical outputs
    q = case.q.copy()
    q[0, 1:4] = q[0, 0]
    out3 = O.paged_decode(layer, q, case.block_tables, case.ctx_lens)
    assert np.array_equal(out3[0, 1], out3[0, 0]) and np.array_equal(out3[0, 3], out3[0, 0])
    # q = 0 -> uniform weights -> mean of V
    out4 = O.paged_decode(layer, np.zeros_like(q), case.block_tables, case.ctx_lens)
    for h in (0, 17):
        V = np.array([[layer.elem(1, case.block_tables[0, t // BS], h // 4, t % BS, d) for d in range(HD)]
                      for t in range(53)], np.float64)
        assert np.max(np.abs(out4[0, h] - V.mean(0))) < 1e-5


def test_decode_empty_context_is_zero():
    case = make_case(O.F16, [5], seed=26)
    layer = oracle_layer(case)
    out = O.paged_decode(layer, case.q, case.block_tables, np.array([0], np.int32))
    assert not out.any()


# -------------------------------------------------------- tree verify ------

def test_tree_verify_reduces_to_decode():
    case = make_case(O.I8_BLK, [40 + 6], n_kv_heads=2, n_heads=8, seed=27)
    layer = oracle_layer(case)
    ctx = 40
    N = 6
    q = synth.normals_f16(N * 8 * HD, 555).reshape(1, N, 8, HD)
    chain = np.array([(1 << (i + 1)) - 1 for i in range(N)], np.uint32)  # node i sees nodes 0..i
    out = O.tree_verify(layer, q, case.block_tables, np.array([ctx], np.int32), chain[None])
    for i in range(N):
        ref = O.paged_decode(layer, q[:, i], case.block_tables, np.array([ctx + i + 1], np.int32))
        assert np.max(np.abs(out[0, i] - ref[0])) < 1e-6
    # an empty mask row attends to the context only
    none = np.zeros((1, N), np.uint32)
    out0 = O.tree_verify(layer, q, case.block_tables, np.array([ctx], np.int32), none)
    ref0 = O.paged_decode(layer, q[:, 2], case.block_tables, np.array([ctx], np.int32))
    assert np.max(np.abs(out0[0, 2] - ref0[0])) < 1e-6


def test_tree_verify_f64_bruteforce_branching_mask():
    case = make_case(O.F16, [20 + 8], n_kv_heads=1, n_heads=2, seed=28)
    layer = oracle_layer(case)
    ctx, N = 20, 8
    parent = [-1, 0, 0, 1, 1, 2, 2, 3]
    mask = np.zeros(N, np.uint32)
    for i in range(N):
        j = i
        while j >= 0:
            mask[i] |= 1 << j
            j = parent[j]
    q = synth.normals_f16(N * 2 * HD, 556).reshape(1, N, 2, HD)
    out = O.tree_verify(layer, q, case.block_tables, np.array([ctx], np.int32), mask[None])
    for i in range(N):
        pos = list(range(ctx)) + [ctx + j for j in range(N) if (mask[i] >> j) & 1]
        for h in range(2):
            K = np.array([[layer.elem(0, case.block_tables[0, t // BS], 0, t % BS, d) for d in range(HD)] for t in pos])
            V = np.array([[layer.elem(1, case.block_tables[0, t // BS], 0, t % BS, d) for d in range(HD)] for t in pos])
            sc = K @ q[0, i, h].astype(np.float64) / np.sqrt(HD)
            p = np.exp(sc - sc.max())
            ref = (p / p.sum()) @ V
            assert np.max(np.abs(out[0, i, h] - ref)) < 2e-5


# -------------------------------------------------------- copy-on-write -----

@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_copy_blocks_invariants(kv):
    case = make_case(kv, [70], n_kv_heads=2, n_heads=4, n_blocks=12, seed=29)
    layer = oracle_layer(case)
    before = layer.copy()
    src = [int(case.block_tables[0, 1]), int(case.block_tables[0, 4])]
    free = [b for b in range(12) if b not in case.block_tables[0, :5]]
    dst = free[:2]
    O.copy_blocks(layer, np.array([[src[0], dst[0]], [src[1], dst[1]]]))
    for s, d in zip(src, dst):
        for h in range(2):
            for t in (0, 7, 15):
                for dd in (0, 64, 127):
                    assert layer.elem(0, d, h, t, dd) == before.elem(0, s, h, t, dd)
                    assert layer.elem(1, d, h, t, dd) == before.elem(1, s, h, t, dd)
    # only the destination blocks changed
    esz = O.ESZ[kv]
    cb = 2 * BS * HD * esz
    changed = np.nonzero(layer.k.reshape(12, cb) != before.k.reshape(12, cb))[0]
    assert set(changed.tolist()) <= set(dst)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_tile_layout_is_a_permutation_with_line_friendly_int8_k(kv, D):
    """Every (token, dim) of a tile has its own offset (a permutation of the
    16 x D tile); int8 K puts the 32 codes of dims 32c..32c+31 of token t in two
    16-byte pieces at (t D/32 + c)*16 and 8 D + (t D/32 + c)*16."""
    L = O.Layer(1, 1, BS, D, kv)
    esz = O.ESZ[kv]
    for is_v in (0, 1):
        idx = O._tile_index(L, is_v)
        assert np.array_equal(np.sort(idx.ravel() // esz), np.arange(BS * D))
    idx = O._tile_index(L, 0)
    if esz == 1:
        n = D // 32
        for t in (0, 7, 15):
            for c in range(n):
                p = (n * t + c) * 16
                assert list(idx[t, 32 * c:32 * c + 16]) == list(range(p, p + 16))
                assert list(idx[t, 32 * c + 16:32 * c + 32]) == list(range(8 * D + p, 8 * D + p + 16))
    else:
        assert np.array_equal(idx, (np.arange(BS)[:, None] * D + np.arange(D)[None, :]) * esz)
    vidx = O._tile_index(L, 1)  # V: token pairs interleaved, [tok/2][D][2]
    t = np.arange(BS)[:, None]
    assert np.array_equal(vidx, (((t >> 1) * D + np.arange(D)[None, :]) * 2 + (t & 1)) * esz)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_head_dim64_layer_equals_zero_padded_128(kv):
    """The oracle at head_dim 64 (16 x 64 tiles) against the oracle at 128 over
    the same rows zero-padded: every (token, dim) holds the same code and scale
    (an int8 scale comes from an absmax, which zero dims do not move), the padded
    dims stay zero, and attention with the 1/sqrt(64) scale is bit for bit the
    same (the zero dims add exact zeros)."""
    D = 64
    case = make_case(kv, [37, 16, 70], n_kv_heads=2, n_heads=4, seed=23, outlier_scale=8.0)
    L64 = O.Layer(case.n_blocks, 2, BS, D, kv)
    L128 = O.Layer(case.n_blocks, 2, BS, HD, kv)
    for sl, kk, vv in (case.prefill_slots(), case.last_slots()):
        O.append(L64, np.ascontiguousarray(kk[..., :D]), np.ascontiguousarray(vv[..., :D]), sl)
        kp, vp = np.zeros_like(kk), np.zeros_like(vv)
        kp[..., :D], vp[..., :D] = kk[..., :D], vv[..., :D]
        O.append(L128, kp, vp, sl)
    used = sorted({int(b) for s in range(case.S) for b in case.block_tables[s, :(int(case.ctx_lens[s]) + BS - 1) // BS]})
    for b in used:
        for h in range(2):
            for is_v in (0, 1):
                t64, t128 = L64.tile_codes(is_v, b, h), L128.tile_codes(is_v, b, h)
                assert np.array_equal(t64, t128[:, :D])
                assert not np.any(t128[:, D:])
    if L64.ks is not None:
        assert np.array_equal(L64.ks, L128.ks) and np.array_equal(L64.vs, L128.vs)
    q64 = np.ascontiguousarray(case.q[..., :D])
    qp = np.zeros_like(case.q)
    qp[..., :D] = q64
    got = O.paged_decode(L64, q64, case.block_tables, case.ctx_lens)
    ref = O.paged_decode(L128, qp, case.block_tables, case.ctx_lens, scale=1.0 / np.sqrt(D))
    assert np.array_equal(got, ref[..., :D])


@pytest.mark.parametrize("hd", [96, 80, 40, 8])
@pytest.mark.parametrize("kv", [O.F32, O.I8_REF])
def test_other_head_dims_padded_layer_equals_reference_restatement(kv, hd):
    """A head_dim that is not 64 or 128 is held in the tiles of the next width (64
    or 128 dims) with zeros past head_dim. Pinned against the restatements of the
    reference's own kernels at that head_dim (kv_update / kv_update_int8 and
    paged_attention_flash[_int8], kernels.metal:440-501, 619-645, 672-732,
    753-802, which take any head_dim up to 128): the padded layer holds the
    reference's codes and scales (an int8 scale comes from the row's absmax,
    which zero dims do not move) and zeros past head_dim, and attention over it
    with the 1/sqrt(head_dim) scale gives the reference's output."""
    T = 64 if hd <= 64 else HD
    n_blocks, Hkv, H = 6, 2, 4
    table = np.array([4, 1, 5], np.uint32)
    row = 4 * hd if kv == O.F32 else hd + 4
    kref = np.zeros(n_blocks * BS * Hkv * row, np.uint8)
    vref = np.zeros_like(kref)
    L = O.Layer(n_blocks, Hkv, BS, T, kv)
    r = np.random.default_rng(31 + hd)
    n_tok = 40
    for pos in range(n_tok):
        k = (r.standard_normal((Hkv, hd)) * r.uniform(0.5, 4)).astype(np.float32)
        v = (r.standard_normal((Hkv, hd)) * r.uniform(0.5, 4)).astype(np.float32)
        if kv == O.F32:
            O.ref_kv_update(kref.view(np.float32), vref.view(np.float32), k, v, 0, table, 3, BS, Hkv, hd, pos)
        else:
            O.ref_kv_update_int8(kref.view(np.int8), vref.view(np.int8), k, v, 0, table, 3, BS, Hkv, hd, pos)
        kp, vp = np.zeros((1, Hkv, T), np.float32), np.zeros((1, Hkv, T), np.float32)
        kp[0, :, :hd], vp[0, :, :hd] = k, v
        O.append(L, kp, vp, [int(table[pos // BS]) * BS + pos % BS])
    for is_v, ref in ((0, kref), (1, vref)):
        got = O.to_reference_layout(L, is_v).reshape(n_blocks * BS * Hkv, -1)
        want = ref.reshape(n_blocks * BS * Hkv, row)
        esz = 4 if kv == O.F32 else 1
        assert np.array_equal(got[:, :hd * esz], want[:, :hd * esz])       # codes (or fp32 values)
        assert not np.any(got[:, hd * esz:T * esz])                         # zeros past head_dim
        if kv == O.I8_REF:
            assert np.array_equal(got[:, T:], want[:, hd:])                  # the per-token fp32 scale
    q = r.standard_normal((H, hd)).astype(np.float32)
    qp = np.zeros((1, H, T), np.float32)
    qp[0, :, :hd] = q
    bt = table[None].astype(np.int32)
    got = O.paged_decode(L, qp.astype(np.float32), bt, np.array([n_tok], np.int32), scale=1.0 / np.sqrt(hd))[0]
    want = O.ref_paged_attention_flash(q, kref.view(np.float32 if kv == O.F32 else np.int8),
                                       vref.view(np.float32 if kv == O.F32 else np.int8), kv == O.I8_REF, hd,
                                       n_tok - 1, 0, table, 3, BS, Hkv, H)
    assert not np.any(got[:, hd:])
    assert np.max(np.abs(got[:, :hd] - want)) < 2e-5


@pytest.mark.parametrize("hd", [96, 40])
def test_other_head_dims_blk_closed_form(hd):
    """I8_BLK over a padded head: one token per block, so each block's scale is
    fp16_rne(amax / 127) over the head's own dims and its codes rne(x / s) clipped
    to +-127 (numpy float16 and rint, no oracle step), zeros past head_dim."""
    T = 64 if hd <= 64 else HD
    r = np.random.default_rng(7 + hd)
    L = O.Layer(8, 1, BS, T, O.I8_BLK)
    for b in range(8):
        x = (r.standard_normal(hd) * r.uniform(0.01, 30)).astype(np.float32)
        xp = np.zeros((1, 1, T), np.float32)
        xp[0, 0, :hd] = x
        O.append(L, xp, xp, [b * BS])
        s = (np.max(np.abs(x)) / np.float32(127)).astype(np.float16)
        assert L.ks.view(np.float16)[b] == s
        c = np.clip(np.rint(x.astype(np.float32) / np.float32(s)), -127, 127).astype(np.int8)
        codes = L.tile_codes(0, b, 0)
        assert np.array_equal(codes[0, :hd], c)
        assert not np.any(codes[0, hd:])
