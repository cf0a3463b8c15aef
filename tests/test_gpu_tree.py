"""GPU parity of tree-verify attention against the oracle (vko_tree_verify:
fp32 two-pass softmax over the committed context plus the mask-selected tree
nodes), within the north-star tolerance, and the config-4 flow: a shared prefix
whose pages alias across sequences, copy-on-write of the partial shared block,
suffix and draft-token appends, then tree verify."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer, tol_check
from test_gpu_append_copy import assert_layer_equal, gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu

KV_TREE = [O.F32, O.F16, O.I8_REF, O.I8_BLK]


def run_tree(ctx, pool, case, q, committed, mask, q_dtype=np.float16, partition_tokens=0, block_tables=None,
             seq_rows=None, layer=0, shared_blocks=0):
    S, N = q.shape[0], q.shape[1]
    qd = q.astype(q_dtype)
    out = ctx.alloc(S * N * case.n_heads * HD * 4)
    bt = case.block_tables if block_tables is None else block_tables
    mk = np.ascontiguousarray(mask, dtype=np.uint32).reshape(S, N)
    ctx.tree_verify(pool, layer, ctx.upload(qd), velokv.DT_F16 if q_dtype == np.float16 else velokv.DT_F32, out,
                    ctx.upload(np.asarray(committed, np.int32)), ctx.upload(mk), S, N, case.n_heads,
                    int(np.max(committed)) if S else 0, block_tables=ctx.upload(bt), bt_stride=bt.shape[1],
                    seq_rows=ctx.upload(seq_rows) if seq_rows is not None else None,
                    partition_tokens=partition_tokens, shared_blocks=shared_blocks)
    ctx.sync()
    return out.download((S, N, case.n_heads, HD), np.float32)


def tree_q(S, N, H, seed):
    return synth.normals_f16(S * N * H * HD, seed).reshape(S, N, H, HD)


def check(got, ref, what):
    ok, err, nbad = tol_check(got, ref)
    assert ok, f"{what}: max err {err:.3g}, {nbad} elements out of tolerance"
    return err


def tree_case(kv, committed, N, G=4, Hkv=8, seed=1, outlier_scale=1.0):
    committed = np.asarray(committed, np.int32)
    return make_case(kv, committed + N, n_kv_heads=Hkv, n_heads=Hkv * G, seed=seed, outlier_scale=outlier_scale)


def mask_222(N):
    return velokv.branching_tree([2, 2, 2, 2, 2], N).ancestor_mask()


@pytest.mark.parametrize("kv", KV_TREE)
@pytest.mark.parametrize("qd", [np.float16, np.float32])
def test_tree_config4_shape_small(ctx, kv, qd):
    """8-node 2-2-2 tree over ragged committed contexts (GQA 4, 8 KV heads)."""
    print(f"tree small kv={kv} q={np.dtype(qd).name}", flush=True)
    committed = [0, 1, 15, 16, 100, 511, 700]
    N = 8
    case = tree_case(kv, committed, N, seed=301, outlier_scale=8.0 if kv != O.F16 else 1.0)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = tree_q(case.S, N, case.n_heads, 3011)
    mask = np.tile(mask_222(N), (case.S, 1))
    got = run_tree(ctx, pool, case, q, committed, mask, q_dtype=qd)
    ref = O.tree_verify(ref_layer, q.astype(qd), case.block_tables, committed, mask)
    check(got, ref, "tree")


@pytest.mark.parametrize("kv", KV_TREE)
@pytest.mark.parametrize("G,N", [(1, 1), (1, 16), (2, 8), (2, 9), (4, 4), (4, 5), (4, 16), (8, 2), (8, 3), (8, 32),
                                 (4, 32)])
def test_tree_row_tiles_and_random_masks(ctx, kv, G, N):
    """Every row-tile shape (rows = N*G from 1 to 256) with random per-sequence
    masks, including rows that see no tree node and, at context 0, nothing."""
    print(f"tree tiles kv={kv} G={G} N={N}", flush=True)
    Hkv = 2
    committed = [0, 3, 33, 250]
    case = tree_case(kv, committed, N, G=G, Hkv=Hkv, seed=302 + 7 * G + N)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = tree_q(case.S, N, case.n_heads, 3021 + N)
    rng = np.random.default_rng(G * 100 + N)
    full = (1 << N) - 1 if N < 32 else 0xFFFFFFFF
    mask = rng.integers(0, 1 << 32, size=(case.S, N), dtype=np.uint64).astype(np.uint32) & np.uint32(full)
    mask[0, 0] = 0  # context 0 and no visible node: output zeros
    got = run_tree(ctx, pool, case, q, committed, mask)
    ref = O.tree_verify(ref_layer, q, case.block_tables, committed, mask)
    check(got, ref, "tree random mask")
    assert np.all(got[0, 0] == 0.0)


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_BLK])
@pytest.mark.parametrize("P", [16, 64, 256, 1024, 0])
def test_tree_split_k(ctx, kv, P):
    print(f"tree split kv={kv} P={P}", flush=True)
    committed = [5, 1000, 2047, 2056, 3000]
    N = 8
    case = tree_case(kv, committed, N, seed=303)
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = tree_q(case.S, N, case.n_heads, 3031)
    mask = np.tile(mask_222(N), (case.S, 1))
    got = run_tree(ctx, pool, case, q, committed, mask, partition_tokens=P)
    ref = O.tree_verify(ref_layer, q, case.block_tables, committed, mask)
    check(got, ref, f"tree P={P}")


@pytest.mark.parametrize("kv", KV_TREE)
def test_tree_single_node_equals_decode(ctx, kv):
    """A one-node tree that sees itself is decode over context + 1 tokens."""
    committed = np.array([0, 16, 77, 600], np.int32)
    case = tree_case(kv, committed, 1, seed=304)
    pool = gpu_pool(ctx, case)
    q = tree_q(case.S, 1, case.n_heads, 3041)
    got = run_tree(ctx, pool, case, q, committed, np.ones((case.S, 1), np.uint32))
    out = ctx.alloc(case.S * case.n_heads * HD * 4)
    ctx.paged_decode(pool, 0, ctx.upload(q[:, 0]), velokv.DT_F16, out, ctx.upload(case.ctx_lens), case.S,
                     case.n_heads, int(case.ctx_lens.max()), block_tables=ctx.upload(case.block_tables),
                     bt_stride=case.block_tables.shape[1])
    ctx.sync()
    dec = out.download((case.S, case.n_heads, HD), np.float32)
    check(got[:, 0], dec, "tree N=1 vs decode")


def test_tree_bad_arguments(ctx):
    case = tree_case(O.F16, [10], 8, seed=305)
    pool = gpu_pool(ctx, case)
    q = ctx.upload(tree_q(1, 8, case.n_heads, 1))
    out = ctx.alloc(8 * case.n_heads * HD * 4)
    cl = ctx.upload(np.array([10], np.int32))
    mk = ctx.upload(np.ones(8, np.uint32))
    bt = ctx.upload(case.block_tables)
    stride = case.block_tables.shape[1]
    with pytest.raises(velokv.VkError) as e:
        ctx.tree_verify(pool, 0, q, velokv.DT_F16, out, cl, mk, 1, 33, case.n_heads, 10, block_tables=bt,
                        bt_stride=stride)
    assert e.value.code == velokv.ERR_BAD_ARG
    with pytest.raises(velokv.VkError) as e:  # context + nodes beyond the table row
        ctx.tree_verify(pool, 0, q, velokv.DT_F16, out, cl, mk, 1, 8, case.n_heads, stride * BS, block_tables=bt,
                        bt_stride=stride)
    assert e.value.code == velokv.ERR_BAD_ARG
    with pytest.raises(velokv.VkError) as e:
        ctx.tree_verify(pool, 0, q, velokv.DT_F16, out, cl, None, 1, 8, case.n_heads, 10, block_tables=bt,
                        bt_stride=stride)
    assert e.value.code == velokv.ERR_BAD_ARG


def config4_flow(ctx, kv, S, prefix_len, max_suffix, N, seed, Hkv=8, G=4, n_layer=1, layer=0):
    """Shared prefix -> fork per sequence -> COW of the partial shared page ->
    suffix + draft appends. Returns (pool, oracle layer, tables, committed, parent
    pages) after checking the pool bytes against the oracle."""
    H = Hkv * G
    rng = np.random.default_rng(seed)
    suffix = rng.integers(0, max_suffix + 1, size=S).astype(np.int32)
    committed = prefix_len + suffix
    total = committed + N
    stride = int((total.max() + BS - 1) // BS)
    need = (prefix_len + BS - 1) // BS + sum((int(t) + BS - 1) // BS for t in total) + S
    n_blocks = need + 64
    bm = velokv.BlockManager(BS, n_blocks)
    parent = bm.allocate(10_000, prefix_len)
    row = Hkv * HD
    pk = synth.normals_f16(prefix_len * row, seed * 10 + 1, row).reshape(prefix_len, Hkv, HD)
    pv = synth.normals_f16(prefix_len * row, seed * 10 + 2, row).reshape(prefix_len, Hkv, HD)
    pool = velokv.Pool(ctx, n_layer, n_blocks, BS, Hkv, HD, kv)
    ref = O.Layer(n_blocks, Hkv, BS, HD, kv)
    ptab = np.array([parent], np.int32)
    psl = synth.slots_for_positions(ptab, np.arange(prefix_len), BS, np.zeros(prefix_len, np.int64))
    ctx.append(pool, layer, ctx.upload(pk), ctx.upload(pv), velokv.DT_F16, ctx.upload(psl), prefix_len)
    O.append(ref, pk, pv, psl)
    tables = np.zeros((S, stride), np.int32)
    pairs = []
    for s in range(S):
        pages = bm.fork(10_000, s, prefix_len, int(total[s]))
        if prefix_len % BS:
            cw = bm.cow(s, prefix_len // BS)
            if cw is not None:
                pairs.append(cw)
                pages = bm.materialize_span(s)
        tables[s, :len(pages)] = pages
    if pairs:
        ctx.copy_blocks(pool, np.array(pairs, np.int32))
        O.copy_blocks(ref, np.array(pairs, np.int32))
    # suffix + draft tokens of every sequence in one append (positions prefix_len .. total-1)
    sl, kk, vv = [], [], []
    for s in range(S):
        n = int(total[s]) - prefix_len
        pos = np.arange(prefix_len, int(total[s]))
        sl.append(synth.slots_for_positions(tables, pos, BS, np.full(n, s)))
        kk.append(synth.normals_f16(n * row, seed * 1000 + 2 * s, row).reshape(n, Hkv, HD))
        vv.append(synth.normals_f16(n * row, seed * 1000 + 2 * s + 1, row).reshape(n, Hkv, HD))
    sl, kk, vv = np.concatenate(sl), np.concatenate(kk), np.concatenate(vv)
    ctx.append(pool, layer, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(sl), len(sl))
    O.append(ref, kk, vv, sl)
    ctx.sync()
    return pool, ref, tables, committed, parent, H


@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
@pytest.mark.parametrize("prefix_len", [4096, 4100])
def test_config4_flow_reduced(ctx, kv, prefix_len):
    """Config 4 at 16 sequences: aliased 4096- (block aligned) or 4100-token
    (partial shared block, so every sequence copies it on write) prefix, suffix
    U[0, 512], 8-node 2-2-2 tree, INT8 KV."""
    print(f"config4 flow kv={kv} prefix={prefix_len}", flush=True)
    S, N = 16, 8
    pool, ref, tables, committed, parent, H = config4_flow(ctx, kv, S, prefix_len, 512, N, seed=306)
    assert_layer_equal(pool, 0, ref)  # appends and COW copies bit-exact, parent pages untouched by children
    q = tree_q(S, N, H, 3061)
    mask = np.tile(mask_222(N), (S, 1))

    class C:
        n_heads = H
        block_tables = tables
    got = run_tree(ctx, pool, C, q, committed, mask)
    expect = O.tree_verify(ref, q, tables, committed, mask)
    check(got, expect, "config4 flow")
    # sequences share the prefix pages (all but the copied partial one)
    shared = prefix_len // BS
    assert np.all(tables[:, :shared] == np.array(parent[:shared], np.int32))


# ---- shared-prefix pass (vk_tree_args.shared_blocks) --------------------------

@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16, O.I8_REF, O.F32])
@pytest.mark.parametrize("prefix_len,S", [(4096, 64), (4100, 16)])
def test_tree_shared_prefix_flow(ctx, kv, prefix_len, S):
    """Config-4 flow with the shared prefix declared: the prefix pass over the
    aliased pages plus the rest of each context must match the oracle and the
    call without the hint (I8_REF pools ignore it). 16 sequences leave few row
    tiles, so the prefix is cut into chunks."""
    print(f"tree shared prefix kv={kv} prefix={prefix_len} S={S}", flush=True)
    N = 8
    pool, ref, tables, committed, parent, H = config4_flow(ctx, kv, S, prefix_len, 512, N, seed=307)
    q = tree_q(S, N, H, 3071)
    mask = np.tile(mask_222(N), (S, 1))

    class C:
        n_heads = H
        block_tables = tables
    shared = prefix_len // BS
    assert np.all(tables[:, :shared] == tables[0, :shared])
    got = run_tree(ctx, pool, C, q, committed, mask, shared_blocks=shared)
    plain = run_tree(ctx, pool, C, q, committed, mask)
    expect = O.tree_verify(ref, q, tables, committed, mask)
    check(got, expect, "shared prefix vs oracle")
    check(got, plain, "shared prefix vs no hint")


@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
@pytest.mark.parametrize("qd", [np.float16, np.float32])
@pytest.mark.parametrize("G,N", [(4, 5), (1, 3), (8, 8)])
def test_tree_shared_prefix_short_contexts(ctx, kv, qd, G, N):
    """Contexts shorter than the shared prefix (0, 5, 16, 639 tokens), equal to
    it and longer, with 40 shared pages cut into two chunks: each row sees only
    its own committed tokens of the shared pages."""
    print(f"tree shared prefix short kv={kv} q={np.dtype(qd).name} G={G} N={N}", flush=True)
    P = 40
    committed = np.array([P * BS + 37, 5, 16, P * BS - 1, P * BS, P * BS + 100, 0, 33], np.int32)
    case = tree_case(kv, committed, N, G=G, Hkv=2, seed=311, outlier_scale=8.0 if kv != O.F16 else 1.0)
    # every row shares row 0's first P pages (row 0 holds the longest context, so they are fully written)
    bt = case.block_tables.copy()
    bt[:, :P] = bt[0, :P]
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = tree_q(case.S, N, case.n_heads, 3111)
    rng = np.random.default_rng(5 + G * N)
    full = (1 << N) - 1
    mask = rng.integers(0, 1 << 32, size=(case.S, N), dtype=np.uint64).astype(np.uint32) & np.uint32(full)
    got = run_tree(ctx, pool, case, q, committed, mask, q_dtype=qd, block_tables=bt, shared_blocks=P)
    ref = O.tree_verify(ref_layer, q.astype(qd), bt, committed, mask)
    check(got, ref, "shared prefix, short contexts")


@pytest.mark.parametrize("kv", [O.I8_BLK, O.F16])
@pytest.mark.parametrize("P", [16, 64, 0])
def test_tree_shared_prefix_partitions(ctx, kv, P):
    """Shared prefix with the rest of each context cut into partitions of P
    tokens (merged by vk_decode_merge after the prefix slots) or, for P = 0, in
    one partition whose kernel folds the prefix partials into the output."""
    print(f"tree shared prefix partitions kv={kv} P={P}", flush=True)
    pb = 24
    committed = np.array([pb * BS + 300, pb * BS, pb * BS + 1, pb * BS + 77, 3 * BS + 5], np.int32)
    N = 8
    case = tree_case(kv, committed, N, Hkv=2, seed=313, outlier_scale=8.0 if kv != O.F16 else 1.0)
    bt = case.block_tables.copy()
    bt[:, :pb] = bt[0, :pb]
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = tree_q(case.S, N, case.n_heads, 3131)
    mask = np.tile(mask_222(N), (case.S, 1))
    got = run_tree(ctx, pool, case, q, committed, mask, block_tables=bt, shared_blocks=pb, partition_tokens=P)
    ref = O.tree_verify(ref_layer, q, bt, committed, mask)
    check(got, ref, "shared prefix partitions")


def test_tree_shared_prefix_bad_arguments(ctx):
    case = tree_case(O.I8_BLK, [64, 80], 4, Hkv=2)
    pool = gpu_pool(ctx, case)
    q = ctx.upload(tree_q(case.S, 4, case.n_heads, 1))
    out = ctx.alloc(case.S * 4 * case.n_heads * HD * 4)
    cl = ctx.upload(np.array([64, 80], np.int32))
    mk = ctx.upload(np.tile(mask_222(4), (case.S, 1)).astype(np.uint32))
    bt = ctx.upload(case.block_tables)
    for shared in (-1, 6):  # 6 pages = 96 tokens > max_context_len 80
        with pytest.raises(velokv.VkError) as e:
            ctx.tree_verify(pool, 0, q, velokv.DT_F16, out, cl, mk, case.S, 4, case.n_heads, 80, block_tables=bt,
                            bt_stride=case.block_tables.shape[1], shared_blocks=shared)
        assert e.value.code == velokv.ERR_BAD_ARG


# The bound of the fp32-q test, 4-5x tighter than the north-star tolerance
# (2e-3 + 1e-2 |ref|); q rounded to fp16 misses it on the test's inputs
TIGHT = {O.F16: dict(atol=5e-4, rtol=2e-3), O.I8_BLK: dict(atol=5e-4, rtol=2e-3)}


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_tree_fp32_q_keeps_its_precision(ctx, kv, shared):
    """An fp32 q with x20 outlier channels (values fp16 does not hold): the tree
    kernels and the shared-prefix pass split q into fp16 hi + lo and take both
    products per score, as the reference's tree kernel computes q.k in fp32
    (kernels.metal:512-599). Outputs match the oracle's fp32-q tree verify within
    the bound TIGHT, which the same q rounded to fp16 misses (checked on the
    oracle itself). K and V have no outlier channels here: the value product's
    fp16 p * v_scale, a rounding apart from q's, grows with |v|."""
    print(f"tree fp32 q precision kv={kv} shared={shared}", flush=True)
    from test_gpu_decode import outlier_q
    N, P = 8, 24
    committed = np.array([P * BS + 300, 1, 15, 16, 100, P * BS + 5, 700, P * BS], np.int32)
    case = tree_case(kv, committed, N, seed=341)
    bt = case.block_tables.copy()
    if shared:  # every row reads row 0's first P pages (row 0 holds the longest context, so they are written)
        bt[:, :P] = bt[0, :P]
    ref_layer = oracle_layer(case)
    pool = gpu_pool(ctx, case)
    q = outlier_q((case.S, N, case.n_heads, HD), 342, 20.0)
    mask = np.tile(mask_222(N), (case.S, 1))
    got = run_tree(ctx, pool, case, q, committed, mask, q_dtype=np.float32, block_tables=bt,
                   shared_blocks=P if shared else 0)
    ref = O.tree_verify(ref_layer, q, bt, committed, mask)
    ok, err, nbad = tol_check(got, ref, **TIGHT[kv])
    print(f"  max abs err {err:.3g}", flush=True)
    assert ok, f"fp32 q: max err {err:.3g}, {nbad} elements out of the tight bound"
    r16 = O.tree_verify(ref_layer, q.astype(np.float16), bt, committed, mask)
    assert not tol_check(r16, ref, **TIGHT[kv])[0], "the bound does not separate fp16-rounded q"
