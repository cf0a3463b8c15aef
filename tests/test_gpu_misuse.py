"""Misuse the kernels detect without trapping (include/velokv.h VK_MISUSE_*): a
block-table page id outside the pool in an attention call, and an INT8
per-block append whose tokens of one block are not adjacent in the call. Each
is fed once on its own and must come back as VK_ERR_BAD_ARG from the next
vk_stream_sync (then cleared); well-formed calls, including ones that revisit
the same blocks in later calls, report nothing. Every kernel exits normally:
out-of-pool page ids are clamped into the pool, so all reads stay in bounds.
The reference rejects the host-visible cases of this kind before dispatch
(metal/runtime.rs:296-302)."""
import numpy as np
import pytest

import pyoracle as O
import velokv
from cases import BS, HD, make_case, oracle_layer
from test_gpu_append_copy import gpu_pool
from velokv import synth

pytestmark = pytest.mark.gpu


def expect_misuse(ctx, flag):
    with pytest.raises(velokv.VkError) as e:
        ctx.sync()
    assert e.value.code == velokv.ERR_BAD_ARG, e.value
    assert f"0x{flag:x}" in str(e.value), str(e.value)
    ctx.sync()  # cleared by the report
    assert ctx.check_misuse() == 0


@pytest.mark.parametrize("impl", ["wg", "packed", "streamk", "split-mfma", "split-valu"])
def test_decode_page_outside_pool_is_reported(ctx, impl):
    print(f"misuse: decode page outside the pool impl={impl}", flush=True)
    kind, sched, P = {"wg": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 0),
                      "packed": (velokv.DECODE_MFMA, velokv.SCHED_PACKED, 0),  # forced
                      "streamk": (velokv.DECODE_MFMA, velokv.SCHED_STREAM, 0),
                      "split-mfma": (velokv.DECODE_MFMA, velokv.SCHED_SPLIT, 64),
                      "split-valu": (velokv.DECODE_VALU, velokv.SCHED_SPLIT, 64)}[impl]
    S = 64 if impl in ("wg", "packed") else 3  # the workgroup splits need a batch that fills the GPU
    lens = [40 + 7 * i for i in range(S)]
    case = make_case(O.I8_BLK, lens, seed=701)
    pool = gpu_pool(ctx, case)
    assert ctx.check_misuse() == 0
    ctx.set_decode_kernel(kind)
    ctx.set_decode_schedule(sched)
    try:
        bt = case.block_tables.copy()
        out = ctx.alloc(S * 32 * HD * 4)
        args = dict(block_tables=None, bt_stride=bt.shape[1], partition_tokens=P)
        # well formed first: nothing to report
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), S, 32,
                         int(max(lens)), **dict(args, block_tables=ctx.upload(bt)))
        ctx.sync()
        if impl in ("wg", "packed"):
            name = ctx.decode_kernel_name(pool, S, 32, int(max(lens)), bt_stride=bt.shape[1])
            assert name.startswith("vk_decode_wg_" if impl == "wg" else "vk_decode_pk_"), name
        bt[1, 2] = pool.n_blocks + 7
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), S, 32,
                         int(max(lens)), **dict(args, block_tables=ctx.upload(bt)))
        expect_misuse(ctx, velokv.MISUSE_PAGE_OUT_OF_POOL)
        bt[1, 2] = -3
        ctx.paged_decode(pool, 0, ctx.upload(case.q), velokv.DT_F16, out, ctx.upload(case.ctx_lens), S, 32,
                         int(max(lens)), **dict(args, block_tables=ctx.upload(bt)))
        expect_misuse(ctx, velokv.MISUSE_PAGE_OUT_OF_POOL)
    finally:
        ctx.set_decode_kernel(velokv.DECODE_AUTO)
        ctx.set_decode_schedule(velokv.SCHED_AUTO)


@pytest.mark.parametrize("shared", [0, 2])
def test_tree_page_outside_pool_is_reported(ctx, shared):
    """Tree verify, with and without the shared-prefix pass (a bad page in the
    prefix row, which every sequence shares)."""
    print(f"misuse: tree page outside the pool shared={shared}", flush=True)
    N = 8
    committed = np.array([40, 40], np.int32)
    case = make_case(O.I8_BLK, committed + N, seed=702)
    pool = gpu_pool(ctx, case)  # each sequence filled through its own pages
    assert ctx.check_misuse() == 0
    bt = case.block_tables.copy()
    if shared:
        # verify as if the sequences shared their first pages (aliasing them before the
        # prefill would put two runs of one block in that append call: reported misuse)
        bt[1, :shared] = bt[0, :shared]
    q = synth.normals_f16(2 * N * 32 * HD, 7021).reshape(2, N, 32, HD)
    mask = np.tile(velokv.branching_tree([2, 2, 2], N).ancestor_mask(), (2, 1)).astype(np.uint32)
    out = ctx.alloc(2 * N * 32 * HD * 4)

    def run(table):
        ctx.tree_verify(pool, 0, ctx.upload(q), velokv.DT_F16, out, ctx.upload(committed), ctx.upload(mask), 2, N, 32,
                        int(committed.max()), block_tables=ctx.upload(table), bt_stride=table.shape[1],
                        shared_blocks=shared)

    run(bt)
    ctx.sync()
    bad = bt.copy()
    bad[:, 0 if shared else 1] = pool.n_blocks + 1
    run(bad)
    expect_misuse(ctx, velokv.MISUSE_PAGE_OUT_OF_POOL)


def test_blk_append_split_run_is_reported(ctx):
    """Tokens of one block not adjacent in a call: two runs would requantize the
    block at the same time. Later calls that continue the same blocks (one run
    each), in this layer and another, report nothing."""
    print("misuse: INT8 block split across runs", flush=True)
    case = make_case(O.I8_BLK, [40, 40], seed=703, outlier_scale=8.0)
    bt = case.block_tables
    pool = velokv.Pool(ctx, 2, case.n_blocks, BS, 8, HD, O.I8_BLK)
    assert ctx.check_misuse() == 0

    def append(layer, seq_pos):
        rows = np.array([s for s, _ in seq_pos])
        pos = np.array([p for _, p in seq_pos])
        sl = synth.slots_for_positions(bt, pos, BS, rows)
        k = np.stack([case.k[s][p] for s, p in seq_pos])
        v = np.stack([case.v[s][p] for s, p in seq_pos])
        ctx.append(pool, layer, ctx.upload(k), ctx.upload(v), velokv.DT_F16, ctx.upload(sl), len(sl))

    # well formed, and continuing the same blocks in later calls and other layers
    append(0, [(0, 0), (0, 1), (0, 2), (1, 0), (1, 1)])
    append(0, [(0, 3), (1, 2), (1, 3)])
    append(1, [(0, 0), (0, 1), (1, 0)])
    ctx.sync()
    # sequence 0's block 0 gets two runs in one call (positions 4, 5 then 6)
    append(0, [(0, 4), (0, 5), (1, 4), (0, 6)])
    expect_misuse(ctx, velokv.MISUSE_BLK_SPLIT_RUN)
    # padding between one block's tokens is allowed (still one run)
    sl = synth.slots_for_positions(bt, np.array([7, 8, 9]), BS, np.array([0, 0, 0]))
    sl = np.array([sl[0], -1, sl[1], -1, -1, sl[2]], np.int64)
    k = np.zeros((6, 8, HD), np.float16)
    ctx.append(pool, 0, ctx.upload(k), ctx.upload(k), velokv.DT_F16, ctx.upload(sl), 6)
    ctx.sync()


def test_folded_append_shared_block_is_reported(ctx):
    """vk_append_decode under the workgroup split, where each sequence's decode
    appends its own new token: two sequences whose new tokens land in the same
    block (the same last page in both table rows) would rewrite it at the same
    time and are reported; the same call with distinct blocks, repeated (a new
    claim epoch per call), reports nothing."""
    print("misuse: folded append, two sequences on one block", flush=True)
    S, H = 64, 32
    lens = np.array([40 + 3 * i for i in range(S)], np.int32)
    case = make_case(O.I8_BLK, lens, seed=705, outlier_scale=8.0)
    pool = gpu_pool(ctx, case, with_last=False)
    sl, kk, vv = case.last_slots()
    out = ctx.alloc(S * H * HD * 4)

    def call(bt, lens):
        ctx.append_decode(pool, 0, ctx.upload(kk), ctx.upload(vv), velokv.DT_F16, ctx.upload(case.q), velokv.DT_F16,
                          out, ctx.upload(lens), S, H, int(lens.max()), block_tables=ctx.upload(bt),
                          bt_stride=bt.shape[1], sum_context_len=int(lens.sum()))

    ctx.set_decode_schedule(velokv.SCHED_SPLIT)
    try:
        pl = ctx.decode_plan(pool, S, H, int(lens.max()), bt_stride=case.block_tables.shape[1],
                             sum_context_len=int(lens.sum()))
        assert pl["schedule"] == velokv.SCHED_WORKGROUP, pl
        for _ in range(2):
            call(case.block_tables, lens)
            ctx.sync()
        assert ctx.check_misuse() == 0
        bt = case.block_tables.copy()
        lens2 = lens.copy()
        lens2[1] = lens2[0]
        bt[1] = bt[0]
        call(bt, lens2)
        expect_misuse(ctx, velokv.MISUSE_BLK_SPLIT_RUN)
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
