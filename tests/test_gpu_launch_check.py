"""Workgroup sizes are checked against each kernel's compiled limit before any
launch (vk_kernel_launch_check, run by every launch of the library): a launch
of vk_decode_merge_sk (compiled for 256 threads) with 1024-thread workgroups
once faulted the device in a throw-away host build; now such a launch is
VK_ERR_BAD_ARG. Nothing here launches a kernel: the planned shape of each
schedule is checked against the limit the context read at creation."""
import numpy as np
import pytest

import velokv

pytestmark = pytest.mark.gpu


def test_oversized_workgroup_is_refused_without_launching(ctx):
    print("launch check: merge kernels at 1024 / 256 threads", flush=True)
    for k in ("vk_decode_merge_sk", "vk_decode_merge"):
        with pytest.raises(velokv.VkError) as e:
            ctx.launch_check(k, 1024)
        assert e.value.code == velokv.ERR_BAD_ARG
        assert k in str(e.value) and "256" in str(e.value)
        assert ctx.launch_check(k, 256) == 256
    with pytest.raises(velokv.VkError) as e:
        ctx.launch_check("vk_decode_merge_sk", 0)
    assert e.value.code == velokv.ERR_BAD_ARG
    with pytest.raises(velokv.VkError) as e:
        ctx.launch_check("vk_no_such_kernel", 64)
    assert e.value.code == velokv.ERR_NOT_WIRED


# (kv type, seqs, heads, context, schedule forced, sum of lengths) -> the planned
# kernel and workgroup size must fit its limit
PLANS = [
    (velokv.KV_I8_BLK, 64, 32, 8192, velokv.SCHED_AUTO, 64 * 8192),        # workgroup split, 4 waves
    (velokv.KV_I8_BLK, 32, 64, 32768, velokv.SCHED_AUTO, 32 * 32768),      # workgroup split, 8 waves
    (velokv.KV_I8_BLK, 64, 32, 8192, velokv.SCHED_AUTO, 64 * 4608),        # stream-K
    (velokv.KV_I8_BLK, 64, 32, 8192, velokv.SCHED_PACKED, 64 * 4608),      # packed, 8 waves
    (velokv.KV_F16, 64, 32, 8192, velokv.SCHED_AUTO, 64 * 8192),           # split-K (dot2)
    (velokv.KV_F32, 64, 32, 8192, velokv.SCHED_AUTO, 64 * 8192),           # fp32 workgroup split
]


@pytest.mark.parametrize("kv,S,H,L,sched,sum_l", PLANS)
def test_planned_shapes_fit_the_kernels(ctx, kv, S, H, L, sched, sum_l):
    print(f"launch check: plan kv={kv} S={S} H={H} L={L} sched={sched}", flush=True)
    pool = velokv.Pool(ctx, 1, 64, 16, 8, 128, kv)
    ctx.set_decode_schedule(sched)
    try:
        pl = ctx.decode_plan(pool, S, H, L, bt_stride=L // 16, sum_context_len=sum_l)
    finally:
        ctx.set_decode_schedule(velokv.SCHED_AUTO)
    threads = 64 * pl["wg_waves"] if pl["wg_waves"] > 0 else 64  # split-K: one wave per workgroup
    if pl["schedule"] == velokv.SCHED_STREAM:
        assert pl["wg_waves"] == 4, pl  # four stream-K workers per workgroup
    assert ctx.launch_check(pl["kernel"], threads) >= threads
    if pl["merge_launch"]:
        merge = "vk_decode_merge_sk" if pl["schedule"] == velokv.SCHED_STREAM else "vk_decode_merge"
        assert ctx.launch_check(merge, 256) == 256
    app = "vk_append_kv%d" % kv
    assert ctx.launch_check(app, 128) == 128
    del pool


def test_tree_plan_shapes_fit_the_kernels(ctx):
    """vk_tree_verify_plan at configuration 4's shape (256 sequences, 8 nodes,
    GQA 4, a 256-page shared prefix): the prefix pass (16 waves per workgroup)
    and the tree kernel (one wave) fit their kernels' limits."""
    print("launch check: tree plan, config 4 shape", flush=True)
    pool = velokv.Pool(ctx, 1, 64, 16, 8, 128, velokv.KV_I8_BLK)
    pl = ctx.tree_plan(pool, 256, 8, 32, 4608, bt_stride=300, shared_blocks=256)
    assert pl["prefix_chunks"] == 1 and pl["prefix_row_tiles"] == 32 and pl["row_tiles"] == 1, pl
    assert pl["rows_per_tile"] == 32 and not pl["merge_launch"], pl
    assert ctx.launch_check(pl["prefix_kernel"], 1024) == 1024
    assert ctx.launch_check(pl["kernel"], 64) >= 64
    del pool
