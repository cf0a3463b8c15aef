#!/usr/bin/env python3
"""Benchmark of the KV-cache hot path on one MI355X.

Metric: paged decode-attention achieved HBM GB/s (% of peak) and
tokens/s at B=64 sequences x 8192 context, Llama-3-8B decode-layer shapes
(32 query heads, 8 KV heads, head_dim 128, block size 16), INT8 KV (per-(block,
head) fp16 scales) as the headline and fp16 KV beside it.

One step = one decode token for all 64 sequences through 32 layers: per layer,
append the new K/V token of every sequence at position 8191 (slot mapping into a
randomly scattered 40k-block pool, on-the-fly INT8 quantization) and run paged
decode attention over the full 8192-token context. With INT8 KV and no RoPE
the layer is one vk_append_decode call, whose decode (workgroup split, or
stream-K for ragged batches, where fp16 KV folds the append too) appends the
new token itself (ms_per_step_two_launches reports the same steps with the
append as a launch of its own). Inputs (pool contents, new
K/V, q) are synthetic (seeded SplitMix64 normals generated on the GPU) and are
resident in HBM before timing starts.

value        = algorithmic bytes of a step / step time (GB/s)
tokens_per_s = 64 / step time (attention-only decode throughput, 32 layers)
roofline     = one vk_paged_decode call (the decode kernel and, when a sequence
               spans several partitions, the merge kernel): algorithmic bytes per
               call / mean call time, against the 8 TB/s HBM peak. The mean call
               time is one pair of HIP events around NL x steps back-to-back calls
               on the bench's stream, divided by their number (an event packet
               between calls adds its own few microseconds, so per-call event
               pairs, reported beside it, read high). The timed step loop holds
               no event packets either: only its start and end are recorded.

--workload tree measures configuration 4 instead: 256 sequences sharing an
aliased 4096-token prefix, suffixes U[0, 512], copy-on-write of every partial
last block, 8 draft tokens appended and an 8-node tree verified per layer, then
the accepted path of every sequence committed in all layers (vk_tree_commit).
--workload nixl measures the NIXL handoff of KV pages: every sequence of the
decode workload packed into wire records (vk_nixl_pack) and unpacked into
other pages (vk_nixl_unpack), all layers.
cpu_baseline = the CPU oracle (oracle/velokv_oracle.c, a C port of the
               reference's CPU attention math on the paged INT8 layout) timed on a
               bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "velo-core_amd"))

import velokv  # noqa: E402
from velokv import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 matrix-core peak
BS, HD = 16, 128


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--kv", choices=["int8", "fp16", "int8ref", "fp32"], default="int8",
                    help="headline KV type (int8: per-(block, head) fp16 scales; int8ref: the reference's "
                         "kv_update_int8 rows, per-(token, head) fp32 scales)")
    ap.add_argument("--also", choices=["fp16", "int8", "fp32", "none"], default="fp16",
                    help="second KV type reported beside")
    ap.add_argument("--seqs", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--kv-heads", type=int, default=8)
    ap.add_argument("--pool-blocks", type=int, default=40000, help="pool capacity in 16-token blocks")
    ap.add_argument("--page", type=int, default=16, help="decode workload: tokens per page (16 k, k = 1..16)")
    ap.add_argument("--head-dim", type=int, default=128, choices=[64, 128], help="decode and tree workloads: head_dim")
    ap.add_argument("--partition", type=int, default=0, help="split-K partition tokens (0 = auto)")
    ap.add_argument("--q-dtype", choices=["fp16", "fp32"], default="fp16",
                    help="decode query dtype (fp32: the reference kernels' float q)")
    ap.add_argument("--ragged", action="store_true", help="context lengths U[1024, ctx] (configs 2/3)")
    ap.add_argument("--decode", choices=["auto", "mfma", "valu"], default="auto",
                    help="decode kernel family (vk_ctx_set_decode_kernel)")
    ap.add_argument("--sched", choices=["auto", "split", "stream", "packed"], default="auto",
                    help="decode work schedule (vk_ctx_set_decode_schedule)")
    ap.add_argument("--rope", choices=["none", "interleaved", "half"], default="none",
                    help="decode step with RoPE at each new token's position: vk_append_rope_decode (K and q "
                         "rotated inside the decode launch) where the plan folds the append, else vk_append_rope "
                         "(K rotated before quantization, q rotated in place) then the decode")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--workload", choices=["decode", "tree", "nixl"], default="decode",
                    help="decode: B x ctx decode (configs 2, 3, 5 by flags); tree: configuration 4; "
                         "nixl: pack + unpack of every sequence's KV pages in the NIXL wire format")
    ap.add_argument("--prefix", type=int, default=4096, help="tree: shared prefix tokens")
    ap.add_argument("--max-suffix", type=int, default=512, help="tree: suffix tokens U[0, max]")
    ap.add_argument("--nodes", type=int, default=8, help="tree: draft-tree nodes")
    ap.add_argument("--no-shared-prefix", action="store_true",
                    help="tree: do not pass the radix cache's shared prefix to vk_tree_verify (shared_blocks = 0)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run one vk_copy_blocks of known size (HBM counter calibration)")
    ap.add_argument("--no-configs", action="store_true",
                    help="decode workload: skip the configurations reported beside the headline in detail "
                         "(configs 2 and 3 with ragged contexts, and the headline with fp32 queries)")
    return ap.parse_args()


def decode_bytes(kv: int, S: int, H: int, Hkv: int, lens: np.ndarray, bt_stride: int, q_esz: int = 2,
                 hd: int = HD, page: int = BS) -> int:
    """Algorithmic HBM bytes of one decode call: each K/V element of every context
    token read once, its scales (one per 16-token tile and head for INT8 BLK), q,
    the output and the block-table entries used (one per page of `page` tokens;
    hd = the pool's head_dim)."""
    tok = int(lens.sum())
    blocks = int(sum(-(-int(L) // BS) for L in lens))
    pages = int(sum(-(-int(L) // page) for L in lens))
    esz = {velokv.KV_F16: 2, velokv.KV_I8_BLK: 1, velokv.KV_I8_REF: 1, velokv.KV_F32: 4}[kv]
    kvb = 2 * tok * Hkv * hd * esz
    if kv == velokv.KV_I8_BLK:
        kvb += 2 * blocks * Hkv * 2
    elif kv == velokv.KV_I8_REF:
        kvb += 2 * tok * Hkv * 4
    return kvb + S * H * hd * q_esz + S * H * hd * 4 + pages * 4 + S * 4


def append_bytes(kv: int, S: int, Hkv: int, hd: int = HD) -> int:
    """New K/V read (fp16), codes written, scales written, slot mapping read."""
    esz = {velokv.KV_F16: 2, velokv.KV_I8_BLK: 1, velokv.KV_I8_REF: 1, velokv.KV_F32: 4}[kv]
    sc = {velokv.KV_I8_BLK: 2, velokv.KV_I8_REF: 4}.get(kv, 0)
    return 2 * S * Hkv * hd * 2 + 2 * S * Hkv * hd * esz + 2 * S * Hkv * sc + S * 8


def measured_traffic(kernel: str, S: int, L: int, H: int, Hkv: int, ragged: bool):
    """HBM bytes per launch of `kernel` on this workload from the committed PMC
    summary (profiles/*.md lines 'traffic <kernel> S=..,L=..,H=..,Hkv=.. <bytes>'), or None.
    Ragged workloads (L = U[1024, ctx], lengths from seed 2024) have keys of their own."""
    key = f"S={S},L={'U[1024,%d]' % L if ragged else L},H={H},Hkv={Hkv}"
    pdir = os.path.join(ROOT, "profiles")
    for fn in sorted(os.listdir(pdir)) if os.path.isdir(pdir) else []:
        if not fn.endswith(".md"):
            continue
        for line in open(os.path.join(pdir, fn)):
            parts = line.split()
            if len(parts) == 4 and parts[0] == "traffic" and parts[1] == kernel and parts[2] == key:
                return int(parts[3])
    return None


def time_calls(ctx, stream, fn, n: int):
    """fn(i) for i < n, twice: back to back between one pair of HIP events on
    `stream` (mean ms per call), then with an event pair around each call
    (per-call ms, which include the event packets' own overhead)."""
    s0, s1 = velokv.Event(ctx), velokv.Event(ctx)
    s0.record(stream)
    for i in range(n):
        fn(i)
    s1.record(stream)
    stream.sync()
    block_ms = s0.elapsed_ms(s1) / n
    evs = [[velokv.Event(ctx), velokv.Event(ctx)] for _ in range(n)]
    for i in range(n):
        evs[i][0].record(stream)
        fn(i)
        evs[i][1].record(stream)
    stream.sync()
    return block_ms, [e[0].elapsed_ms(e[1]) for e in evs]


def run_gpu(ctx, args, kv_name: str):
    kv = {"int8": velokv.KV_I8_BLK, "int8ref": velokv.KV_I8_REF, "fp32": velokv.KV_F32}.get(kv_name, velokv.KV_F16)
    S, H, Hkv, L, NL = args.seqs, args.heads, args.kv_heads, args.ctx, args.layers
    D, PG = args.head_dim, args.page  # head_dim and tokens per page of the pool
    n_pages = args.pool_blocks * BS // PG
    if args.ragged:
        lens = synth.rng(2024).integers(1024, L + 1, S).astype(np.int32)
    else:
        lens = np.full(S, L, np.int32)
    pages = [-(-int(x) // PG) for x in lens]
    bt = synth.scatter_block_tables(n_pages, pages, seed=11, stride=-(-L // PG))
    pool = velokv.Pool(ctx, NL, n_pages, PG, Hkv, D, kv)

    # ---- fill the pool: tokens 0 .. base-1 of every sequence, per layer, base the
    # first position of the sequence's last 16-token block ----
    base = (BS * ((lens.astype(np.int64) - 1) // BS)).astype(np.int32)
    n_pre = int(base.sum())
    rows = np.repeat(np.arange(S), base)
    pos = np.concatenate([np.arange(int(x)) for x in base])
    pre_slots = ctx.upload(synth.slots_for_positions(bt, pos, PG, rows))
    kbuf = ctx.alloc(max(1, n_pre) * Hkv * D * 2)
    vbuf = ctx.alloc(max(1, n_pre) * Hkv * D * 2)
    outlier = 8.0 if kv in (velokv.KV_I8_BLK, velokv.KV_I8_REF) else 1.0
    for layer in range(NL):
        ctx.fill_normal_f16(kbuf, n_pre * Hkv * D, 1000 + 2 * layer, Hkv * D, outlier)
        ctx.fill_normal_f16(vbuf, n_pre * Hkv * D, 1001 + 2 * layer, Hkv * D, outlier)
        ctx.append(pool, layer, kbuf, vbuf, velokv.DT_F16, pre_slots, n_pre)
    ctx.sync()
    kbuf.free()
    vbuf.free()

    # ---- per-step inputs ----
    # Step i appends every sequence's new token at offset o = i % 16 of its last
    # block (position base + o, context base + o + 1), so consecutive steps walk
    # the block as a real decode does: the int8 block scale restarts at offset 0
    # and grows (requantizing the earlier codes) whenever a new row's absmax needs
    # it. New rows, q and K/V come from R input sets rotated per step.
    R = 4
    W = BS
    walk_lens = [base + o + 1 for o in range(W)]
    d_walk = [ctx.upload(x.astype(np.int32)) for x in walk_lens]
    walk_slots = [ctx.upload(synth.slots_for_positions(bt, (base + o).astype(np.int64), PG)) for o in range(W)]
    walk_max = int((base + W).max())
    new_slots = ctx.upload(synth.slots_for_positions(bt, lens.astype(np.int64) - 1, PG))
    qs, ks, vs = [], [], []
    qdt = velokv.DT_F32 if args.q_dtype == "fp32" else velokv.DT_F16
    for r in range(R):
        if qdt == velokv.DT_F32:  # seeded normals made on the host (1 MB per set at the headline shape)
            q = ctx.upload(synth.rng(7000 + r).standard_normal(S * H * D).astype(np.float32))
        else:
            q = ctx.alloc(S * H * D * 2)
            ctx.fill_normal_f16(q, S * H * D, 7000 + r, H * D)
        k = ctx.alloc(S * Hkv * D * 2)
        ctx.fill_normal_f16(k, S * Hkv * D, 8000 + r, Hkv * D, outlier)
        v = ctx.alloc(S * Hkv * D * 2)
        ctx.fill_normal_f16(v, S * Hkv * D, 9000 + r, Hkv * D, outlier)
        qs.append(q); ks.append(k); vs.append(v)
    out = ctx.alloc(S * H * D * 4)
    d_lens = ctx.upload(lens)
    d_bt = ctx.upload(bt)
    stream = velokv.Stream(ctx)
    rope = {"none": 0, "interleaved": velokv.ROPE_INTERLEAVED, "half": velokv.ROPE_HALF}[args.rope]
    if rope:
        n_pos = max(int(lens.max()), walk_max)
        d_table = ctx.upload(velokv.rope_table(n_pos, D, 500000.0))
        d_pos = ctx.upload(lens.astype(np.int32) - 1)
        d_walk_pos = [ctx.upload((base + o).astype(np.int32)) for o in range(W)]

    plan = ctx.decode_plan(pool, S, H, int(lens.max()), bt_stride=bt.shape[1], partition_tokens=args.partition,
                           q_dtype=qdt, sum_context_len=int(lens.sum()))

    def decode(layer, r, cl=None, cmax=None, csum=None):
        ctx.paged_decode(pool, layer, qs[r], qdt, out, d_lens if cl is None else cl, S, H,
                         int(lens.max()) if cmax is None else cmax,
                         block_tables=d_bt, bt_stride=bt.shape[1], partition_tokens=args.partition,
                         stream=stream, sum_context_len=int(lens.sum()) if csum is None else csum)

    # INT8 (I8_BLK) under the workgroup split or stream-K, fp16 under stream-K:
    # vk_append_decode, whose decode appends each sequence's new token itself (one
    # launch per layer), with RoPE vk_append_rope_decode, whose decode also rotates
    # the new K row and q; otherwise the append and the decode are two launches
    fused = ((kv == velokv.KV_I8_BLK and plan["schedule"] == velokv.SCHED_WORKGROUP) or
             (kv in (velokv.KV_I8_BLK, velokv.KV_F16) and plan["schedule"] == velokv.SCHED_STREAM))

    def append_decode(layer, r, o=None):
        cl, cmax, csum = ((d_lens, int(lens.max()), int(lens.sum())) if o is None else
                          (d_walk[o], walk_max, int(walk_lens[o].sum())))
        if rope:
            ctx.append_rope_decode(pool, layer, ks[r], vs[r], velokv.DT_F16, d_table, n_pos, rope, qs[r], qdt, out,
                                   cl, S, H, cmax, block_tables=d_bt, bt_stride=bt.shape[1],
                                   partition_tokens=args.partition, stream=stream, sum_context_len=csum)
            return
        ctx.append_decode(pool, layer, ks[r], vs[r], velokv.DT_F16, qs[r], qdt, out, cl, S, H, cmax,
                          block_tables=d_bt, bt_stride=bt.shape[1], partition_tokens=args.partition, stream=stream,
                          sum_context_len=csum)

    def step(i, app_evs=None, one_launch=fused, walk=True):
        """One decode step over all layers; walk: the new token at offset i % 16
        of the last block (else at position L - 1, the same every step)."""
        r = i % R
        o = i % W if walk else None
        for layer in range(NL):
            if one_launch and app_evs is None:
                append_decode(layer, r, o)
                continue
            if app_evs is not None:
                app_evs[layer][0].record(stream)
            sl = new_slots if o is None else walk_slots[o]
            if rope:
                ctx.append_rope(pool, layer, ks[r], vs[r], velokv.DT_F16, d_pos if o is None else d_walk_pos[o], sl,
                                S, d_table, n_pos, rope, q=qs[r], q_dtype=qdt, n_heads=H, stream=stream)
            else:
                ctx.append(pool, layer, ks[r], vs[r], velokv.DT_F16, sl, S, stream=stream)
            if app_evs is not None:
                app_evs[layer][1].record(stream)
            if o is None:
                decode(layer, r)
            else:
                decode(layer, r, d_walk[o], walk_max, int(walk_lens[o].sum()))

    # warm-up walks the whole last block once (every position holds a token
    # before any step is timed), then W more steps
    n_warm = max(args.warmup, 0) + W
    for i in range(n_warm):
        step(i)
    stream.sync()
    ctx.sync()

    start, end = velokv.Event(ctx), velokv.Event(ctx)
    start.record(stream)
    for i in range(args.steps):
        step(n_warm + i)
    end.record(stream)
    stream.sync()
    ctx.sync()
    total_ms = start.elapsed_ms(end)
    timed_offsets = [(n_warm + i) % W for i in range(args.steps)]
    two_ms = None
    if fused:  # the same steps with the append in a launch of its own (untimed for the value)
        start.record(stream)
        for i in range(args.steps):
            step(n_warm + i, one_launch=False)
        end.record(stream)
        stream.sync()
        two_ms = start.elapsed_ms(end) / args.steps
    # the same number of steps with every new token at position L - 1 (after the
    # first pass the block scales stop growing: the append never requantizes)
    start.record(stream)
    for i in range(args.steps):
        step(i, walk=False)
    end.record(stream)
    stream.sync()
    rep_ms = start.elapsed_ms(end) / args.steps
    # decode calls alone at the full context lengths: NL x steps back-to-back
    # calls (layers and input sets rotating)
    dec_mean_ms, dec_ms = time_calls(ctx, stream, lambda i: decode(i % NL, (i // NL) % R), NL * args.steps)
    fold_ms = (time_calls(ctx, stream, lambda i: append_decode(i % NL, (i // NL) % R, ((i // NL) % W)),
                          NL * args.steps)[0] if fused else None)
    # append time per layer, from two more (untimed) steps with events around the appends only
    app_evs = [[[velokv.Event(ctx), velokv.Event(ctx)] for _ in range(NL)] for _ in range(2)]
    for i in range(2):
        step(i, app_evs[i])
    stream.sync()
    app_ms = [app_evs[i][l][0].elapsed_ms(app_evs[i][l][1]) for i in range(2) for l in range(NL)]

    ms_step = total_ms / args.steps
    q_esz = 4 if qdt == velokv.DT_F32 else 2
    dbytes = decode_bytes(kv, S, H, Hkv, lens, bt.shape[1], q_esz, D, PG)  # one call at the full lengths
    walk_dbytes = float(np.mean([decode_bytes(kv, S, H, Hkv, walk_lens[o], bt.shape[1], q_esz, D, PG)
                                 for o in timed_offsets]))
    abytes = append_bytes(kv, S, Hkv, D)
    if rope and fused:  # one table row (D/2 cos, sin pairs) per token; q is rotated in registers
        abytes += S * D * 4
    elif rope:  # q read and written, positions, one table row per token
        abytes += 2 * S * H * D * (4 if qdt == velokv.DT_F32 else 2) + S * 4 + S * D * 4
    step_bytes = NL * (walk_dbytes + abytes)
    achieved = dbytes / (dec_mean_ms * 1e-3) / 1e9
    kname = plan["kernel"]
    res = {
        "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 2),
        "ms_per_step": round(ms_step, 4),
        "tokens_per_s": round(S / (ms_step * 1e-3), 1),
        "frac_of_peak": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "decode_bytes_per_launch": dbytes,
        "append_bytes_per_launch": abytes,
        "append": {"kernel": "vk_append_kv%d" % kv, "call": "vk_append_rope" if rope else "vk_append",
                   "rope": args.rope, "ms_mean": round(float(np.mean(app_ms)), 5),
                   "q_rotated_heads": S * H if rope else 0},
        "step_call": ("vk_append_rope_decode (RoPE and append folded into the decode launch)" if fused and rope else
                      "vk_append_decode (append folded into the decode launch)" if fused else
                      "RoPE append + decode" if rope else "append + decode"),
        "step_positions": "new token at offset i % 16 of each sequence's last block (context base + o + 1); "
                          "the block scale restarts at offset 0 and grows as the rows require",
        "step_bytes": int(step_bytes),
        "append_decode_ms_mean": round(fold_ms, 5) if fused else None,
        "ms_per_step_two_launches": round(two_ms, 4) if fused else None,
        "ms_per_step_repeated_position": round(rep_ms, 4),
        "plan": plan,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (measured_traffic(kname, S, L, H, Hkv, args.ragged)
                                 if (D, PG) == (HD, BS) else None),
                     "kernel": kname,
                     "launch_ms_mean": round(dec_mean_ms, 5), "launch_ms_min": round(float(np.min(dec_ms)), 5),
                     "launches": len(dec_ms), "call_ms_events_mean": round(float(np.mean(dec_ms)), 5)},
        "pool_gb": round(pool.nbytes / 1e9, 2),
        "workload": "S=%d, L=%s, H=%d/Hkv=%d, D=%d, page %d, %s KV, q %s" % (
            S, "U[1024,%d]" % L if args.ragged else str(L), H, Hkv, D, PG, kv_name, args.q_dtype),
        "sum_context_len": int(lens.sum()),
    }
    if args.calibrate:
        # plain copy of known size: n_pairs blocks x all layers x (K + V codes and scales)
        used = set(bt[bt >= 0].ravel().tolist())
        free = [b for b in range(args.pool_blocks) if b not in used]
        n = min(2048, len(free))
        pairs = np.stack([np.array(free[:n]), np.array(free[n:2 * n] if len(free) >= 2 * n else free[:n])], 1)
        pairs = pairs[:len(free) // 2] if len(free) < 2 * n else pairs
        ctx.copy_blocks(pool, pairs.astype(np.int32))
        ctx.sync()
        desc_tile = HD * BS * {velokv.KV_F16: 2, velokv.KV_F32: 4}.get(kv, 1)
        sc = {velokv.KV_I8_BLK: 2}.get(kv, 0)
        res["calibration_copy_bytes_read"] = int(len(pairs) * NL * 2 * Hkv * (desc_tile + sc))
    del pool
    return res


def run_tree(ctx, args):
    """Configuration 4. Per step: one copy-on-write launch for the partial last
    block of every sequence (all layers), then per layer the append of the N draft
    tokens of every sequence and one tree-verify call."""
    S, H, Hkv, NL, N = args.seqs, args.heads, args.kv_heads, args.layers, args.nodes
    D = args.head_dim  # 128, or 64 (the 64-dim tree kernels)
    kv = velokv.KV_I8_BLK if args.kv == "int8" else velokv.KV_F16
    prefix = args.prefix
    if prefix % BS:
        raise SystemExit("--prefix must be a multiple of the block size (16): the shared pages are whole blocks")
    suffix = synth.rng(4).integers(0, args.max_suffix + 1, S).astype(np.int32)
    committed = prefix + suffix
    total = committed + N
    stride = int(-(-int(total.max()) // BS))
    # Pages from the radix prefix cache (vk_radix_cache_sequence): the prefix is
    # cached once; every prompt (prefix + its own suffix) aliases the prefix's
    # pages and gets fresh pages for its suffix, then grows by the N draft slots.
    # The cache keeps a second handle on every prompt's pages, so a partially
    # filled last prompt page is shared and is copied on write (vk_bm_cow) before
    # the drafts are appended: that copy is the step's vk_copy_blocks.
    budget = -(-prefix // BS) + int(sum(-(-int(t) // BS) + 1 for t in total))
    bm = velokv.BlockManager(BS, budget)
    rc = velokv.RadixCache(bm)
    prefix_tokens = list(range(prefix))
    t0 = time.perf_counter()
    rc.cache_sequence(prefix_tokens, seq_handle=1 << 40, cache_handle=(1 << 40) + 1)
    bm.release(1 << 40)
    tables = np.zeros((S, stride), np.int32)
    fill_tables = np.zeros((S, stride), np.int32)
    pairs = []
    for s_ in range(S):
        toks = prefix_tokens + [10 ** 6 + s_ * 1000 + t for t in range(int(suffix[s_]))]
        r = rc.cache_sequence(toks, seq_handle=2 * s_, cache_handle=2 * s_ + 1)
        pages = bm.extend(2 * s_, int(total[s_]))
        fill_tables[s_, :len(pages)] = pages
        c = int(committed[s_])
        if c % BS:
            cw = bm.cow(2 * s_, c // BS)
            if cw is not None:
                pairs.append(cw)
            pages = bm.materialize_span(2 * s_)
        tables[s_, :len(pages)] = pages
    host_ms = (time.perf_counter() - t0) * 1e3
    used_pages = budget - bm.free_pages()
    reference_pages = -(-prefix // BS) + int(sum(-(-int(t) // BS) for t in total))  # a fresh page list per prompt
    n_blocks = int(max(tables.max(), fill_tables.max(), max((max(p_) for p_ in pairs), default=0))) + 1
    pblocks = -(-prefix // BS)
    perm = synth.rng(5).permutation(n_blocks).astype(np.int32)  # scatter pages over the pool
    tables, fill_tables = perm[tables], perm[fill_tables]
    pairs = perm[np.array(pairs, np.int64)] if pairs else np.zeros((0, 2), np.int32)
    pool = velokv.Pool(ctx, NL, n_blocks, BS, Hkv, D, kv)

    # ---- fill: prefix once through sequence 0's row, then every suffix ----
    outlier = 8.0 if kv == velokv.KV_I8_BLK else 1.0
    rows = np.concatenate([np.zeros(prefix, np.int64)] + [np.full(int(x), i) for i, x in enumerate(suffix)])
    pos = np.concatenate([np.arange(prefix)] + [np.arange(prefix, int(c)) for c in committed])
    fill_slots = ctx.upload(synth.slots_for_positions(fill_tables, pos, BS, rows))
    n_fill = len(pos)
    kbuf, vbuf = ctx.alloc(n_fill * Hkv * D * 2), ctx.alloc(n_fill * Hkv * D * 2)
    for layer in range(NL):
        ctx.fill_normal_f16(kbuf, n_fill * Hkv * D, 3000 + 2 * layer, Hkv * D, outlier)
        ctx.fill_normal_f16(vbuf, n_fill * Hkv * D, 3001 + 2 * layer, Hkv * D, outlier)
        ctx.append(pool, layer, kbuf, vbuf, velokv.DT_F16, fill_slots, n_fill)
    ctx.sync()
    kbuf.free()
    vbuf.free()

    # every table row starts with the prefix's pages (the radix cache aliases them)
    shared_blocks = 0 if args.no_shared_prefix else prefix // BS
    assert np.all(tables[:, :prefix // BS] == tables[0, :prefix // BS])
    dpos = (committed[:, None] + np.arange(N)[None, :]).reshape(-1)
    draft_slots = ctx.upload(synth.slots_for_positions(tables, dpos, BS, np.repeat(np.arange(S), N)))
    mask = np.tile(velokv.branching_tree([2, 2, 2, 2, 2], N).ancestor_mask(), S)
    R = 2
    qs, ks, vs = [], [], []
    qdt = velokv.DT_F32 if args.q_dtype == "fp32" else velokv.DT_F16
    for r in range(R):
        if qdt == velokv.DT_F32:  # seeded normals made on the host
            q = ctx.upload(synth.rng(7100 + r).standard_normal(S * N * H * D).astype(np.float32))
        else:
            q = ctx.alloc(S * N * H * D * 2)
            ctx.fill_normal_f16(q, S * N * H * D, 7100 + r, H * D)
        k = ctx.alloc(S * N * Hkv * D * 2)
        ctx.fill_normal_f16(k, S * N * Hkv * D, 8100 + r, Hkv * D, outlier)
        v = ctx.alloc(S * N * Hkv * D * 2)
        ctx.fill_normal_f16(v, S * N * Hkv * D, 9100 + r, Hkv * D, outlier)
        qs.append(q); ks.append(k); vs.append(v)
    out = ctx.alloc(S * N * H * D * 4)
    d_committed, d_mask, d_bt = ctx.upload(committed), ctx.upload(mask.astype(np.uint32)), ctx.upload(tables)
    # accepted path per sequence: root to node s % N (what find_best_path returns
    # when the target agrees along that branch)
    tree = velokv.branching_tree([2, 2, 2, 2, 2], N)
    acc_rows = [tree.path_nodes(s_ % N) for s_ in range(S)]
    acc = np.full((S, 32), -1, np.int32)
    n_acc = np.array([len(a) for a in acc_rows], np.int32)
    for s_, a in enumerate(acc_rows):
        acc[s_, :len(a)] = a
    d_acc, d_nacc = ctx.upload(acc), ctx.upload(n_acc)
    moved_tok = sum(len(a) - next((d for d, x in enumerate(a) if x != d), len(a)) for a in acc_rows)
    stream = velokv.Stream(ctx)

    def verify(layer, r):
        ctx.tree_verify(pool, layer, qs[r], qdt, out, d_committed, d_mask, S, N, H,
                        int(committed.max()), block_tables=d_bt, bt_stride=stride,
                        partition_tokens=args.partition, stream=stream, shared_blocks=shared_blocks)

    def step(i, app_evs=None, commit_evs=None):
        r = i % R
        if len(pairs):
            ctx.copy_blocks(pool, pairs, stream=stream)
        for layer in range(NL):
            if app_evs is not None:
                app_evs[layer][0].record(stream)
            ctx.append(pool, layer, ks[r], vs[r], velokv.DT_F16, draft_slots, S * N, stream=stream)
            if app_evs is not None:
                app_evs[layer][1].record(stream)
            verify(layer, r)
        # the accepted paths move to committed + 0, 1, ... in every layer
        if commit_evs is not None:
            commit_evs[0].record(stream)
        ctx.tree_commit(pool, d_bt, stride, d_committed, d_acc, 32, d_nacc, S, stream=stream)
        if commit_evs is not None:
            commit_evs[1].record(stream)

    for i in range(args.warmup):
        step(i)
    stream.sync()
    start, end = velokv.Event(ctx), velokv.Event(ctx)
    start.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    end.record(stream)
    stream.sync()
    total_ms = start.elapsed_ms(end)
    # verify calls alone: NL x steps back-to-back calls (layers and input sets rotating)
    tv_mean, tv_ms = time_calls(ctx, stream, lambda i: verify(i % NL, (i // NL) % R), NL * args.steps)
    # draft-append time per layer and commit time per step, from two more
    # (untimed) steps with events around the appends and the commit only
    app_evs = [[[velokv.Event(ctx), velokv.Event(ctx)] for _ in range(NL)] for _ in range(2)]
    commit_evs = [[velokv.Event(ctx), velokv.Event(ctx)] for _ in range(2)]
    for i in range(2):
        step(i, app_evs[i], commit_evs[i])
    stream.sync()
    append_ms = float(np.mean([app_evs[i][l][0].elapsed_ms(app_evs[i][l][1]) for i in range(2) for l in range(NL)]))
    commit_ms = float(np.mean([e[0].elapsed_ms(e[1]) for e in commit_evs]))

    esz = 1 if kv == velokv.KV_I8_BLK else 2
    sc = 2 if kv == velokv.KV_I8_BLK else 0
    tile = BS * D * esz
    uniq_tok = prefix + int((total - prefix).sum())
    uniq_blk = pblocks + int(sum(-(-int(t) // BS) - pblocks for t in total))
    logical_tok = int(total.sum())
    logical_blk = int(sum(-(-int(t) // BS) for t in total))
    qo = S * N * H * D * ((4 if qdt == velokv.DT_F32 else 2) + 4) + S * N * 4 + S * 4 + logical_blk * 4
    uniq = 2 * uniq_tok * Hkv * D * esz + 2 * uniq_blk * Hkv * sc + qo
    logical = 2 * logical_tok * Hkv * D * esz + 2 * logical_blk * Hkv * sc + qo
    G = H // Hkv
    rows = -(-N * G // 16) * 16
    flops = 4 * rows * D * logical_tok * Hkv  # QK and PV over every visible-or-not row of each unit
    cow_bytes = 2 * len(pairs) * NL * 2 * Hkv * (tile + sc)
    # commit: each moved token's K and V rows read and written once per layer
    commit_bytes = NL * moved_tok * 2 * 2 * Hkv * (D * esz + sc)
    step_bytes = cow_bytes + commit_bytes + NL * (uniq + append_bytes(kv, S * N, Hkv, D))
    ms_step = total_ms / args.steps
    ach = uniq / (tv_mean * 1e-3) / 1e9
    rt = 2 if N * G > 16 else 1
    qsfx = 0 if qdt == velokv.DT_F32 else 1
    gtag = "gx_d64" if D == 64 else "g%d" % G
    kname = "vk_tree_kv%d_%s_r%d_q%d" % (kv, gtag, rt, qsfx)
    call_kernels = [kname, "vk_decode_merge"]
    if shared_blocks and kv in (velokv.KV_I8_BLK, velokv.KV_F16):
        # the rest of each context runs in one partition (no merge) while it fits 4096 tokens
        rest = max(int(committed.max()) - shared_blocks * BS, BS - 1) + N
        call_kernels = ["vk_tree_pfx_kv%d_%s_q%d" % (kv, gtag, qsfx), kname] + (["vk_decode_merge"] if rest > 4096 else [])
    tflops = flops / (tv_mean * 1e-3) / 1e12
    return {
        "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 2),
        "ms_per_step": round(ms_step, 4),
        "tokens_per_s": round(S / (ms_step * 1e-3), 1),
        "draft_tokens_per_s": round(S * N / (ms_step * 1e-3), 1),
        "unique_bytes_per_launch": uniq, "logical_bytes_per_launch": logical, "cow_pairs": int(len(pairs)),
        "radix": {"host_ms": round(host_ms, 3), "pages": int(used_pages), "pages_without_aliasing": int(reference_pages),
                  "pool_gb": round(pool.nbytes / 1e9, 3),
                  "pool_gb_without_aliasing": round(pool.nbytes / 1e9 * reference_pages / used_pages, 3)},
        "draft_append": {"kernel": "vk_append_kv%d" % kv, "ms_mean": round(append_ms, 5), "tokens": S * N},
        "commit": {"kernel": "vk_tree_commit_kv%d" % kv, "ms_mean": round(commit_ms, 5), "layers": NL,
                   "accepted_tokens": int(n_acc.sum()), "moved_tokens": int(moved_tok)},
        "logical_gbs": round(logical / (tv_mean * 1e-3) / 1e9, 2),
        "mfma_tflops": round(tflops, 2),
        "shared_blocks": shared_blocks,
        "call_kernels": call_kernels,
        # One vk_tree_verify call (all of call_kernels, timed together) against
        # the matrix cores' dense fp16 peak: QK and PV of every row over its
        # committed context and the tree nodes. The shared prefix stays in L2, so
        # the call is bound by matrix and vector issue, not by HBM; the HBM view
        # (unique bytes over the same time) is kept beside it.
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "vk_tree_verify call: " + " + ".join(call_kernels),
                     "flops_per_launch": int(flops),
                     "launch_ms_mean": round(tv_mean, 5), "launch_ms_min": round(float(np.min(tv_ms)), 5),
                     "launches": len(tv_ms), "call_ms_events_mean": round(float(np.mean(tv_ms)), 5)},
        "roofline_hbm": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "bytes_per_launch": uniq},
        "pool_gb": round(pool.nbytes / 1e9, 2),
        "workload": "S=%d, prefix %d (aliased%s), suffix U[0,%d], %d-node tree, H=%d/Hkv=%d, D=%d, %s KV, %d layers" %
                    (S, prefix, ", shared_blocks %d" % shared_blocks if shared_blocks else "", args.max_suffix, N, H,
                     Hkv, D, args.kv, NL),
    }


def run_nixl(ctx, args):
    """NIXL handoff of the decode workload's KV: one record per sequence (all
    layers, ceil(L/16) pages) packed from the pool into a wire buffer in HBM, then
    unpacked into a second set of pages of the same pool. Bytes per call = payload
    read + payload written + headers."""
    kv = velokv.KV_I8_BLK if args.kv == "int8" else velokv.KV_F16
    S, Hkv, L, NL = args.seqs, args.kv_heads, args.ctx, args.layers
    if args.ragged:
        lens = synth.rng(2024).integers(1024, L + 1, S).astype(np.int32)
    else:
        lens = np.full(S, L, np.int32)
    pages = [-(-int(x) // BS) for x in lens]
    need = 2 * sum(pages)
    if "--pool-blocks" not in sys.argv:
        args.pool_blocks = max(args.pool_blocks, need)
    if need > args.pool_blocks:
        raise SystemExit(f"--pool-blocks {args.pool_blocks} < {need} pages (source and destination)")
    perm = synth.rng(12).permutation(args.pool_blocks).astype(np.int32)
    src_pages, dst_pages = perm[:need // 2], perm[need // 2:need]
    pool = velokv.Pool(ctx, NL, args.pool_blocks, BS, Hkv, HD, kv)
    # fill the source pages of every layer with synthetic K/V through the append path
    n_tok = int(lens.sum())
    firsts = np.concatenate([[0], np.cumsum(pages)[:-1]]).astype(np.int64)
    bt = np.zeros((S, max(pages)), np.int32)
    for s_ in range(S):
        bt[s_, :pages[s_]] = src_pages[firsts[s_]:firsts[s_] + pages[s_]]
    rows = np.repeat(np.arange(S), lens)
    pos = np.concatenate([np.arange(int(x)) for x in lens])
    slots = ctx.upload(synth.slots_for_positions(bt, pos, BS, rows))
    kbuf, vbuf = ctx.alloc(n_tok * Hkv * HD * 2), ctx.alloc(n_tok * Hkv * HD * 2)
    outlier = 8.0 if kv == velokv.KV_I8_BLK else 1.0
    for layer in range(NL):
        ctx.fill_normal_f16(kbuf, n_tok * Hkv * HD, 5000 + 2 * layer, Hkv * HD, outlier)
        ctx.fill_normal_f16(vbuf, n_tok * Hkv * HD, 5001 + 2 * layer, Hkv * HD, outlier)
        ctx.append(pool, layer, kbuf, vbuf, velokv.DT_F16, slots, n_tok)
    ctx.sync()
    kbuf.free()
    vbuf.free()
    items, off = [], 0
    for s_ in range(S):
        items.append((s_, int(lens[s_]), int(firsts[s_]), off))
        off += 16 + pool.nixl_payload_bytes(int(lens[s_]))
        off = (off + 255) // 256 * 256
    wire_bytes = off
    payload = sum(pool.nixl_payload_bytes(int(x)) for x in lens)
    wire = ctx.alloc(wire_bytes)
    d_src, d_dst = ctx.upload(src_pages), ctx.upload(dst_pages)
    st = ctx.alloc(4 * S)
    stream = velokv.Stream(ctx)

    def step(evs=None):
        if evs is not None:
            evs[0].record(stream)
        ctx.nixl_pack(pool, items, d_src, len(src_pages), wire, wire_bytes, st, stream=stream)
        if evs is not None:
            evs[1].record(stream)
        ctx.nixl_unpack(pool, items, d_dst, len(dst_pages), wire, wire_bytes, st, stream=stream)
        if evs is not None:
            evs[2].record(stream)

    for _ in range(args.warmup):
        step()
    stream.sync()
    status = st.download((S,), np.int32)
    if np.any(status != velokv.NIXL_OK):
        raise SystemExit(f"nixl statuses not OK: {np.unique(status)}")
    evs = [[velokv.Event(ctx) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(evs[i])
    stream.sync()
    pack_ms = [e[0].elapsed_ms(e[1]) for e in evs]
    unpack_ms = [e[1].elapsed_ms(e[2]) for e in evs]
    call_bytes = 2 * payload + 16 * S
    pk, up = float(np.mean(pack_ms)), float(np.mean(unpack_ms))
    ms_step = pk + up
    ach = call_bytes / (pk * 1e-3) / 1e9
    return {
        "value": round(2 * call_bytes / (ms_step * 1e-3) / 1e9, 2),
        "ms_per_step": round(ms_step, 4),
        "payload_bytes": int(payload), "records": S,
        "pack": {"ms_mean": round(pk, 4), "gbs": round(call_bytes / (pk * 1e-3) / 1e9, 2)},
        "unpack": {"ms_mean": round(up, 4), "gbs": round(call_bytes / (up * 1e-3) / 1e9, 2)},
        "handles_per_s": round(S / (ms_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("vk_nixl_copy", S, L, args.heads, Hkv, args.ragged),
                     "kernel": "vk_nixl_copy",
                     "launch_ms_mean": round(pk, 5), "launch_ms_min": round(float(np.min(pack_ms)), 5),
                     "launches": len(pack_ms)},
        "pool_gb": round(pool.nbytes / 1e9, 2), "wire_gb": round(wire_bytes / 1e9, 2),
        "workload": "%d records, L=%s, Hkv=%d, D=128, bs=16, %s KV, %d layers, pack then unpack into other pages" %
                    (S, "U[1024,%d]" % L if args.ragged else str(L), Hkv, args.kv, NL),
    }


def cpu_baseline(args):
    """The oracle's paged INT8 decode (llama_cpu.rs math on the paged layout) on a
    bounded sample: 4 sequences x 8192 context x 32 heads, one layer."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O
    Ssmp, L, H, Hkv = 4, args.ctx, args.heads, args.kv_heads
    lens = np.full(Ssmp, L, np.int32)
    pages = [-(-L // BS)] * Ssmp
    nb = sum(pages)
    bt = synth.scatter_block_tables(nb, pages, seed=3)
    layer = O.Layer(nb, Hkv, BS, HD, O.I8_BLK)
    row = Hkv * HD
    for s in range(Ssmp):
        k = synth.normals_f16(L * row, 50 + 2 * s, row, 8.0).reshape(L, Hkv, HD)
        v = synth.normals_f16(L * row, 51 + 2 * s, row, 8.0).reshape(L, Hkv, HD)
        O.append(layer, k, v, synth.slots_for_positions(bt, np.arange(L), BS, np.full(L, s)))
    q = synth.normals_f16(Ssmp * H * HD, 77).reshape(Ssmp, H, HD)
    nbytes = decode_bytes(velokv.KV_I8_BLK, Ssmp, H, Hkv, lens, bt.shape[1])

    def timed(threads):
        O.set_threads(threads)
        ts = []
        t_end = time.time() + args.cpu_seconds / 2
        while len(ts) < 3 or (time.time() < t_end and len(ts) < 9):
            t0 = time.perf_counter()
            O.paged_decode(layer, q, bt, lens)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    cores = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    t1 = timed(1)
    tn = timed(cores)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(nbytes / tn / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
        "tokens_per_s": round(Ssmp / (tn * args.layers), 3),
        "sample": f"oracle paged INT8 decode, {Ssmp} seqs x {L} ctx x {H} heads, 1 layer, median of runs; "
                  f"tokens/s scaled to {args.layers} layers",
        "single_thread": {"value": round(nbytes / t1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                          "seconds_per_layer": round(t1, 4)},
        "seconds_per_layer": round(tn, 4), "cpu_model": model,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this build is the "
              "single-GPU KV-cache hot path (no collectives)", file=sys.stderr)
        sys.exit(2)
    ctx = velokv.Context(0)
    ctx.set_decode_kernel({"auto": velokv.DECODE_AUTO, "mfma": velokv.DECODE_MFMA,
                           "valu": velokv.DECODE_VALU}[args.decode])
    ctx.set_decode_schedule({"auto": velokv.SCHED_AUTO, "split": velokv.SCHED_SPLIT,
                             "stream": velokv.SCHED_STREAM, "packed": velokv.SCHED_PACKED}[args.sched])
    if args.workload == "tree":
        if args.seqs == 64 and "--seqs" not in sys.argv:
            args.seqs = 256
        t = run_tree(ctx, args)
        print(json.dumps({
            "metric": "tree-verify attention GB/s (unique bytes) + tokens/s, configuration 4",
            "value": t["value"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": t["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "i8" if args.kv == "int8" else "f16", "data": "synthetic",
            "config": {"workload": t["workload"], "global_batch": args.seqs, "seq_len": args.prefix,
                       "parallelism": "single GPU"},
            "tokens_per_s": t["tokens_per_s"], "roofline": t["roofline"], "cpu_baseline": None, "detail": t}))
        return
    if args.workload == "nixl":
        t = run_nixl(ctx, args)
        print(json.dumps({
            "metric": "NIXL KV-page pack + unpack GB/s (bytes read + written)",
            "value": t["value"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": t["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "u8", "data": "synthetic",
            "config": {"workload": t["workload"], "global_batch": args.seqs, "seq_len": args.ctx,
                       "parallelism": "single GPU"},
            "roofline": t["roofline"], "cpu_baseline": None, "detail": t}))
        return
    head = run_gpu(ctx, args, args.kv)
    also = None
    if args.also != "none" and args.also != args.kv:
        also = run_gpu(ctx, args, args.also)
    configs = {}
    if (not args.no_configs and not args.ragged and args.kv == "int8" and args.q_dtype == "fp16"
            and (args.page, args.head_dim) == (BS, HD)):
        # benchmark configurations 2 (fp16) and 3 (INT8 with outliers): the same shapes with
        # L ~ U[1024, ctx]; and the headline with the reference kernels' fp32 q
        import copy
        rag = copy.copy(args)
        rag.ragged, rag.steps, rag.warmup = True, min(args.steps, 10), min(args.warmup, 2)
        configs["config2_fp16_ragged"] = run_gpu(ctx, rag, "fp16")
        configs["config3_int8_ragged"] = run_gpu(ctx, rag, "int8")
        f32 = copy.copy(args)
        f32.q_dtype, f32.steps, f32.warmup = "fp32", min(args.steps, 10), min(args.warmup, 2)
        configs["headline_int8_fp32q"] = run_gpu(ctx, f32, "int8")
        # the reference's default cache type (fp32 K/V, fp32 q) at the headline shape
        configs["headline_fp32_kv"] = run_gpu(ctx, f32, "fp32")
        # benchmark configuration 4: radix-shared 4096-token prefix, 256 sequences, 8-node tree verify + commit
        c4 = copy.copy(args)
        c4.seqs, c4.steps, c4.warmup = 256, min(args.steps, 10), min(args.warmup, 2)
        configs["config4_tree"] = run_tree(ctx, c4)
        # benchmark configuration 5, one GPU's share: 32 x 32768, 64 / 8 heads, INT8, 80 layers, 65,536-block pool
        c5 = copy.copy(args)
        c5.seqs, c5.ctx, c5.heads, c5.layers, c5.pool_blocks = 32, 32768, 64, 80, 65536
        c5.steps, c5.warmup = min(args.steps, 10), min(args.warmup, 2)
        configs["config5_s32_ctx32k"] = run_gpu(ctx, c5, "int8")
    cpu = None if args.no_cpu else cpu_baseline(args)
    workload = ("S=%d, L=%s, H=%d/Hkv=%d, D=%d, bs=%d, %s KV, %d layers, %sappend+decode per layer, pool %d blocks" %
                (args.seqs, "U[1024,%d]" % args.ctx if args.ragged else str(args.ctx), args.heads, args.kv_heads,
                 args.head_dim, args.page,
                 {"int8": "INT8 per-(block,head) fp16-scale", "int8ref": "INT8 per-(token,head) fp32-scale (reference rows)",
                  "fp32": "fp32"}.get(args.kv, "fp16"), args.layers,
                 "" if args.rope == "none" else "RoPE(%s)+" % args.rope, args.pool_blocks * BS // args.page))
    line = {
        "metric": "paged decode-attn achieved HBM GB/s (% peak) + tokens/s, B=64 ctx=8k, fp16/INT8 KV",
        "value": head["value"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "i8" if args.kv.startswith("int8") else {"fp32": "f32"}.get(args.kv, "f16"),
        "data": "synthetic (seeded SplitMix64 normals, 1% outlier channels x8 for INT8, random block scatter)",
        "config": {"workload": workload, "global_batch": args.seqs, "seq_len": args.ctx, "parallelism": "single GPU"},
        "tokens_per_s": head["tokens_per_s"], "frac_of_peak": head["frac_of_peak"],
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "detail": {args.kv: head, **({args.also: also} if also else {}), **configs},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
