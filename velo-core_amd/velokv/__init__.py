"""velokv -- MI355X (gfx950) KV-cache hot path of Velo-Core behind a C ABI.

Python host mirror of the reference's memory boundary (runtime.rs:8-42,
paged_attention.rs:92-212, metal/runtime.rs:274-324): a HIP context, K/V pools
in HBM with a slot block table, the block manager, and the three hot-path
operations (append with INT8 quantization, paged decode attention, copy-on-write
block copy) plus tree-verify attention, the accepted-path commit of a verified
tree, and NIXL wire-record pack/unpack of KV pages. Every compute call goes to the gfx950
code object through libvelokv.so.
"""
from ._capi import (  # noqa: F401
    DT_F16, DT_F32, DECODE_AUTO, DECODE_MFMA, DECODE_VALU, SCHED_AUTO, SCHED_SPLIT, SCHED_STREAM, SCHED_WORKGROUP, SCHED_PACKED, NOALLOC_SCRATCH_BYTES, KV_F16, KV_F32, KV_I8_BLK, KV_I8_REF, VkError,
    ERR_BAD_ARG, ERR_INVALID_BLOCK_SIZE, ERR_OUT_OF_PAGES, ERR_TOO_MANY_PAGES, ERR_NO_FREE_SLOTS,
    ERR_NOT_WIRED, ERR_NO_DEVICE, ERR_HIP, ERR_UNSUPPORTED, ERR_UNKNOWN_HANDLE,
    NIXL_HEADER_BYTES, NIXL_OK, NIXL_SHORT_HEADER, NIXL_TRUNCATED, NIXL_HANDLE_MISMATCH, NIXL_LENGTH_MISMATCH,
    NIXL_BAD_PAGE, ROPE_HALF, ROPE_INTERLEAVED, COMMIT_OK, COMMIT_BAD_ROW, COMMIT_PAST_TABLE, COMMIT_BAD_PAGE,
    MISUSE_PAGE_OUT_OF_POOL, MISUSE_BLK_SPLIT_RUN,
)
from .runtime import (  # noqa: F401
    BlockManager, CacheLookup, CachedSequence, Context, DeviceBuffer, Event, HipMemoryRuntime, KvCacheType,
    MemoryRuntimeConfig, Pool, RadixCache,
    SlotPool, Stream, kv_bytes_per_token_per_head, rope_table,
)
from .tree import SpeculativeTree, TreeNode, TreeVerifyResult, branching_tree  # noqa: F401
