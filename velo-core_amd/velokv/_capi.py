"""ctypes declarations of include/velokv.h and the loader of libvelokv.so.

The product path is HIP only: importing works everywhere (so CPU tests can check
the exported symbols), but creating a context without a gfx950 device or
without the built code object raises VkError -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# VELOKV_SANITIZE=1 selects the host library built under AddressSanitizer + UBSan
# (velo-core_amd/build.py --sanitize; CPU tests only)
LIB_PATH = os.path.join(HERE, "libvelokv_asan.so" if os.environ.get("VELOKV_SANITIZE") == "1" else "libvelokv.so")
CODE_OBJECT_PATH = os.path.join(HERE, "velokv_gfx950.co")

# status codes (velokv.h)
OK = 0
ERR_BAD_ARG = -1
ERR_INVALID_BLOCK_SIZE = -2
ERR_OUT_OF_PAGES = -3
ERR_TOO_MANY_PAGES = -4
ERR_NO_FREE_SLOTS = -5
ERR_NOT_WIRED = -6
ERR_NO_DEVICE = -7
ERR_HIP = -8
ERR_UNSUPPORTED = -9
ERR_UNKNOWN_HANDLE = -10

STATUS_NAMES = {
    OK: "OK", ERR_BAD_ARG: "BAD_ARG", ERR_INVALID_BLOCK_SIZE: "INVALID_BLOCK_SIZE",
    ERR_OUT_OF_PAGES: "OUT_OF_PAGES", ERR_TOO_MANY_PAGES: "TOO_MANY_PAGES",
    ERR_NO_FREE_SLOTS: "NO_FREE_SLOTS", ERR_NOT_WIRED: "NOT_WIRED", ERR_NO_DEVICE: "NO_DEVICE",
    ERR_HIP: "HIP", ERR_UNSUPPORTED: "UNSUPPORTED", ERR_UNKNOWN_HANDLE: "UNKNOWN_HANDLE",
}

# KV storage types and caller dtypes
KV_F32, KV_F16, KV_I8_REF, KV_I8_BLK = 0, 1, 2, 3
DECODE_AUTO, DECODE_VALU, DECODE_MFMA = 0, 1, 2
SCHED_AUTO, SCHED_SPLIT, SCHED_STREAM = 0, 1, 2
SCHED_WORKGROUP = 3  # reported by vk_paged_decode_plan for the workgroup split
SCHED_PACKED = 4
NOALLOC_SCRATCH_BYTES = 64 << 20  # VK_NOALLOC_SCRATCH_BYTES
DT_F32, DT_F16 = 0, 1
NIXL_HEADER_BYTES = 16
ROPE_INTERLEAVED, ROPE_HALF = 1, 2
NIXL_OK, NIXL_SHORT_HEADER, NIXL_TRUNCATED, NIXL_HANDLE_MISMATCH, NIXL_LENGTH_MISMATCH, NIXL_BAD_PAGE = range(6)
# misuse flags reported by vk_stream_sync / vk_ctx_check
MISUSE_PAGE_OUT_OF_POOL, MISUSE_BLK_SPLIT_RUN = 1, 2
# per-sequence status of vk_tree_commit
COMMIT_OK, COMMIT_BAD_ROW, COMMIT_PAST_TABLE, COMMIT_BAD_PAGE = range(4)


class VkError(RuntimeError):
    """A negative status from the C ABI, with the library's message."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.status = STATUS_NAMES.get(code, str(code))
        super().__init__(f"[{self.status}] {message}")


class PoolDesc(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("n_blocks", C.c_int32), ("block_size", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("kv_type", C.c_int32),
                ("max_slots", C.c_int32), ("max_pages_per_slot", C.c_int32)]


class LayerView(C.Structure):
    _fields_ = [("k_codes", C.c_void_p), ("v_codes", C.c_void_p), ("k_scales", C.c_void_p),
                ("v_scales", C.c_void_p), ("codes_bytes", C.c_uint64), ("scales_bytes", C.c_uint64),
                ("scale_step", C.c_uint32)]


class DecodeArgs(C.Structure):
    _fields_ = [("layer", C.c_int32), ("q", C.c_void_p), ("q_dtype", C.c_int32), ("out", C.c_void_p),
                ("block_tables", C.c_void_p), ("bt_stride", C.c_int32), ("seq_rows", C.c_void_p),
                ("context_lens", C.c_void_p), ("n_seqs", C.c_int32), ("n_heads", C.c_int32),
                ("max_context_len", C.c_int32), ("scale", C.c_float), ("partition_tokens", C.c_int32),
                ("workspace", C.c_void_p), ("workspace_bytes", C.c_uint64), ("sum_context_len", C.c_int64)]


class DecodePlan(C.Structure):
    _fields_ = [("kernel", C.c_char * 64), ("schedule", C.c_int32), ("wg_waves", C.c_int32),
                ("partition_tokens", C.c_int32), ("max_partitions", C.c_int32), ("n_workers", C.c_int32),
                ("max_blocks_per_wave", C.c_int32), ("workspace_bytes", C.c_uint64), ("merge_launch", C.c_int32)]


class TreePlan(C.Structure):
    _fields_ = [("kernel", C.c_char * 64), ("prefix_kernel", C.c_char * 64), ("prefix_chunks", C.c_int32),
                ("prefix_row_tiles", C.c_int32), ("row_tiles", C.c_int32), ("rows_per_tile", C.c_int32),
                ("partition_tokens", C.c_int32), ("max_partitions", C.c_int32), ("workspace_bytes", C.c_uint64),
                ("merge_launch", C.c_int32)]


class TreeArgs(C.Structure):
    _fields_ = [("layer", C.c_int32), ("q", C.c_void_p), ("q_dtype", C.c_int32), ("out", C.c_void_p),
                ("block_tables", C.c_void_p), ("bt_stride", C.c_int32), ("seq_rows", C.c_void_p),
                ("context_lens", C.c_void_p), ("tree_mask", C.c_void_p), ("n_seqs", C.c_int32),
                ("n_nodes", C.c_int32), ("n_heads", C.c_int32), ("max_context_len", C.c_int32),
                ("scale", C.c_float), ("partition_tokens", C.c_int32), ("workspace", C.c_void_p),
                ("workspace_bytes", C.c_uint64), ("shared_blocks", C.c_int32)]


class NixlItem(C.Structure):
    _fields_ = [("block_id", C.c_uint64), ("token_len", C.c_uint32), ("first_page", C.c_int32),
                ("wire_offset", C.c_uint64)]


P = C.c_void_p
I32 = C.c_int32
U32 = C.c_uint32
I64 = C.c_int64
U64 = C.c_uint64
PP = C.POINTER(C.c_void_p)
PI32 = C.POINTER(C.c_int32)
PU32 = C.POINTER(C.c_uint32)

# name -> argtypes (all return int32 status unless noted)
PROTOTYPES = {
    "vk_ctx_create": [C.c_int, C.c_char_p, PP],
    "vk_ctx_destroy": [P],
    "vk_ctx_arch": [P, C.c_char_p, C.c_size_t],
    "vk_kernel_launch_check": [P, C.c_char_p, I32, PI32],
    "vk_workspace_grow_bytes": [U64, U64],
    "vk_ctx_set_decode_kernel": [P, C.c_int],
    "vk_ctx_set_decode_schedule": [P, C.c_int],
    "vk_pool_create": [P, C.POINTER(PoolDesc), PP],
    "vk_pool_destroy": [P],
    "vk_pool_get_desc": [P, C.POINTER(PoolDesc)],
    "vk_pool_layer_view": [P, I32, C.POINTER(LayerView)],
    "vk_pool_block_table": [P, PP, PI32],
    "vk_pool_bytes": [P, C.POINTER(U64)],
    "vk_bind_slot": [P, U32, PU32, I32],
    "vk_slot_mapping": [P, P, P, I32, P, P, I32, P, P],
    "vk_append": [P, P, I32, P, P, I32, P, I32, P],
    "vk_rope_table": [C.POINTER(C.c_float), I32, I32, C.c_float],
    "vk_append_rope": [P, P, I32, P, I32, I32, P, P, I32, P, P, I32, P, I32, I32, P],
    "vk_paged_decode_workspace": [P, C.POINTER(DecodeArgs), C.POINTER(U64)],
    "vk_paged_decode": [P, P, C.POINTER(DecodeArgs), P],
    "vk_paged_decode_kernel": [P, C.POINTER(DecodeArgs), C.c_char_p, C.c_size_t],
    "vk_paged_decode_plan": [P, C.POINTER(DecodeArgs), C.POINTER(DecodePlan)],
    "vk_paged_decode_noalloc": [P, P, C.POINTER(DecodeArgs), P],
    "vk_append_decode": [P, P, P, P, I32, C.POINTER(DecodeArgs), P],
    "vk_append_rope_decode": [P, P, P, P, I32, P, I32, I32, C.POINTER(DecodeArgs), P],
    "vk_append_rope_decode_workspace": [P, C.POINTER(DecodeArgs), C.POINTER(U64)],
    "vk_tree_verify_workspace": [P, C.POINTER(TreeArgs), C.POINTER(U64)],
    "vk_tree_verify_plan": [P, C.POINTER(TreeArgs), C.POINTER(TreePlan)],
    "vk_tree_verify": [P, P, C.POINTER(TreeArgs), P],
    "vk_tree_mask": [PI32, I32, PU32],
    "vk_copy_blocks": [P, P, PI32, I32, P],
    "vk_tree_commit": [P, P, I32, I32, P, I32, P, P, I32, P, I32, P, P],
    "vk_nixl_payload_bytes": [P, I32, U32, C.POINTER(U64)],
    "vk_nixl_pack": [P, P, I32, I32, C.POINTER(NixlItem), I32, P, I32, P, U64, P, P],
    "vk_nixl_unpack": [P, P, I32, I32, C.POINTER(NixlItem), I32, P, I32, P, U64, P, P],
    "vk_bm_create": [I32, I32, PP],
    "vk_bm_destroy": [P],
    "vk_bm_free_pages": [P, PI32],
    "vk_bm_allocate": [P, U64, I64, PU32, I32, PI32],
    "vk_bm_release": [P, U64],
    "vk_bm_pages": [P, U64, PU32, I32, PI32],
    "vk_bm_fork": [P, U64, U64, I64, I64, PU32, I32, PI32],
    "vk_bm_cow": [P, U64, I32, PI32, PI32, PI32],
    "vk_bm_refcount": [P, U32, PI32],
    "vk_bm_block_size": [P, PI32],
    "vk_bm_extend": [P, U64, I64, PU32, I32, PI32],
    "vk_radix_create": [P, I64, PP],
    "vk_radix_destroy": [P],
    "vk_radix_insert": [P, PU32, I32, U64, C.POINTER(U64), PI32],
    "vk_radix_lookup": [P, PU32, I32, PI32, C.POINTER(U64), PI32],
    "vk_radix_len": [P, PI32],
    "vk_radix_resident_tokens": [P, C.POINTER(I64)],
    "vk_radix_capacity_tokens": [P, C.POINTER(I64)],
    "vk_radix_set_capacity": [P, I64],
    "vk_radix_evict_coldest": [P, I64, C.POINTER(U64), I32, PI32],
    "vk_radix_cache_sequence": [P, PU32, I32, U64, U64, PI32, PU32, I32, PI32, PI32, PI32, PI32],
    "vk_dev_alloc": [P, U64, PP],
    "vk_dev_free": [P, P],
    "vk_memcpy_h2d": [P, P, P, U64],
    "vk_memcpy_d2h": [P, P, P, U64],
    "vk_memset_d": [P, P, C.c_int, U64],
    "vk_stream_create": [P, PP],
    "vk_stream_destroy": [P, P],
    "vk_stream_sync": [P, P],
    "vk_ctx_check": [P, C.POINTER(U32)],
    "vk_event_create": [P, PP],
    "vk_event_destroy": [P, P],
    "vk_event_record": [P, P, P],
    "vk_event_elapsed_ms": [P, P, P, C.POINTER(C.c_float)],
    "vk_fill_normal_f16": [P, P, U64, U64, I32, C.c_float, P],
}
# entries that return something other than an int32 status
RESTYPES = {"vk_workspace_grow_bytes": C.c_uint64}

_lib = None


def lib():
    """Load libvelokv.so (built in-tree by velo-core_amd/build.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VkError(ERR_NOT_WIRED, f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, argtypes in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, C.c_int)
        L.vk_last_error.argtypes = []
        L.vk_last_error.restype = C.c_char_p
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise VkError(rc, lib().vk_last_error().decode(errors="replace"))
