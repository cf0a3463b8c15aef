"""Host objects over the C ABI, named after the reference's memory boundary.

Reference interfaces mirrored here:
  KvCacheType            paged_attention.rs:27-35
  MemoryRuntimeConfig    runtime.rs:44-88
  MemoryRuntime          runtime.rs:24-42 (store / allocator / bind_slot)
  PagedBlockAllocator    runtime.rs:14-22, PagedAttentionBlockManager paged_attention.rs:92-212
  KvBlockStore           runtime.rs:8-12, InMemoryKvStore kv_store.rs:25-93
  SlotPool               slot_manager.rs:20-60
  kv_bytes_per_token_per_head  model_loader.rs:129-140
"""
from __future__ import annotations

import ctypes as C
import enum
from collections import deque
from dataclasses import dataclass

import numpy as np

from . import _capi
from ._capi import DT_F16, DT_F32, KV_F16, KV_F32, KV_I8_BLK, KV_I8_REF, VkError, check, lib


class KvCacheType(enum.Enum):
    """paged_attention.rs:27-35 plus the two types this build adds."""
    Fp32 = "fp32"
    Int8 = "int8"          # per-(token, head) fp32 scale (kernels.metal:753-802)
    Fp8 = "fp8"            # routed to the Int8 kernels, as metal/model.rs:404,442 does
    Fp16 = "fp16"
    Int8Block = "int8blk"  # per-(block, head) fp16 scale, round-half-even codes

    @property
    def code(self) -> int:
        return {KvCacheType.Fp32: KV_F32, KvCacheType.Int8: KV_I8_REF, KvCacheType.Fp8: KV_I8_REF,
                KvCacheType.Fp16: KV_F16, KvCacheType.Int8Block: KV_I8_BLK}[self]


def kv_bytes_per_token_per_head(head_dim: int, kv_type: KvCacheType, block_size: int = 16) -> float:
    """model_loader.rs:129-140: Fp32 4*D, Int8/Fp8 D+4. Fp16 2*D; Int8Block D codes
    plus one 2-byte scale per block (2/block_size per token)."""
    return {KvCacheType.Fp32: 4 * head_dim, KvCacheType.Int8: head_dim + 4, KvCacheType.Fp8: head_dim + 4,
            KvCacheType.Fp16: 2 * head_dim, KvCacheType.Int8Block: head_dim + 2.0 / block_size}[kv_type]


def _dtype_code(a: np.dtype) -> int:
    a = np.dtype(a)
    if a == np.float16:
        return DT_F16
    if a == np.float32:
        return DT_F32
    raise VkError(_capi.ERR_BAD_ARG, f"unsupported element type {a}")


class Context:
    """A HIP device with the gfx950 code object loaded (vk_ctx_create)."""

    def __init__(self, device: int = 0, code_object: str | None = None):
        h = C.c_void_p()
        path = code_object.encode() if code_object else None
        check(lib().vk_ctx_create(device, path, C.byref(h)))
        self.h = h
        self.device = device

    def close(self):
        if self.h:
            lib().vk_ctx_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_decode_kernel(self, kind: int):
        """_capi.DECODE_AUTO / DECODE_VALU / DECODE_MFMA (vk_ctx_set_decode_kernel)."""
        check(lib().vk_ctx_set_decode_kernel(self.h, kind))

    def set_decode_schedule(self, schedule: int):
        """_capi.SCHED_AUTO / SCHED_SPLIT / SCHED_STREAM (vk_ctx_set_decode_schedule)."""
        check(lib().vk_ctx_set_decode_schedule(self.h, schedule))

    @property
    def arch(self) -> str:
        buf = C.create_string_buffer(64)
        check(lib().vk_ctx_arch(self.h, buf, 64))
        return buf.value.decode()

    # ---- memory helpers ----
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = DeviceBuffer(self, max(a.nbytes, 1))
        b.upload(a)
        b.shape, b.dtype = a.shape, a.dtype
        return b

    def sync(self, stream=None):
        """vk_stream_sync: raises VkError (ERR_BAD_ARG) when a kernel reported misuse."""
        check(lib().vk_stream_sync(self.h, _sptr(stream)))

    def check_misuse(self) -> int:
        """vk_ctx_check: waits for the device, returns the misuse flags read (and clears
        them) without raising."""
        f = C.c_uint32()
        lib().vk_ctx_check(self.h, C.byref(f))
        return f.value

    # ---- hot path ----
    def slot_mapping(self, pool: "Pool", positions, block_tables=None, bt_stride=0, seq_rows=None,
                     out=None, stream=None):
        n = positions.nbytes // 4
        out = out if out is not None else self.alloc(8 * max(n, 1))
        check(lib().vk_slot_mapping(self.h, pool.h, _bptr(block_tables), bt_stride, _bptr(seq_rows),
                                    _bptr(positions), n, _bptr(out), _sptr(stream)))
        return out

    def append(self, pool: "Pool", layer: int, k, v, in_dtype: int, slot_mapping, n_tok: int, stream=None):
        check(lib().vk_append(self.h, pool.h, layer, _bptr(k), _bptr(v), in_dtype, _bptr(slot_mapping), n_tok,
                              _sptr(stream)))

    def append_rope(self, pool: "Pool", layer: int, k, v, in_dtype: int, positions, slot_mapping, n_tok: int,
                    cos_sin, n_pos: int, style: int, q=None, q_dtype: int = DT_F16, n_heads: int = 0, stream=None):
        """vk_append_rope: K rotated by position and appended, q (optional) rotated in place."""
        check(lib().vk_append_rope(self.h, pool.h, layer, _bptr(q), q_dtype, n_heads, _bptr(k), _bptr(v), in_dtype,
                                   _bptr(positions), _bptr(slot_mapping), n_tok, _bptr(cos_sin), n_pos, style,
                                   _sptr(stream)))

    def paged_decode(self, pool: "Pool", layer: int, q, q_dtype: int, out, context_lens, n_seqs: int, n_heads: int,
                     max_context_len: int, block_tables=None, bt_stride: int = 0, seq_rows=None, scale: float = 0.0,
                     partition_tokens: int = 0, workspace=None, workspace_bytes: int = 0, stream=None,
                     sum_context_len: int = 0):
        a = _capi.DecodeArgs(layer, _bptr(q), q_dtype, _bptr(out), _bptr(block_tables), bt_stride, _bptr(seq_rows),
                             _bptr(context_lens), n_seqs, n_heads, max_context_len, scale, partition_tokens,
                             _bptr(workspace), workspace_bytes, sum_context_len)
        check(lib().vk_paged_decode(self.h, pool.h, C.byref(a), _sptr(stream)))

    def append_decode(self, pool: "Pool", layer: int, k_new, v_new, in_dtype: int, q, q_dtype: int, out,
                      context_lens, n_seqs: int, n_heads: int, max_context_len: int, block_tables=None,
                      bt_stride: int = 0, seq_rows=None, scale: float = 0.0, partition_tokens: int = 0,
                      workspace=None, workspace_bytes: int = 0, stream=None, sum_context_len: int = 0):
        """vk_append_decode: the new token of every sequence appended at context_len - 1, then decode."""
        a = _capi.DecodeArgs(layer, _bptr(q), q_dtype, _bptr(out), _bptr(block_tables), bt_stride, _bptr(seq_rows),
                             _bptr(context_lens), n_seqs, n_heads, max_context_len, scale, partition_tokens,
                             _bptr(workspace), workspace_bytes, sum_context_len)
        check(lib().vk_append_decode(self.h, pool.h, _bptr(k_new), _bptr(v_new), in_dtype, C.byref(a),
                                     _sptr(stream)))

    def append_rope_decode(self, pool: "Pool", layer: int, k_new, v_new, in_dtype: int, cos_sin, n_pos: int,
                           rope_style: int, q, q_dtype: int, out, context_lens, n_seqs: int, n_heads: int,
                           max_context_len: int, block_tables=None, bt_stride: int = 0, seq_rows=None,
                           scale: float = 0.0, partition_tokens: int = 0, workspace=None, workspace_bytes: int = 0,
                           stream=None, sum_context_len: int = 0):
        """vk_append_rope_decode: RoPE at context_len - 1 of the new K rows and of q (q left unchanged), the
        append, then decode over the rotated q."""
        a = _capi.DecodeArgs(layer, _bptr(q), q_dtype, _bptr(out), _bptr(block_tables), bt_stride, _bptr(seq_rows),
                             _bptr(context_lens), n_seqs, n_heads, max_context_len, scale, partition_tokens,
                             _bptr(workspace), workspace_bytes, sum_context_len)
        check(lib().vk_append_rope_decode(self.h, pool.h, _bptr(k_new), _bptr(v_new), in_dtype, _bptr(cos_sin),
                                          n_pos, rope_style, C.byref(a), _sptr(stream)))

    def paged_decode_noalloc(self, pool: "Pool", layer: int, q, q_dtype: int, out, context_lens, n_seqs: int,
                             n_heads: int, max_context_len: int, block_tables=None, bt_stride: int = 0,
                             seq_rows=None, scale: float = 0.0, partition_tokens: int = 0, stream=None,
                             sum_context_len: int = 0):
        """vk_paged_decode_noalloc: the same decode with its split-K scratch in the library's
        per-device array (allocates nothing)."""
        a = _capi.DecodeArgs(layer, _bptr(q), q_dtype, _bptr(out), _bptr(block_tables), bt_stride, _bptr(seq_rows),
                             _bptr(context_lens), n_seqs, n_heads, max_context_len, scale, partition_tokens,
                             None, 0, sum_context_len)
        check(lib().vk_paged_decode_noalloc(self.h, pool.h, C.byref(a), _sptr(stream)))

    def decode_plan(self, pool: "Pool", n_seqs, n_heads, max_context_len, bt_stride=0, partition_tokens=0,
                    q_dtype=DT_F16, sum_context_len=0) -> dict:
        """vk_paged_decode_plan as a dict (kernel, schedule, waves, partitions, blocks per wave, workspace)."""
        a = _capi.DecodeArgs(0, None, q_dtype, None, C.c_void_p(1) if bt_stride else None, bt_stride, None, None,
                             n_seqs, n_heads, max_context_len, 0.0, partition_tokens, None, 0, sum_context_len)
        p = _capi.DecodePlan()
        check(lib().vk_paged_decode_plan(pool.h, C.byref(a), C.byref(p)))
        return {"kernel": p.kernel.decode(), "schedule": p.schedule, "wg_waves": p.wg_waves,
                "partition_tokens": p.partition_tokens, "max_partitions": p.max_partitions,
                "n_workers": p.n_workers, "max_blocks_per_wave": p.max_blocks_per_wave,
                "workspace_bytes": p.workspace_bytes, "merge_launch": bool(p.merge_launch)}

    def launch_check(self, kernel: str, threads: int) -> int:
        """vk_kernel_launch_check: the kernel's workgroup limit; raises VkError when
        `threads` exceeds it (nothing is launched)."""
        mx = C.c_int32()
        check(lib().vk_kernel_launch_check(self.h, kernel.encode(), threads, C.byref(mx)))
        return mx.value

    def decode_workspace_bytes(self, pool: "Pool", n_seqs, n_heads, max_context_len, bt_stride=0,
                               partition_tokens=0, q_dtype=DT_F16, sum_context_len=0) -> int:
        a = _capi.DecodeArgs(0, None, q_dtype, None, C.c_void_p(1) if bt_stride else None, bt_stride, None, None,
                             n_seqs, n_heads, max_context_len, 0.0, partition_tokens, None, 0, sum_context_len)
        n = C.c_uint64()
        check(lib().vk_paged_decode_workspace(pool.h, C.byref(a), C.byref(n)))
        return n.value

    def append_rope_decode_workspace_bytes(self, pool: "Pool", n_seqs, n_heads, max_context_len, bt_stride=0,
                                           partition_tokens=0, q_dtype=DT_F16, sum_context_len=0) -> int:
        """vk_append_rope_decode_workspace: the decode's workspace, plus the rotated
        q rows when the RoPE is not folded into the decode kernel."""
        a = _capi.DecodeArgs(0, None, q_dtype, None, C.c_void_p(1) if bt_stride else None, bt_stride, None, None,
                             n_seqs, n_heads, max_context_len, 0.0, partition_tokens, None, 0, sum_context_len)
        n = C.c_uint64()
        check(lib().vk_append_rope_decode_workspace(pool.h, C.byref(a), C.byref(n)))
        return n.value

    def decode_kernel_name(self, pool: "Pool", n_seqs, n_heads, max_context_len, bt_stride=0, partition_tokens=0,
                           q_dtype=DT_F16, sum_context_len=0) -> str:
        """The attention kernel vk_paged_decode would launch (vk_paged_decode_kernel)."""
        a = _capi.DecodeArgs(0, None, q_dtype, None, C.c_void_p(1) if bt_stride else None, bt_stride, None, None,
                             n_seqs, n_heads, max_context_len, 0.0, partition_tokens, None, 0, sum_context_len)
        buf = C.create_string_buffer(128)
        check(lib().vk_paged_decode_kernel(pool.h, C.byref(a), buf, 128))
        return buf.value.decode()

    def tree_verify(self, pool: "Pool", layer: int, q, q_dtype: int, out, context_lens, tree_mask, n_seqs: int,
                    n_nodes: int, n_heads: int, max_context_len: int, block_tables=None, bt_stride: int = 0,
                    seq_rows=None, scale: float = 0.0, partition_tokens: int = 0, workspace=None,
                    workspace_bytes: int = 0, stream=None, shared_blocks: int = 0):
        """vk_tree_verify; shared_blocks = leading table pages every row shares (radix-cache prefix)."""
        a = _capi.TreeArgs(layer, _bptr(q), q_dtype, _bptr(out), _bptr(block_tables), bt_stride, _bptr(seq_rows),
                           _bptr(context_lens), _bptr(tree_mask), n_seqs, n_nodes, n_heads, max_context_len, scale,
                           partition_tokens, _bptr(workspace), workspace_bytes, shared_blocks)
        check(lib().vk_tree_verify(self.h, pool.h, C.byref(a), _sptr(stream)))

    def tree_workspace_bytes(self, pool: "Pool", n_seqs, n_nodes, n_heads, max_context_len, bt_stride=0,
                             partition_tokens=0, q_dtype=DT_F16, shared_blocks: int = 0) -> int:
        a = _capi.TreeArgs(0, None, q_dtype, None, C.c_void_p(1) if bt_stride else None, bt_stride, None, None, None,
                           n_seqs, n_nodes, n_heads, max_context_len, 0.0, partition_tokens, None, 0, shared_blocks)
        n = C.c_uint64()
        check(lib().vk_tree_verify_workspace(pool.h, C.byref(a), C.byref(n)))
        return n.value

    def tree_plan(self, pool: "Pool", n_seqs, n_nodes, n_heads, max_context_len, bt_stride=0, partition_tokens=0,
                  q_dtype=DT_F16, shared_blocks: int = 0) -> dict:
        """vk_tree_verify_plan as a dict (kernels, prefix chunks and row tiles, partitions, workspace)."""
        a = _capi.TreeArgs(0, None, q_dtype, None, C.c_void_p(1) if bt_stride else None, bt_stride, None, None, None,
                           n_seqs, n_nodes, n_heads, max_context_len, 0.0, partition_tokens, None, 0, shared_blocks)
        p = _capi.TreePlan()
        check(lib().vk_tree_verify_plan(pool.h, C.byref(a), C.byref(p)))
        return {"kernel": p.kernel.decode(), "prefix_kernel": p.prefix_kernel.decode(),
                "prefix_chunks": p.prefix_chunks, "prefix_row_tiles": p.prefix_row_tiles, "row_tiles": p.row_tiles,
                "rows_per_tile": p.rows_per_tile, "partition_tokens": p.partition_tokens,
                "max_partitions": p.max_partitions, "workspace_bytes": p.workspace_bytes,
                "merge_launch": bool(p.merge_launch)}

    def copy_blocks(self, pool: "Pool", pairs, stream=None):
        p = np.ascontiguousarray(np.asarray(pairs, dtype=np.int32).reshape(-1))
        check(lib().vk_copy_blocks(self.h, pool.h, p.ctypes.data_as(C.POINTER(C.c_int32)), len(p) // 2,
                                   _sptr(stream)))

    def tree_commit(self, pool: "Pool", block_tables, bt_stride: int, context_lens, accept, accept_stride: int,
                    n_accept, n_seqs: int, layer0: int = 0, n_layers: int | None = None, status=None, stream=None):
        """vk_tree_commit: move the accepted path's K/V to context_len + d (device arrays); status
        (optional device int32 [n_seqs]) receives COMMIT_* per sequence."""
        n_layers = pool.n_layer - layer0 if n_layers is None else n_layers
        check(lib().vk_tree_commit(self.h, pool.h, layer0, n_layers, _bptr(block_tables), bt_stride,
                                   _bptr(context_lens), _bptr(accept), accept_stride, _bptr(n_accept), n_seqs,
                                   _bptr(status), _sptr(stream)))

    @staticmethod
    def _nixl_items(items):
        arr = (_capi.NixlItem * max(1, len(items)))()
        for i, (bid, tl, fp, off) in enumerate(items):
            arr[i] = _capi.NixlItem(bid, tl, fp, off)
        return arr

    def nixl_pack(self, pool: "Pool", items, pages, n_pages: int, wire, wire_bytes: int, status, layer0: int = 0,
                  n_layers: int | None = None, stream=None):
        """vk_nixl_pack: items are (block_id, token_len, first_page, wire_offset) on the host;
        pages, wire and status are device buffers."""
        n_layers = pool.n_layer - layer0 if n_layers is None else n_layers
        check(lib().vk_nixl_pack(self.h, pool.h, layer0, n_layers, self._nixl_items(items), len(items),
                                 _bptr(pages), n_pages, _bptr(wire), wire_bytes, _bptr(status), _sptr(stream)))

    def nixl_unpack(self, pool: "Pool", items, pages, n_pages: int, wire, wire_bytes: int, status, layer0: int = 0,
                    n_layers: int | None = None, stream=None):
        """vk_nixl_unpack: the inverse of nixl_pack, with per-record status."""
        n_layers = pool.n_layer - layer0 if n_layers is None else n_layers
        check(lib().vk_nixl_unpack(self.h, pool.h, layer0, n_layers, self._nixl_items(items), len(items),
                                   _bptr(pages), n_pages, _bptr(wire), wire_bytes, _bptr(status), _sptr(stream)))

    def fill_normal_f16(self, buf: "DeviceBuffer", n: int, seed: int, row_len: int, outlier_scale: float = 1.0,
                        stream=None):
        check(lib().vk_fill_normal_f16(self.h, _bptr(buf), n, seed & 0xFFFFFFFFFFFFFFFF, row_len, outlier_scale,
                                       _sptr(stream)))


def rope_table(n_pos: int, head_dim: int, freq_base: float) -> np.ndarray:
    """vk_rope_table: float32 [n_pos][head_dim/2][2] cos, sin (host)."""
    out = np.zeros((n_pos, head_dim // 2, 2), np.float32)
    check(lib().vk_rope_table(out.ctypes.data_as(C.POINTER(C.c_float)), n_pos, head_dim, freq_base))
    return out


def _bptr(b):
    if b is None:
        return None
    if isinstance(b, DeviceBuffer):
        return C.c_void_p(b.ptr)
    if isinstance(b, int):
        return C.c_void_p(b)
    return b


def _sptr(s):
    if s is None:
        return None
    if isinstance(s, Stream):
        return s.h
    return C.c_void_p(int(s))


class DeviceBuffer:
    """Device memory from vk_dev_alloc, freed with the object."""

    def __init__(self, ctx: Context, nbytes: int, ptr: int | None = None, owned: bool = True):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.owned = owned and ptr is None
        self.shape = None
        self.dtype = None
        if ptr is None:
            h = C.c_void_p()
            check(lib().vk_dev_alloc(ctx.h, max(self.nbytes, 1), C.byref(h)))
            self.ptr = h.value
        else:
            self.ptr = int(ptr)

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise VkError(_capi.ERR_BAD_ARG, "upload overruns the buffer")
        check(lib().vk_memcpy_h2d(self.ctx.h, C.c_void_p(self.ptr + offset), a.ctypes.data_as(C.c_void_p), a.nbytes))

    def download(self, shape=None, dtype=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype if dtype is not None else (self.dtype if self.dtype is not None else np.uint8))
        shape = shape if shape is not None else (self.shape if self.shape is not None else (self.nbytes // dtype.itemsize,))
        out = np.empty(shape, dtype)
        if offset + out.nbytes > self.nbytes:
            raise VkError(_capi.ERR_BAD_ARG, "download overruns the buffer")
        check(lib().vk_memcpy_d2h(self.ctx.h, out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset), out.nbytes))
        return out

    def zero(self):
        check(lib().vk_memset_d(self.ctx.h, C.c_void_p(self.ptr), 0, self.nbytes))

    def free(self):
        if self.owned and self.ptr:
            lib().vk_dev_free(self.ctx.h, C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.h = C.c_void_p()
        check(lib().vk_stream_create(ctx.h, C.byref(self.h)))

    def sync(self):
        check(lib().vk_stream_sync(self.ctx.h, self.h))

    def __del__(self):
        try:
            if self.h:
                lib().vk_stream_destroy(self.ctx.h, self.h)
        except Exception:
            pass


class Event:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.h = C.c_void_p()
        check(lib().vk_event_create(ctx.h, C.byref(self.h)))

    def record(self, stream=None):
        check(lib().vk_event_record(self.ctx.h, self.h, _sptr(stream)))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().vk_event_elapsed_ms(self.ctx.h, self.h, end.h, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.h:
                lib().vk_event_destroy(self.ctx.h, self.h)
        except Exception:
            pass


class Pool:
    """K/V pools of all layers plus the slot block table (vk_pool_create)."""

    def __init__(self, ctx: Context, n_layer: int, n_blocks: int, block_size: int, n_kv_heads: int, head_dim: int,
                 kv_type: int, max_slots: int = 0, max_pages_per_slot: int = 0):
        self.ctx = ctx
        d = _capi.PoolDesc(n_layer, n_blocks, block_size, n_kv_heads, head_dim, kv_type, max_slots, max_pages_per_slot)
        h = C.c_void_p()
        check(lib().vk_pool_create(ctx.h, C.byref(d), C.byref(h)))
        self.h = h
        out = _capi.PoolDesc()
        check(lib().vk_pool_get_desc(self.h, C.byref(out)))
        self.desc = out
        self.n_layer, self.n_blocks, self.block_size = n_layer, n_blocks, block_size
        self.n_kv_heads, self.head_dim, self.kv_type = n_kv_heads, head_dim, kv_type

    def close(self):
        if self.h:
            lib().vk_pool_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def nbytes(self) -> int:
        n = C.c_uint64()
        check(lib().vk_pool_bytes(self.h, C.byref(n)))
        return n.value

    def nixl_payload_bytes(self, token_len: int, n_layers: int | None = None) -> int:
        """Payload bytes of one NIXL record of token_len tokens (vk_nixl_payload_bytes)."""
        n = C.c_uint64()
        check(lib().vk_nixl_payload_bytes(self.h, self.n_layer if n_layers is None else n_layers, token_len,
                                          C.byref(n)))
        return n.value

    def layer_view(self, layer: int) -> _capi.LayerView:
        v = _capi.LayerView()
        check(lib().vk_pool_layer_view(self.h, layer, C.byref(v)))
        return v

    def block_table(self):
        p = C.c_void_p()
        st = C.c_int32()
        check(lib().vk_pool_block_table(self.h, C.byref(p), C.byref(st)))
        return p.value, st.value

    def bind_slot(self, slot: int, pages):
        arr = np.ascontiguousarray(np.asarray(pages, dtype=np.uint32))
        check(lib().vk_bind_slot(self.h, slot, arr.ctypes.data_as(C.POINTER(C.c_uint32)), len(arr)))

    def download_layer(self, layer: int) -> dict:
        """Raw bytes of one layer: k, v codes and ks, vs scales (None if absent),
        each kind's scales as one contiguous array (I8_BLK pools interleave the K
        and V scale of a (block, head) in one word; they are split here)."""
        v = self.layer_view(layer)
        def dl(ptr, n):
            if not ptr or n == 0:
                return None
            b = DeviceBuffer(self.ctx, n, ptr=ptr, owned=False)
            return b.download((n,), np.uint8)
        out = {"k": dl(v.k_codes, v.codes_bytes), "v": dl(v.v_codes, v.codes_bytes)}
        if v.k_scales and v.scale_step == 4:
            w = dl(v.k_scales, 2 * v.scales_bytes).view(np.uint16).reshape(-1, 2)
            out["ks"] = np.ascontiguousarray(w[:, 0]).view(np.uint8)
            out["vs"] = np.ascontiguousarray(w[:, 1]).view(np.uint8)
        else:
            out["ks"], out["vs"] = dl(v.k_scales, v.scales_bytes), dl(v.v_scales, v.scales_bytes)
        return out

    def upload_layer(self, layer: int, parts: dict):
        """Write parts of one layer given as download_layer returns them."""
        v = self.layer_view(layer)
        for key, ptr, n in (("k", v.k_codes, v.codes_bytes), ("v", v.v_codes, v.codes_bytes)):
            if parts.get(key) is not None and ptr:
                a = np.ascontiguousarray(parts[key]).view(np.uint8).reshape(-1)
                assert a.nbytes == n, (key, a.nbytes, n)
                DeviceBuffer(self.ctx, n, ptr=ptr, owned=False).upload(a)
        if not v.k_scales or (parts.get("ks") is None and parts.get("vs") is None):
            return
        n = v.scales_bytes
        if v.scale_step == 4:  # interleaved (K, V) words: keep the half not given
            cur = self.download_layer(layer)
            ks = np.ascontiguousarray(parts["ks"] if parts.get("ks") is not None else cur["ks"]).view(np.uint8)
            vs = np.ascontiguousarray(parts["vs"] if parts.get("vs") is not None else cur["vs"]).view(np.uint8)
            assert ks.nbytes == n and vs.nbytes == n, (ks.nbytes, vs.nbytes, n)
            w = np.stack([ks.reshape(-1).view(np.uint16), vs.reshape(-1).view(np.uint16)], 1)
            DeviceBuffer(self.ctx, 2 * n, ptr=v.k_scales, owned=False).upload(np.ascontiguousarray(w).view(np.uint8))
            return
        for key, ptr in (("ks", v.k_scales), ("vs", v.v_scales)):
            if parts.get(key) is not None:
                a = np.ascontiguousarray(parts[key]).view(np.uint8).reshape(-1)
                assert a.nbytes == n, (key, a.nbytes, n)
                DeviceBuffer(self.ctx, n, ptr=ptr, owned=False).upload(a)


class BlockManager:
    """PagedAttentionBlockManager (paged_attention.rs:92-212) with page refcounts."""

    def __init__(self, block_size: int, total_pages: int):
        h = C.c_void_p()
        check(lib().vk_bm_create(block_size, total_pages, C.byref(h)))
        self.h = h
        self.block_size = block_size
        self.total_pages = total_pages

    def __del__(self):
        try:
            if self.h:
                lib().vk_bm_destroy(self.h)
        except Exception:
            pass

    def pages_for_tokens(self, token_len: int) -> int:
        return -(-token_len // self.block_size)

    def free_pages(self) -> int:
        n = C.c_int32()
        check(lib().vk_bm_free_pages(self.h, C.byref(n)))
        return n.value

    def _pages_call(self, fn, *args, cap=None):
        cap = cap if cap is not None else self.total_pages
        buf = (C.c_uint32 * max(cap, 1))()
        n = C.c_int32()
        check(fn(self.h, *args, buf, cap, C.byref(n)))
        return [buf[i] for i in range(n.value)]

    def allocate(self, handle: int, token_len: int) -> list[int]:
        return self._pages_call(lib().vk_bm_allocate, handle, token_len)

    def release(self, handle: int):
        check(lib().vk_bm_release(self.h, handle))

    def materialize_span(self, handle: int) -> list[int]:
        return self._pages_call(lib().vk_bm_pages, handle)

    def fork(self, parent: int, child: int, shared_tokens: int, token_len: int) -> list[int]:
        return self._pages_call(lib().vk_bm_fork, parent, child, shared_tokens, token_len)

    def extend(self, handle: int, token_len: int) -> list[int]:
        """Grow the handle's pages to cover token_len tokens (vk_bm_extend)."""
        return self._pages_call(lib().vk_bm_extend, C.c_uint64(handle), C.c_int64(token_len))

    def cow(self, handle: int, page_idx: int):
        s, d, c = C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().vk_bm_cow(self.h, handle, page_idx, C.byref(s), C.byref(d), C.byref(c)))
        return (s.value, d.value) if c.value else None

    def refcount(self, page: int) -> int:
        n = C.c_int32()
        check(lib().vk_bm_refcount(self.h, page, C.byref(n)))
        return n.value


@dataclass
class CacheLookup:
    """radix_cache.rs:11-15: matched tokens and the handle of the longest cached prefix."""
    matched_tokens: int
    handle: int | None


@dataclass
class CachedSequence:
    """Result of RadixCache.cache_sequence: the sequence's pages and the copy to
    issue (vk_copy_blocks) before it writes into its shared partial page."""
    matched_tokens: int
    pages: list
    cow: tuple | None


def _tokens(tokens):
    a = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
    return a, a.ctypes.data_as(C.POINTER(C.c_uint32))


class RadixCache:
    """RadixCache (radix_cache.rs:28-264) over block-manager handles
    (vk_radix_*). With a BlockManager the cache owns the handles inserted into
    it and releases replaced and evicted ones; without one handles are opaque
    ids, as in the reference."""

    def __init__(self, block_manager: "BlockManager | None" = None, capacity_tokens: int | None = None):
        h = C.c_void_p()
        self.bm = block_manager
        check(lib().vk_radix_create(block_manager.h if block_manager else None,
                                    -1 if capacity_tokens is None else capacity_tokens, C.byref(h)))
        self.h = h

    @classmethod
    def with_capacity_tokens(cls, capacity_tokens: int, block_manager=None) -> "RadixCache":
        return cls(block_manager, capacity_tokens)

    def close(self):
        if self.h:
            lib().vk_radix_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def insert(self, tokens, handle: int) -> int | None:
        """Insert tokens -> handle; returns the replaced handle (CacheInsert.replaced)."""
        a, p = _tokens(tokens)
        old, has = C.c_uint64(), C.c_int32()
        check(lib().vk_radix_insert(self.h, p, len(a), handle, C.byref(old), C.byref(has)))
        return old.value if has.value else None

    def lookup(self, tokens) -> CacheLookup:
        a, p = _tokens(tokens)
        m, hd, has = C.c_int32(), C.c_uint64(), C.c_int32()
        check(lib().vk_radix_lookup(self.h, p, len(a), C.byref(m), C.byref(hd), C.byref(has)))
        return CacheLookup(m.value, hd.value if has.value else None)

    def __len__(self) -> int:
        n = C.c_int32()
        check(lib().vk_radix_len(self.h, C.byref(n)))
        return n.value

    def is_empty(self) -> bool:
        return len(self) == 0

    def resident_tokens(self) -> int:
        n = C.c_int64()
        check(lib().vk_radix_resident_tokens(self.h, C.byref(n)))
        return n.value

    def capacity_tokens(self) -> int | None:
        n = C.c_int64()
        check(lib().vk_radix_capacity_tokens(self.h, C.byref(n)))
        return None if n.value < 0 else n.value

    def set_capacity_tokens(self, capacity_tokens: int | None):
        check(lib().vk_radix_set_capacity(self.h, -1 if capacity_tokens is None else capacity_tokens))

    def evict_coldest(self, tokens_to_evict: int) -> list[int]:
        n = C.c_int32()
        cap = max(1, len(self))
        out = (C.c_uint64 * cap)()
        check(lib().vk_radix_evict_coldest(self.h, tokens_to_evict, out, cap, C.byref(n)))
        return [out[i] for i in range(n.value)]

    def cache_sequence(self, tokens, seq_handle: int, cache_handle: int) -> CachedSequence:
        """Prefill with the cached prefix's pages aliased (vk_radix_cache_sequence)."""
        a, p = _tokens(tokens)
        cap = max(1, (len(a) + self.bm.block_size - 1) // self.bm.block_size)
        pages = (C.c_uint32 * cap)()
        m, n, src, dst, has = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().vk_radix_cache_sequence(self.h, p, len(a), seq_handle, cache_handle, C.byref(m), pages, cap,
                                            C.byref(n), C.byref(src), C.byref(dst), C.byref(has)))
        return CachedSequence(m.value, [pages[i] for i in range(n.value)],
                              (src.value, dst.value) if has.value else None)


class SlotPool:
    """slot_manager.rs:20-60: FIFO slot ids, the row index of the block table."""

    def __init__(self, max_slots: int):
        self.max_slots = max_slots
        self.free = deque(range(max_slots))

    def alloc(self):
        return self.free.popleft() if self.free else None

    def release(self, slot: int):
        if not (0 <= slot < self.max_slots):
            raise ValueError(f"Invalid slot ID: {slot} is out of bounds for capacity {self.max_slots}")
        self.free.append(slot)


class InMemoryKvStore:
    """kv_store.rs:25-93: handle bookkeeping with bytes accounting, no KV data."""

    def __init__(self, bytes_per_token: int):
        self.next_block_id = 1
        self.bytes_per_token = bytes_per_token
        self.blocks: dict[int, int] = {}

    def allocate(self, token_len: int) -> int:
        if token_len == 0:
            raise VkError(_capi.ERR_BAD_ARG, "KV block must contain at least one token")
        h = self.next_block_id
        self.next_block_id += 1
        self.blocks[h] = token_len * self.bytes_per_token
        return h

    def release(self, handle: int):
        if handle not in self.blocks:
            raise VkError(_capi.ERR_UNKNOWN_HANDLE, f"unknown KV handle {handle}")
        del self.blocks[handle]

    def allocated_bytes(self) -> int:
        return sum(self.blocks.values())


@dataclass
class MemoryRuntimeConfig:
    """runtime.rs:44-88."""
    bytes_per_token: int
    paged_block_size: int
    paged_total_pages: int
    n_layer: int
    max_slots: int
    n_kv_heads: int = 8
    head_dim: int = 128
    kv_type: KvCacheType = KvCacheType.Fp32
    unified_memory: bool = False


class HipMemoryRuntime:
    """MemoryRuntime (runtime.rs:24-42) on one MI355X: store + allocator + bind_slot,
    with the pool in HBM. MetalMemoryRuntime::new's validation (metal/runtime.rs:146-165)."""

    def __init__(self, config: MemoryRuntimeConfig, ctx: Context | None = None):
        if config.bytes_per_token == 0:
            raise VkError(_capi.ERR_BAD_ARG, "memory.bytes_per_token must be greater than zero")
        if config.paged_block_size == 0:
            raise VkError(_capi.ERR_INVALID_BLOCK_SIZE, "block size must be greater than zero")
        if config.paged_total_pages == 0:
            raise VkError(_capi.ERR_BAD_ARG, "memory.paged_total_pages must be greater than zero")
        self.config = config
        self.ctx = ctx if ctx is not None else Context(0)
        self._store = InMemoryKvStore(config.bytes_per_token)
        self._allocator = BlockManager(config.paged_block_size, config.paged_total_pages)
        self.pool = Pool(self.ctx, config.n_layer, config.paged_total_pages, config.paged_block_size,
                         config.n_kv_heads, config.head_dim, config.kv_type.code, config.max_slots)

    def store(self):
        return self._store

    def allocator(self):
        return self._allocator

    def bind_slot(self, slot: int, pages):
        self.pool.bind_slot(slot, pages)
