"""C ABI and host-side logic, without a GPU: the library loads, exports every
function include/velokv.h declares, and the host block manager / runtime
mirror the reference's behaviour (paged_attention.rs tests 237-305,
metal/runtime.rs tests 334-349, slot_manager.rs)."""
import ctypes as C
import os
import re

import pytest

import velokv
from velokv import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "velokv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _capi.lib()
    names = declared_functions()
    assert len(names) >= 35
    for n in names:
        assert hasattr(lib, n), f"{n} declared in velokv.h but not exported"
    # and the ctypes prototypes cover them all
    assert set(names) - set(_capi.PROTOTYPES) <= {"vk_last_error"}


def test_code_object_is_built_for_gfx950():
    assert os.path.exists(_capi.CODE_OBJECT_PATH)
    data = open(_capi.CODE_OBJECT_PATH, "rb").read()
    assert data[:4] == b"\x7fELF"
    assert b"gfx950" in data
    for kernel in (b"vk_decode_kv3_g4_q1", b"vk_decode_mfma_kv3_g4", b"vk_decode_merge", b"vk_append_kv3", b"vk_copy_blocks"):
        assert kernel in data


def test_no_device_is_a_loud_error_not_a_fallback():
    try:
        ctx = velokv.Context(0)
    except velokv.VkError as e:
        assert e.code in (velokv.ERR_NO_DEVICE, velokv.ERR_UNSUPPORTED)
    else:  # running on a GPU box
        assert ctx.arch == "gfx950"
        ctx.close()


def test_null_arguments_are_rejected():
    lib = _capi.lib()
    assert lib.vk_pool_create(None, None, None) == velokv.ERR_NOT_WIRED
    assert lib.vk_paged_decode(None, None, None, None) == velokv.ERR_NOT_WIRED
    assert lib.vk_append(None, None, 0, None, None, 0, None, 0, None) == velokv.ERR_NOT_WIRED
    assert lib.vk_copy_blocks(None, None, None, 0, None) == velokv.ERR_NOT_WIRED
    assert b"null" in lib.vk_last_error()


# ---------------- block manager: paged_attention.rs:237-305 ----------------

def test_allocates_pages_from_a_fixed_budget():
    bm = velokv.BlockManager(16, 4)
    pages = bm.allocate(1, 24)
    assert len(pages) == 2
    assert bm.free_pages() == 2
    assert bm.materialize_span(1) == pages
    assert pages == [0, 1]  # FIFO from the front


def test_release_returns_pages_to_pool():
    bm = velokv.BlockManager(8, 2)
    bm.allocate(2, 8)
    bm.release(2)
    assert bm.free_pages() == 2


def test_rejects_oversized_allocations():
    bm = velokv.BlockManager(32, 1)
    with pytest.raises(velokv.VkError) as e:
        bm.allocate(3, 64)
    assert e.value.code == velokv.ERR_OUT_OF_PAGES
    assert "requested 2 pages but only 1 are available" in str(e.value)


def test_unknown_handle_and_invalid_block_size():
    bm = velokv.BlockManager(16, 32)
    with pytest.raises(velokv.VkError) as e:
        bm.release(1)
    assert e.value.code == velokv.ERR_UNKNOWN_HANDLE
    with pytest.raises(velokv.VkError) as e:
        velokv.BlockManager(0, 32)
    assert e.value.code == velokv.ERR_INVALID_BLOCK_SIZE


def test_fifo_reuse_order():
    bm = velokv.BlockManager(16, 6)
    a = bm.allocate(1, 32)   # 0, 1
    b = bm.allocate(2, 16)   # 2
    bm.release(1)            # free: 3, 4, 5, 0, 1
    c = bm.allocate(3, 80)   # 3, 4, 5, 0, 1
    assert a == [0, 1] and b == [2] and c == [3, 4, 5, 0, 1]


def test_fork_shares_prefix_pages_and_cow_unshares():
    bm = velokv.BlockManager(16, 16)
    parent = bm.allocate(1, 70)            # 5 pages: 0..4
    child = bm.fork(1, 2, 70, 90)           # shares 5 pages, 1 fresh
    assert child[:5] == parent and len(child) == 6
    assert all(bm.refcount(p) == 2 for p in parent)
    assert bm.free_pages() == 16 - 6
    # appending into the child's page 4 (partially filled, shared) needs a copy
    src, dst = bm.cow(2, 4)
    assert src == parent[4] and dst not in parent
    assert bm.refcount(parent[4]) == 1 and bm.refcount(dst) == 1
    assert bm.materialize_span(2)[4] == dst
    # a private page needs no copy
    assert bm.cow(2, 5) is None
    # releasing the parent keeps the still-shared pages alive
    bm.release(1)
    assert all(bm.refcount(p) == 1 for p in parent[:4])
    assert bm.refcount(parent[4]) == 0
    bm.release(2)
    assert bm.free_pages() == 16


def test_kv_bytes_per_token_per_head():
    # model_loader.rs:129-140, tests/kv_compression.rs:23-29
    from velokv import KvCacheType, kv_bytes_per_token_per_head as f
    assert f(128, KvCacheType.Fp32) == 512
    assert f(128, KvCacheType.Int8) == 132
    assert f(128, KvCacheType.Fp8) == 132
    assert f(128, KvCacheType.Fp16) == 256
    assert KvCacheType.Fp8.code == velokv.KV_I8_REF  # metal/model.rs:404,442


def test_runtime_config_validation():
    # metal/runtime.rs:334-349
    from velokv import HipMemoryRuntime, MemoryRuntimeConfig
    with pytest.raises(velokv.VkError) as e:
        HipMemoryRuntime(MemoryRuntimeConfig(0, 16, 32, 1, 32))
    assert "bytes_per_token" in str(e.value)
    with pytest.raises(velokv.VkError) as e:
        HipMemoryRuntime(MemoryRuntimeConfig(64, 0, 32, 1, 32))
    assert e.value.code == velokv.ERR_INVALID_BLOCK_SIZE
    with pytest.raises(velokv.VkError):
        HipMemoryRuntime(MemoryRuntimeConfig(64, 16, 0, 1, 32))


def test_slot_pool_fifo():
    sp = velokv.SlotPool(3)
    assert [sp.alloc(), sp.alloc(), sp.alloc(), sp.alloc()] == [0, 1, 2, None]
    sp.release(1)
    assert sp.alloc() == 1
    with pytest.raises(ValueError):
        sp.release(7)


def test_decode_workspace_query_needs_no_gpu_for_validation():
    lib = _capi.lib()
    n = C.c_uint64()
    assert lib.vk_paged_decode_workspace(None, None, C.byref(n)) == velokv.ERR_BAD_ARG


def test_workspace_growth_keeps_retired_buffers_below_the_live_one():
    """The context's own split-K workspace grows at least geometrically, so the
    outgrown buffers it keeps until vk_ctx_destroy sum to less than the live
    one. Needs as stream-K plans them when max_context_len grows 16 tokens at a
    time past the point where the workers outnumber the resident waves
    (S=64, Hkv=8, G=4: ceil(units / 256) workers, 2 partial rows of G per worker)."""
    grow = _capi.lib().vk_workspace_grow_bytes
    assert grow(0, 1000) == 1024
    assert grow(4096, 100) == 4096
    assert grow(4096, 5000) == 8192
    assert grow(4096, 9000) == 9216
    S, Hkv, G, pen = 64, 8, 4, 8
    cur, retired, allocs = 0, 0, 0
    for L in range(16384, 32769, 16):
        units = S * Hkv * (L // 16 + pen)
        nw = max(2048, -(-units // 256))
        prow = nw * 2 * G
        need = -(-prow * 128 * 4 // 256) * 256 + -(-prow * 2 * 4 // 256) * 256 + -(-(S + 1) * 4 // 256) * 256
        nxt = grow(cur, need)
        assert nxt >= need
        if nxt != cur:
            retired += cur
            cur = nxt
            allocs += 1
    assert retired < cur
    assert allocs <= 4  # 1025 growing calls, a handful of allocations
