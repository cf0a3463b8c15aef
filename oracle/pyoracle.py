"""ctypes wrapper of the CPU oracle (oracle/velokv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline. The
product (velokv) never imports it.

Layer arrays use the build layout (see include/velokv.h) as numpy uint8 buffers
so GPU pools can be compared byte for byte.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# VELOKV_SANITIZE=1 selects the AddressSanitizer + UBSan build (make asan)
LIB_PATH = os.path.join(HERE, "build", "libvelokv_oracle_asan.so" if os.environ.get("VELOKV_SANITIZE") == "1"
                        else "libvelokv_oracle.so")

F32, F16, I8_REF, I8_BLK = 0, 1, 2, 3
ESZ = {F32: 4, F16: 2, I8_REF: 1, I8_BLK: 1}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.vko_f16_to_f32.argtypes = [C.c_uint16]
        L.vko_f16_to_f32.restype = C.c_float
        L.vko_f32_to_f16.argtypes = [C.c_float]
        L.vko_f32_to_f16.restype = C.c_uint16
        L.vko_append.restype = C.c_int
        L.vko_splitmix64.argtypes = [C.c_uint64]
        L.vko_splitmix64.restype = C.c_uint64
        L.vko_load_elem.restype = C.c_float
        L.vko_get_threads.restype = C.c_int
        _lib = L
    return _lib


class VkoLayer(C.Structure):
    _fields_ = [("n_blocks", C.c_int32), ("n_kv_heads", C.c_int32), ("block_size", C.c_int32),
                ("head_dim", C.c_int32), ("kv_type", C.c_int32),
                ("k", C.c_void_p), ("v", C.c_void_p), ("ks", C.c_void_p), ("vs", C.c_void_p)]


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


class Layer:
    """One layer of a KV pool in host memory, build layout."""

    def __init__(self, n_blocks, n_kv_heads, block_size, head_dim, kv_type):
        self.n_blocks, self.n_kv_heads, self.block_size, self.head_dim, self.kv_type = (
            n_blocks, n_kv_heads, block_size, head_dim, kv_type)
        codes = n_blocks * n_kv_heads * block_size * head_dim * ESZ[kv_type]
        self.k = np.zeros(codes, np.uint8)
        self.v = np.zeros(codes, np.uint8)
        sb = {I8_BLK: 2, I8_REF: 4 * block_size}.get(kv_type, 0) * n_blocks * n_kv_heads
        self.ks = np.zeros(sb, np.uint8) if sb else None
        self.vs = np.zeros(sb, np.uint8) if sb else None

    def struct(self):
        return VkoLayer(self.n_blocks, self.n_kv_heads, self.block_size, self.head_dim, self.kv_type,
                        _ptr(self.k), _ptr(self.v), _ptr(self.ks), _ptr(self.vs))

    def copy(self):
        o = Layer(self.n_blocks, self.n_kv_heads, self.block_size, self.head_dim, self.kv_type)
        o.k[:] = self.k
        o.v[:] = self.v
        if self.ks is not None:
            o.ks[:] = self.ks
            o.vs[:] = self.vs
        return o

    def tile_codes(self, is_v, blk, h):
        """Codes of one (block, head) tile as [block_size][head_dim] elements
        (int8 / uint16 fp16 bits / float32), gathered through the build layout."""
        idx = _tile_index(self, is_v)
        esz = ESZ[self.kv_type]
        raw = self.v if is_v else self.k
        tile = self.block_size * self.head_dim * esz
        base = (blk * self.n_kv_heads + h) * tile
        b = raw[base:base + tile]
        if esz == 1:
            return b.view(np.int8)[idx]
        dt = np.uint16 if esz == 2 else np.float32
        return b.view(dt)[idx // esz]

    def elem(self, is_v, blk, h, tok, d):
        s = self.struct()
        return lib().vko_load_elem(C.byref(s), int(is_v), C.c_int64(blk), h, tok, d)


_TILE_INDEX = {}


def _tile_index(layer, is_v):
    """[block_size][head_dim] byte offsets of a tile's elements (vko_elem_offset)."""
    key = (layer.kv_type, layer.block_size, layer.head_dim, int(is_v))
    if key not in _TILE_INDEX:
        lib().vko_elem_offset.restype = C.c_uint64
        one = Layer(1, 1, layer.block_size, layer.head_dim, layer.kv_type)
        s = one.struct()
        _TILE_INDEX[key] = np.array([[lib().vko_elem_offset(C.byref(s), int(is_v), C.c_int64(0), 0, t, d)
                                      for d in range(layer.head_dim)] for t in range(layer.block_size)], np.int64)
    return _TILE_INDEX[key]


def f16_to_f32(bits):
    return lib().vko_f16_to_f32(int(bits))


def f32_to_f16(x):
    return lib().vko_f32_to_f16(float(x))


def splitmix64(x):
    return lib().vko_splitmix64(C.c_uint64(x & 0xFFFFFFFFFFFFFFFF))


def _in_dtype(a):
    if a.dtype == np.float16:
        return F16
    assert a.dtype == np.float32
    return F32


def append(layer: Layer, k, v, slot_mapping):
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    s = layer.struct()
    rc = lib().vko_append(C.byref(s), _ptr(k), _ptr(v), _in_dtype(k), _ptr(sm), C.c_int(len(sm)))
    if rc != 0:
        raise RuntimeError(f"vko_append failed ({rc})")


def paged_decode(layer: Layer, q, block_tables, ctx_lens, scale=None):
    q = np.ascontiguousarray(q)
    S, H, D = q.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    out = np.zeros((S, H, D), np.float32)
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    s = layer.struct()
    lib().vko_paged_decode(C.byref(s), _ptr(q), _in_dtype(q), _ptr(out), _ptr(bt), C.c_int(bt.shape[1]),
                           _ptr(cl), C.c_int(S), C.c_int(H), C.c_float(scale))
    return out


def paged_decode_f64(layer: Layer, q, block_tables, ctx_lens, scale=None):
    q = np.ascontiguousarray(q)
    S, H, D = q.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    out = np.zeros((S, H, D), np.float64)
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    s = layer.struct()
    lib().vko_paged_decode_f64(C.byref(s), _ptr(q), _in_dtype(q), _ptr(out), _ptr(bt), C.c_int(bt.shape[1]),
                               _ptr(cl), C.c_int(S), C.c_int(H), C.c_double(scale))
    return out


def tree_verify(layer: Layer, q, block_tables, ctx_lens, mask, scale=None):
    q = np.ascontiguousarray(q)
    S, N, H, D = q.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    mk = np.ascontiguousarray(mask, dtype=np.uint32)
    out = np.zeros((S, N, H, D), np.float32)
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    s = layer.struct()
    lib().vko_tree_verify(C.byref(s), _ptr(q), _in_dtype(q), _ptr(out), _ptr(bt), C.c_int(bt.shape[1]),
                          _ptr(cl), _ptr(mk), C.c_int(S), C.c_int(N), C.c_int(H), C.c_float(scale))
    return out


def copy_blocks(layer: Layer, pairs):
    p = np.ascontiguousarray(pairs, dtype=np.int32).reshape(-1)
    s = layer.struct()
    lib().vko_copy_blocks(C.byref(s), _ptr(p), C.c_int(len(p) // 2))


def to_reference_layout(layer: Layer, is_v):
    D = layer.head_dim
    row = 4 * D if layer.kv_type == F32 else D + 4
    dst = np.zeros(layer.n_blocks * layer.block_size * layer.n_kv_heads * row, np.uint8)
    s = layer.struct()
    lib().vko_to_reference_layout(C.byref(s), C.c_int(int(is_v)), _ptr(dst))
    return dst


# ---- reference-layout restatements ------------------------------------------

def ref_kv_update(k_cache, v_cache, k_in, v_in, slot_id, table, max_pages, block_size, n_head, head_dim, pos):
    lib().vko_ref_kv_update(_ptr(k_cache), _ptr(v_cache), _ptr(k_in), _ptr(v_in), C.c_uint32(slot_id), _ptr(table),
                            C.c_uint32(max_pages), C.c_uint32(block_size), C.c_uint32(n_head),
                            C.c_uint32(head_dim), C.c_uint32(pos))


def ref_kv_update_int8(k_cache, v_cache, k_in, v_in, slot_id, table, max_pages, block_size, n_head, head_dim, pos):
    lib().vko_ref_kv_update_int8(_ptr(k_cache), _ptr(v_cache), _ptr(k_in), _ptr(v_in), C.c_uint32(slot_id),
                                 _ptr(table), C.c_uint32(max_pages), C.c_uint32(block_size), C.c_uint32(n_head),
                                 C.c_uint32(head_dim), C.c_uint32(pos))


def ref_paged_attention_flash(q, k_cache, v_cache, int8, head_dim, pos, slot_id, table, max_pages, block_size,
                              n_head_kv, n_head):
    out = np.zeros(n_head * head_dim, np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    lib().vko_ref_paged_attention_flash(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), C.c_int(int(int8)),
                                        C.c_uint32(head_dim), C.c_uint32(pos), C.c_uint32(slot_id), _ptr(table),
                                        C.c_uint32(max_pages), C.c_uint32(block_size), C.c_uint32(n_head_kv),
                                        C.c_uint32(n_head))
    return out.reshape(n_head, head_dim)


def ref_cpu_attention(q, k, v, n_head, n_head_kv, head_dim):
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n_seq = k.size // (n_head_kv * head_dim)
    out = np.zeros(n_head * head_dim, np.float32)
    lib().vko_ref_cpu_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), C.c_uint32(n_seq), C.c_uint32(n_head),
                                C.c_uint32(n_head_kv), C.c_uint32(head_dim))
    return out.reshape(n_head, head_dim)


def set_threads(n):
    lib().vko_set_threads(C.c_int(n))


def get_threads():
    return lib().vko_get_threads()


# ---- accepted-path commit of a draft tree ------------------------------------

def tree_commit(layer: Layer, block_table_row, ctx_len, accept):
    """vko_tree_commit on one sequence of one layer; returns 0, or 1 when the row
    is rejected and the layer left untouched."""
    bt = np.ascontiguousarray(block_table_row, dtype=np.int32)
    a = np.ascontiguousarray(accept, dtype=np.int32)
    s = layer.struct()
    return lib().vko_tree_commit(C.byref(s), _ptr(bt), C.c_int(len(bt)), C.c_int(int(ctx_len)), _ptr(a),
                                 C.c_int(len(a)))


# ---- NIXL wire records (nixl.rs:24-61) -----------------------------------------

NIXL_OK, NIXL_SHORT_HEADER, NIXL_TRUNCATED, NIXL_HANDLE_MISMATCH, NIXL_LENGTH_MISMATCH, NIXL_BAD_PAGE = range(6)


def nixl_serialize(block_id, token_len, payload):
    """serialize_block (nixl.rs:36-43) -> bytes."""
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    out = np.zeros(16 + payload.size, np.uint8)
    n = lib().vko_nixl_serialize(C.c_uint64(block_id), C.c_uint32(token_len), _ptr(payload),
                                 C.c_uint32(payload.size), _ptr(out))
    assert n == out.size
    return out


def nixl_deserialize(buf):
    """deserialize_block (nixl.rs:49-61): None, or (block_id, token_len, payload)."""
    buf = np.ascontiguousarray(buf, dtype=np.uint8)
    bid, tl, bl = C.c_uint64(), C.c_uint32(), C.c_uint32()
    ok = lib().vko_nixl_deserialize(_ptr(buf) if buf.size else None, C.c_uint64(buf.size), C.byref(bid),
                                    C.byref(tl), C.byref(bl))
    if not ok:
        return None
    return bid.value, tl.value, buf[16:16 + bl.value]


def _layers_array(layers):
    arr = (VkoLayer * len(layers))()
    for i, L in enumerate(layers):
        arr[i] = L.struct()
    return arr


def nixl_payload_bytes(layer: Layer, n_layers, token_len):
    lib().vko_nixl_payload_bytes.restype = C.c_uint64
    s = layer.struct()
    return lib().vko_nixl_payload_bytes(C.byref(s), C.c_int(n_layers), C.c_uint32(token_len))


def nixl_gather(layers, pages):
    pages = np.ascontiguousarray(pages, dtype=np.int32)
    n = nixl_payload_bytes(layers[0], len(layers), len(pages) * layers[0].block_size)
    out = np.zeros(n, np.uint8)
    arr = _layers_array(layers)
    lib().vko_nixl_move(arr, C.c_int(len(layers)), _ptr(pages), C.c_int(len(pages)), _ptr(out), C.c_int(0))
    return out


def nixl_scatter(layers, pages, payload):
    pages = np.ascontiguousarray(pages, dtype=np.int32)
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    arr = _layers_array(layers)
    lib().vko_nixl_move(arr, C.c_int(len(layers)), _ptr(pages), C.c_int(len(pages)), _ptr(payload), C.c_int(1))


def nixl_pack(layers, items, pages, wire):
    """Multi-record pack into `wire` (uint8 array, modified in place); items are
    (block_id, token_len, first_page, wire_offset). Returns the status list."""
    bs, nb = layers[0].block_size, layers[0].n_blocks
    status = []
    for bid, tl, fp, off in items:
        pg = np.asarray(pages[fp:fp + (tl + bs - 1) // bs], np.int64)
        if np.any((pg < 0) | (pg >= nb)):
            status.append(NIXL_BAD_PAGE)
            continue
        rec = nixl_serialize(bid, tl, nixl_gather(layers, pg))
        wire[off:off + rec.size] = rec
        status.append(NIXL_OK)
    return status


def nixl_unpack(layers, items, pages, wire):
    """Multi-record unpack from `wire` into `layers` (modified in place); returns
    the status list (header checks in deserialize_block's order, then ours)."""
    bs, nb = layers[0].block_size, layers[0].n_blocks
    status = []
    for bid, tl, fp, off in items:
        if off > wire.size or wire.size - off < 16:
            status.append(NIXL_SHORT_HEADER)
            continue
        r = nixl_deserialize(wire[off:])
        if r is None:
            status.append(NIXL_TRUNCATED)
            continue
        rbid, rtl, payload = r
        if rbid != bid or rtl != tl:
            status.append(NIXL_HANDLE_MISMATCH)
            continue
        if payload.size != nixl_payload_bytes(layers[0], len(layers), tl):
            status.append(NIXL_LENGTH_MISMATCH)
            continue
        pg = np.asarray(pages[fp:fp + (tl + bs - 1) // bs], np.int64)
        if np.any((pg < 0) | (pg >= nb)):
            status.append(NIXL_BAD_PAGE)
            continue
        nixl_scatter(layers, pg, payload)
        status.append(NIXL_OK)
    return status


# ---- RoPE ------------------------------------------------------------------------

ROPE_INTERLEAVED, ROPE_HALF = 1, 2


def rope_table(n_pos, head_dim, freq_base):
    out = np.zeros((n_pos, head_dim // 2, 2), np.float32)
    lib().vko_rope_table(_ptr(out), C.c_int(n_pos), C.c_int(head_dim), C.c_float(freq_base))
    return out


def rope_apply(x, positions, style, table):
    """Rotate rows x[..., n, head, D] (fp32) of token n by positions[n] (copy)."""
    x = np.array(x, dtype=np.float32, copy=True)
    n_tok = x.shape[0]
    D = x.shape[-1]
    rows = x.reshape(n_tok, -1, D)
    tb = np.ascontiguousarray(table, dtype=np.float32)
    for n in range(n_tok):
        for h in range(rows.shape[1]):
            r = np.ascontiguousarray(rows[n, h])
            lib().vko_rope_apply(_ptr(r), C.c_int(D), C.c_int(int(positions[n])), C.c_int(style), _ptr(tb))
            rows[n, h] = r
    return rows.reshape(x.shape)


def ref_rope_cpu(x, pos, freq_base):
    """llama_cpu.rs:113-131 on one head row (fp32)."""
    r = np.array(x, dtype=np.float32, copy=True)
    lib().vko_ref_rope_cpu(_ptr(r), C.c_int(r.size), C.c_int(pos), C.c_float(freq_base))
    return r


def ref_rope_metal(x, pos, freq_base):
    """kernels.metal:103-131 on one head row (fp32)."""
    r = np.array(x, dtype=np.float32, copy=True)
    lib().vko_ref_rope_metal(_ptr(r), C.c_int(r.size), C.c_int(pos), C.c_float(freq_base))
    return r


def append_rope(layer: Layer, k, v, slot_mapping, positions, style, table, q=None):
    """The fused RoPE + append: K rows rotated in fp32 then appended (V as is);
    tokens with positions outside the table are skipped. Returns the rotated q
    (in q's dtype) or None."""
    n_pos = table.shape[0]
    pos = np.asarray(positions, np.int64)
    ok = (pos >= 0) & (pos < n_pos)
    sm = np.where(ok, np.asarray(slot_mapping, np.int64), -1)
    kr = rope_apply(np.asarray(k, np.float32), np.where(ok, pos, 0), style, table)
    append(layer, np.ascontiguousarray(kr), np.ascontiguousarray(np.asarray(v, np.float32)), sm)
    if q is None:
        return None
    qr = rope_apply(np.asarray(q, np.float32), np.where(ok, pos, 0), style, table).astype(q.dtype)
    return np.where(ok.reshape((-1,) + (1,) * (q.ndim - 1)), qr, q)
