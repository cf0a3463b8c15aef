"""CPU pins of the oracle's NIXL wire records and accepted-path commit.

NIXL: the reference's own unit tests of the wire format (nixl.rs:491-525 --
round trip, short header, truncated payload, empty payload, and the 64-byte
payload of dma_write_and_read_back, nixl.rs:529-548) restated as known answers,
plus the little-endian header layout of serialize_block (nixl.rs:36-43) checked
against struct.pack, and gather/scatter invariants of the page payload.

Tree commit (no reference counterpart): closed forms -- moves that keep the
block scale move codes exactly; a destination at block offset 0 starts the
scale fp16(amax/127) of the moved tokens; the identity path and rejected rows
leave the pool untouched; every moved token dequantizes to within half a
quantization step of its source.
"""
import struct

import numpy as np
import pytest

import pyoracle as O
from cases import BS, HD
from velokv import synth


# ---- NIXL wire format ---------------------------------------------------------

def test_wire_round_trip_known_answer():
    # nixl.rs:491-500: handle (42, 8), payload 0xAB x 64
    wire = O.nixl_serialize(42, 8, np.full(64, 0xAB, np.uint8))
    assert wire.size == 16 + 64
    assert bytes(wire[:16]) == struct.pack("<QII", 42, 8, 64)
    bid, tl, payload = O.nixl_deserialize(wire)
    assert (bid, tl) == (42, 8)
    assert np.array_equal(payload, np.full(64, 0xAB, np.uint8))


def test_wire_rejects_short_header():
    # nixl.rs:502-505: 15 zero bytes -> None
    assert O.nixl_deserialize(np.zeros(15, np.uint8)) is None
    assert O.nixl_deserialize(np.zeros(0, np.uint8)) is None


def test_wire_rejects_truncated_payload():
    # nixl.rs:507-514: handle (1, 4), 32-byte payload, last byte cut
    wire = O.nixl_serialize(1, 4, np.zeros(32, np.uint8))
    assert O.nixl_deserialize(wire[:-1]) is None
    assert O.nixl_deserialize(wire) is not None


def test_wire_empty_payload():
    # nixl.rs:516-524: handle (7, 0), empty payload -> 16-byte record
    wire = O.nixl_serialize(7, 0, np.zeros(0, np.uint8))
    assert wire.size == 16
    bid, tl, payload = O.nixl_deserialize(wire)
    assert (bid, tl, payload.size) == (7, 0, 0)


def test_wire_header_is_little_endian_for_large_values():
    bid, tl = 0x0123456789ABCDEF, 0xFEDCBA98
    wire = O.nixl_serialize(bid, tl, np.arange(5, dtype=np.uint8))
    assert bytes(wire[:16]) == struct.pack("<QII", bid, tl, 5)
    assert O.nixl_deserialize(wire)[:2] == (bid, tl)


def _random_layers(kv, n_layers, n_blocks, n_kv_heads, seed):
    rng = np.random.default_rng(seed)
    layers = []
    for _ in range(n_layers):
        L = O.Layer(n_blocks, n_kv_heads, BS, HD, kv)
        for key in ("k", "v", "ks", "vs"):
            a = getattr(L, key)
            if a is not None:
                a[:] = rng.integers(0, 256, a.size, dtype=np.uint8)
        layers.append(L)
    return layers


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_payload_size_and_layout(kv):
    layers = _random_layers(kv, 3, 12, 2, seed=5)
    pages = [7, 2, 9]
    payload = O.nixl_gather(layers, pages)
    esz = O.ESZ[kv]
    cb = 2 * BS * HD * esz
    sb = {O.I8_BLK: 2 * 2, O.I8_REF: 2 * 4 * BS}.get(kv, 0)
    assert payload.size == 3 * 3 * 2 * (cb + sb)
    assert payload.size == O.nixl_payload_bytes(layers[0], 3, 3 * BS)
    assert O.nixl_payload_bytes(layers[0], 3, 3 * BS - 5) == payload.size  # whole pages travel
    # tiles of (page i, layer l) sit at ((i * n_layers + l) * 2) * cb: K then V
    i, l = 1, 2
    off = (i * 3 + l) * 2 * cb
    assert np.array_equal(payload[off:off + cb], layers[l].k[pages[i] * cb:(pages[i] + 1) * cb])
    assert np.array_equal(payload[off + cb:off + 2 * cb], layers[l].v[pages[i] * cb:(pages[i] + 1) * cb])
    if sb:
        soff = 3 * 3 * 2 * cb + (i * 3 + l) * 2 * sb
        assert np.array_equal(payload[soff:soff + sb], layers[l].ks[pages[i] * sb:(pages[i] + 1) * sb])
        assert np.array_equal(payload[soff + sb:soff + 2 * sb], layers[l].vs[pages[i] * sb:(pages[i] + 1) * sb])


@pytest.mark.parametrize("kv", [O.F16, O.I8_BLK])
def test_pack_unpack_round_trip_moves_only_target_pages(kv):
    src = _random_layers(kv, 2, 16, 2, seed=6)
    dst = _random_layers(kv, 2, 16, 2, seed=7)
    before = [L.copy() for L in dst]
    items = [(11, 40, 0, 0), (12, 0, 3, 4096 * 64), (13, 16, 3, 4096 * 128)]
    src_pages = np.array([1, 5, 9, 14], np.int32)
    dst_pages = np.array([3, 0, 8, 2], np.int32)
    wire = np.full(4096 * 192, 0xEE, np.uint8)
    assert O.nixl_pack(src, items, src_pages, wire) == [O.NIXL_OK] * 3
    assert O.nixl_unpack(dst, items, dst_pages, wire) == [O.NIXL_OK] * 3
    moved = {3: 1, 0: 5, 8: 9, 2: 14}  # dst page -> src page (item 11: pages 0..2, item 13: page 3)
    for L, S0, B in zip(dst, src, before):
        cb = L.k.size // L.n_blocks
        for blk in range(L.n_blocks):
            exp = S0 if blk in moved else B
            sblk = moved.get(blk, blk)
            assert np.array_equal(L.k[blk * cb:(blk + 1) * cb], exp.k[sblk * cb:(sblk + 1) * cb])
            assert np.array_equal(L.v[blk * cb:(blk + 1) * cb], exp.v[sblk * cb:(sblk + 1) * cb])


def test_unpack_statuses_follow_deserialize_order():
    layers = _random_layers(O.I8_BLK, 1, 8, 2, seed=8)
    wire = np.zeros(16384, np.uint8)
    rec = O.nixl_serialize(5, 16, O.nixl_gather(layers, [1]))
    wire[:rec.size] = rec
    pages = np.array([2], np.int32)
    assert O.nixl_unpack(layers, [(5, 16, 0, 16384 - 8)], pages, wire) == [O.NIXL_SHORT_HEADER]
    assert O.nixl_unpack(layers, [(5, 16, 0, 0)], pages, wire[:rec.size - 1]) == [O.NIXL_TRUNCATED]
    assert O.nixl_unpack(layers, [(6, 16, 0, 0)], pages, wire) == [O.NIXL_HANDLE_MISMATCH]
    two = _random_layers(O.I8_BLK, 2, 8, 2, seed=9)
    assert O.nixl_unpack(two, [(5, 16, 0, 0)], pages, wire) == [O.NIXL_LENGTH_MISMATCH]
    assert O.nixl_unpack(layers, [(5, 16, 0, 0)], np.array([8], np.int32), wire) == [O.NIXL_BAD_PAGE]


# ---- accepted-path commit -------------------------------------------------------

def _commit_case(kv, ctx, n_nodes, seed, scale_spread=False):
    """One sequence: committed context ctx followed by n_nodes tree tokens, appended
    through the oracle's append (so I8_BLK scales follow the append rule)."""
    L_tot = ctx + n_nodes
    n_pages = (L_tot + BS - 1) // BS
    bt = synth.scatter_block_tables(3 * n_pages + 4, [n_pages], seed)[0]
    L = O.Layer(3 * n_pages + 4, 2, BS, HD, kv)
    row = 2 * HD
    k = synth.normals_f16(L_tot * row, seed, row, 8.0).reshape(L_tot, 2, HD)
    v = synth.normals_f16(L_tot * row, seed + 1, row, 8.0).reshape(L_tot, 2, HD)
    if scale_spread:  # tree tokens much larger than the context: moves raise scales
        k[ctx:] = (k[ctx:].astype(np.float32) * 6).astype(np.float16)
        v[ctx:] = (v[ctx:].astype(np.float32) * 6).astype(np.float16)
    slots = synth.slots_for_positions(bt[None, :], np.arange(L_tot), BS, np.zeros(L_tot, np.int64))
    O.append(L, k, v, slots)
    return L, bt


def _deq(L, bt, pos, is_v):
    return np.array([[L.elem(is_v, bt[pos // BS], h, pos % BS, d) for d in range(HD)] for h in range(2)])


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF])
def test_commit_moves_rows_exactly(kv):
    L, bt = _commit_case(kv, 29, 8, seed=21)
    before = L.copy()
    accept = [0, 2, 5, 6]
    assert O.tree_commit(L, bt, 29, accept) == 0
    for d, a in enumerate(accept):
        for is_v in (0, 1):
            assert np.array_equal(_deq(L, bt, 29 + d, is_v), _deq(before, bt, 29 + a, is_v))
    for p in range(29):  # committed context untouched
        assert np.array_equal(_deq(L, bt, p, 0), _deq(before, bt, p, 0))


@pytest.mark.parametrize("kv", [O.F32, O.F16, O.I8_REF, O.I8_BLK])
def test_commit_identity_and_rejected_rows_leave_pool_untouched(kv):
    L, bt = _commit_case(kv, 40, 8, seed=22)
    before = L.copy()
    for accept in ([0, 1, 2], [0], [], [1, 1], [2, 1], [0, 40], [0, 3, 2]):
        rc = O.tree_commit(L, bt, 40, accept)
        assert rc == (0 if accept in ([0, 1, 2], [0], []) else 1), accept
        for key in ("k", "v", "ks", "vs"):
            if getattr(L, key) is not None:
                assert np.array_equal(getattr(L, key), getattr(before, key)), (accept, key)
    # positions past the table row are rejected
    assert O.tree_commit(L, bt, len(bt) * BS - 2, [0, 5]) == 1


def test_commit_blk_within_one_block_moves_codes_exactly():
    # context 33 (offset 1 of block 2), nodes at 33..40 stay in block 2: the scale
    # cannot grow, so codes move unchanged
    L, bt = _commit_case(O.I8_BLK, 33, 8, seed=23)
    before = L.copy()
    accept = [0, 3, 4, 7]
    assert O.tree_commit(L, bt, 33, accept) == 0
    blk = bt[33 // BS]
    sb = 2 * 2
    assert np.array_equal(L.ks[blk * sb:(blk + 1) * sb], before.ks[blk * sb:(blk + 1) * sb])
    for d, a in enumerate(accept):
        for is_v in (0, 1):
            assert np.array_equal(_deq(L, bt, 33 + d, is_v), _deq(before, bt, 33 + a, is_v))


def test_commit_blk_block_start_takes_fresh_scale_and_stays_within_half_step():
    # context 32 = block boundary and node 0 rejected: the first destination is
    # offset 0, so the block's scale restarts; with every moved token in that
    # block the final scale is max_d fp16(amax_d / 127) exactly
    L, bt = _commit_case(O.I8_BLK, 32, 8, seed=24, scale_spread=True)
    before = L.copy()
    accept = [1, 2, 3, 6]
    src = {(d, is_v): _deq(before, bt, 32 + a, is_v) for d, a in enumerate(accept) for is_v in (0, 1)}
    assert O.tree_commit(L, bt, 32, accept) == 0
    blk = bt[2]
    for is_v, sc in ((0, L.ks), (1, L.vs)):
        for h in range(2):
            need = max(np.float16(np.float32(np.abs(src[(d, is_v)][h]).max()) / np.float32(127.0))
                       for d in range(4))
            s = sc[(blk * 2 + h) * 2:(blk * 2 + h) * 2 + 2].view(np.float16)[0]
            assert s == need
            for d in range(4):
                got = _deq(L, bt, 32 + d, is_v)[h]
                # token d is rounded once at its own scale and once more each time a
                # later token raises the scale (at most 3 - d times), each rounding at
                # most half a step of a scale <= s
                assert np.abs(got - src[(d, is_v)][h]).max() <= 0.5 * (4 - d) * float(s) + 1e-6
            last = _deq(L, bt, 32 + 3, is_v)[h]  # the largest-scale token is rounded once
            if need == np.float16(np.float32(np.abs(src[(3, is_v)][h]).max()) / np.float32(127.0)):
                assert np.abs(last - src[(3, is_v)][h]).max() <= 0.5 * float(s) + 1e-6


def test_commit_blk_equals_reappending_dequantized_sources():
    # the definition, checked across a block boundary (context 14: tree spans blocks 0 and 1)
    L, bt = _commit_case(O.I8_BLK, 14, 8, seed=25, scale_spread=True)
    before = L.copy()
    accept = [0, 1, 4, 7]
    assert O.tree_commit(L, bt, 14, accept) == 0
    ref = before.copy()
    xk = np.stack([_deq(before, bt, 14 + a, 0) for a in accept[2:]]).astype(np.float32)
    xv = np.stack([_deq(before, bt, 14 + a, 1) for a in accept[2:]]).astype(np.float32)
    slots = synth.slots_for_positions(bt[None, :], np.array([16, 17]), BS, np.zeros(2, np.int64))
    O.append(ref, xk, xv, slots)
    for key in ("k", "v", "ks", "vs"):
        assert np.array_equal(getattr(L, key), getattr(ref, key)), key
