"""Seeded test cases shared by the CPU and GPU tests (inputs only; the expected
values always come from the oracle)."""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import pyoracle as O
from velokv import synth

BS, HD = 16, 128


@dataclass
class Case:
    kv_type: int
    n_blocks: int
    n_kv_heads: int
    n_heads: int
    ctx_lens: np.ndarray            # tokens per sequence, including the appended one
    block_tables: np.ndarray        # [S][stride] int32
    k: list = field(default_factory=list)   # per sequence [L][Hkv][D] fp16
    v: list = field(default_factory=list)
    q: np.ndarray = None            # [S][H][D] fp16

    @property
    def S(self):
        return len(self.ctx_lens)

    def prefill_slots(self):
        """Flat slots and rows of tokens 0..L-2 of every sequence (sequence-major)."""
        sl, kk, vv = [], [], []
        for s in range(self.S):
            n = int(self.ctx_lens[s]) - 1
            if n <= 0:
                continue
            sl.append(synth.slots_for_positions(self.block_tables, np.arange(n), BS, np.full(n, s)))
            kk.append(self.k[s][:n])
            vv.append(self.v[s][:n])
        if not sl:
            return np.zeros(0, np.int64), np.zeros((0, self.n_kv_heads, HD), np.float16), np.zeros((0, self.n_kv_heads, HD), np.float16)
        return np.concatenate(sl), np.concatenate(kk), np.concatenate(vv)

    def last_slots(self):
        """Slot, K and V of the appended token (position L-1) of every sequence."""
        pos = self.ctx_lens.astype(np.int64) - 1
        sl = synth.slots_for_positions(self.block_tables, pos, BS)
        kk = np.stack([self.k[s][int(pos[s])] for s in range(self.S)])
        vv = np.stack([self.v[s][int(pos[s])] for s in range(self.S)])
        return sl, kk, vv


def make_case(kv_type, ctx_lens, n_kv_heads=8, n_heads=32, n_blocks=None, seed=1, outlier_scale=1.0,
              stride=None):
    ctx_lens = np.asarray(ctx_lens, np.int32)
    pages = [(int(L) + BS - 1) // BS for L in ctx_lens]
    need = sum(pages)
    n_blocks = n_blocks if n_blocks is not None else max(2 * need, 8)
    bt = synth.scatter_block_tables(n_blocks, pages, seed, stride)
    c = Case(kv_type, n_blocks, n_kv_heads, n_heads, ctx_lens, bt)
    row = n_kv_heads * HD
    for s, L in enumerate(ctx_lens):
        L = int(L)
        c.k.append(synth.normals_f16(L * row, seed * 1000 + 2 * s, row, outlier_scale).reshape(L, n_kv_heads, HD))
        c.v.append(synth.normals_f16(L * row, seed * 1000 + 2 * s + 1, row, outlier_scale).reshape(L, n_kv_heads, HD))
    c.q = synth.normals_f16(c.S * n_heads * HD, seed * 1000 + 999).reshape(c.S, n_heads, HD)
    return c


def oracle_layer(case: Case, with_last=True):
    L = O.Layer(case.n_blocks, case.n_kv_heads, BS, HD, case.kv_type)
    sl, kk, vv = case.prefill_slots()
    if len(sl):
        O.append(L, kk, vv, sl)
    if with_last:
        sl, kk, vv = case.last_slots()
        O.append(L, kk, vv, sl)
    return L


def tol_check(got, ref, atol=2e-3, rtol=1e-2):
    """The north-star tolerance: |got - ref| <= atol + rtol * |ref| elementwise."""
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = atol + rtol * np.abs(ref.astype(np.float64))
    bad = err > bound
    return (not bad.any()), float(err.max(initial=0.0)), int(bad.sum())


def ref_codes_closed_form(x):
    """kv_update_int8's codes restated in numpy fp32 (kernels.metal:783-797):
    inv = 127 / amax rounded to fp32 once, each x * inv rounded to fp32, then the
    (char) cast truncates toward zero. No step is shared with the C oracle."""
    x32 = np.asarray(x, np.float32)
    amax = np.max(np.abs(x32), axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    prod = (x32 * inv).astype(np.float32)
    return np.trunc(prod).astype(np.int8), (amax[..., 0] / np.float32(127)).astype(np.float32)
