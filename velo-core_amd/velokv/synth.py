"""Seeded synthetic workloads (host side) for tests and the benchmark.

Generators:
  splitmix64 / normals_f16: counter-based SplitMix64 -> Box-Muller -> fp16 RNE,
    the same stream vk_fill_normal_f16 produces on the GPU (up to the last bit of
    the transcendental functions).
  scatter_block_tables: a Fisher-Yates permutation of the pool handed out to the
    sequences in order (each sequence's table is a random scatter).
"""
from __future__ import annotations

import numpy as np

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
OUTLIER_SALT = 0x6F75746C69657273


def splitmix64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = x + np.uint64(0x9E3779B97F4A7C15)
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return x ^ (x >> np.uint64(31))


def normals_f16(n: int, seed: int, row_len: int = 1, outlier_scale: float = 1.0, start: int = 0) -> np.ndarray:
    """fp16 N(0,1) samples i = start .. start+n-1; channels i % row_len whose
    SplitMix64(seed ^ OUTLIER_SALT ^ channel) % 100 == 0 are scaled by outlier_scale."""
    i = np.arange(start, start + n, dtype=np.uint64)
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    r1 = splitmix64(s ^ (np.uint64(2) * i))
    r2 = splitmix64(s ^ (np.uint64(2) * i + np.uint64(1)))
    u1 = ((r1 >> np.uint64(40)).astype(np.float64) + 1.0) / 16777216.0
    u2 = (r2 >> np.uint64(40)).astype(np.float64) / 16777216.0
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    if outlier_scale != 1.0:
        ch = i % np.uint64(row_len)
        out = (splitmix64(s ^ np.uint64(OUTLIER_SALT) ^ ch) % np.uint64(100)) == 0
        z = np.where(out, z * outlier_scale, z)
    return z.astype(np.float32).astype(np.float16)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def scatter_block_tables(n_blocks_pool: int, pages_per_seq, seed: int, stride: int | None = None) -> np.ndarray:
    """Random scatter: one permutation of the pool, consumed sequence by sequence."""
    pages_per_seq = [int(p) for p in pages_per_seq]
    need = sum(pages_per_seq)
    if need > n_blocks_pool:
        raise ValueError(f"{need} pages needed, pool has {n_blocks_pool}")
    perm = rng(seed).permutation(n_blocks_pool).astype(np.int32)
    stride = stride if stride is not None else max(pages_per_seq + [1])
    bt = np.zeros((len(pages_per_seq), stride), np.int32)
    off = 0
    for s, n in enumerate(pages_per_seq):
        bt[s, :n] = perm[off:off + n]
        off += n
    return bt


def slots_for_positions(block_tables: np.ndarray, positions, block_size: int, rows=None) -> np.ndarray:
    """Flat slots table[row][pos // bs] * bs + pos % bs (kernels.metal:637-640)."""
    positions = np.asarray(positions, dtype=np.int64)
    rows = np.arange(len(positions)) if rows is None else np.asarray(rows)
    blk = block_tables[rows, positions // block_size].astype(np.int64)
    return blk * block_size + positions % block_size
