"""CPU pins of the RoPE oracle and of the host table function vk_rope_table.

- the table: cos / sin of p * base^(-2i/D) computed in float64 by numpy and
  rounded to fp32 once, equal to the oracle's and to vk_rope_table's (the
  C ABI's host function, callable without a GPU);
- the reference's own test rope_does_not_change_norm (llama_cpu.rs:557-564),
  plus norm preservation at other positions;
- agreement with the restatements of both reference paths (llama_cpu.rs:113-131
  half-split, kernels.metal:103-131 interleaved, fp32 angles) at small
  positions, where their fp32 angle is accurate;
- the rotation itself against a float64 rotation of the same inputs;
- half-split equals interleaved under the pair permutation, exactly (catches a
  wrong partner index);
- position 0 is the identity, exactly; scores depend only on relative position.
"""
import numpy as np
import pytest

import pyoracle as O
import velokv

D = 128


def test_table_matches_numpy_and_the_c_abi():
    n_pos, base = 3000, 500000.0
    ref = np.zeros((n_pos, D // 2, 2), np.float32)
    i = np.arange(D // 2, dtype=np.float64)
    inv = np.power(float(np.float32(base)), -2.0 * i / D)
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None, :]
    ref[:, :, 0] = np.cos(ang).astype(np.float32)
    ref[:, :, 1] = np.sin(ang).astype(np.float32)
    got = O.rope_table(n_pos, D, base)
    host = velokv.rope_table(n_pos, D, base)
    assert np.array_equal(got, host)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1


def test_reference_norm_test_and_identity_at_position_zero():
    # llama_cpu.rs:557-564: q = [1, 0, 0, 1], k = [.5, .5, -.5, -.5], pos 0, D 4
    t4 = O.rope_table(8, 4, 10000.0)
    q = np.array([[[1.0, 0.0, 0.0, 1.0]]], np.float32)
    for style in (O.ROPE_HALF, O.ROPE_INTERLEAVED):
        r = O.rope_apply(q, [0], style, t4)
        assert np.array_equal(r, q)  # cos 0 = 1, sin 0 = 0: exact
        r = O.rope_apply(q, [5], style, t4)
        assert abs(np.linalg.norm(r) - np.linalg.norm(q)) < 1e-4


@pytest.mark.parametrize("style", [O.ROPE_HALF, O.ROPE_INTERLEAVED])
def test_rotation_against_float64_and_norm(style):
    rng = np.random.default_rng(3)
    n_pos = 9000
    t = O.rope_table(n_pos, D, 10000.0)
    pos = np.array([0, 1, 17, 511, 4095, 8191, 8999])
    x = rng.standard_normal((len(pos), 2, D)).astype(np.float32)
    got = O.rope_apply(x, pos, style, t)
    tt = t.astype(np.float64)
    for n, p in enumerate(pos):
        c, s = tt[p, :, 0], tt[p, :, 1]
        for h in range(2):
            v = x[n, h].astype(np.float64)
            if style == O.ROPE_HALF:
                a, b = v[:D // 2], v[D // 2:]
                ref = np.concatenate([a * c - b * s, a * s + b * c])
            else:
                a, b = v[0::2], v[1::2]
                ref = np.empty(D)
                ref[0::2], ref[1::2] = a * c - b * s, a * s + b * c
            assert np.abs(got[n, h] - ref).max() <= 4e-6 * (1 + np.abs(ref).max())
            assert abs(np.linalg.norm(got[n, h]) - np.linalg.norm(v)) <= 1e-5 * np.linalg.norm(v)


def test_agrees_with_both_reference_paths_at_small_positions():
    rng = np.random.default_rng(4)
    t = O.rope_table(64, D, 10000.0)
    for p in (1, 7, 31, 63):
        x = rng.standard_normal(D).astype(np.float32)
        cpu = O.ref_rope_cpu(x, p, 10000.0)
        metal = O.ref_rope_metal(x, p, 10000.0)
        half = O.rope_apply(x[None, None], [p], O.ROPE_HALF, t)[0, 0]
        inter = O.rope_apply(x[None, None], [p], O.ROPE_INTERLEAVED, t)[0, 0]
        assert np.abs(half - cpu).max() < 2e-5
        assert np.abs(inter - metal).max() < 2e-5
        assert np.abs(half - inter).max() > 1e-2  # the two reference paths really differ


def test_half_split_is_interleaved_under_the_pair_permutation():
    rng = np.random.default_rng(5)
    t = O.rope_table(5000, D, 10000.0)
    x = rng.standard_normal((3, 4, D)).astype(np.float32)
    pos = [3, 1000, 4999]
    perm = np.empty(D, np.int64)
    perm[0::2], perm[1::2] = np.arange(D // 2), np.arange(D // 2) + D // 2  # interleaved slot -> half-split dim
    half = O.rope_apply(x, pos, O.ROPE_HALF, t)
    inter = O.rope_apply(x[..., perm], pos, O.ROPE_INTERLEAVED, t)
    assert np.array_equal(half[..., perm], inter)


def test_scores_depend_on_relative_position_only():
    rng = np.random.default_rng(6)
    t = O.rope_table(6000, D, 10000.0)
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)
    for style in (O.ROPE_HALF, O.ROPE_INTERLEAVED):
        s = [float(np.dot(O.rope_apply(q, [a + 40], style, t).ravel(), O.rope_apply(k, [a], style, t).ravel()))
             for a in (0, 100, 2500, 5900)]
        assert max(s) - min(s) < 1e-3 * (1 + abs(s[0]))
