"""Pins of the sampling oracle (oracle/sampling.py): Triton's Philox stream against the
published known-answer vectors, the uniform map's end points and range, the normals'
moments and Box-Muller in float64, the keyed noise's seed arithmetic, the argmax rule,
and the Gumbel-max sampler's frequencies against softmax(logits / T)."""

import math

import numpy as np
import pytest

from oracle import sampling as S

# Random123 kat_vectors, philox4x32_10: counter words, key words -> output words
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = S.philox4x32(*(np.uint32(c) for c in ctr), np.uint32(key[0]), np.uint32(key[1]))
    assert tuple(int(x) for x in got) == want


def test_counter_and_key_words():
    # seed 0x243F6A8885A308D3 -> key (low, high); offset -> counter (low, 0 | high, 0, 0)
    seed = np.int64(0x243F6A8885A308D3)
    w = S.randint4x(seed, np.int64(0x13198A2E))
    ref = S.philox4x32(np.uint32(0x13198A2E), np.uint32(0), np.uint32(0), np.uint32(0),
                       np.uint32(0x85A308D3), np.uint32(0x243F6A88))
    assert all(int(a) == int(b) for a, b in zip(w, ref))
    off = np.arange(5, dtype=np.int64) + (3 << 32)
    narrow = S.randint4x(np.int64(7), off)  # int32 offsets: the high word is dropped
    wide = S.randint4x(np.int64(7), off, wide=True)
    low = S.randint4x(np.int64(7), off & 0xFFFFFFFF, wide=True)
    assert all((a == b).all() for a, b in zip(narrow, low)) and not (narrow[0] == wide[0]).all()


def test_uniform_map():
    words = np.array([0, 0xFFFFFFFF, 0x7FFFFFFF, 0x80000000, 1, 0xFFFFFFFE], dtype=np.uint32)
    u = S.uniform(words)
    assert u[0] == 0 and u[1] == 0  # 0 and -1 fold to 0
    assert u[2] == u[3] and u[2] < 1.0  # INT_MAX and INT_MIN fold to the largest value, below 1
    assert u[4] == u[5] == np.float32(np.float32(1) * np.float32(4.6566127342e-10))
    r = S.rand(np.int64(12345), np.arange(200000))
    assert r.dtype == np.float32 and r.min() >= 0 and r.max() < 1
    assert abs(r.mean() - 0.5) < 0.005 and abs(r.var() - 1 / 12) < 0.002


def test_normals_moments_and_box_muller():
    off = np.arange(200000)
    z = S.randn(np.int64(99), off)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1) < 0.02
    assert abs((z ** 3).mean()) < 0.03 and abs((z ** 4).mean() - 3) < 0.08
    w = S.randint4x(np.int64(99), off)
    u1 = np.maximum(1e-7, S.uniform(w[0]).astype(np.float64))
    u2 = S.uniform(w[1]).astype(np.float64)
    z64 = np.sqrt(-2 * np.log(u1)) * np.cos(2 * math.pi * u2)
    assert np.abs(z - z64).max() < 2e-5


def test_seeded_normal_keys():
    seeds = np.array([5, (1 << 62) + 3, -7], dtype=np.int64)
    rows = np.array([1, -1, 2, 0])
    pos = np.array([10, 4, 9, 0])
    z = S.seeded_normal(seeds, rows, pos, 64, scale=0.5)
    for i in range(4):
        seed = int(seeds[rows[i]]) if rows[i] >= 0 else 0
        key = (seed * 1000003 + int(pos[i])) % (1 << 64)  # int64 wrapping
        key = key - (1 << 64) if key >= (1 << 63) else key
        assert np.array_equal(z[i], (S.randn(np.int64(key), np.arange(64)) * np.float32(0.5)).astype(np.float32))


def test_argmax_rule():
    x = np.array([[1, 3, 3, 2], [-np.inf] * 4, [1, np.nan, 5, np.nan], [0, 0, 0, 0]], dtype=np.float32)
    assert S.argmax_first(x).tolist() == [1, 0, 1, 0]


def test_sampler_greedy_rows_and_frequencies():
    logits = np.array([1.0, 0.5, 0.0, -0.5, 2.0, 1.0], dtype=np.float32)
    rows, t = 30000, 0.7
    x = np.tile(logits, (rows, 1))
    greedy = np.zeros(rows, dtype=bool)
    greedy[:5] = True
    got = S.sample_rows(x, np.full(rows, t), greedy, seed=2024)
    assert (got[:5] == 4).all()
    p = np.exp(logits / t) / np.exp(logits / t).sum()
    counts = np.bincount(got[5:], minlength=6)
    expected = p * (rows - 5)
    chi2 = ((counts - expected) ** 2 / expected).sum()
    assert chi2 < 25.0  # 5 degrees of freedom: p < 1.4e-4 above this
    # another seed gives other samples with the same law
    again = S.sample_rows(x[:2000], np.full(2000, t), np.zeros(2000, bool), seed=2025)
    assert (again != got[:2000]).mean() > 0.5
