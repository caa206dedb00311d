"""CPU restatement of the draft step's sampling and noise kernels (numpy, exact integer
arithmetic for the random stream).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference's kernels draw their randomness with Triton's Philox generator
(``tl.rand`` / ``tl.randn``; Triton 3.x, ``triton/language/random.py``, the version in this
image is 3.6.0): Philox-4x32 with 10 rounds (Salmon et al., "Parallel random numbers: as
easy as 1, 2, 3", SC 2011), key = (seed low 32 bits, seed high 32 bits), counter =
(offset low 32 bits, offset high 32 bits, 0, 0); ``rand`` maps the first output word ``x``
(as int32) to ``(x < 0 ? -x - 1 : x) * 4.6566127342e-10`` in float32; ``randn`` takes the
first two words to uniforms ``u1, u2`` and returns ``sqrt(-2 log(max(u1, 1e-7))) *
cos(6.283185307179586 * u2)`` (Box-Muller) in float32.

Pinned by (tests/test_oracle_sampling.py): the Philox known-answer vectors published with
Random123 (kat_vectors, philox4x32_10); the uniform map's end points and range; the
normal's moments and the Box-Muller identity in float64; the Gumbel-max sample's
frequencies against softmax(logits / T) (chi-square); argmax ties to the first index.
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)  # Philox-4x32 multipliers
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)  # Weyl key increments
W1 = np.uint32(0xBB67AE85)
MASK32 = np.uint64(0xFFFFFFFF)
UNIFORM_SCALE = np.float32(4.6566127342e-10)
TWO_PI = np.float32(6.283185307179586)


def philox4x32(c0, c1, c2, c3, k0, k1, rounds: int = 10):
    """Philox-4x32 on uint32 arrays (broadcast): per round
    ``(c0, c1, c2, c3) <- (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0))``,
    then the key gains the Weyl increments (triton/language/random.py: philox_impl).
    Pinned by: the Random123 known-answer vectors."""
    c0, c1, c2, c3 = (np.asarray(x, dtype=np.uint32) for x in (c0, c1, c2, c3))
    k0, k1 = np.asarray(k0, dtype=np.uint32), np.asarray(k1, dtype=np.uint32)
    for _ in range(rounds):
        p0 = c0.astype(np.uint64) * M0
        p1 = c2.astype(np.uint64) * M1
        n0 = ((p1 >> np.uint64(32)).astype(np.uint32)) ^ c1 ^ k0
        n2 = ((p0 >> np.uint64(32)).astype(np.uint32)) ^ c3 ^ k1
        c1 = (p1 & MASK32).astype(np.uint32)
        c3 = (p0 & MASK32).astype(np.uint32)
        c0, c2 = n0, n2
        k0 = ((k0.astype(np.uint64) + np.uint64(W0)) & MASK32).astype(np.uint32)
        k1 = ((k1.astype(np.uint64) + np.uint64(W1)) & MASK32).astype(np.uint32)
    return c0, c1, c2, c3


def _seed_words(seed):
    s = np.asarray(seed).astype(np.int64).astype(np.uint64)
    return (s & MASK32).astype(np.uint32), (s >> np.uint64(32)).astype(np.uint32)


def randint4x(seed, offset, wide: bool = False):
    """The four words for int64 ``seed`` and integer ``offset`` arrays: counter = (offset's
    low word, its high word if the offsets are 64-bit (``wide``) else 0, 0, 0). Both
    reference kernels pass int32 offsets. Pinned by: the counter and key words of a known-answer
    vector (test_counter_and_key_words)."""
    off = np.asarray(offset).astype(np.int64).astype(np.uint64)
    k0, k1 = _seed_words(seed)
    zero = np.zeros(off.shape, dtype=np.uint32)
    hi = (off >> np.uint64(32)).astype(np.uint32) if wide else zero
    return philox4x32((off & MASK32).astype(np.uint32), hi, zero, zero, k0, k1)


def uniform(x):
    """uint32 words -> float32 in [0, 1): the word as int32, negatives folded by -x - 1. Pinned
    by: its end points (0, -1, INT_MAX, INT_MIN) and range."""
    i = np.asarray(x, dtype=np.uint32).view(np.int32).astype(np.int64)
    i = np.where(i < 0, -i - 1, i)
    return i.astype(np.float32) * UNIFORM_SCALE


def rand(seed, offset):
    """``tl.rand``: the uniform of the first word. Pinned by: range and moments over 200000
    offsets (test_uniform_map)."""
    return uniform(randint4x(seed, offset)[0])


def randn(seed, offset):
    """``tl.randn``: Box-Muller of the first two words' uniforms. Pinned by: moments, and
    the same words in float64 (test_normals_moments_and_box_muller)."""
    w = randint4x(seed, offset)
    u1, u2 = uniform(w[0]), uniform(w[1])
    u1 = np.maximum(np.float32(1e-7), u1)
    th = TWO_PI * u2
    r = np.sqrt(np.float32(-2.0) * np.log(u1))
    return (r * np.cos(th)).astype(np.float32)


def seeded_normal(seeds, rows, positions, n_cols: int, scale: float = 1.0):
    """flashmap/vllm/kernels.py:367-410: row ``i`` of ``(len(rows), n_cols)`` float32
    standard normals times ``scale``, keyed by ``seeds[rows[i]] * 1000003 + positions[i]``
    (int64, wrapping; seed 0 where ``rows[i] < 0``), column ``j`` at offset ``j``. Pinned
    by: each row against randn at the key computed in Python integers modulo 2^64
    (test_seeded_normal_keys)."""
    seeds = np.asarray(seeds, dtype=np.int64)
    rows = np.asarray(rows).astype(np.int64)
    pos = np.asarray(positions).astype(np.int64)
    seed = np.where(rows >= 0, seeds[np.maximum(rows, 0)], 0).astype(np.int64)
    with np.errstate(over="ignore"):
        key = (seed.astype(np.uint64) * np.uint64(1000003) + pos.astype(np.uint64)).astype(np.int64)
    cols = np.arange(n_cols, dtype=np.int64)
    out = randn(key[:, None], cols[None, :])
    return (out * np.float32(scale)).astype(np.float32)


def argmax_first(x):
    """Per row, the index of the largest value, the first among equals (torch.argmax's
    rule; a NaN counts as the largest, the first NaN wins). Pinned by: hand-checked rows
    (ties, -inf, NaN) (test_argmax_rule)."""
    x = np.asarray(x, dtype=np.float32)
    nan = np.isnan(x)
    idx = np.argmax(np.where(nan, -np.inf, x), axis=-1)
    has_nan = nan.any(axis=-1)
    return np.where(has_nan, np.argmax(nan, axis=-1), idx).astype(np.int64)


def split_argmax(logits):
    """flashmap/vllm/fold.py:117-128: ``logits.argmax(-1)`` (chunked on the GPU; the chunks
    do not change the result). Pinned by: argmax_first."""
    return argmax_first(logits)


def sample_keys(logits, temperatures, greedy, seed: int, row0: int = 0):
    """The keys flashmap/sglang/kernels.py:195-247 takes the argmax of, for rows
    ``row0 ..`` of the batch: a greedy row's key is its logit (float32), another row's
    ``logit / T - log(-log(u))`` with ``u = rand(seed, row * V + col)``, the offset in int32
    arithmetic as the reference's kernel forms it (low word, high word 0). Pinned by: the sampler's
    frequencies against softmax(logits / T) (chi-square) and its greedy rows."""
    x = np.asarray(logits, dtype=np.float32)
    rows, vocab = x.shape
    t = np.asarray(temperatures, dtype=np.float32)
    g = np.asarray(greedy).astype(bool)
    off = (np.arange(row0, row0 + rows, dtype=np.int64)[:, None] * vocab + np.arange(vocab, dtype=np.int64)[None, :])
    u = rand(np.int64(seed), off & 0xFFFFFFFF)
    with np.errstate(divide="ignore"):  # u = 0 gives key -inf, as on the GPU
        noisy = x / t[:, None] - np.log(-np.log(u))
    return np.where(g[:, None], x, noisy.astype(np.float32))


def sample_rows(logits, temperatures, greedy, seed: int, row0: int = 0):
    """flashmap/sglang/kernels.py:195-247: per row, the argmax of :func:`sample_keys`, the
    first index among equals (Gumbel-max: a sample of softmax(logits / T) for the
    non-greedy rows). Pinned by: as sample_keys."""
    return argmax_first(sample_keys(logits, temperatures, greedy, seed, row0))
