"""The Barrett reduction of the NTT engine's `-barrett` lowerings (no GPU
needed): the device formula restated step by step in exact integers, with
every intermediate truncated to the word as the kernel truncates it, checked
against a w mod q.

For a modulus q of bit length b (q < 2^(k - 2), k the word size) and
mu = floor(2^(2b+1) / q): P = a w, t = floor(P / 2^(b-2)),
Q = floor(t mu / 2^(b+3)), r = P - Q q modulo 2^k, then one conditional
subtraction. The claim the kernels rely on: for canonical a, w < q the
estimate Q is floor(P / q) or one less, so r < 2q before the subtraction and
the result is canonical. Pinned by exhaustion over every a, w for q < 400, by
random and boundary operands for every bit length up to k - 2, and a planted
mistake (mu one bit short) must fail the same check."""
import random

import pytest


def device_barrett(a, w, q, k, mu_shift=1):
    """The kernel's steps (csrc/ntt_kernels.hpp `barrett`), word size k."""
    mask = (1 << k) - 1
    b = q.bit_length()
    mu = ((1 << (2 * b + mu_shift)) // q) & mask
    if k == 32:
        p = a * w                                   # 64-bit product
        t = (p >> (b - 2)) & mask
        quo = ((t * mu) >> (b + 3)) & mask
        r = ((p & mask) - quo * q) & mask
    else:
        lo, hi = (a * w) & mask, (a * w) >> 64
        s = b - 2
        t = ((lo >> s) | (((hi << 1) & mask) << (63 - s))) & mask
        plo, phi = (t * mu) & mask, (t * mu) >> 64
        s2 = b + 3
        quo = (phi >> (s2 - 64)) if s2 >= 64 else ((plo >> s2) | (((phi << 1) & mask) << (63 - s2))) & mask
        r = (lo - quo * q) & mask
    before = r
    return (r - q if r >= q else r), before


def check(a, w, q, k, mu_shift=1):
    r, before = device_barrett(a, w, q, k, mu_shift)
    return before < 2 * q and r == (a * w) % q


@pytest.mark.parametrize("k", [32, 64])
def test_random_and_boundary_operands_every_bit_length(k):
    rng = random.Random(k)
    for b in range(2, k - 1):
        for _ in range(40):
            q = rng.randrange(1 << (b - 1), 1 << b) | 1
            q = max(q, 3)
            operands = [0, 1, q - 1, q - 2, q // 2, rng.randrange(q), rng.randrange(q)]
            for a in operands:
                for w in operands:
                    assert check(a, w, q, k), (k, q, a, w)


def test_exhaustive_small_moduli():
    for q in range(3, 400):
        for a in range(q):
            for w in range(q):
                assert check(a, w, q, 32), (q, a, w)


def test_c4_moduli_and_reference_primes():
    from cubutterfly_amd import workloads
    rng = random.Random(4)
    for q in list(workloads.c4_moduli()) + [1152921504577486849, 576460756061519873]:
        for _ in range(2000):
            a, w = rng.randrange(q), rng.randrange(q)
            assert check(a, w, q, 64), (q, a, w)
        assert check(q - 1, q - 1, q, 64)


def test_planted_short_mu_is_caught():
    # mu = floor(2^(2b) / q), one bit short: the estimate then falls short by
    # more than one, and the same check must fail somewhere.
    rng = random.Random(7)
    failures = 0
    for _ in range(200):
        q = rng.randrange(1 << 59, 1 << 60) | 1
        a, w = rng.randrange(q), rng.randrange(q)
        failures += not check(a, w, q, 64, mu_shift=0)
    assert failures > 0
