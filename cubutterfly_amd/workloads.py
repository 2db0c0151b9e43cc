"""Seeded synthetic inputs for the five benchmark configurations (host side, numpy).

Portable generators (splitmix64, mt19937_64) so the same inputs can be rebuilt
anywhere. The NTT inputs follow the reference benchmark's make_input rule
(benchmarks/crypto_ntt/crypto_ntt_bench.cu:436-448): an mt19937_64 stream
seeded with seed ^ (0x9e3779b97f4a7c15 * (channel + 1)), the first four words of
the channel fixed to {0, 1, q-1, q-2}, then random() % q.
"""
import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def _u64(x):
    return np.uint64(x & M64)


def splitmix64(seed, count, offset=0):
    """Outputs offset..offset+count-1 of the splitmix64 stream started at `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = _u64(seed) + i * _u64(GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _u64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * _u64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


class MT19937_64:
    """The 64-bit Mersenne Twister (Matsumoto & Nishimura 2000), as std::mt19937_64.

    Blocks of 312 outputs are produced with three vectorised twist slices.
    """
    N, M = 312, 156
    A = 0xB5026F5AA96619E9
    UPPER, LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF

    def __init__(self, seed):
        state = [seed & M64]
        for i in range(1, self.N):
            prev = state[-1]
            state.append((6364136223846793005 * (prev ^ (prev >> 62)) + i) & M64)
        self.state = np.array(state, dtype=np.uint64)
        self.index = self.N

    def _twist(self):
        s = self.state
        n, m = self.N, self.M
        upper, lower, a = _u64(self.UPPER), _u64(self.LOWER), _u64(self.A)
        one = np.uint64(1)

        def step(i0, i1, nxt, far):
            x = (s[i0:i1] & upper) | (nxt & lower)
            return far ^ (x >> one) ^ np.where((x & one) != 0, a, np.uint64(0))

        s[0:n - m] = step(0, n - m, s[1:n - m + 1], s[m:n])
        s[n - m:n - 1] = step(n - m, n - 1, s[n - m + 1:n], s[0:m - 1])
        s[n - 1:n] = step(n - 1, n, s[0:1], s[m - 1:m])
        self.index = 0

    def _temper(self, y):
        y = y ^ ((y >> np.uint64(29)) & _u64(0x5555555555555555))
        y = y ^ ((y << np.uint64(17)) & _u64(0x71D67FFFEDA60000))
        y = y ^ ((y << np.uint64(37)) & _u64(0xFFF7EEE000000000))
        return y ^ (y >> np.uint64(43))

    def random(self, count):
        out = np.empty(count, dtype=np.uint64)
        filled = 0
        while filled < count:
            if self.index >= self.N:
                self._twist()
            take = min(self.N - self.index, count - filled)
            out[filled:filled + take] = self._temper(self.state[self.index:self.index + take])
            self.index += take
            filled += take
        return out


def ntt_input(log_n, batch, modulus, seed=1, channel=0):
    """uint64 [batch, n] per the reference make_input rule (random pattern)."""
    n = 1 << log_n
    count = batch * n
    values = np.empty(count, dtype=np.uint64)
    boundary = [0, 1 % modulus, modulus - 1, modulus - 2]
    head = min(4, count)
    values[:head] = boundary[:head]
    if count > 4:
        rng = MT19937_64(seed ^ ((GOLDEN * (channel + 1)) & M64))
        values[4:] = rng.random(count - 4) % np.uint64(modulus)
    return values.reshape(batch, n)


def fwht_integer_input(log_n, batch, seed=1):
    """fp32 [batch, n], (splitmix64 mod 17) - 8: exact FWHT sums in fp32."""
    n = 1 << log_n
    raw = splitmix64(seed, batch * n) % np.uint64(17)
    return (raw.astype(np.int64) - 8).astype(np.float32).reshape(batch, n)


def _uniform01(seed, count, offset=0):
    return (splitmix64(seed, count, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal_pairs(seed, count):
    """Box-Muller: `count` pairs of N(0,1) doubles from splitmix64."""
    u1 = _uniform01(seed, count, 0)
    u2 = _uniform01(seed, count, count)
    r = np.sqrt(-2.0 * np.log1p(-u1))
    theta = 2.0 * math.pi * u2
    return r * np.cos(theta), r * np.sin(theta)


def complex_input(log_n, batch, seed=1):
    """complex64 [batch, n] with i.i.d. N(0,1) real and imaginary parts."""
    n = 1 << log_n
    re, im = normal_pairs(seed, batch * n)
    out = np.empty(batch * n, dtype=np.complex64)
    out.real = re.astype(np.float32)
    out.imag = im.astype(np.float32)
    return out.reshape(batch, n)


def _box_muller_part(seed, pairs, first, count, imaginary):
    """The real (cos) or imaginary (sin) parts of pairs first..first+count-1
    of normal_pairs(seed, pairs)."""
    u1 = _uniform01(seed, count, first)
    u2 = _uniform01(seed, count, pairs + first)
    r = np.sqrt(-2.0 * np.log1p(-u1))
    theta = 2.0 * math.pi * u2
    return r * (np.sin(theta) if imaginary else np.cos(theta))


def _workers():
    return max(1, min(16, os.cpu_count() or 1))


def quarot_input(rows, n, seed=1, outlier_seed=7, chunk=1 << 21):
    """fp16 [rows, n]: N(0,1), columns with splitmix64 % 1000 == 0 scaled x50 (RNE).

    Element k of the flat array is the real part of Box-Muller pair k for
    k < P = ceil(rows * n / 2), else the imaginary part of pair k - P (the
    real parts of all pairs, then their imaginary parts). Chunks of `chunk`
    elements are generated on a thread pool (numpy releases the GIL); the
    values are those of one sequential pass."""
    total = rows * n
    pairs = (total + 1) // 2
    scale = np.where((splitmix64(outlier_seed, n) % np.uint64(1000)) == 0, 50.0, 1.0)
    out = np.empty(total, dtype=np.float16)

    def fill(start):
        stop = min(total, start + chunk)
        part = np.empty(stop - start)
        lo, hi = start, min(stop, pairs)
        if lo < hi:
            part[: hi - lo] = _box_muller_part(seed, pairs, lo, hi - lo, False)
        lo = max(start, pairs)
        if lo < stop:
            part[lo - start:] = _box_muller_part(seed, pairs, lo - pairs, stop - lo, True)
        part *= scale[np.arange(start, stop) % n]
        out[start:stop] = part.astype(np.float32).astype(np.float16)

    with ThreadPoolExecutor(_workers()) as pool:
        list(pool.map(fill, range(0, total, chunk)))
    return out.reshape(rows, n)


def _is_prime(q):
    if q < 2:
        return False
    for p in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37):
        if q % p == 0:
            return q == p
    d, s = q - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for a in (2, 325, 9375, 28178, 450775, 9780504, 1795265022):
        a %= q
        if a == 0:
            continue
        x = pow(a, d, q)
        if x in (1, q - 1):
            continue
        for _ in range(s - 1):
            x = x * x % q
            if x == q - 1:
                break
        else:
            return False
    return True


def ntt_primes(count, bits, log_order):
    """The `count` largest primes below 2^bits with q = 1 mod 2^log_order."""
    step = 1 << log_order
    k = ((1 << bits) - 2) // step
    primes = []
    while len(primes) < count and k > 0:
        q = k * step + 1
        if q < (1 << bits) and _is_prime(q):
            primes.append(q)
        k -= 1
    return primes


# BASELINE configurations (seeded, portable).
C2_MODULUS = 1073479681  # 2^30 - 2^18 + 1; reference fixture tests/test_ntt.cpp:251


def c4_moduli():
    return ntt_primes(32, 60, 17)
