"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something other than a retyping of its
own loop: the reference's own known answers, closed forms, brute force by
definition (Python big integers / numpy float64), the reference test-side
formulations, and library routines (numpy float16, numpy.fft). Each check is
chosen so that a plausible mistake -- a dropped term, a wrong sign or index, a
transposed operand, a different stage order or root -- fails it.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from cubutterfly_amd import ntt_roots, workloads

# Reference moduli fixtures: tests/test_ntt.cpp:251 and friends,
# tests/test_rns_ntt.cu:19, tests/test_crypto_ntt_host.py:21-26, include/cuntt/ntt.hpp:17.
MODULI = [998244353, 1073479681, 2013265921, 8380417, 2130706433,
          576460756061519873, 1152921504577486849, 1152921504606584833]


@pytest.fixture(scope="module", autouse=True)
def built():
    oracle.build()


# ---------------------------------------------------------------- FWHT

def test_fwht_reference_known_answers():
    # reference_fwht({1..8}) as printed by the reference's own C++ oracle
    # (compiled and run once during the survey of the reference).
    np.testing.assert_array_equal(oracle.fwht_f32(np.arange(1, 9, dtype=np.float32)),
                                  [36, -4, -8, 0, -16, 0, 0, 0])
    # tests/test_c_api.c:1031-1058: eight ones -> output[0] == 8 (rest 0).
    np.testing.assert_array_equal(oracle.fwht_f32(np.ones(8, np.float32)), [8, 0, 0, 0, 0, 0, 0, 0])


def sylvester(n):
    h = np.array([[1]], dtype=np.int64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("log_n", [1, 2, 3, 5, 6])
def test_fwht_matches_sylvester_matrix(log_n):
    n = 1 << log_n
    x = workloads.fwht_integer_input(log_n, 7, seed=log_n)
    expected = (sylvester(n) @ x.astype(np.int64).T).T  # natural (Sylvester) ordering
    np.testing.assert_array_equal(oracle.fwht_f32(x), expected.astype(np.float32))


def test_fwht_inverse_normalised_round_trip():
    x = workloads.fwht_integer_input(9, 5, seed=3)
    y = oracle.fwht_f32(x)
    np.testing.assert_array_equal(oracle.fwht_f32(y, inverse=True, normalize=True), x)  # H H = n I
    np.testing.assert_array_equal(oracle.fwht_f32(y, inverse=True, normalize=False), x * 512)


def reference_test_fwht_stages(x):
    """Stage loop in the formulation of tests/test_fwht_final_storage.py:28-40:
    for width = 1, 2, 4, ...: view rows as (-1, 2*width), left+right | left-right."""
    result = x.astype(np.float32)
    rows, n = result.shape
    width = 1
    while width < n:
        paired = result.reshape(rows, -1, 2 * width)
        left, right = paired[..., :width], paired[..., width:]
        result = np.concatenate((left + right, left - right), axis=-1).reshape(rows, n)
        width *= 2
    return result


def test_fwht_stage_order_is_pinned_on_random_floats():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((16, 1024)) * np.exp(rng.standard_normal((16, 1024)) * 4)).astype(np.float32)
    got = oracle.fwht_f32(x)
    np.testing.assert_array_equal(got, reference_test_fwht_stages(x))
    # Sensitivity: the same network with bits processed high-to-low rounds differently.
    flipped = reference_test_fwht_stages(x.reshape(16, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2)
                                         .transpose(0, *range(10, 0, -1)).reshape(16, 1024))
    flipped = flipped.reshape(16, *([2] * 10)).transpose(0, *range(10, 0, -1)).reshape(16, 1024)
    assert not np.array_equal(got, flipped)


# ---------------------------------------------------------------- binary16

def test_f16_to_f32_all_patterns():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle._lib().cbo_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(expected)
    np.testing.assert_array_equal(got[finite].view(np.uint32), expected[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]) == np.isnan(expected[~finite]))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(5)
    # Random bit patterns over the whole exponent range plus every tie pattern
    # around the subnormal, normal and overflow boundaries.
    patterns = rng.integers(0, 1 << 32, 60000, dtype=np.uint64).astype(np.uint32)
    specials = []
    for exponent in range(96, 146):
        for low in (0x0000, 0x0FFF, 0x1000, 0x1001, 0x2000, 0x3000, 0x1FFF):
            for mant_hi in (0, 1, 0x3FF):
                specials.append((exponent << 23) | (mant_hi << 13) | low)
    patterns = np.concatenate([patterns, np.array(specials, dtype=np.uint32),
                               np.array(specials, dtype=np.uint32) | np.uint32(0x80000000)])
    values = patterns.view(np.float32)
    values = values[~np.isnan(values)]
    with np.errstate(over="ignore"):
        expected = values.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_f16_bits(values), expected)


def test_fwht_fp16_final_storage_matches_reference_test_oracle():
    # tests/test_fwht_final_storage.py:22-40: dyadic inputs, fp32 stages, x scale, .half().
    rng = np.random.default_rng(61013)
    for n, inverse, normalize, scale in [(32, False, False, 1.0), (64, False, True, 0.375),
                                         (128, True, False, -0.75), (128, True, True, 0.375),
                                         (4096, False, False, 1 / 64)]:
        x = (rng.integers(-1024, 1025, (3, n)).astype(np.float32) / 1024).astype(np.float16)
        y = reference_test_fwht_stages(x.astype(np.float32))
        if inverse and normalize:
            y = y / np.float32(n)
        expected = (y * np.float32(scale)).astype(np.float16)
        got = oracle.fwht_f16_final(x, scale, inverse=inverse, normalize=normalize)
        np.testing.assert_array_equal(got.view(np.uint16), expected.view(np.uint16))


def test_fwht_fp16_final_storage_quarot_rows():
    x = workloads.quarot_input(8, 4096, seed=2)
    y = reference_test_fwht_stages(x.astype(np.float32)) * np.float32(1 / 64)
    np.testing.assert_array_equal(oracle.fwht_f16_final(x, 1 / 64).view(np.uint16),
                                  y.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- FFT

@pytest.mark.parametrize("log_n", [1, 4, 10, 14])
def test_fft_matches_numpy_float64(log_n):
    x = workloads.complex_input(log_n, 3, seed=log_n)
    ref = np.fft.fft(x.astype(np.complex128), axis=-1)
    got = oracle.fft_c64(x)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 2e-7
    inv = oracle.fft_c64(got, inverse=True, normalize=True)
    assert np.linalg.norm(inv - x) / np.linalg.norm(x) < 2e-7
    raw = oracle.fft_c64(got, inverse=True, normalize=False)
    assert np.linalg.norm(raw - x * (1 << log_n)) / np.linalg.norm(x * (1 << log_n)) < 2e-7


def test_fft_closed_forms():
    n = 256
    impulse = np.zeros(n, np.complex64)
    impulse[0] = 1
    np.testing.assert_array_equal(oracle.fft_c64(impulse), np.ones(n, np.complex64))
    const = np.ones(n, np.complex64)
    expected = np.zeros(n, np.complex64)
    expected[0] = n
    np.testing.assert_allclose(oracle.fft_c64(const), expected, atol=1e-4)
    # Forward sign convention: X_k = sum_j x_j exp(-2 pi i jk/n) -> a tone at +k0 lands on bin k0.
    k0 = 5
    tone = np.exp(2j * np.pi * k0 * np.arange(n) / n).astype(np.complex64)
    spectrum = oracle.fft_c64(tone)
    assert abs(spectrum[k0] - n) < 1e-3 and np.max(np.abs(np.delete(spectrum, k0))) < 1e-3


# ---------------------------------------------------------------- roots

def brute_root(log_n, q):
    """Smallest c >= 2 whose c^((q-1)/n) has exact order n, by definition."""
    n = 1 << log_n
    for c in range(2, 1 << 20):
        w = pow(c, (q - 1) // n, q)
        if pow(w, n, q) == 1 and pow(w, n // 2, q) != 1:
            return w
    raise AssertionError("no root")


def brute_psi(log_n, q, w):
    order = 2 << log_n
    cands = []
    for c in range(2, 1 << 20):
        psi = pow(c, (q - 1) // order, q)
        if pow(psi, order, q) == 1 and pow(psi, order // 2, q) != 1:
            cands.append(psi)
            if psi * psi % q == w:
                # The default (first candidate) wins when it squares to w.
                return cands[0] if cands[0] * cands[0] % q == w else psi
    raise AssertionError("no psi")


@pytest.mark.parametrize("q", MODULI)
def test_is_prime_and_roots(q):
    assert oracle.is_prime(q) and not oracle.is_prime(q * 3) and not oracle.is_prime(q - 1)
    for log_n in (1, 3, 8, 13):
        if (q - 1) % (1 << (log_n + 1)):
            continue
        w = oracle.find_primitive_root(log_n, q)
        assert w == brute_root(log_n, q)
        assert oracle.find_psi(log_n, q, w) == brute_psi(log_n, q, w)


GOLDEN = Path(__file__).resolve().parent / "golden"


def test_roots_match_the_references_recorded_roots():
    # The reference's benchmark runner records the root it handed each timed
    # NTT backend (experiments/snapshots/*/identities.json, snapshot.json):
    # find_primitive_power_of_two_root(log2 n, q) for 11 (q, n) pairs, C2's
    # modulus at n = 2^16 among them. tests/golden/extract_reference_roots.py
    # wrote them; the root convention every bit-exact NTT test rests on is
    # pinned by these values, not only by brute_root's restatement.
    records = json.loads((GOLDEN / "reference_roots.json").read_text())["records"]
    assert len(records) == 11 and any(r["modulus"] == workloads.C2_MODULUS and r["n"] == 1 << 16 for r in records)
    for r in records:
        log_n = r["n"].bit_length() - 1
        assert oracle.find_primitive_root(log_n, r["modulus"]) == r["root"], r
        assert ntt_roots.primitive_root(log_n, r["modulus"]) == r["root"], r


def test_is_prime_small_range():
    def naive(v):
        return v >= 2 and all(v % d for d in range(2, int(v ** 0.5) + 1))
    for v in range(0, 3000):
        assert oracle.is_prime(v) == naive(v), v
    assert not oracle.is_prime(3215031751)  # strong pseudoprime to bases 2, 3, 5, 7


# ---------------------------------------------------------------- NTT

def naive_cyclic(x, w, q):
    n = len(x)
    return [sum(int(x[j]) * pow(w, j * k, q) for j in range(n)) % q for k in range(n)]


@pytest.mark.parametrize("q", [998244353, 1073479681, 576460756061519873, 1152921504606584833])
@pytest.mark.parametrize("log_n", [1, 3, 5])
def test_cyclic_ntt_is_the_dft_with_the_reference_root(q, log_n):
    n = 1 << log_n
    x = workloads.ntt_input(log_n, 2, q, seed=9)
    w = brute_root(log_n, q)
    got = oracle.ntt_cyclic(x, q)
    for row in range(2):
        assert [int(v) for v in got[row]] == naive_cyclic(x[row], w, q)
    back = oracle.ntt_cyclic(got, q, inverse=True)
    np.testing.assert_array_equal(back, x)
    # The inverse is the DFT with w^-1, times n^-1.
    inv_n = pow(n, q - 2, q)
    expect = [v * inv_n % q for v in naive_cyclic(x[0], pow(w, q - 2, q), q)]
    assert [int(v) for v in oracle.ntt_cyclic(x, q, inverse=True)[0]] == expect


def naive_negacyclic(x, psi, q):
    n = len(x)
    return [sum(int(x[j]) * pow(psi, j * (2 * k + 1), q) for j in range(n)) % q for k in range(n)]


@pytest.mark.parametrize("q", [1073479681, 998244353, 1152921504606584833])
@pytest.mark.parametrize("log_n", [2, 4, 6, 9])
def test_negacyclic_matches_definition(q, log_n):
    n = 1 << log_n
    x = workloads.ntt_input(log_n, 2, q, seed=4)
    w = brute_root(log_n, q)
    psi = brute_psi(log_n, q, w)
    fwd = oracle.ntt_negacyclic(x, q)
    assert [int(v) for v in fwd[1]] == naive_negacyclic(x[1], psi, q)
    np.testing.assert_array_equal(oracle.ntt_negacyclic(fwd, q, inverse=True), x)


def test_negacyclic_convolution_theorem():
    q, log_n = 1073479681, 5
    n = 1 << log_n
    a = workloads.ntt_input(log_n, 1, q, seed=1)[0]
    b = workloads.ntt_input(log_n, 1, q, seed=2)[0]
    prod = [0] * n
    for i in range(n):
        for j in range(n):
            k, s = (i + j) % n, -1 if i + j >= n else 1
            prod[k] = (prod[k] + s * int(a[i]) * int(b[j])) % q
    fa = oracle.ntt_negacyclic(a[None], q)[0]
    fb = oracle.ntt_negacyclic(b[None], q)[0]
    pointwise = np.array([int(x) * int(y) % q for x, y in zip(fa, fb)], dtype=np.uint64)
    assert [int(v) for v in oracle.ntt_negacyclic(pointwise[None], q, inverse=True)[0]] == prod


# ---------------------------------------------------------------- RNS

def bitrev(i, bits):
    return int(format(i, f"0{bits}b")[::-1], 2) if bits else 0


@pytest.mark.parametrize("in_rev,out_rev", [(0, 1), (1, 0), (0, 0), (1, 1)])
def test_rns_reference_orders_and_roots(in_rev, out_rev):
    # tests/test_rns_ntt.cu:113-140: explicit root fixtures psi = primitive^3, ^5.
    log_n = 5
    n = 1 << log_n
    primes = [1152921504577486849, 576460756061519873]
    roots = [pow(brute_root(log_n + 1, q), e, q) for q, e in zip(primes, (3, 5))]
    x = np.stack([workloads.ntt_input(log_n, 1, q, seed=3 + i)[0] for i, q in enumerate(primes)])
    got = oracle.rns(x, primes, roots, input_bit_reversed=in_rev, output_bit_reversed=out_rev)
    for p, (q, psi) in enumerate(zip(primes, roots)):
        logical = [int(x[p][bitrev(j, log_n) if in_rev else j]) for j in range(n)]
        expect = naive_negacyclic(logical, psi, q)
        physical = [expect[bitrev(j, log_n)] if out_rev else expect[j] for j in range(n)]
        assert [int(v) for v in got[p]] == physical
    back = oracle.rns(got, primes, roots, inverse=True, input_bit_reversed=out_rev, output_bit_reversed=in_rev)
    np.testing.assert_array_equal(back, x)


def test_rns_cyclic_matches_dft():
    q, log_n = 576460756061519873, 4
    w = pow(brute_root(log_n, q), 3, q)
    x = workloads.ntt_input(log_n, 1, q, seed=8)
    got = oracle.rns(x, [q], [w], negacyclic=False)
    assert [int(v) for v in got[0]] == naive_cyclic(x[0], w, q)


def test_rns_agrees_with_negacyclic_channel_for_the_benchmark_root():
    # With psi chosen by the crypto-benchmark rule, the RNS negacyclic reference
    # (natural order) equals the benchmark composition twist + cyclic NTT.
    q, log_n = 1152921504606584833, 8
    w = brute_root(log_n, q)
    psi = brute_psi(log_n, q, w)
    x = workloads.ntt_input(log_n, 2, q, seed=6)
    np.testing.assert_array_equal(oracle.rns(x, [q, q], [psi, psi]), oracle.ntt_negacyclic(x, q))


# ---------------------------------------------------------------- input generators

def test_mt19937_64_matches_the_cpp_standard():
    # [rand.predef]: the 10000th consecutive output of a default-constructed
    # std::mt19937_64 (seed 5489) is 9981545732273789042. Every NTT input
    # (the reference's make_input, crypto_ntt_bench.cu:436-448) comes from
    # this generator.
    values = workloads.MT19937_64(5489).random(10000)
    assert int(values[-1]) == 9981545732273789042
    # Drawing in pieces gives the same stream as one draw.
    g = workloads.MT19937_64(5489)
    pieces = np.concatenate([g.random(k) for k in (1, 311, 312, 313, 9063)])
    np.testing.assert_array_equal(pieces, values)


def test_ntt_input_follows_make_input():
    # First four words {0, 1, q-1, q-2}, then mt19937_64 % q from the seed
    # seed ^ (0x9e3779b97f4a7c15 * (channel + 1)) (crypto_ntt_bench.cu:436-448).
    q = workloads.C2_MODULUS
    x = workloads.ntt_input(4, 2, q, seed=7, channel=3)
    assert list(map(int, x.ravel()[:4])) == [0, 1, q - 1, q - 2]
    g = workloads.MT19937_64(7 ^ ((0x9E3779B97F4A7C15 * 4) & ((1 << 64) - 1)))
    np.testing.assert_array_equal(x.ravel()[4:], g.random(28) % np.uint64(q))
