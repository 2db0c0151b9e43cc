"""The 32-register FWHT kernel for short FP16 rows (csrc/fwht.hip,
fwht_short_kernel and ShortMap: 4096-element tiles of 2^(12 - log n) whole
rows, 128 threads x 32 registers, one LDS exchange), restated here:

* both phase maps (thread t, register r) -> tile element are bijections;
* flipping register bit j flips exactly the element bit that phase
  butterflies (phase 0: bits 0-4 on register bits 0-4; phase 1: bits
  5 .. log n - 1 on register bits P .. 4, P = 10 - log n), so the stages run
  0, 1, ..., log n - 1 in order (the reference's stage order,
  src/butterfly_reference.cpp:349-369);
* phase 1's registers below bit P are element bits 0 .. P - 1: aligned runs
  of 2^P consecutive results, stored at the row / column the kernel computes;
* the swizzled LDS image (low five word bits XORed with bits 5-9 rotated
  right by log n - 5) is a bijection, linear over disjoint bits (the kernel
  adds a per-thread base and a per-register offset by XOR), and puts every
  32-lane group of both accesses on 32 distinct banks (distinct modulo 32,
  hence also modulo 64), where the plain image does not.

A layout change in the kernel must change these maps too."""
import pytest

THREADS, REGS, TILE = 128, 32, 4096


def params(log_n):
    return 10 - log_n, log_n - 5  # passenger bits P, phase-1 butterfly thread bits


def lds_word(i, log_n):
    _, b1 = params(log_n)
    hi = (i >> 5) & 31
    return i ^ (((hi >> b1) | (hi << (5 - b1))) & 31)


def i0(t, r):
    return (t << 5) | r


def i1(t, r, log_n):
    p, b1 = params(log_n)
    thread = ((t & ((1 << b1) - 1)) << p) | ((t >> b1) << log_n)
    register = (r & ((1 << p) - 1)) | ((r >> p) << 5)
    return thread | register


LOGS = [7, 8]


@pytest.mark.parametrize("log_n", LOGS)
def test_maps_are_bijections_with_the_stage_order(log_n):
    p, _ = params(log_n)
    f1 = lambda t, r: i1(t, r, log_n)
    for f in (i0, f1):
        assert sorted(f(t, r) for t in range(THREADS) for r in range(REGS)) == list(range(TILE))
    for t in range(THREADS):
        for r in range(REGS):
            for j in range(5):
                assert i0(t, r ^ (1 << j)) == i0(t, r) ^ (1 << j)
            for j in range(p, 5):
                assert f1(t, r ^ (1 << j)) == f1(t, r) ^ (1 << (5 + j - p))
    stages = list(range(5)) + [5 + j - p for j in range(p, 5)]
    assert stages == list(range(log_n))


@pytest.mark.parametrize("log_n", LOGS)
def test_phase_zero_reads_whole_rows(log_n):
    # Thread t loads 32 consecutive elements of one row: row t >> (log n - 5),
    # columns from (t mod 2^(log n - 5)) * 32.
    _, b1 = params(log_n)
    for t in range(THREADS):
        row, col = t >> b1, (t & ((1 << b1) - 1)) << 5
        assert [i0(t, r) for r in range(REGS)] == [row * (1 << log_n) + col + r for r in range(REGS)]


@pytest.mark.parametrize("log_n", LOGS)
def test_phase_one_runs_are_the_kernel_stores(log_n):
    p, b1 = params(log_n)
    n = 1 << log_n
    for t in range(THREADS):
        out_row, out_col = t >> b1, (t & ((1 << b1) - 1)) << p
        for g in range(REGS >> p):
            run = [i1(t, (g << p) | k, log_n) for k in range(1 << p)]
            assert run == list(range(run[0], run[0] + (1 << p)))
            assert run[0] % (1 << p) == 0  # aligned: one 8- to 32-byte vector store
            assert run[0] == out_row * n + out_col + (g << 5)


@pytest.mark.parametrize("log_n", LOGS)
def test_image_is_a_bijection_linear_over_the_split(log_n):
    assert sorted(lds_word(i, log_n) for i in range(TILE)) == list(range(TILE))
    for t in range(THREADS):
        for r in range(REGS):
            assert lds_word(i0(t, r), log_n) == lds_word(t << 5, log_n) ^ r
            assert lds_word(i1(t, r, log_n), log_n) == lds_word(i1(t, 0, log_n), log_n) ^ lds_word(
                i1(0, r, log_n), log_n)


def distinct_banks(addr, f, lanes, banks):
    worst = lanes
    for r in range(REGS):
        for g in range(0, THREADS, lanes):
            worst = min(worst, len({addr(f(t, r)) % banks for t in range(g, g + lanes)}))
    return worst


@pytest.mark.parametrize("log_n", LOGS)
def test_exchange_is_conflict_free(log_n):
    swizzled = lambda i: lds_word(i, log_n)
    for f in (i0, lambda t, r: i1(t, r, log_n)):
        assert distinct_banks(swizzled, f, 32, 32) == 32
    # Unswizzled, both accesses pile lanes onto shared banks.
    plain = lambda i: i
    assert distinct_banks(plain, i0, 32, 32) == 1
    assert distinct_banks(plain, lambda t, r: i1(t, r, log_n), 32, 32) < 32
