"""The 32-register FWHT kernel's index maps and LDS image (csrc/fwht.hip,
WideMap and wide_lds_addr), restated here:

* each phase's map (thread t, register r) -> element index is a bijection;
* flipping register bit j flips exactly the element bit that phase butterflies
  (phase 0: bits 0-4, phase 1: bits 5-9, phase 2: bits 10.. log n - 1 on
  register bits P..4), so the three phases run stages 0, 1, ..., log n - 1 in
  order (the reference's stage order, src/butterfly_reference.cpp:349-369);
* the registers of phase 2 below bit P (P = 15 - log n) are element bits
  0..P-1, so each thread's results form runs of 2^P consecutive elements;
* each LDS word splits into a per-thread base plus a register offset;
* every 32-lane group of the four exchange accesses (phase-0 write, phase-1
  read and write, phase-2 read) lands on 32 distinct banks of the padded image
  addr = i + i/32.

A layout change in the kernel must change these maps too."""
import pytest


def maps(log_n):
    p = 5 - (log_n - 10)
    i0 = lambda t, r: (t << 5) | r
    i1 = lambda t, r: (t & 31) | (r << 5) | ((t >> 5) << 10)
    i2 = lambda t, r: (r & ((1 << p) - 1)) | (t << p) | ((r >> p) << 10)
    return p, 1 << (log_n - 5), (i0, i1, i2)


def lds_addr(i):
    return i + (i >> 5)


@pytest.mark.parametrize("log_n", [11, 12, 13])
def test_maps_are_bijections_with_the_stage_order(log_n):
    p, threads, (i0, i1, i2) = maps(log_n)
    for f in (i0, i1, i2):
        assert sorted(f(t, r) for t in range(threads) for r in range(32)) == list(range(1 << log_n))
    stages = []
    for t in range(threads):
        for r in range(32):
            for j in range(5):
                assert i0(t, r ^ (1 << j)) == i0(t, r) ^ (1 << j)
                assert i1(t, r ^ (1 << j)) == i1(t, r) ^ (1 << (5 + j))
            for j in range(p, 5):
                assert i2(t, r ^ (1 << j)) == i2(t, r) ^ (1 << (10 + j - p))
    stages = list(range(5)) + list(range(5, 10)) + [10 + j - p for j in range(p, 5)]
    assert stages == list(range(log_n))


@pytest.mark.parametrize("log_n", [11, 12, 13])
def test_phase_two_runs_are_consecutive(log_n):
    p, threads, (_, _, i2) = maps(log_n)
    for t in range(threads):
        for g in range(32 >> p):
            run = [i2(t, (g << p) | k) for k in range(1 << p)]
            assert run == list(range(run[0], run[0] + (1 << p)))
            assert run[0] % (1 << p) == 0  # aligned: one 8- to 64-byte vector store


@pytest.mark.parametrize("log_n", [11, 12, 13])
def test_exchanges_are_conflict_free(log_n):
    _, threads, (i0, i1, i2) = maps(log_n)
    for f in (i0, i1, i2):
        for r in range(32):
            for g in range(0, threads, 32):
                banks = {lds_addr(f(t, r)) % 32 for t in range(g, min(g + 32, threads))}
                assert len(banks) == min(32, threads - g)


def test_the_padded_image_fits_the_kernel_array():
    for log_n in (11, 12, 13):
        n = 1 << log_n
        assert max(lds_addr(i) for i in range(n)) < n + (n >> 5)


@pytest.mark.parametrize("log_n", [11, 12, 13])
def test_lds_words_split_into_thread_and_register_parts(log_n):
    # The kernel addresses element I(t, r) at lds_addr(I(t, 0)) +
    # lds_addr(I(0, r)) (WideMap::lds_word): a per-thread base plus a
    # compile-time register offset. That equals lds_addr(I(t, r)) for every
    # map, thread and register.
    _, threads, (i0, i1, i2) = maps(log_n)
    for f in (i0, i1, i2):
        for t in range(threads):
            for r in range(32):
                assert lds_addr(f(t, 0)) + lds_addr(f(0, r)) == lds_addr(f(t, r))
