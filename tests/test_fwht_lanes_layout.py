"""The 64-elements-per-lane FWHT kernel (csrc/fwht.hip, fwht_lane_kernel,
lane_element, register_element, swap_lane_bit) replayed on the CPU for one
wave's 4096 elements: the same fp32 operations in the same order, on numpy
float32 (IEEE round-to-nearest-even per operation, like the VALU), with the
two lane-swap instructions modelled as measured on gfx950 with a one-wave
probe (lane l of the first operand holding l, of the second 100 + l):

* v_permlane32_swap(a, b) -> (a[0:32] ++ b[0:32], a[32:64] ++ b[32:64]);
* v_permlane16_swap(a, b) -> (a[0:16] ++ b[0:16] ++ a[32:48] ++ b[32:48],
  a[16:32] ++ b[16:32] ++ a[48:64] ++ b[48:64]).

The replay must equal the stage-ordered oracle (src/butterfly_reference.cpp:
349-369) bit for bit, so the element map, the swaps and the butterfly order
are pinned without a GPU. A swap model with the halves exchanged (a
plausible misreading of the instructions) must fail. The element map must
also keep every 16-byte access instruction on as few 128-byte lines as the
16-register kernel's."""
import numpy as np
import pytest

import oracle

LANES, REGS = 64, 64


def lane_element(lane):
    return (((lane >> 4) & 3) << 4) | ((lane & 15) << 8)


def register_element(r):
    return (r & 15) | ((r >> 4) << 6)


def element(lane, r):
    return lane_element(lane) | register_element(r)


def swap32(a, b):
    return np.concatenate([a[:32], b[:32]]), np.concatenate([a[32:], b[32:]])


def swap16(a, b):
    return (np.concatenate([a[0:16], b[0:16], a[32:48], b[32:48]]),
            np.concatenate([a[16:32], b[16:32], a[48:64], b[48:64]]))


def misread(fn):
    def swapped(a, b):
        x, y = fn(a, b)
        return y, x
    return swapped


def stages(v, lo, hi):
    for j in range(lo, hi):
        d = 1 << j
        for r in range(REGS):
            if not r & d:
                a, b = v[r].copy(), v[r + d].copy()
                v[r], v[r + d] = a + b, a - b


def swap_bit(v, rb, fn):
    for r in range(REGS):
        if not (r >> rb) & 1:
            v[r], v[r | (1 << rb)] = fn(v[r], v[r | (1 << rb)])


def replay(x, log_n, s32=swap32, s16=swap16):
    """x: 4096 float32 (4096 / n rows) -> the kernel's 4096 results."""
    idx = [np.array([element(lane, r) for lane in range(LANES)]) for r in range(REGS)]
    v = [x[i].astype(np.float32) for i in idx]  # v[r][lane]
    stages(v, 0, 4)
    swap_bit(v, 0, s16)
    stages(v, 0, 1)
    if log_n >= 6:
        swap_bit(v, 1, s32)
        stages(v, 1, 2)
    if log_n >= 7:
        stages(v, 4, log_n - 2)
    if log_n >= 6:
        swap_bit(v, 1, s32)
    swap_bit(v, 0, s16)
    out = np.empty(4096, np.float32)
    for r in range(REGS):
        out[idx[r]] = v[r]
    return out


def wave_input(seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(4096) * 3 + rng.integers(-4, 5, 4096)).astype(np.float32)


def test_element_map_is_a_bijection():
    assert sorted(element(lane, r) for lane in range(LANES) for r in range(REGS)) == list(range(4096))


@pytest.mark.parametrize("elements_per_access,lines_per_access", [(8, 16), (4, 32)])  # fp16, fp32
def test_accesses_touch_few_lines(elements_per_access, lines_per_access):
    # As many lines as the 16-register kernel's accesses (16 or 32 consecutive
    # bytes per lane): 16 lines for fp16, 32 for fp32.
    bytes_per_element = 16 // elements_per_access
    for a in range(REGS // elements_per_access):
        r0 = a * elements_per_access
        lines = set()
        for lane in range(LANES):
            first = element(lane, r0)
            # one access: consecutive registers are consecutive elements
            assert [element(lane, r0 + k) for k in range(elements_per_access)] == \
                list(range(first, first + elements_per_access))
            lines.add(first * bytes_per_element // 128)
        assert len(lines) == lines_per_access


@pytest.mark.parametrize("log_n", [5, 6, 7, 8])
def test_replay_matches_the_stage_ordered_oracle(log_n):
    x = wave_input(seed=log_n)
    got = replay(x, log_n)
    want = oracle.fwht_f32(x.reshape(-1, 1 << log_n)).reshape(-1)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("which", ["swap32", "swap16"])
def test_misread_swap_fails(which):
    x = wave_input(seed=1)
    want = oracle.fwht_f32(x.reshape(-1, 256)).reshape(-1)
    kw = {"s32": misread(swap32)} if which == "swap32" else {"s16": misread(swap16)}
    assert not np.array_equal(replay(x, 8, **kw).view(np.uint32), want.view(np.uint32))
