"""The LDS image of the NTT's 4-byte row tiles of 2^8-point rows
(csrc/ntt_kernels.hpp, Lds<..., BANKED>), modelled on the CPU: every access
these tiles make covers 32 distinct four-byte banks per 32-lane half-wave,
and the image is injective over the tile (no GPU needed).

A tile of 2^8 x 2^LI words (LI = 4 or 5, 16 words per thread, 2^(4 + LI)
threads) is touched in three layouts, each as eight `ds_*2_b32` instructions
(two dwords per lane, the register parts in the immediate offsets):
* the exchange layouts phase_index<S>(t, r) for the windows S = 0 and 4;
* the staged boundary permutation of rows read or written at bit-reversed
  positions: element g = t + T r of the enumeration is tile index
  bitrev_8(g >> LI) | (g mod 2^LI) << 8.
The bank model (32 banks of 4 bytes, the 32 lanes of each half-wave served
together, one extra cycle per additional lane on a bank) reproduces the 4
conflict cycles per instruction that rocprofv3 measured with the single row
pitch of 273 words; the per-bit row offsets bring every layout to 0, which
the same counter confirmed on the GPU."""
import pytest

ROW_BITS = 8
DIGIT = 4


def brev(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def phase_index(s, t, r):
    return (t & ((1 << s) - 1)) | (r << s) | ((t >> s) << (s + DIGIT))


def staged(li, g):
    return brev(g >> li, ROW_BITS) | ((g & ((1 << li) - 1)) << ROW_BITS)


def banked(i):
    """The kernel's image: 272 (rr & 1) + 545 (rr >> 1) + x + x / 16."""
    x, rr = i & 0xFF, i >> ROW_BITS
    return 272 * (rr & 1) + 545 * (rr >> 1) + x + (x >> 4)


def pitched(i):
    """The previous image: one row pitch of 2^8 + 2^4 + 1 words."""
    x, rr = i & 0xFF, i >> ROW_BITS
    return rr * 273 + x + (x >> 4)


def conflict_cycles(addrs):
    extra = 0
    for half in (addrs[:32], addrs[32:]):
        banks = {}
        for a in half:
            banks[a % 32] = banks.get(a % 32, 0) + 1
        extra += max(banks.values()) - 1
    return extra


def layouts(li):
    threads = 1 << (DIGIT + li)
    yield "exchange S=0", lambda t, r: phase_index(0, t, r)
    yield "exchange S=4", lambda t, r: phase_index(4, t, r)
    yield "staged rows", lambda t, r: staged(li, t + threads * r)


def cycles_per_instruction(image, li):
    """Average conflict cycles of a ds_*2_b32 (two dwords per lane) per layout."""
    threads = 1 << (DIGIT + li)
    out = {}
    for name, index in layouts(li):
        total = 0
        for r in range(16):
            for w in range(threads // 64):
                total += conflict_cycles([image(index(64 * w + l, r)) for l in range(64)])
        out[name] = 2 * total / (16 * (threads // 64))
    return out


@pytest.mark.parametrize("li", [4, 5])
def test_banked_image_is_injective_and_sized(li):
    addrs = [banked(i) for i in range(1 << (ROW_BITS + li))]
    assert len(set(addrs)) == len(addrs)
    # Lds::kWords: the last row's offset plus one row's span.
    assert max(addrs) + 1 == 272 + 545 * ((1 << (li - 1)) - 1) + 256 + 16 - 1


@pytest.mark.parametrize("li", [4, 5])
def test_banked_image_is_conflict_free(li):
    assert set(cycles_per_instruction(banked, li).values()) == {0.0}


def test_model_reproduces_the_measured_conflicts_of_the_pitched_image():
    # rocprofv3 read SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS = 4.00 for both row
    # passes of the 2^16-point u32 NTT (16-row tiles) with the pitched image.
    assert cycles_per_instruction(pitched, 4) == {"exchange S=0": 4.0, "exchange S=4": 4.0, "staged rows": 4.0}


def test_additive_split_holds():
    # addr(a | b) = addr(a) + addr(b) for disjoint a, b: the kernels add a
    # per-thread base and a compile-time per-register offset.
    for a in range(0, 1 << 13, 37):
        for b in (1, 2, 16, 255, 256, 512, 768, 1024, 4096):
            if a & b == 0:
                assert banked(a | b) == banked(a) + banked(b)
