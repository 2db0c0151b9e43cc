"""The one-row FFT tiles' LDS image (csrc/fft.hip, FftLds with kXor): the
address map is a bijection on the tile, and every access pattern of these
tiles (each digit phase's exchange, the bit-reversed final read) gives each
16-lane group of a 64-bit LDS access 16 distinct low word bits, i.e. all 32
banks. The map and the patterns restate the kernel's (phase_index, staged);
a layout change there must change them here."""
import pytest


def brev(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def addr(i, lt, db):
    return i ^ (((i >> db) ^ (i >> (lt - 4))) & 15)


def patterns(lt, db):
    threads = 1 << (lt - db)
    phases = (lt + db - 1) // db
    out = []
    for p in range(phases):
        s = max(lt - db * (p + 1), 0)
        out.append(lambda t, r, s=s: (t & ((1 << s) - 1)) | (r << s) | ((t >> s) << (s + db)))
    out.append(lambda t, r: brev((t + threads * r) & ((1 << lt) - 1), lt))
    return threads, out


@pytest.mark.parametrize("lt,db", [(12, 4), (13, 5), (14, 5)])
def test_bijective_and_conflict_free(lt, db):
    assert sorted(addr(i, lt, db) for i in range(1 << lt)) == list(range(1 << lt))
    threads, pats = patterns(lt, db)
    for f in pats:
        for r in range(1 << db):
            for g in range(0, threads, 16):
                low = {addr(f(t, r), lt, db) & 15 for t in range(g, g + 16)}
                assert len(low) == 16


def test_padded_layout_conflicted_the_final_read():
    # The former 1-in-16 padded image: every lane of a group on one bank pair.
    lt, db = 14, 5
    threads, pats = patterns(lt, db)
    final = pats[-1]
    low = {((i := final(t, 0)) + (i >> 4)) & 15 for t in range(16)}
    assert len(low) == 1
