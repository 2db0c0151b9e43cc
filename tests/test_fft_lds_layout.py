"""The one-row FFT tiles' LDS image (csrc/fft.hip, FftLds with kXor): the
address map is a bijection on the tile, and every access pattern of these
tiles (each digit phase's exchange, the paired final store's bit-reversed
reads of outputs 2j and 2j + 1) gives each 16-lane group of a 64-bit LDS
access 16 distinct low word bits, i.e. all 32 banks. The paired reads of a
bit-reversed output order (outputs 2j, 2j + 1 read as they are, j varying in
its low four bits) leave at most two lanes of a group on one bank pair. The
map and the patterns restate the kernel's (phase_index, store_pairs); a
layout change there must change them here."""
import pytest


def brev(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def addr(i, lt, db):
    return i ^ (((i >> db) ^ (i >> (lt - 5))) & 15)


def patterns(lt, db):
    """(name, registers, tile index of (thread, register)) per LDS access."""
    threads = 1 << (lt - db)
    phases = (lt + db - 1) // db
    out = []
    for p in range(phases):
        s = max(lt - db * (p + 1), 0)
        out.append((f"phase {p}", 1 << db, lambda t, r, s=s: (t & ((1 << s) - 1)) | (r << s) | ((t >> s) << (s + db))))
    for b in (0, 1):  # pair j = t + T r, r < 2^db / 2
        out.append((f"paired read {b}", 1 << (db - 1), lambda t, r, b=b: brev(2 * (t + threads * r) + b, lt)))
        out.append((f"paired read {b}, bit-reversed order", 1 << (db - 1),
                    lambda t, r, b=b: 2 * (t + threads * r) + b))
    return threads, out


@pytest.mark.parametrize("lt,db", [(12, 4), (13, 5), (14, 5)])
def test_bijective_and_conflict_free(lt, db):
    assert sorted(addr(i, lt, db) for i in range(1 << lt)) == list(range(1 << lt))
    threads, pats = patterns(lt, db)
    for name, regs, f in pats:
        for r in range(regs):
            for g in range(0, threads, 16):
                low = {addr(f(t, r), lt, db) & 15 for t in range(g, g + 16)}
                assert len(low) >= (8 if "bit-reversed order" in name else 16), (name, r, g)


def test_padded_layout_conflicted_the_unpaired_final_read():
    # The former 1-in-16 padded image: every lane of a group on one bank pair
    # for the unpaired bit-reversed read.
    lt, threads = 14, 512
    low = {((i := brev(t, lt)) + (i >> 4)) & 15 for t in range(16)}
    assert len(low) == 1


def test_top_four_bit_key_conflicted_the_paired_read():
    # Keyed on the top four index bits, the paired reads of 2^14-point tiles
    # (varying bits 9-12) shared bank pairs.
    lt, db, threads = 14, 5, 512
    old = lambda i: i ^ (((i >> db) ^ (i >> (lt - 4))) & 15)
    low = {old(brev(2 * t, lt)) & 15 for t in range(16)}
    assert len(low) < 16


def column_addr(i, li, paired):
    """FftLds for column tiles: rows padded by one word, the column index
    XOR-swizzled by the row's bits from 3 up, and for paired-column tiles
    first rotated (bit 0 to the top)."""
    cc, x = i & ((1 << li) - 1), i >> li
    if paired:
        cc = (cc >> 1) | ((cc & 1) << (li - 1))
    return x * ((1 << li) + 1) + (cc ^ ((x >> 3) & ((1 << li) - 1)))


def test_paired_column_tiles_are_conflict_free():
    # 64-column tiles of 2^8 rows (C3a's column passes), 1024 threads whose
    # lane l holds logical column 2 (l mod 32) + l / 32 (FftPass::
    # logical_thread); the two digit layouts. The rotation keeps every 16-lane
    # group on 16 distinct bank pairs, where the unrotated image put it on 8.
    lt, li, db, threads = 8, 6, 4, 1024
    logical = lambda tid: (tid & ~63) | (2 * (tid & 31)) | ((tid >> 5) & 1)
    phase = lambda s, t, r: (t & ((1 << s) - 1)) | (r << s) | ((t >> s) << (s + db))
    words = 1 << (lt + li)
    assert sorted(column_addr(i, li, True) for i in range(words)) == sorted(column_addr(i, li, False) for i in range(words))
    for paired, distinct in [(True, 16), (False, 8)]:
        worst = 16
        for s in (li + 4, li):
            for r in range(1 << db):
                for g in range(0, threads, 16):
                    low = {column_addr(phase(s, logical(t), r), li, paired) % 16 for t in range(g, g + 16)}
                    worst = min(worst, len(low))
        assert worst == distinct


def last_thread_index(t, lt):
    """FftPass::last_thread_index: the relabelled last phase of one-row 5-bit
    tiles (direct stores)."""
    l, w = t & 63, t >> 6
    return (((l & 1) << (lt - 2)) | (((l >> 1) & 1) << (lt - 3)) | (((l >> 2) & 1) << (lt - 4)) |
            (((l >> 3) & 1) << (lt - 5)) | (((l >> 4) & 1) << (lt - 1)) | (((l >> 5) & 1) << (lt - 6)) | (w << 5))


@pytest.mark.parametrize("lt", [13, 14])
def test_direct_store_relabelling(lt):
    # One-row tiles of 2^13 / 2^14 points store their results from registers:
    # thread t, register r holds tile position last_thread_index(t) | r, whose
    # output index is its bit reversal. The relabelling is a bijection, every
    # register of a wave stores 64 consecutive outputs (512 contiguous bytes),
    # and its LDS reads keep each 16-lane group on 16 distinct bank pairs.
    db, threads = 5, 1 << (lt - 5)
    assert sorted(last_thread_index(t, lt) | r for t in range(threads) for r in range(32)) == list(range(1 << lt))
    for r in range(32):
        for w in range(threads // 64):
            ks = sorted(brev(last_thread_index(64 * w + l, lt) | r, lt) for l in range(64))
            assert ks == list(range(ks[0], ks[0] + 64)) and ks[0] % 64 == 0
        for g in range(0, threads, 16):
            low = {addr(last_thread_index(t, lt) | r, lt, db) & 15 for t in range(g, g + 16)}
            assert len(low) == 16, (r, g)
    # A relabelling with lanes on position bits LT-4..LT-1 (the plain reversal
    # of output bits 0-3) would leave two lanes per bank pair.
    plain = lambda t: ((int(format(t & 15, "04b")[::-1], 2)) << (lt - 4)) | ((t >> 4) << 5)
    assert min(len({addr(plain(t) | 0, lt, db) & 15 for t in range(g, g + 16)}) for g in range(0, threads, 16)) < 16
