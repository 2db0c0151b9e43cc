"""The persistent walk of the one-row FFT tiles (csrc/fft.hip, FftPass::run /
step / process / exchange), modelled on the CPU: the LDS protocol across
consecutive tiles has no hazard between waves, whatever order the final
store reads its staged results in.

Each tile runs, per wave: digit 0 in registers; for every later digit an
exchange (barrier, LDS writes in the previous digit's layout, barrier, LDS
reads in the next one's) and the digit; then the final store (barrier, LDS
writes in the last digit's layout, barrier, LDS reads in store order, global
stores); then the next tile, whose first LDS access follows its first
exchange's barrier. Every barrier is `s_waitcnt lgkmcnt(0); s_barrier`, so a
wave's LDS accesses are complete before it arrives. The model replays that
sequence for every wave of two consecutive tiles with the kernel's index maps
(phase_index, the XOR-swizzled image, the staged store enumeration) and
checks, per interval between barriers:
* no interval holds both LDS writes and LDS reads;
* the writes of an interval hit each word once;
* every read hits a word written in the latest write interval of the same
  tile (no stale word from the previous tile or an earlier phase).

The natural-order 2^13 / 2^14-point tiles store straight from registers
instead (FftPass::kDirectStore): their last exchange reads with relabelled
threads and no final store exchange follows; the model covers that walk too.

The same holds for an enumeration in which each lane stores two neighbouring
outputs (the removed "paired final stores" variant's read pattern): its
reads still sit in the one read interval that the next tile's first barrier
closes. So the LDS protocol of the walk that C3b runs is not where that
variant's wrong results on later tiles came from; they belonged to the
variant's own code, which was removed (its exact source is not kept).
"""
import pytest


def brev(x, bits):
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


def swizzled(i, lt, db):
    """FftLds<...>::split for one-row tiles: the unpadded XOR-swizzled image."""
    return i ^ (((i >> db) ^ (i >> (lt - 5))) & 15)


def phase_index(s, db, t, r):
    return (t & ((1 << s) - 1)) | (r << s) | ((t >> s) << (s + db))


def window(lt, db, p):
    return max(lt - db * (p + 1), 0)


def last_thread_index(t, lt):
    """FftPass::last_thread_index (one-row 5-bit tiles with direct stores)."""
    l, w = t & 63, t >> 6
    return (((l & 1) << (lt - 2)) | (((l >> 1) & 1) << (lt - 3)) | (((l >> 2) & 1) << (lt - 4)) |
            (((l >> 3) & 1) << (lt - 5)) | (((l >> 4) & 1) << (lt - 1)) | (((l >> 5) & 1) << (lt - 6)) | (w << 5))


def walk(lt, db, tiles, store_order, direct=False):
    """Per-interval LDS events of `tiles` consecutive tiles: a list of
    intervals, each a list of (tile, kind, wave, word, tag) with kind 'w' or
    'r' and tag naming the layout step a read must see. direct: the last
    phase's reads take the relabelled threads and the results leave from
    registers (no final store exchange)."""
    threads = 1 << (lt - db)
    regs = 1 << db
    phases = (lt + db - 1) // db
    intervals = []
    for tile in range(tiles):
        for p in range(phases):
            last = p == phases - 1
            if last and direct:
                break
            # barrier, writes of digit p's layout, barrier, reads
            writes, reads = [], []
            s_from = window(lt, db, p)
            for t in range(threads):
                for r in range(regs):
                    writes.append((tile, "w", t // 64, swizzled(phase_index(s_from, db, t, r), lt, db), p))
            if not last:
                s_to = window(lt, db, p + 1)
                for t in range(threads):
                    for r in range(regs):
                        i = (last_thread_index(t, lt) | r) if direct and p + 1 == phases - 1 else \
                            phase_index(s_to, db, t, r)
                        reads.append((tile, "r", t // 64, swizzled(i, lt, db), p))
            else:
                for t, words in store_order(threads, regs):
                    for i in words:
                        reads.append((tile, "r", t // 64, swizzled(i, lt, db), p))
            intervals.append(writes)
            intervals.append(reads)
    return intervals


def natural_store(lt):
    """staged(): element g = t + T r of the tile, bit-reversed position."""
    def order(threads, regs):
        for t in range(threads):
            yield t, [brev((t + threads * r) & ((1 << lt) - 1), lt) for r in range(regs)]
    return order


def paired_store(lt):
    """Two neighbouring natural-order outputs per lane and store."""
    def order(threads, regs):
        for t in range(threads):
            words = []
            for r in range(regs // 2):
                j = t + threads * r
                words += [brev(2 * j, lt), brev(2 * j + 1, lt)]
            yield t, words
    return order


def check(intervals):
    latest = {}  # word -> (tile, tag) of its latest write
    for events in intervals:
        kinds = {e[1] for e in events}
        assert len(kinds) <= 1, "an interval mixes LDS reads and writes"
        if kinds == {"w"}:
            words = [e[3] for e in events]
            assert len(words) == len(set(words)), "two writes of one word in an interval"
            for tile, _, _, word, tag in events:
                latest[word] = (tile, tag)
        elif kinds == {"r"}:
            for tile, _, _, word, tag in events:
                assert latest.get(word) == (tile, tag), f"stale read of word {word} (tile {tile}, step {tag})"


@pytest.mark.parametrize("lt,db", [(14, 5), (12, 4)])
@pytest.mark.parametrize("order", ["natural", "paired"])
def test_walk_lds_protocol_has_no_hazard(lt, db, order):
    store = natural_store(lt) if order == "natural" else paired_store(lt)
    check(walk(lt, db, 2, store))


@pytest.mark.parametrize("lt", [14, 13])
def test_walk_with_direct_stores_has_no_hazard(lt):
    # The one-row 5-bit tiles' default (natural order): the relabelled last
    # exchange, then stores from registers; the next tile's first exchange
    # barrier closes the last read interval.
    check(walk(lt, 5, 3, None, direct=True))


def test_model_catches_a_missing_barrier():
    # Planted on the CPU: merge the final store's reads with the next tile's
    # first exchange writes (no barrier between them); the check must fail.
    lt, db = 12, 4
    intervals = walk(lt, db, 2, natural_store(lt))
    phases = (lt + db - 1) // db
    first_tile_last_reads = 2 * phases - 1
    merged = intervals[:first_tile_last_reads] + [intervals[first_tile_last_reads] + intervals[first_tile_last_reads + 1]] \
        + intervals[first_tile_last_reads + 2:]
    with pytest.raises(AssertionError):
        check(merged)


@pytest.mark.parametrize("lt,db", [(14, 5), (13, 5), (12, 4)])
@pytest.mark.parametrize("bitrev_out", [False, True])
def test_paired_store_addresses(lt, db, bitrev_out):
    # FftPass::store_pairs: pair j = t + T r holds outputs 2j, 2j + 1; their
    # LDS words come from a thread part (index of 2t) and a register part
    # (index of 2 T r), XOR-combined, the second output's by one more bit.
    # That must equal the swizzled word of each output's own tile index, and
    # the pairs must cover every output once.
    threads = 1 << (lt - db)
    regs = 1 << db

    def index(g):
        return g if bitrev_out else brev(g, lt)

    second = 1 if bitrev_out else 1 << (lt - 1)
    seen = set()
    for t in range(threads):
        it = index(2 * t)
        for r in range(regs // 2):
            ir = index(2 * threads * r)
            assert it & ir == 0 and (it | ir) & second == 0
            j = t + threads * r
            assert swizzled(it, lt, db) ^ swizzled(ir, lt, db) == swizzled(index(2 * j), lt, db)
            assert swizzled(it, lt, db) ^ swizzled(ir | second, lt, db) == swizzled(index(2 * j + 1), lt, db)
            seen.update((2 * j, 2 * j + 1))
    assert seen == set(range(1 << lt))
