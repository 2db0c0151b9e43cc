// Device code of the NTT engine: the templated pass kernel, Shoup arithmetic,
// the twiddle-chunk geometry shared with the host table builder, and the
// registry of instantiated pass shapes. Included by ntt.hip (host side) and by
// the ntt_u{32,64}_{lazy,strict}.hip translation units, which instantiate the
// kernels in parallel builds.
//
// Memory access: every tile addresses one polynomial (or, for one-pass tiles,
// one run of dense polynomials) through a buffer resource whose base and
// range are that span, so each load and store is a 32-bit lane offset from a
// uniform base (no 64-bit address arithmetic), and an access outside the span
// reads 0 / is dropped by the hardware range check instead of touching other
// memory.
//
// Twiddles: a radix-16 phase of the merged-twist transform needs, per thread,
// the 15 (or fewer) table entries of one block of the stage tree (its
// "chunk", in stage execution order, padded to whole 16-byte pieces). A
// phase's chunks are stored piece-major: piece e of every chunk of the phase,
// in chunk order, then piece e + 1. Threads that hold consecutive chunks
// (the lanes of a row pass, where every lane has its own block) then read
// piece e as one contiguous run per load instruction -- 1 KiB over 8 cache
// lines for a wave -- instead of 64 pieces one chunk apart (64 or more lines
// per instruction, which filled the address unit's queue).
#pragma once

#include <hip/hip_runtime.h>

#include "buffer.hpp"
#include "ntt_engine.hpp"

#include <cstddef>
#include <map>
#include <tuple>
#include <type_traits>
#include <vector>

namespace cbw {
namespace ntt_detail {

constexpr int kLE = 4;
constexpr int kE = 1 << kLE;

// A twiddle and its Shoup factor floor(w 2^k / q). Tables of lazy
// Cooley-Tukey passes hold -w mod 2^k in place of w (see ct_butterfly).
template <class W>
struct alignas(2 * sizeof(W)) TwPair {
    W w, wp;
};

// Arithmetic of a pass: Shoup products on fully reduced values ([0, 2q)
// between stages), Shoup products on lazy ranges, or Barrett products on
// canonical values with one constant per domain instead of a Shoup factor per
// twiddle (tables of single words).
constexpr int kStrict = 0, kLazy = 1, kBarrett = 2;

// A twiddle table entry: a Shoup pair, or the bare twiddle for Barrett.
template <class W, int AR>
using Entry = std::conditional_t<AR == kBarrett, W, TwPair<W>>;

template <class W>
struct DeviceDomain {
    W q, q2, nq, rwp;     // modulus, 2q, -q mod 2^k, floor(2^k / q) (Shoup factor of 1)
    TwPair<W> ninv;       // n^-1 with its Shoup factor
    TwPair<W> last;       // Tinv[1] * n^-1 (final inverse stage)
    W mu;                 // Barrett: floor(2^(2b+1) / q), b = qbits
    std::uint32_t qbits;  // Barrett: bit length of q
    std::uint64_t tw;     // offset of this domain's chunk tables in PassArgs::tw (entries)
};

template <class W>
struct PassArgs {
    const W* in;
    W* out;
    const DeviceDomain<W>* domains;
    const void* tw;                    // all domains' chunk tables (Entry), concatenated
    const std::uint32_t* poly_domain;  // per polynomial (null: domain 0)
    const std::uint64_t* in_off;       // per polynomial word offset (null: p << log n)
    const std::uint64_t* out_off;
    std::uint32_t polys, tiles;
    std::uint32_t reduce_input;
    std::uint32_t phase_off[3];  // chunk array of each phase, entries from the domain's table start
    std::uint32_t tw_bytes;      // bytes of one domain's chunk tables (buffer range of the twiddle reads)
};

// ---- phase geometry (host and device) ---------------------------------------
//
// A pass butterflies LT transform bits in phases of a 4-bit register window.
// Cooley-Tukey (CT) walks the bits high -> low, windows [LT-4(P+1), LT-4P)
// clamped at 0; Gentleman-Sande (GS) walks low -> high, windows [4P, 4P+4)
// clamped at LT-4. A clamped window re-covers bits of its neighbour; only the
// bits not yet done ("active" stages) are butterflied there.

constexpr int num_phases(int lt) { return (lt + kLE - 1) / kLE; }
constexpr int imin(int a, int b) { return a < b ? a : b; }
constexpr int imax(int a, int b) { return a > b ? a : b; }

constexpr int window_start(int lt, bool ct, int p) {
    return ct ? imax(lt - kLE * (p + 1), 0) : (kLE * p < lt - kLE ? kLE * p : imax(lt - kLE, 0));
}
constexpr int stage_hi(int lt, bool ct, int p) {
    const int ws = window_start(lt, ct, p);
    return ct ? imin(imin(ws + 3, lt - 1), lt - kLE * p - 1) : imin(ws + 3, lt - 1);
}
constexpr int stage_lo(int lt, bool ct, int p) {
    const int ws = window_start(lt, ct, p);
    return ct ? ws : imax(ws, kLE * p);
}
// Stage k of the phase at window ws: its twiddle for register group g is
// table[(head >> (k+1)) + (g & gmask)], head = (prefix << lt) | (window bits
// clear). Distinct entries per thread: 2^min(ws+3-k, lt-1-k). All of a
// phase's entries hang off the block index head >> chunk_shift.
constexpr int stage_count(int lt, int ws, int k) { return 1 << imin(ws + 3 - k, lt - 1 - k); }
constexpr int chunk_shift(int lt, bool ct, int p) { return imin(window_start(lt, ct, p) + kLE, lt); }
// The final GS stage of a transform multiplies by n^-1 (no table entries).
constexpr bool scale_stage(int lt, bool ct, bool last, int k) { return !ct && last && k == lt - 1; }
// k of the s-th executed stage of a phase.
constexpr int exec_stage(int lt, bool ct, int p, int s) { return ct ? stage_hi(lt, ct, p) - s : stage_lo(lt, ct, p) + s; }
constexpr int active_stages(int lt, bool ct, int p) { return stage_hi(lt, ct, p) - stage_lo(lt, ct, p) + 1; }
// Entry offset of the s-th executed stage within the chunk, and the chunk size.
constexpr int chunk_offset(int lt, bool ct, bool last, int p, int s) {
    int off = 0;
    for (int e = 0; e < s; ++e) {
        const int k = exec_stage(lt, ct, p, e);
        if (!scale_stage(lt, ct, last, k)) off += stage_count(lt, window_start(lt, ct, p), k);
    }
    return off;
}
constexpr int chunk_entries(int lt, bool ct, bool last, int p) {
    return chunk_offset(lt, ct, last, p, active_stages(lt, ct, p));
}
// Chunk stride in entries: a multiple of 16 bytes.
constexpr int chunk_stride(int lt, bool ct, bool last, int p, int entry_bytes) {
    const int per16 = 16 / entry_bytes > 0 ? 16 / entry_bytes : 1;
    const int e = chunk_entries(lt, ct, last, p);
    return (e + per16 - 1) / per16 * per16;
}
// Chunks of one phase: one per block of the stage tree at chunk_shift,
// over the 2^(prefix_bits + lt) entries the pass covers.
constexpr std::uint64_t chunk_count(int lt, int prefix_bits, bool ct, int p) {
    return (std::uint64_t{1} << (prefix_bits + lt)) >> chunk_shift(lt, ct, p);
}

// Appends one pass's twiddle chunks (piece-major, layout above) to `out` and
// records each phase's offset from `base`. prefix_bits: 0 for column and
// one-pass tiles, l1 for row tiles (their block index carries 2^l1 + row).
template <class E>
void append_pass_chunks(std::vector<E>& out, std::size_t base, const std::vector<E>& table, int lt,
                        int prefix_bits, bool ct, bool last, std::uint32_t (&phase_off)[3]) {
    constexpr std::size_t per16 = 16 / sizeof(E) > 0 ? 16 / sizeof(E) : 1;
    for (int p = 0; p < num_phases(lt); ++p) {
        phase_off[p] = static_cast<std::uint32_t>(out.size() - base);
        const int entries = chunk_entries(lt, ct, last, p);
        if (entries == 0) continue;
        const int shift = chunk_shift(lt, ct, p);
        const int stride = chunk_stride(lt, ct, last, p, int(sizeof(E)));
        const int ws = window_start(lt, ct, p);
        const std::uint64_t count = chunk_count(lt, prefix_bits, ct, p);
        const std::size_t start = out.size();
        out.resize(start + std::size_t(count) * std::size_t(stride), E{});
        for (std::uint64_t c = 0; c < count; ++c) {
            const std::uint64_t idx = count + c;  // block index in the stage tree
            std::size_t e = 0;
            for (int s = 0; s < active_stages(lt, ct, p); ++s) {
                const int k = exec_stage(lt, ct, p, s);
                if (scale_stage(lt, ct, last, k)) continue;
                for (int j = 0; j < stage_count(lt, ws, k); ++j, ++e) {
                    const std::size_t piece = e / per16, slot = e % per16;
                    out[start + (piece * std::size_t(count) + std::size_t(c)) * per16 + slot] =
                        table.at((idx << (shift - k - 1)) + std::uint64_t(j));
                }
            }
        }
    }
}

// ---- arithmetic -------------------------------------------------------------

__device__ __forceinline__ std::uint32_t mulhi(std::uint32_t a, std::uint32_t b) { return __umulhi(a, b); }
__device__ __forceinline__ std::uint64_t mulhi(std::uint64_t a, std::uint64_t b) { return __umul64hi(a, b); }

// x - m if x >= m else x (x < 2m).
__device__ __forceinline__ std::uint32_t csub(std::uint32_t x, std::uint32_t m) { return min(x, x - m); }
// 64-bit: add the wave-uniform -m (formed once in scalar registers) rather
// than subtract m, so the result is one 64-bit add (v_lshl_add_u64) with no
// carry chain through VCC.
__device__ __forceinline__ std::uint64_t csub(std::uint64_t x, std::uint64_t m) {
    std::uint64_t nm = std::uint64_t(0) - m;
    asm("" : "+s"(nm));  // keeps the optimiser from folding the add back into a subtract
    return x + (x >= m ? nm : std::uint64_t(0));
}

// (a b + c) mod 2^k as one multiply-add (v_mad_u64_u32 for 32-bit words,
// where a 32-bit multiply and a separate add would take two instructions).
__device__ __forceinline__ std::uint32_t mul_add(std::uint32_t a, std::uint32_t b, std::uint32_t c) {
    return static_cast<std::uint32_t>(std::uint64_t(a) * b + c);
}
__device__ __forceinline__ std::uint64_t mul_add(std::uint64_t a, std::uint64_t b, std::uint64_t c) {
    return a * b + c;
}

// Shoup: a w - floor(a wp / 2^k) q, in [0, 2q) for any word a; written with
// nq = -q so the subtraction folds into the multiply-add.
template <class W>
__device__ __forceinline__ W shoup(W a, W w, W wp, W nq) {
    return mul_add(mulhi(a, wp), nq, a * w);
}
// -shoup(a, w, ...) modulo the word, from nw = -w: the lazy butterfly then
// folds the sign into its subtraction and three-input add.
template <class W>
__device__ __forceinline__ W neg_shoup(W a, W nw, W wp, W q) {
    return mul_add(mulhi(a, wp), q, a * nw);
}

// Lazy: x, y in [0, 4q) -> [0, 4q), table entries hold -w. Strict: [0, 2q)
// -> [0, 2q), entries hold w.
template <class W, bool LAZY>
__device__ __forceinline__ void ct_butterfly(W& x, W& y, TwPair<W> t, const DeviceDomain<W>& d) {
    if constexpr (LAZY) {
        const W u = csub(x, d.q2);
        const W nv = neg_shoup(y, t.w, t.wp, d.q);  // -v, v in [0, 2q)
        x = u - nv;
        y = u + d.q2 + nv;
    } else {
        const W u = csub(x, d.q);
        const W v = csub(shoup(y, t.w, t.wp, d.nq), d.q);
        x = u + v;
        y = u - v + d.q;
    }
}

template <class W, bool LAZY>
__device__ __forceinline__ void gs_butterfly(W& x, W& y, TwPair<W> t, const DeviceDomain<W>& d) {
    if constexpr (LAZY) {  // x, y in [0, 2q)
        const W u = x, v = y;
        x = csub(u + v, d.q2);
        y = shoup(u - v + d.q2, t.w, t.wp, d.nq);
    } else {
        const W u = csub(x, d.q), v = csub(y, d.q);
        x = u + v;
        y = shoup(u - v + d.q, t.w, t.wp, d.nq);
    }
}

// Final inverse stage: both outputs also multiplied by n^-1.
template <class W, bool LAZY>
__device__ __forceinline__ void gs_scale_butterfly(W& x, W& y, const DeviceDomain<W>& d) {
    W u = x, v = y;
    if constexpr (!LAZY) {
        u = csub(u, d.q);
        v = csub(v, d.q);
    }
    const W span = LAZY ? d.q2 : d.q;
    x = shoup(u + v, d.ninv.w, d.ninv.wp, d.nq);
    y = shoup(u - v + span, d.last.w, d.last.wp, d.nq);
}

// Barrett (the constants of the reference's GPU-NTT-compatible provider,
// src/ntt_hybrid2d.cuh:53-71, mu = floor(2^(2b+1) / q) for the bit length b
// of q, q < 2^(k-2)): for canonical a, w < q, P = a w < 2^(2b),
// t = floor(P / 2^(b-2)) < 2^(b+2) and Q = floor(t mu / 2^(b+3)) satisfy
// floor(P / q) - 1 <= Q <= floor(P / q), so P - Q q (formed modulo the word)
// lies in [0, 2q) and one conditional subtraction makes it canonical.
__device__ __forceinline__ std::uint32_t barrett(std::uint32_t a, std::uint32_t w, const DeviceDomain<std::uint32_t>& d) {
    const std::uint64_t p = std::uint64_t(a) * w;
    const std::uint32_t t = std::uint32_t(p >> (d.qbits - 2u));
    const std::uint32_t quo = std::uint32_t((std::uint64_t(t) * d.mu) >> (d.qbits + 3u));
    return min(std::uint32_t(p) - quo * d.q, std::uint32_t(p) - quo * d.q - d.q);
}
__device__ __forceinline__ std::uint64_t barrett(std::uint64_t a, std::uint64_t w, const DeviceDomain<std::uint64_t>& d) {
    const std::uint64_t lo = a * w, hi = __umul64hi(a, w);
    const std::uint32_t s = d.qbits - 2u;  // 0 .. 60; (hi << 1) << (63 - s) is hi << (64 - s), 0 at s = 0
    const std::uint64_t t = (lo >> s) | ((hi << 1) << (63u - s));
    const std::uint64_t plo = t * d.mu, phi = __umul64hi(t, d.mu);
    const std::uint32_t s2 = d.qbits + 3u;  // 5 .. 65 (wave-uniform)
    const std::uint64_t quo = s2 >= 64u ? phi >> (s2 - 64u) : (plo >> s2) | ((phi << 1) << (63u - s2));
    const std::uint64_t r = lo - quo * d.q;
    return r >= d.q ? r - d.q : r;
}

// x - m if x >= m else x (x < 2m), with no register-class constraint on m
// (the u64 csub pins -m to scalar registers, which some kernels of this
// arithmetic cannot satisfy).
__device__ __forceinline__ std::uint32_t reduce_once(std::uint32_t x, std::uint32_t m) { return min(x, x - m); }
__device__ __forceinline__ std::uint64_t reduce_once(std::uint64_t x, std::uint64_t m) { return x >= m ? x - m : x; }

// Barrett butterflies keep every value canonical (inputs and outputs in [0, q)).
template <class W>
__device__ __forceinline__ void ct_barrett(W& x, W& y, W w, const DeviceDomain<W>& d) {
    const W u = x, v = barrett(y, w, d);
    x = reduce_once(u + v, d.q);
    y = reduce_once(u - v + d.q, d.q);
}
template <class W>
__device__ __forceinline__ void gs_barrett(W& x, W& y, W w, const DeviceDomain<W>& d) {
    const W u = x, v = y;
    x = reduce_once(u + v, d.q);
    y = barrett(reduce_once(u - v + d.q, d.q), w, d);
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Orders one wave's LDS accesses around an exchange that stays inside the
// wave: a wave's LDS instructions execute in issue order, so only the
// compiler has to be kept from moving reads above writes (no code).
__device__ __forceinline__ void wave_lds_fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ std::uint32_t brev(std::uint32_t x, std::uint32_t bits) {
    return bits ? __brev(x) >> (32 - bits) : 0u;
}

// Tile index of (thread t, register r) when registers span tile bits [S, S+4).
template <int S>
__device__ __forceinline__ std::uint32_t phase_index(std::uint32_t t, std::uint32_t r) {
    const std::uint32_t lo = t & ((1u << S) - 1u);
    return lo | (r << S) | ((t >> S) << (S + kLE));
}

// Padded LDS image of a tile. Column tiles that stage a bit-reversed boundary
// also swizzle the column by the top transform bits (lanes then walk rows in
// bit-reversed order, which a plain stride maps onto few banks).
//
// Row tiles of 2^8-point rows in 4-byte words (BANKED) give each row bit its
// own offset instead of one row pitch: 272, 545, 1090, 2180, 4360 words,
// which are 16, 1, 2, 4, 8 modulo the 32 four-byte banks, at least 272 words
// apart (a row spans 271). A 32-lane half of every access these tiles make
// then covers 32 distinct banks: the exchanges' phase layouts (lanes over
// index bits 4-8, or 0-3 and 8) and the staged boundary permutation (lanes
// over the row bits and index bit 7), where the single pitch of 273 words
// (17 modulo 32) put two lanes on each bank (4 conflict cycles per ds_*2_b32
// instruction, measured, and reproduced by enumerating the accesses).
template <bool COL, bool SWZ, int LT, int LI, bool BANKED = false>
struct Lds {
    static_assert(!BANKED || (!COL && LT == 8 && LI <= 5), "banked row offsets cover 2^8-point rows, up to 32");
    // Row bit j > 0 contributes 545 * 2^(j - 1): the bits above bit 0 are
    // one multiple of 545.
    static __host__ __device__ constexpr std::uint32_t row_offset(std::uint32_t rr) {
        return 272u * (rr & 1u) + 545u * (rr >> 1);
    }
    // Without the swizzle, addr() is a sum of terms over disjoint index bit
    // fields, so addr(a | b) = addr(a) + addr(b) for disjoint a, b.
    static constexpr bool kLinear = !(COL && SWZ);
    static constexpr std::uint32_t kWords =
        COL      ? (1u << LT) * ((1u << LI) + 1u)
        : BANKED ? row_offset((1u << LI) - 1u) + (1u << LT) + (1u << LT >> 4) - 1u
                 : (1u << LI) * ((1u << LT) + (1u << LT >> 4) + 1u);
    static __device__ __forceinline__ std::uint32_t addr(std::uint32_t i) {
        if constexpr (COL) {
            const std::uint32_t cc = i & ((1u << LI) - 1u), x = i >> LI;
            if constexpr (SWZ) {
                constexpr int top = LT > LI ? LT - LI : 0;
                return x * ((1u << LI) + 1u) + (cc ^ ((x >> top) & ((1u << LI) - 1u)));
            } else {
                return x * ((1u << LI) + 1u) + cc;
            }
        } else if constexpr (BANKED) {
            const std::uint32_t x = i & ((1u << LT) - 1u), rr = i >> LT;
            return row_offset(rr) + x + (x >> 4);
        } else {
            const std::uint32_t x = i & ((1u << LT) - 1u), rr = i >> LT;
            return rr * ((1u << LT) + (1u << LT >> 4) + 1u) + x + (x >> 4);
        }
    }
    // Address of element phase_index<S>(t, r): a per-thread base plus a
    // compile-time offset per register where the layout is linear.
    template <int S>
    static __device__ __forceinline__ std::uint32_t at(std::uint32_t t, int r) {
        if constexpr (kLinear) return addr(phase_index<S>(t, 0)) + addr(phase_index<S>(0, std::uint32_t(r)));
        else return addr(phase_index<S>(t, std::uint32_t(r)));
    }
};

// ---- the pass ---------------------------------------------------------------
//
// A workgroup owns a tile of 2^(LT+LI) words = 2^LT transform points x 2^LI
// lines, 16 words per thread. COL tiles hold 2^LI adjacent columns (stride
// 2^L2) of the high L1 bits; ROW tiles hold 2^LI rows of the low L2 bits; one
// -pass (SINGLE) tiles hold 2^LI whole polynomials (L1 = 0, L2 = LT).
template <class W, int AR, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE, int L1, int L2>
struct Pass {
    static constexpr bool LAZY = AR == kLazy;
    static constexpr bool BARRETT = AR == kBarrett;
    using E = Entry<W, AR>;
    static constexpr int LB = LT + LI;
    static constexpr std::uint32_t T = 1u << (LB - kLE);
    static constexpr int kPhases = num_phases(LT);
    static constexpr int kLogN = L1 + L2;
    static constexpr bool kFirst = SINGLE || (COL == CT);
    static constexpr bool kLast = SINGLE || (COL != CT);
    // Rows of a permuted two-pass ROW tile are bitrev(k0 + rr).
    static constexpr bool kPermRows = !COL && !SINGLE && (PIN || POUT);
    static constexpr std::uint32_t kPolyBytes = std::uint32_t(sizeof(W)) << kLogN;
    using L = Lds<COL, COL && (PIN || POUT), LT, LI, !COL && sizeof(W) == 4 && LT == 8 && LI <= 5>;
    // Stores of two-pass inverse (Gentleman-Sande) tiles write through the L2
    // (sc0 sc1), so the end-of-kernel write-back has little left to flush;
    // measured 5-6% faster per C2 / C4 step. Forward passes keep write-back
    // stores: write-through made them slower (partial-line segments that
    // the L2 would otherwise merge).
    // (Nontemporal final stores measured slower for C4, whose bit-reversed
    // output lands in 8-byte segments: 60.6 -> 71-73 us.) Forward column
    // passes whose tiles write whole 128-byte lines per row (u32 32-column,
    // u64 16-column tiles) store the intermediate nontemporally: C4 56.5 ->
    // 54.9 us, C2 unchanged. Forward row passes that stage their stores
    // (natural output through the LDS permutation, or native output through
    // the wave's own rows, kStagedAux) write through as well: C2 38.6 ->
    // 37.3 us, C4 54.2 -> 52.0 us.
    static constexpr int kStoreAux = (!CT && !SINGLE) || (CT && !SINGLE && !COL && POUT) ? 17
                                     : (COL && CT && !SINGLE && (sizeof(W) << LI) >= 128) ? 2
                                                                                          : 0;
    // Row tiles of at most 2^10-point rows: every phase layout keeps a row in
    // 2^(LT-4) <= 64 consecutive threads (phase_index puts the row bits at
    // t >> (LT - 4)), so the register-window exchanges never leave a wave.
    // Their barriers would only hold the workgroup's waves in step; a wave
    // that has its data computes while the others still wait for theirs.
    // The staged boundary permutations (PIN / POUT) mix rows across waves
    // and keep their barriers.
    static constexpr bool kWaveLocal = !COL && LT - kLE <= 6;
    // Forward row tiles whose output stays in the transform's native order
    // end with every thread holding 16 consecutive outputs of one row, so a
    // store instruction would put its 64 lanes 16 words apart (64 cache lines
    // per instruction). A wave's 1024 outputs are one contiguous run, and
    // they go through the wave's own LDS rows instead: each 16-byte store
    // instruction then covers 64 x 16 contiguous bytes.
    static constexpr bool kStagedStore = !COL && CT && kLast && !POUT && kWaveLocal && LT + LI >= 10;
    static constexpr int kStagedAux = SINGLE ? 0 : 17;
    // (The mirror image, the first inverse pass loading its native-order rows
    // as contiguous runs and moving them into the phase-0 layout through the
    // wave's rows, measured no faster: C4 52.7 against 52.0-52.2 us.)
    static constexpr int kPer = 16 / int(sizeof(W));  // words per 16-byte access

    // Staged store run: lane l of wave w moves tile elements g0 + 64 kPer k + e
    // (e < kPer), g0 = 1024 w + kPer l. The thread, lane and register parts
    // lie in disjoint index bits, so the LDS address and the word in the
    // span (row k0 + rr at stride 2^L2 = 2^LT, or the dense one-pass element)
    // split into a thread part plus a compile-time offset, and kPer
    // consecutive words never cross the image's 1-in-16 pad.
    static __device__ __forceinline__ std::uint32_t run_first(std::uint32_t t) {
        return (t >> 6) * 1024u + std::uint32_t(kPer) * (t & 63u);
    }
    static constexpr std::uint32_t run_offset(int k) { return 64u * std::uint32_t(kPer) * std::uint32_t(k); }
    static_assert(SINGLE ? (L1 == 0 && L2 == LT) : (COL ? LT == L1 : LT == L2), "pass bits");
    static_assert(LT >= 1 && LB >= kLE && LB <= 13, "tile shape");

    template <int P>
    static constexpr int tile_window() {
        return (COL ? LI : 0) + window_start(LT, CT, P);
    }

    struct Tile {
        std::uint32_t poly;  // COL / two-pass ROW: the polynomial; SINGLE: the first polynomial
        std::uint32_t c0;    // COL: first column
        std::uint32_t k0;    // ROW: first row (or bit-reversed row index)
        std::uint32_t lines; // SINGLE: polynomials in this tile
    };

    static __device__ __forceinline__ Tile decode(const PassArgs<W>& a, std::uint32_t tile) {
        // A tile is wave-uniform; saying so keeps its fields (and the buffer
        // resources and domain record derived from them) in scalar registers
        // inside the persistent loop.
        tile = uniform(tile);
        Tile tl{};
        if constexpr (COL) {
            constexpr int shift = L2 - LI;
            tl.poly = tile >> shift;
            tl.c0 = (tile & ((1u << shift) - 1u)) << LI;
        } else if constexpr (SINGLE) {
            tl.poly = tile << LI;
            tl.lines = min(1u << LI, a.polys - tl.poly);
        } else {
            constexpr int shift = L1 - LI;
            tl.poly = tile >> shift;
            tl.k0 = (tile & ((1u << shift) - 1u)) << LI;
        }
        return tl;
    }

    // Buffer over the tile's span: its polynomial (two-pass, or one-pass with
    // explicit offsets, where a tile holds one polynomial) or its run of dense
    // polynomials (one-pass).
    static __device__ __forceinline__ __amdgpu_buffer_rsrc_t span(const W* base, const std::uint64_t* off,
                                                                  const Tile& tl) {
        // Offsets are read back into scalar registers (see domain_of).
        if constexpr (SINGLE) {
            if (off) return make_rsrc(base + uniform(off[tl.poly]), kPolyBytes);
            return make_rsrc(base + (std::uint64_t(tl.poly) << kLogN), tl.lines * kPolyBytes);
        } else {
            return make_rsrc(base + (off ? uniform(off[tl.poly]) : std::uint64_t(tl.poly) << kLogN), kPolyBytes);
        }
    }

    // Logical row of line rr in a ROW tile.
    static __device__ __forceinline__ std::uint32_t row_of(const Tile& tl, std::uint32_t rr) {
        if constexpr (SINGLE) return 0;
        else if constexpr (kPermRows) return brev(tl.k0 + rr, L1);
        else return tl.k0 + rr;
    }

    // Word (relative to the span) of tile element i, natural side.
    static __device__ __forceinline__ std::uint32_t natural_word(const Tile& tl, std::uint32_t i) {
        if constexpr (COL) {
            const std::uint32_t cc = i & ((1u << LI) - 1u), x = i >> LI;
            return tl.c0 + cc + (x << L2);
        } else if constexpr (SINGLE) {
            return i;  // rows are consecutive polynomials of 2^LT words
        } else {
            const std::uint32_t x = i & ((1u << LT) - 1u), rr = i >> LT;
            return (row_of(tl, rr) << L2) + x;
        }
    }

    // natural_word of element phase_index<S>(t, r) as a per-thread word plus
    // a per-register word: every natural_word layout is a sum of terms over
    // disjoint index bit fields (row bit reversal included, as k0 is a
    // multiple of 2^LI), and the tile's own origin sits in the thread part.
    template <int S>
    static __device__ __forceinline__ std::uint32_t thread_word(const Tile& tl, std::uint32_t t) {
        return natural_word(tl, phase_index<S>(t, 0));
    }
    template <int S>
    static __device__ __forceinline__ std::uint32_t register_word(int r) {
        return natural_word(Tile{}, phase_index<S>(0, std::uint32_t(r)));
    }

    // Access of the word at lane_bytes + reg_bytes (reg_bytes compile-time
    // per register). Small register offsets stay in the lane offset, where
    // they fold into the instruction's immediate and neighbouring registers
    // merge into wide accesses; large ones go to the scalar offset. A
    // one-pass tile may be partial and relies on the range check, which
    // sees only the lane offset, so it never uses the scalar offset.
    static __device__ __forceinline__ W load_at(__amdgpu_buffer_rsrc_t src, std::uint32_t lane_bytes,
                                                std::uint32_t reg_bytes) {
        if (SINGLE || reg_bytes < 4096u) return buffer_load<W>(src, lane_bytes + reg_bytes);
        return buffer_load<W>(src, lane_bytes, reg_bytes);
    }
    static __device__ __forceinline__ void store_at(W x, __amdgpu_buffer_rsrc_t dst, std::uint32_t lane_bytes,
                                                    std::uint32_t reg_bytes) {
        if (SINGLE || reg_bytes < 4096u) buffer_store<W, kStoreAux>(x, dst, lane_bytes + reg_bytes);
        else buffer_store<W, kStoreAux>(x, dst, lane_bytes, reg_bytes);
    }

    // Staged (permuted) enumeration: element g of the tile in physical
    // contiguity order -> (tile index i, word relative to the span).
    static __device__ __forceinline__ void permuted(const Tile& tl, std::uint32_t g, std::uint32_t& i,
                                                    std::uint32_t& word) {
        if constexpr (COL) {  // each column is a contiguous bit-reversed block of 2^L1 words
            const std::uint32_t rp = g & ((1u << LT) - 1u), cc = g >> LT;
            i = cc | (brev(rp, LT) << LI);
            word = (brev(tl.c0 + cc, L2) << L1) + rp;
        } else if constexpr (SINGLE) {  // in-row bit reversal, rows are polynomials
            const std::uint32_t xp = g & ((1u << LT) - 1u), rr = g >> LT;
            i = brev(xp, LT) | (rr << LT);
            word = (rr << LT) + xp;
        } else {  // rows bitrev(k0 + rr): lanes over rr are contiguous words
            const std::uint32_t rr = g & ((1u << LI) - 1u), cp = g >> LI;
            i = brev(cp, LT) | (rr << LT);
            word = (cp << L1) + tl.k0 + rr;
        }
    }

    // permuted() of g = t + T * r, split like thread_word / register_word:
    // each output is a sum over disjoint bit fields of g, and the tile origin
    // enters only through the thread part.
    struct Staged {
        std::uint32_t i, word;  // thread part
        std::uint32_t lds;      // LDS address of the thread part (linear layouts)
    };
    static __device__ __forceinline__ Staged staged_base(const Tile& tl, std::uint32_t t) {
        Staged b;
        permuted(tl, t, b.i, b.word);
        b.lds = L::addr(b.i);
        return b;
    }
    static __device__ __forceinline__ std::uint32_t staged_lds(const Staged& b, int r) {
        std::uint32_t i, word;
        permuted(Tile{}, T * std::uint32_t(r), i, word);
        if constexpr (L::kLinear) return b.lds + L::addr(i);
        else return L::addr(b.i + i);
    }
    static __device__ __forceinline__ std::uint32_t staged_word(int r) {
        std::uint32_t i, word;
        permuted(Tile{}, T * std::uint32_t(r), i, word);
        return word;
    }

    // Block index of this thread's phase-P twiddle chunk.
    template <int P>
    static __device__ __forceinline__ std::uint32_t chunk_index(const Tile& tl, std::uint32_t t) {
        const std::uint32_t i0 = phase_index<tile_window<P>()>(t, 0);
        const std::uint32_t x0 = COL ? (i0 >> LI) : (i0 & ((1u << LT) - 1u));
        // Prefix: 1 for columns and one-pass rows, 2^L1 + row for two-pass
        // rows (the row is the same for all registers since LT >= 4 there).
        const std::uint32_t prefix = (COL || SINGLE) ? 1u : ((1u << L1) + row_of(tl, i0 >> LT));
        const std::uint32_t head = (prefix << LT) | x0;
        constexpr int shift = chunk_shift(LT, CT, P);
        constexpr std::uint32_t first = ((COL || SINGLE) ? (1u << LT) : (1u << (L1 + LT))) >> shift;
        return (head >> shift) - first;
    }

    using V4 = __attribute__((ext_vector_type(4))) std::uint32_t;
    // 16-byte loads that hold one phase's chunk.
    template <int P>
    static constexpr int chunk_loads() {
        return (chunk_entries(LT, CT, kLast, P) * int(sizeof(E)) + 15) / 16;
    }
    template <int P>
    struct Chunk {
        V4 raw[chunk_loads<P>() > 0 ? chunk_loads<P>() : 1];
    };

    template <int P>
    static __device__ __forceinline__ void load_chunk(Chunk<P>& c, const PassArgs<W>& a, const Tile& tl,
                                                      std::uint32_t t, __amdgpu_buffer_rsrc_t tw) {
        if constexpr (P < kPhases) {
            // Piece e of chunk c sits at (e * count + c) * 16 bytes from the
            // phase's table: the per-piece step is a compile-time constant
            // (scalar offset), the chunk a lane offset.
            constexpr std::uint32_t step = 16u * std::uint32_t(chunk_count(LT, (COL || SINGLE) ? 0 : L1, CT, P));
            const std::uint32_t base =
                a.phase_off[P] * std::uint32_t(sizeof(E)) + 16u * chunk_index<P>(tl, t);
#pragma unroll
            for (int e = 0; e < chunk_loads<P>(); ++e)
                c.raw[e] = __builtin_amdgcn_raw_buffer_load_b128(tw, int(base), int(step * std::uint32_t(e)), 0);
        }
    }

    template <int P>
    static __device__ __forceinline__ void stages(W (&v)[kE], const Chunk<P>& c, const DeviceDomain<W>& d) {
        constexpr int ws = window_start(LT, CT, P);
#pragma unroll
        for (int s = 0; s < active_stages(LT, CT, P); ++s) {
            const int k = exec_stage(LT, CT, P, s);
            const int jb = k - ws;
            const std::uint32_t gmask = (1u << (LT - 1 - k)) - 1u;
            const bool scale = scale_stage(LT, CT, kLast, k);
            const int off = chunk_offset(LT, CT, kLast, P, s);
#pragma unroll
            for (int g = 0; g < (1 << (kLE - 1 - jb)); ++g) {
                TwPair<W> tp{};
                if (!scale) {
                    const int e = off + int(std::uint32_t(g) & gmask);
                    if constexpr (BARRETT && sizeof(W) == 4) {
                        tp.w = c.raw[e >> 2][e & 3];
                    } else if constexpr (BARRETT) {
                        tp.w = (std::uint64_t(c.raw[e >> 1][(e & 1) * 2 + 1]) << 32) | c.raw[e >> 1][(e & 1) * 2];
                    } else if constexpr (sizeof(W) == 4) {
                        tp.w = c.raw[e >> 1][(e & 1) * 2];
                        tp.wp = c.raw[e >> 1][(e & 1) * 2 + 1];
                    } else {
                        tp.w = (std::uint64_t(c.raw[e][1]) << 32) | c.raw[e][0];
                        tp.wp = (std::uint64_t(c.raw[e][3]) << 32) | c.raw[e][2];
                    }
                }
#pragma unroll
                for (int lo = 0; lo < (1 << jb); ++lo) {
                    const int r = (g << (jb + 1)) | lo;
                    const int r2 = r | (1 << jb);
                    if constexpr (CT && BARRETT) {
                        ct_barrett<W>(v[r], v[r2], tp.w, d);
                    } else if constexpr (CT) {
                        ct_butterfly<W, LAZY>(v[r], v[r2], tp, d);
                    } else if (scale) {
                        // The final inverse stage scales by n^-1 with the
                        // domain's Shoup pairs in every arithmetic ([0, 2q):
                        // the last pass's final reduction follows).
                        gs_scale_butterfly<W, LAZY>(v[r], v[r2], d);
                    } else if constexpr (BARRETT) {
                        gs_barrett<W>(v[r], v[r2], tp.w, d);
                    } else {
                        gs_butterfly<W, LAZY>(v[r], v[r2], tp, d);
                    }
                }
            }
        }
    }

    // Register window FROM -> TO through the LDS image. `between` runs
    // between the writes and the second barrier: the next phase's twiddle
    // loads go there, so their latency overlaps the barrier wait and their
    // registers are only live from the phase that uses them (loading every
    // phase's chunk up front kept them all live and cost occupancy).
    template <int FROM, int TO, class Between>
    static __device__ __forceinline__ void exchange(W (&v)[kE], W* lds, std::uint32_t t, Between&& between) {
        if constexpr (kWaveLocal) wave_lds_fence();
        else lds_barrier();
#pragma unroll
        for (int r = 0; r < kE; ++r) lds[L::template at<FROM>(t, r)] = v[r];
        between();
        if constexpr (kWaveLocal) wave_lds_fence();
        else lds_barrier();
#pragma unroll
        for (int r = 0; r < kE; ++r) v[r] = lds[L::template at<TO>(t, r)];
    }

    // The tile's 16 input words, raw (boundary permutation and reduction
    // happen in process()).
    static __device__ __forceinline__ void load_tile(const PassArgs<W>& a, const Tile& tl, std::uint32_t t,
                                                     W (&v)[kE]) {
        const __amdgpu_buffer_rsrc_t src = span(a.in, a.in_off, tl);
        constexpr int S = tile_window<0>();
        constexpr std::uint32_t B = sizeof(W);
        const std::uint32_t tw = PIN ? staged_base(tl, t).word : thread_word<S>(tl, t);
#pragma unroll
        for (int r = 0; r < kE; ++r) {
            const std::uint32_t rw = PIN ? staged_word(r) : register_word<S>(r);
            v[r] = load_at(src, tw * B, rw * B);
        }
    }

    static __device__ __forceinline__ __amdgpu_buffer_rsrc_t twiddles(const PassArgs<W>& a, const DeviceDomain<W>& d) {
        return make_rsrc(static_cast<const E*>(a.tw) + d.tw, a.tw_bytes);
    }

    // The tile's butterflies and its store. c0 holds phase 0's twiddle chunk;
    // later phases load theirs during the preceding exchange.
    static __device__ __forceinline__ void process(const PassArgs<W>& a, const Tile& tl, std::uint32_t t, W (&v)[kE],
                                                   const Chunk<0>& c0, const DeviceDomain<W>& d, W* lds) {
        if constexpr (PIN) {  // physical order -> phase-0 layout through LDS
            lds_barrier();
            const Staged b = staged_base(tl, t);
#pragma unroll
            for (int r = 0; r < kE; ++r) lds[staged_lds(b, r)] = v[r];
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kE; ++r) v[r] = lds[L::template at<tile_window<0>()>(t, r)];
        }
        if (kFirst && a.reduce_input) {
            // Arbitrary input words -> [0, 2q). A Cooley-Tukey first stage
            // multiplies its upper operands by Shoup twiddles (any word is
            // fine there), so only the lower half needs it. Barrett products
            // need canonical operands: every word is reduced to [0, q).
            constexpr int top = CT ? stage_hi(LT, CT, 0) - window_start(LT, CT, 0) : kLE;
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                if constexpr (BARRETT) v[r] = reduce_once(shoup(v[r], W(1), d.rwp, d.nq), d.q);
                else if (!CT || LT < kLE || !((r >> top) & 1)) v[r] = shoup(v[r], W(1), d.rwp, d.nq);
            }
        }
        stages<0>(v, c0, d);
        if constexpr (kPhases > 1) {
            Chunk<1> c1;
            exchange<tile_window<0>(), tile_window<1>()>(v, lds, t,
                                                         [&] { load_chunk<1>(c1, a, tl, t, twiddles(a, d)); });
            stages<1>(v, c1, d);
        }
        if constexpr (kPhases > 2) {
            Chunk<2> c2;
            exchange<tile_window<1>(), tile_window<2>()>(v, lds, t,
                                                         [&] { load_chunk<2>(c2, a, tl, t, twiddles(a, d)); });
            stages<2>(v, c2, d);
        }
        constexpr int wl = tile_window<kPhases - 1>();
        if constexpr (kLast) {
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                W x = v[r];
                if constexpr (CT && LAZY) x = csub(x, d.q2);
                v[r] = csub(x, d.q);
            }
        }
        const __amdgpu_buffer_rsrc_t dst = span(a.out, a.out_off, tl);
        if constexpr (POUT) {
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kE; ++r) lds[L::template at<wl>(t, r)] = v[r];
            lds_barrier();
            constexpr std::uint32_t B = sizeof(W);
            const Staged b = staged_base(tl, t);
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                store_at(lds[staged_lds(b, r)], dst, b.word * B, staged_word(r) * B);
            }
        } else if constexpr (kStagedStore) {
            constexpr std::uint32_t B = sizeof(W);
            wave_lds_fence();
#pragma unroll
            for (int r = 0; r < kE; ++r) lds[L::template at<wl>(t, r)] = v[r];
            wave_lds_fence();
            const std::uint32_t g0 = run_first(t);
            const std::uint32_t a0 = L::addr(g0);
            const std::uint32_t w0 = natural_word(tl, g0) * B;
#pragma unroll
            for (int k = 0; k < kE / kPer; ++k) {
                const std::uint32_t gk = run_offset(k);
                const std::uint32_t ak = a0 + L::addr(gk);
                using V4 = __attribute__((ext_vector_type(4))) std::uint32_t;
                W x[kPer];
#pragma unroll
                for (int e = 0; e < kPer; ++e) x[e] = lds[ak + std::uint32_t(e)];
                buffer_store<V4, kStagedAux>(__builtin_bit_cast(V4, x), dst, w0, gk * B);
            }
        } else {
            constexpr std::uint32_t B = sizeof(W);
            const std::uint32_t tw = thread_word<wl>(tl, t);
#pragma unroll
            for (int r = 0; r < kE; ++r) store_at(v[r], dst, tw * B, register_word<wl>(r) * B);
        }
    }

    // One domain per tile (the planner keeps mixed-domain tiles apart). The
    // record is wave-uniform; it comes back through vector loads (the
    // kernel's stores could alias it as far as the compiler knows), so each
    // field is read back into a scalar register.
    static __device__ __forceinline__ DeviceDomain<W> domain_of(const PassArgs<W>& a, const Tile& tl) {
        const std::uint32_t dom = a.poly_domain ? uniform(a.poly_domain[tl.poly]) : 0u;
        const DeviceDomain<W> d = a.domains[dom];
        DeviceDomain<W> u;
        u.q = uniform(d.q);
        u.q2 = uniform(d.q2);
        u.nq = uniform(d.nq);
        u.rwp = uniform(d.rwp);
        u.ninv = {uniform(d.ninv.w), uniform(d.ninv.wp)};
        u.last = {uniform(d.last.w), uniform(d.last.wp)};
        u.mu = uniform(d.mu);
        u.qbits = uniform(d.qbits);
        u.tw = uniform(d.tw);
        return u;
    }

    // One tile: its words, its twiddle chunks, the butterflies and the
    // store. `lds` holds at least L::kWords words.
    static __device__ __forceinline__ void tile(const PassArgs<W>& a, std::uint32_t index, W* lds) {
        const std::uint32_t t = threadIdx.x;
        const Tile tl = decode(a, index);
        W v[kE];
        load_tile(a, tl, t, v);
        const DeviceDomain<W> d = domain_of(a, tl);
        Chunk<0> c0;
        load_chunk<0>(c0, a, tl, t, twiddles(a, d));
        process(a, tl, t, v, c0, d, lds);
    }

    // One tile per workgroup. (Every tile of a 2^16 x 64 pass is resident at
    // once on 256 CUs; persistent prefetching variants measured slower.)
    static __device__ void run(const PassArgs<W>& a) {
        __shared__ W lds[L::kWords];
        const std::uint32_t b = blockIdx.x;
        // XCD-contiguous tile order: blocks are dealt to the 8 XCDs
        // round-robin, so block b walks tile (b mod 8) * tiles/8 + b/8 and the
        // tiles sharing cache lines and twiddle rows meet in one L2.
        const std::uint32_t index =
            (a.tiles & 7u) == 0 && (gridDim.x & 7u) == 0 ? (b & 7u) * (a.tiles >> 3) + (b >> 3) : b;
        tile(a, index, lds);
    }
};

template <class W, int AR, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE, int L1, int L2>
__global__ __launch_bounds__(1 << (LT + LI - kLE)) void ntt_pass_kernel(PassArgs<W> a) {
    Pass<W, AR, LT, LI, COL, CT, PIN, POUT, SINGLE, L1, L2>::run(a);
}

// ---- launcher registry -----------------------------------------------------

template <class W>
using PassLaunch = void (*)(const PassArgs<W>&, unsigned grid, hipStream_t);

struct PassKey {
    int arith;  // kStrict, kLazy or kBarrett
    int log_n, lt, li;
    bool col, ct, pin, pout, single;
    bool operator<(const PassKey& o) const {
        return std::tie(arith, log_n, lt, li, col, ct, pin, pout, single) <
               std::tie(o.arith, o.log_n, o.lt, o.li, o.col, o.ct, o.pin, o.pout, o.single);
    }
};

template <class W, int AR, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE, int L1, int L2>
void launch_pass(const PassArgs<W>& a, unsigned grid, hipStream_t stream) {
    hipLaunchKernelGGL((ntt_pass_kernel<W, AR, LT, LI, COL, CT, PIN, POUT, SINGLE, L1, L2>), dim3(grid),
                       dim3(1u << (LT + LI - kLE)), 0, stream, a);
}

// One table per word type, filled once by the per-arithmetic translation units.
template <class W>
std::map<PassKey, PassLaunch<W>>& registry();
template <>
std::map<PassKey, PassLaunch<std::uint32_t>>& registry<std::uint32_t>();
template <>
std::map<PassKey, PassLaunch<std::uint64_t>>& registry<std::uint64_t>();

template <class W, int AR, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE, int L1, int L2>
void add() {
    registry<W>()[PassKey{AR, L1 + L2, LT, LI, COL, CT, PIN, POUT, SINGLE}] =
        &launch_pass<W, AR, LT, LI, COL, CT, PIN, POUT, SINGLE, L1, L2>;
}

// Boundary-permutation variants of one pass shape: a first pass may permute
// its input, a last pass its output.
template <class W, int AR, int LT, int LI, bool COL, bool CT, bool SINGLE, int L1, int L2>
void add_variants() {
    constexpr bool first = SINGLE || (COL == CT);
    constexpr bool last = SINGLE || (COL != CT);
    add<W, AR, LT, LI, COL, CT, false, false, SINGLE, L1, L2>();
    if constexpr (first) add<W, AR, LT, LI, COL, CT, true, false, SINGLE, L1, L2>();
    if constexpr (last) add<W, AR, LT, LI, COL, CT, false, true, SINGLE, L1, L2>();
    if constexpr (first && last) add<W, AR, LT, LI, COL, CT, true, true, SINGLE, L1, L2>();
}

template <class W, int AR, int LT, int LB>
void add_single() {
    add_variants<W, AR, LT, LB - LT, false, true, true, 0, LT>();
    add_variants<W, AR, LT, LB - LT, false, false, true, 0, LT>();
}

// Two-pass split used by the planner: l1 = min(8, log n / 2) high bits;
// column tiles of 2^COL_LI lines, row tiles of as many rows as fit 2^LB words.
constexpr int split_l1(int log_n) { return log_n / 2 < 8 ? log_n / 2 : 8; }
constexpr int kTileLog = 12;
constexpr int kColLines = 4;
// u32 column tiles may also hold 32 columns (128-byte row segments, 2^(l1+5)
// words, up to 512 threads): the `-c32` lowering.
constexpr int kWideColLines = 5;
constexpr int row_lines(int l1, int l2) { return l1 < kTileLog - l2 ? l1 : kTileLog - l2; }

// Column passes of one split with 32-column tiles, where they fit.
template <class W, int AR, int L1, int L2>
void add_wide_columns() {
    if constexpr (L1 + kWideColLines <= 13 && L2 >= kWideColLines) {
        add_variants<W, AR, L1, kWideColLines, true, true, false, L1, L2>();
        add_variants<W, AR, L1, kWideColLines, true, false, false, L1, L2>();
    }
}

// Column passes of one split: 16-column tiles, and 32-column tiles (WIDE).
template <class W, int AR, int L1, int L2, bool WIDE>
void add_columns() {
    add_variants<W, AR, L1, kColLines, true, true, false, L1, L2>();
    add_variants<W, AR, L1, kColLines, true, false, false, L1, L2>();
    if constexpr (WIDE) add_wide_columns<W, AR, L1, L2>();
}

template <class W, int AR, int L1, int L2>
void add_rows() {
    constexpr int rli = row_lines(L1, L2);
    add_variants<W, AR, L2, rli, false, true, false, L1, L2>();
    add_variants<W, AR, L2, rli, false, false, false, L1, L2>();
}

// The planner's split (l1 = split_l1): u32 with 16- and 32-column tiles,
// u64 with 16 (32-column u64 tiles and other splits are instantiated by
// ntt_alt_u32.hip and ntt_alt_u64.hip).
template <class W, int AR, int LOG_N>
void add_two_pass() {
    constexpr int l1 = split_l1(LOG_N), l2 = LOG_N - l1;
    add_columns<W, AR, l1, l2, sizeof(W) == 4>();
    add_rows<W, AR, l1, l2>();
}

// Another split of LOG_N (both tile widths), for MEASURE and RNS Prepare.
template <class W, int AR, int LOG_N, int L1>
void add_split() {
    static_assert(L1 >= 4 && LOG_N - L1 >= 4 && LOG_N - L1 <= kTileLog, "split shape");
    add_columns<W, AR, L1, LOG_N - L1, true>();
    add_rows<W, AR, L1, LOG_N - L1>();
}

// 4 KiWord tiles; columns of 64 B (u32) / 128 B (u64).
template <class W, int AR>
void register_all() {
    constexpr int LB = kTileLog;
    add_single<W, AR, 1, LB>();
    add_single<W, AR, 2, LB>();
    add_single<W, AR, 3, LB>();
    add_single<W, AR, 4, LB>();
    add_single<W, AR, 5, LB>();
    add_single<W, AR, 6, LB>();
    add_single<W, AR, 7, LB>();
    add_single<W, AR, 8, LB>();
    add_single<W, AR, 9, LB>();
    add_single<W, AR, 10, LB>();
    add_single<W, AR, 11, LB>();
    add_single<W, AR, 12, LB>();
    add_two_pass<W, AR, 13>();
    add_two_pass<W, AR, 14>();
    add_two_pass<W, AR, 15>();
    add_two_pass<W, AR, 16>();
    add_two_pass<W, AR, 17>();
    add_two_pass<W, AR, 18>();
    add_two_pass<W, AR, 19>();
    add_two_pass<W, AR, 20>();
}

void register_u32_lazy();
void register_u32_strict();
void register_u64_lazy();
void register_u64_strict();
void register_u32_barrett();
void register_u64_barrett();
void register_alt_u32();
void register_alt_u64();

// Splits l1 of two-pass lengths with kernels: the planner's split_l1 and the
// neighbouring ones that ntt_alt_u32.hip and ntt_alt_u64.hip instantiate.
constexpr bool alt_split(int log_n, int l1) {
    return log_n >= 15 && log_n <= 17 && (l1 == split_l1(log_n) - 1 || l1 == split_l1(log_n) + 1);
}

}  // namespace ntt_detail
}  // namespace cbw
