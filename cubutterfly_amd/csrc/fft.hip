// Complex FFT (COMPLEX_FP32, natural order in and out) for gfx950.
//
// Decimation in frequency over digits of DB bits (5 on one-pass 2^13- and
// 2^14-point tiles, 4 elsewhere), top digit first. A workgroup holds a tile of 2^LB complex
// values = 2^LT transform points x 2^LI lines, 2^DB per thread. For each
// digit: an in-register radix-2^r DIF codelet with compile-time twiddles
// (r = DB, the last digit r = 1..DB), then every element is multiplied by
// w_{2^h}^(j_low * c): j_low = the element's index bits below the digit, c =
// its digit output, h = the digit's top bit + 1 (the four-step twiddle of
// that level). LDS exchanges regroup the data between digits. The result
// lands in bit-reversed position (digit reversal with each digit
// bit-reversed), so the final pass stores through an LDS-staged
// bit-reversal; two-pass lengths also transpose the 2^l1 x 2^l2 grid there.
//
// Level twiddles come from two 4096-entry tables (w^f = A[f >> 12] B[f & 4095],
// entries rounded from double), so lengths up to 2^24 need 64 KB of tables.
// Lengths <= 2^14 run in one pass; up to 2^24 in two.
#include <hip/hip_runtime.h>

#include "buffer.hpp"
#include "json.hpp"
#include "planner.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

// Complex products may fuse into FMAs here: FFT accuracy is specified as a
// relative L2 bound, and fused products are the more accurate ones.
#pragma clang fp contract(fast)

namespace cbw {
namespace {

struct FftArgs {
    const float2* in;
    float2* out;
    const float2* twa;  // w^(4096 k), k < 4096
    const float2* twb;  // w^k, k < 4096
    std::uint32_t l1, l2;  // high / low index bits (l1 = 0: one pass)
    // Column passes: the low cbits bits of the column index number
    // independent transforms (the other axis of a rank-2 block) and stay out
    // of the level twiddles; 0 for a one-dimensional transform.
    std::uint32_t cbits;
    std::uint32_t rows, tiles;
    float scale;  // 1/n for the normalised inverse on the final store, else 1
    // Elements between consecutive transforms of the input / output buffer:
    // n when packed, a caller's row pitch otherwise (one transform per tile).
    std::uint64_t in_pitch, out_pitch;
};

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ std::uint32_t brev(std::uint32_t x, std::uint32_t bits) {
    return bits ? __brev(x) >> (32 - bits) : 0u;
}

// Hides a value from the optimiser (no code): keeps computations that use it
// where they are written.
__device__ __forceinline__ void opaque(float2& x) { asm volatile("" : "+v"(x.x), "+v"(x.y)); }

constexpr std::uint32_t brev_const(std::uint32_t x, int bits) {
    std::uint32_t r = 0;
    for (int i = 0; i < bits; ++i) r |= ((x >> i) & 1u) << (bits - 1 - i);
    return r;
}

// Tile index of (thread t, register r) when the DB register bits sit at
// tile bits [S, S + DB).
template <int S, int DB>
__device__ __forceinline__ std::uint32_t phase_index(std::uint32_t t, std::uint32_t r) {
    return (t & ((1u << S) - 1u)) | (r << S) | ((t >> S) << (S + DB));
}

// cos(2 pi j / 32) for j = 0..31 (decimal expansions of the exact values).
constexpr double kCos32[32] = {
    1.0, 9.80785280403230449126e-1, 9.23879532511286756128e-1, 8.31469612302545237079e-1,
    7.07106781186547524401e-1, 5.55570233019602224743e-1, 3.82683432365089771728e-1, 1.95090322016128267848e-1,
    0.0, -1.95090322016128267848e-1, -3.82683432365089771728e-1, -5.55570233019602224743e-1,
    -7.07106781186547524401e-1, -8.31469612302545237079e-1, -9.23879532511286756128e-1, -9.80785280403230449126e-1,
    -1.0, -9.80785280403230449126e-1, -9.23879532511286756128e-1, -8.31469612302545237079e-1,
    -7.07106781186547524401e-1, -5.55570233019602224743e-1, -3.82683432365089771728e-1, -1.95090322016128267848e-1,
    0.0, 1.95090322016128267848e-1, 3.82683432365089771728e-1, 5.55570233019602224743e-1,
    7.07106781186547524401e-1, 8.31469612302545237079e-1, 9.23879532511286756128e-1, 9.80785280403230449126e-1};

// x * w_len^j with w = exp(-+2 pi i / len) (forward / inverse), constants folded.
template <int LEN, int J, bool INV>
__device__ __forceinline__ float2 twiddle_const(float2 x) {
    constexpr int e = (J * (32 / LEN)) & 31;  // angle index in 32nds of a turn
    if constexpr (e == 0) {
        return x;
    } else if constexpr (e == 8) {  // -i (forward) / +i (inverse)
        return INV ? make_float2(-x.y, x.x) : make_float2(x.y, -x.x);
    } else if constexpr (e == 16) {
        return make_float2(-x.x, -x.y);
    } else if constexpr (e == 24) {
        return INV ? make_float2(x.y, -x.x) : make_float2(-x.y, x.x);
    } else {
        constexpr float c = float(kCos32[e]);
        constexpr float s = float(INV ? kCos32[(e + 24) & 31] : -kCos32[(e + 24) & 31]);  // +-sin
        return make_float2(x.x * c - x.y * s, x.x * s + x.y * c);
    }
}

// One radix-2 DIF stage (pairs R, R + 2^B inside each group), unrolled over
// the registers at compile time.
template <int E, int B, int R, bool INV>
__device__ __forceinline__ void codelet_stage(float2 (&v)[E]) {
    constexpr int half = 1 << B;
    if constexpr (!(R & half)) {
        const float2 u = v[R], w = v[R + half];
        v[R] = make_float2(u.x + w.x, u.y + w.y);
        v[R + half] = twiddle_const<2 * half, (R & (half - 1)), INV>(make_float2(u.x - w.x, u.y - w.y));
    }
    if constexpr (R + 1 < E) codelet_stage<E, B, R + 1, INV>(v);
}

// Radix-2^DS DIF on register bits [0, DS) of each 2^DS group (bit-reversed out).
template <int E, int DS, bool INV>
__device__ __forceinline__ void codelet(float2 (&v)[E]) {
    codelet_stage<E, DS - 1, 0, INV>(v);
    if constexpr (DS > 1) codelet<E, DS - 1, INV>(v);
}

constexpr int digit_bits_for(int lb, bool single);

// LDS image of a tile (8-byte complex words).
//
// One-pass tiles of one whole row of 2^12 .. 2^14 points are unpadded, with
// the low four word bits XORed with index bits [DB, DB + 4) and
// [LT - 5, LT - 1) (DB the digit width). A 16-lane group of a 64-bit LDS
// access covers all banks when its 16 words differ in those four low bits,
// and every access of these tiles varies across a group in one of the three
// fields: the lowest four index bits (phase exchanges with the register
// window above them), the digit's lowest four bits (the exchange into the
// last digit), or bits LT - 5 .. LT - 2 (the bit-reversed reads of the paired
// final store: outputs 2j and 2j + 1, j varying in its low four bits). The
// XOR of the varying field with the others, constant or overlapping in one
// bit, stays a bijection on it (checked by enumeration for 2^12, 2^13 and
// 2^14 points). Keyed on the top four bits instead, the paired reads of
// 2^14-point tiles fell on 8 bank pairs per group; a plain 1-in-16 pad left
// the unpaired bit-reversed read on one.
//
// Other row tiles pad each row by 1/16 and 1 word; column tiles pad rows and
// swizzle columns. Column tiles whose lanes hold every other column (PAIRED:
// FftPass::logical_thread) also rotate the column index (bit 0 to the top),
// so a 16-lane group's columns 2c + h, c consecutive, land on 16 distinct
// 8-byte bank pairs again instead of 8 (checked by enumeration).
template <bool COL, int LT, int LI, bool SINGLE, bool PAIRED = false, int DBX = 0>
struct FftLds {
    static constexpr int DB = DBX ? DBX : digit_bits_for(LT + LI, SINGLE);
    static constexpr bool kXor = SINGLE && LI == 0 && LT >= DB + 8;
    // Row layouts are sums of terms over disjoint index bit fields, so
    // addr(a | b) = addr(a) + addr(b) for disjoint a, b; the XOR layout is
    // linear over bits, addr(a | b) = addr(a) ^ addr(b); the column layout's
    // swizzle is neither.
    static constexpr bool kLinear = !COL && !kXor;
    static constexpr std::uint32_t kWords =
        kXor ? (1u << LT)
             : COL ? (1u << LT) * ((1u << LI) + 1u) : (1u << LI) * ((1u << LT) + (1u << LT >> 4) + 1u);
    static __device__ __forceinline__ std::uint32_t addr(std::uint32_t i) {
        if constexpr (kXor) {
            return i ^ (((i >> DB) ^ (i >> (LT - 5))) & 15u);
        } else if constexpr (COL) {
            std::uint32_t cc = i & ((1u << LI) - 1u);
            const std::uint32_t x = i >> LI;
            if constexpr (PAIRED) cc = (cc >> 1) | ((cc & 1u) << (LI - 1));
            return x * ((1u << LI) + 1u) + (cc ^ ((x >> 3) & ((1u << LI) - 1u)));
        } else {
            const std::uint32_t x = i & ((1u << LT) - 1u), rr = i >> LT;
            return rr * ((1u << LT) + (1u << LT >> 4) + 1u) + x + (x >> 4);
        }
    }
    // addr(it | ir) for disjoint thread and register parts.
    static __device__ __forceinline__ std::uint32_t split(std::uint32_t it, std::uint32_t ir) {
        if constexpr (kXor) return addr(it) ^ addr(ir);
        else if constexpr (kLinear) return addr(it) + addr(ir);
        else return addr(it | ir);
    }
};

// One-pass tiles of 2^13 and 2^14 points (LDS-bound to one or two per CU)
// use 5-bit digits, 32 values per thread, and prefetch the next tile into
// registers (2 waves per SIMD leave room for both tiles). Other tiles use
// 4-bit digits and 16 values per thread. Two-pass tiles at m = 24 measured
// slower with 5-bit digits and prefetching (their 32-byte column segments,
// not the VALU, bound them), so they keep the 4-bit layout.
constexpr int digit_bits_for(int lb, bool single) { return single && lb >= 13 ? 5 : 4; }
// A pass's digit width: ORD bit 4 asks one-pass tiles of 2^13 / 2^14 points
// for 4-bit digits (16 values per thread, twice the threads per tile).
constexpr int pass_digit_bits(int lb, bool single, int ord) { return (ord & 16) ? 4 : digit_bits_for(lb, single); }

// One FFT pass over LT transform bits. COL: high bits, tile of 2^LI columns;
// ROW: low bits, tile of 2^LI rows (the final pass, storing in natural order);
// SINGLE: a one-pass transform, 2^LI whole rows per tile.
// ORD: for one-pass tiles, bit 0 reads the input in bit-reversed logical
// order and bit 1 writes the output in bit-reversed order (the DIF result's
// own order, so the final store skips the reversal); for row passes, bit 2
// reads the block's rows in natural order (a row-major 2^l1 x 2^l2 block
// whose row transforms are written transposed: the rank-2 axis step), and
// bit 3 writes row k of the block's bit-reversed row order back as row k,
// transformed, in natural order (the last step of a rank-2 transform whose
// first axis ran as column passes). Bit 4 gives one-pass tiles of 2^13 and
// 2^14 points 4-bit digits (pass_digit_bits). Bit 5 makes the final row pass
// of a two- or three-pass transform write the bit-reversed logical order:
// output k = k1 + 2^l1 k2 belongs at bitrev(k) = bitrev(k1) 2^l2 +
// bitrev(k2), and the row pass reads tile row k1 from row bitrev(k1) of the
// intermediate, so each row goes back to the row it came from, in the DIF
// result's own order (no reversal, no transpose).
template <int LT, int LI, bool COL, bool SINGLE, bool INV, int ORD = 0>
struct FftPass {
    static constexpr int LB = LT + LI;
    static constexpr int DB = pass_digit_bits(LB, SINGLE, ORD);
    static constexpr int kE = 1 << DB;
    static constexpr std::uint32_t T = 1u << (LB - DB);
    static constexpr int kPhases = (LT + DB - 1) / DB;
    // Prefetching needs registers for two tiles: with 16 values per thread
    // that fits the 128-register budget for passes of at most two digits,
    // and for the 4-bit one-pass tiles of 2^13 / 2^14 points, whose bases
    // beyond the third are fetched digit by digit.
    static constexpr bool kPrefetch = DB == 5 || kPhases <= 2 || (ORD & 16) != 0;
    static constexpr bool kPairedColumns = COL && LI == 6 && kE == 16;
    using L = FftLds<COL, LT, LI, SINGLE, kPairedColumns, DB>;

    template <int P>
    static constexpr int window() {  // transform-relative register window start
        return LT - DB * (P + 1) > 0 ? LT - DB * (P + 1) : 0;
    }
    template <int P>
    static constexpr int digit_bits() {
        return LT - DB * P < DB ? LT - DB * P : DB;
    }
    template <int P>
    static constexpr int tile_window() {
        return (COL ? LI : 0) + window<P>();
    }
    template <int S>
    static __device__ __forceinline__ std::uint32_t index(std::uint32_t t, std::uint32_t r) {
        return phase_index<S, DB>(t, r);
    }

    // Whether digit P is followed by a level twiddle (not for the last digit
    // of the whole transform, whose lowest bit is bit 0).
    template <int P>
    static constexpr bool twiddled() {
        return COL || window<P>() > 0;
    }

    // Level twiddle base of digit P for thread t: register r (digit output
    // c = bitrev(r)) is multiplied by base^c, base = w^(j_low << (m - h)),
    // j_low = the element's index bits below the digit, h = the digit's top
    // bit + 1 (the four-step twiddle of that level). One table pair per
    // thread and digit: w^f = A[f >> 12] * B[f & 4095].
    template <int P>
    static __device__ __forceinline__ float2 level_base(const FftArgs& a, std::uint32_t t, std::uint32_t c0,
                                                        std::uint32_t m) {
        if constexpr (!twiddled<P>()) {
            return make_float2(1.f, 0.f);
        } else {
            constexpr int ws = window<P>(), ds = digit_bits<P>();
            const std::uint32_t lo_rel = std::uint32_t(ws);
            const std::uint32_t lo = COL ? a.l2 - a.cbits + lo_rel : lo_rel;
            const std::uint32_t h = lo + ds;
            const std::uint32_t i0 = index<tile_window<P>()>(t, 0);
            // Index bits below the digit: for columns, the low transform bits
            // of the column index and the column's transform bits (the column
            // without its low cbits); for rows, the low bits.
            const std::uint32_t x0 = COL ? (i0 >> LI) : (i0 & ((1u << LT) - 1u));
            std::uint32_t jl = x0 & ((1u << lo_rel) - 1u);
            if (COL) jl = (jl << (a.l2 - a.cbits)) | ((c0 + (i0 & ((1u << LI) - 1u))) >> a.cbits);
            const std::uint32_t f = jl << (m - h);
            const __amdgpu_buffer_rsrc_t ta = make_rsrc(a.twa, 4096u * 8u), tb = make_rsrc(a.twb, 4096u * 8u);
            return cmul(buffer_load<float2>(ta, (f >> 12) * 8u), buffer_load<float2>(tb, (f & 4095u) * 8u));
        }
    }

    // Digit P: codelet, then the level twiddle base^c on each register.
    template <int P>
    static __device__ __forceinline__ void digit(float2 (&v)[kE], float2 base) {
        constexpr int ds = digit_bits<P>();
        codelet<kE, ds, INV>(v);
        if constexpr (twiddled<P>()) {
            // base^c for c = 1 .. 2^ds - 1, streamed: only base^1,2,3,4,8,16
            // stay live; every other power is at most three products of those,
            // applied as soon as it is formed.
            float2 p1 = base;
            float2 p2 = ds > 1 ? cmul(p1, p1) : p1;
            float2 p3 = ds > 1 ? cmul(p2, p1) : p1;
            float2 p4 = ds > 2 ? cmul(p2, p2) : p1;
            float2 p8 = ds > 3 ? cmul(p4, p4) : p1;
            float2 p16 = ds > 4 ? cmul(p8, p8) : p1;
            // Row passes compute their bases once per thread; in the tile loop
            // the optimiser would otherwise also hoist all 2^ds - 1 products
            // out of it and hold them in registers across it.
            if constexpr (kPrefetch) {
                opaque(p1);
                opaque(p2);
                opaque(p3);
                opaque(p4);
                opaque(p8);
                opaque(p16);
            }
            apply_powers<0, ds>(v, p1, p2, p3, p4, p8, p16);
        }
    }

    // v[R] *= base^c, c = bitrev(R's digit bits) known at compile time; bits of
    // R above the digit (only in a short last digit) are earlier digits.
    template <int R, int DS>
    static __device__ __forceinline__ void apply_powers(float2 (&v)[kE], float2 p1, float2 p2, float2 p3, float2 p4,
                                                        float2 p8, float2 p16) {
        constexpr int c = int(brev_const(std::uint32_t(R) & ((1u << DS) - 1u), DS));
        if constexpr (c != 0) {
            constexpr int lo = c & 7;
            float2 w;
            if constexpr (lo == 0) w = (c & 8) ? p8 : p16;
            else if constexpr (lo == 1) w = p1;
            else if constexpr (lo == 2) w = p2;
            else if constexpr (lo == 3) w = p3;
            else if constexpr (lo == 4) w = p4;
            else if constexpr (lo == 5) w = cmul(p4, p1);
            else if constexpr (lo == 6) w = cmul(p4, p2);
            else w = cmul(p4, p3);
            if constexpr (lo != 0 && (c & 8)) w = cmul(p8, w);
            if constexpr ((c & 16) && (lo != 0 || (c & 8))) w = cmul(p16, w);
            v[R] = cmul(v[R], w);
        }
        if constexpr (R + 1 < kE) apply_powers<R + 1, DS>(v, p1, p2, p3, p4, p8, p16);
    }

    // `between` runs after this wave's LDS writes, before the barrier.
    // RELABEL: the reading threads take the last phase's relabelled
    // positions (last_thread_index).
    template <int FROM, int TO, bool RELABEL = false, class Between>
    static __device__ __forceinline__ void exchange(float2 (&v)[kE], float2* lds, std::uint32_t t,
                                                    Between&& between) {
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kE; ++r) lds[L::split(index<FROM>(t, 0), index<FROM>(0, r))] = v[r];
        between();
        lds_barrier();
        const std::uint32_t it = RELABEL ? last_thread_index(t) : index<TO>(t, 0);
#pragma unroll
        for (int r = 0; r < kE; ++r) v[r] = lds[L::split(it, index<TO>(0, r))];
    }

    // One-row 5-bit tiles store their results straight from registers. The
    // last phase holds tile positions 0-4 in registers (p = thread part |
    // r), and its threads are relabelled so that for every register the 64
    // lanes of a wave hold 64 consecutive outputs (output k = bitrev(p)):
    // lane bits 0-3 take position bits LT-2..LT-5 (output bits 1-4), lane
    // bit 4 position bit LT-1 (output bit 0), lane bit 5 position bit LT-6
    // (output bit 5), the wave index bits 5 and up. Each store instruction
    // then writes 512 contiguous bytes, and the final LDS round trip is gone
    // (C3b 55.9-56.1 -> 54.5-54.7 us against the paired stores through LDS).
    // The relabelled reads keep every 16-lane group on 16 distinct bank
    // pairs of the XOR image: its lanes vary position bits LT-5..LT-2, the
    // image's second key field.
    static constexpr bool kDirectStore = SINGLE && LI == 0 && ORD == 0 && DB == 5;
    static __device__ __forceinline__ std::uint32_t last_thread_index(std::uint32_t t) {
        const std::uint32_t l = t & 63u, w = t >> 6;
        return ((l & 1u) << (LT - 2)) | (((l >> 1) & 1u) << (LT - 3)) | (((l >> 2) & 1u) << (LT - 4)) |
               (((l >> 3) & 1u) << (LT - 5)) | (((l >> 4) & 1u) << (LT - 1)) | (((l >> 5) & 1u) << (LT - 6)) |
               (w << 5);
    }

    struct Tile {
        std::uint32_t row0;  // ROW: first global row (= transform for one pass)
        std::uint32_t c0;    // COL: first column
        std::uint64_t base;  // COL: the tile's transform
    };

    static __device__ __forceinline__ Tile decode(const FftArgs& a, std::uint32_t tile, std::uint32_t m) {
        Tile tl{};
        if constexpr (COL) {
            const std::uint32_t shift = a.l2 - LI;
            tl.c0 = (tile & ((1u << shift) - 1u)) << LI;
            tl.base = tile >> shift;
        } else {
            tl.row0 = tile << LI;
        }
        return tl;
    }

    // Uniform base of the tile's span in a buffer whose transforms lie
    // `pitch` elements apart, and the 32-bit element offset of tile element i
    // on the natural (load) side.
    static __device__ __forceinline__ std::uint64_t span_base(const FftArgs& a, const Tile& tl, std::uint64_t pitch) {
        if constexpr (COL) return tl.base * pitch;
        else if constexpr (SINGLE) return std::uint64_t(tl.row0) * pitch;
        else return std::uint64_t((tl.row0 >> LI) >> (a.l1 - LI)) * pitch;  // the transform of the tile's rows
    }
    static __device__ __forceinline__ std::uint32_t natural_offset(const FftArgs& a, const Tile& tl, std::uint32_t i) {
        if constexpr (COL) {
            return tl.c0 + (i & ((1u << LI) - 1u)) + ((i >> LI) << a.l2);
        } else if constexpr (SINGLE) {  // rows are consecutive transforms of 2^LT points
            if constexpr ((ORD & 1) != 0) {  // element x of a row sits at bitrev(x)
                const std::uint32_t x = i & ((1u << LT) - 1u);
                return (i - x) | brev(x, LT);
            }
            return i;
        } else if constexpr ((ORD & 4) != 0) {  // rows k0 + rr of a row-major block, in natural order
            const std::uint32_t k0 = tl.row0 & ((1u << a.l1) - 1u);
            return ((k0 + (i >> LT)) << a.l2) + (i & ((1u << LT) - 1u));
        } else {  // rows bitrev(k0 + rr) of one transform, matching the transposing store
            const std::uint32_t k0 = tl.row0 & ((1u << a.l1) - 1u);
            return (brev(k0 + (i >> LT), a.l1) << a.l2) + (i & ((1u << LT) - 1u));
        }
    }

    // Bytes of the tile's span: a one-pass tile's existing rows (the range
    // check zero-fills loads and drops stores past them), else its transform.
    static __device__ __forceinline__ std::uint32_t span_bytes(const FftArgs& a, const Tile& tl, std::uint32_t m) {
        if constexpr (SINGLE) return min(1u << LI, a.rows - tl.row0) << (LT + 3);
        else return 8u << m;
    }

    // Element offsets split into a per-thread part and a wave-uniform
    // per-register part: natural_offset is a sum over disjoint index bit
    // fields (row bit reversal included, as k0 is a multiple of 2^LI), and
    // the tile origin enters only the thread part. A partial one-pass tile
    // keeps the whole offset in the lane offset, which the range check sees.
    static constexpr bool kLaneOnly = SINGLE && LI > 0;
    // One-pass tiles read the caller's input once: nontemporal loads (C3b
    // 56.2-56.3 -> 55.6-55.8 us). Multi-pass tiles keep the default policy
    // (their later passes read the intermediate back from the caches; C3a
    // measured slower with nontemporal loads).
    static constexpr int kLoadAux = SINGLE ? 2 : 0;
    // (Two-pass register offsets depend on l1 / l2 at run time, so the choice
    // is a wave-uniform branch there; keeping small offsets in the lane offset
    // measured faster than always using the scalar offset.)
    static __device__ __forceinline__ float2 load_at(__amdgpu_buffer_rsrc_t src, std::uint32_t lane_bytes,
                                                     std::uint32_t reg_bytes) {
        if (kLaneOnly || reg_bytes < 4096u) return buffer_load<float2, kLoadAux>(src, lane_bytes + reg_bytes);
        return buffer_load<float2, kLoadAux>(src, lane_bytes, reg_bytes);
    }
    // Final-pass stores (the caller's output, written once) are nontemporal
    // where a wave's stores form segments of at least 512 bytes: one-pass
    // rows, and transposing row passes with 2^6 or more rows per tile (C3a:
    // 168.7 -> 156.4 us; on the 32-byte segments of 4096-point transposing
    // rows the hint measured 2.6x slower). Column passes write the
    // intermediate the next pass reads (nontemporal there: C3a 183 us).
    static constexpr int kStoreAux = !COL && (SINGLE || LI >= 6 || (ORD & 40) != 0) ? 2 : 0;
    static __device__ __forceinline__ void store_at(float2 x, __amdgpu_buffer_rsrc_t dst, std::uint32_t lane_bytes,
                                                    std::uint32_t reg_bytes) {
        if (kLaneOnly || reg_bytes < 4096u) buffer_store<float2, kStoreAux>(x, dst, lane_bytes + reg_bytes);
        else buffer_store<float2, kStoreAux>(x, dst, lane_bytes, reg_bytes);
    }
    // Two consecutive outputs as one 16-byte store.
    static __device__ __forceinline__ void store2_at(float2 x0, float2 x1, __amdgpu_buffer_rsrc_t dst,
                                                     std::uint32_t lane_bytes, std::uint32_t reg_bytes) {
        const float4 x = make_float4(x0.x, x0.y, x1.x, x1.y);
        if (kLaneOnly || reg_bytes < 4096u) buffer_store<float4, kStoreAux>(x, dst, lane_bytes + reg_bytes);
        else buffer_store<float4, kStoreAux>(x, dst, lane_bytes, reg_bytes);
    }

    // Column tiles of 64 columns (a wave's width) move two neighbouring
    // columns per lane and access: 16-byte loads and stores, half as many
    // instructions (C3a 147 -> 138.5 us for the loads alone at equal bytes).
    // Lane l of a wave holds logical column 2 (l mod 32) + l / 32, i.e. the
    // tile's logical thread index is logical_thread(threadIdx.x), and all
    // index maps use it. Register pair (2k, 2k + 1) of a column tile's
    // digit-0 layout is rows x = w + 16 (2k) and w + 16 (2k + 1) (w: the
    // wave's transform bits). Lanes 0-31 load row 2k and lanes 32-63 row
    // 2k + 1 of columns 2c, 2c + 1 (c = l mod 32); v_permlane32_swap of the
    // two column values (a 2 x 2 transpose of lane bit 5 with the column bit)
    // leaves each lane both rows of its own column. The stores run the same
    // transpose backwards on the last digit's register pairs.
    static __device__ __forceinline__ std::uint32_t logical_thread(std::uint32_t tid) {
        if constexpr (kPairedColumns) return (tid & ~63u) | (2u * (tid & 31u)) | ((tid >> 5) & 1u);
        else return tid;
    }
    static __device__ __forceinline__ void swap_halves(float2& a, float2& b) {
        const auto re = __builtin_amdgcn_permlane32_swap(__float_as_uint(a.x), __float_as_uint(b.x), false, false);
        const auto im = __builtin_amdgcn_permlane32_swap(__float_as_uint(a.y), __float_as_uint(b.y), false, false);
        a = make_float2(__uint_as_float(re[0]), __uint_as_float(im[0]));
        b = make_float2(__uint_as_float(re[1]), __uint_as_float(im[1]));
    }
    // Byte offset (from the span) of columns 2c, 2c + 1 of tile row x, lane l.
    static __device__ __forceinline__ std::uint32_t pair_column_bytes(const FftArgs& a, const Tile& tl, std::uint32_t l,
                                                                      std::uint32_t x) {
        return (tl.c0 + 2u * (l & 31u) + (x << a.l2)) * 8u;
    }

    // Registers [R0, R1) of a tile. `valid` false: an empty buffer range, so
    // every load returns zero without touching memory (keeps a prefetch
    // unconditional, see step()).
    template <int R0 = 0, int R1 = kE>
    static __device__ __forceinline__ void load(const FftArgs& a, const Tile& tl, std::uint32_t t, std::uint32_t m,
                                                float2 (&v)[kE], bool valid = true) {
        constexpr int w0 = tile_window<0>();
        const __amdgpu_buffer_rsrc_t src =
            make_rsrc(a.in + span_base(a, tl, a.in_pitch), valid ? span_bytes(a, tl, m) : 0u);
        if constexpr (kPairedColumns) {
            static_assert(R0 % 2 == 0 && R1 % 2 == 0, "register pairs");
            static_assert(w0 == LI + 4, "digit 0 holds the top four of eight row bits");
            const std::uint32_t l = threadIdx.x & 63u, h = l >> 5, w = t >> 6;
#pragma unroll
            for (int k = R0 / 2; k < R1 / 2; ++k) {
                const std::uint32_t x = w | ((2u * std::uint32_t(k) + h) << 4);
                const auto q = __builtin_amdgcn_raw_buffer_load_b128(
                    src, static_cast<int>(pair_column_bytes(a, tl, l, x)), 0, 0);
                float2 e = make_float2(__uint_as_float(q[0]), __uint_as_float(q[1]));
                float2 o = make_float2(__uint_as_float(q[2]), __uint_as_float(q[3]));
                swap_halves(e, o);
                v[2 * k] = e;
                v[2 * k + 1] = o;
            }
            return;
        }
        const std::uint32_t tb = natural_offset(a, tl, index<w0>(t, 0)) * 8u;
#pragma unroll
        for (int r = R0; r < R1; ++r) v[r] = load_at(src, tb, natural_offset(a, Tile{}, index<w0>(0, r)) * 8u);
    }

    static __device__ __forceinline__ void bases_of(float2 (&bs)[3], const FftArgs& a, std::uint32_t t,
                                                    std::uint32_t c0, std::uint32_t m) {
        bs[0] = level_base<0>(a, t, c0, m);
        if constexpr (kPhases > 1) bs[1] = level_base<1>(a, t, c0, m);
        if constexpr (kPhases > 2) bs[2] = level_base<2>(a, t, c0, m);
    }
    static_assert(kPhases <= 4, "at most four digits per pass");

    // `at(K)` (K an std::integral_constant) runs at hook point K: 2P right
    // after digit P, 2P + 1 between this wave's LDS writes and the barrier of
    // the exchange that follows digit P (for the last digit, the final
    // store's; a column pass has none and runs it before its stores). Every
    // point 0 .. 2 kPhases - 1 runs once per tile. The persistent walk issues
    // slices of the next tile's loads there.
    template <class At>
    static __device__ __forceinline__ void process(const FftArgs& a, const Tile& tl, std::uint32_t t, std::uint32_t m,
                                                   float2 (&v)[kE], const float2 (&bs)[3], float2* lds, At&& at) {
        using std::integral_constant;
        digit<0>(v, bs[0]);
        at(integral_constant<int, 0>{});
        if constexpr (kPhases > 1) {
            exchange<tile_window<0>(), tile_window<1>()>(v, lds, t, [&] { at(integral_constant<int, 1>{}); });
            digit<1>(v, bs[1]);
            at(integral_constant<int, 2>{});
        }
        if constexpr (kPhases > 2) {
            static_assert(!kDirectStore || kPhases == 3, "the relabelled phase is the last of three");
            exchange<tile_window<1>(), tile_window<2>(), kDirectStore>(v, lds, t,
                                                                     [&] { at(integral_constant<int, 3>{}); });
            digit<2>(v, bs[2]);
            at(integral_constant<int, 4>{});
        }
        if constexpr (kPhases > 3) {
            // A fourth digit (4-bit digits over 13 or 14 bits) fetches its
            // base here, keeping the bases held across the tile to three.
            exchange<tile_window<2>(), tile_window<3>()>(v, lds, t, [&] { at(integral_constant<int, 5>{}); });
            digit<3>(v, level_base<3>(a, t, tl.c0, m));
            at(integral_constant<int, 6>{});
        }
        constexpr int wl = tile_window<kPhases - 1>();
        const __amdgpu_buffer_rsrc_t dst = make_rsrc(a.out + span_base(a, tl, a.out_pitch), span_bytes(a, tl, m));
        if constexpr (COL) {  // intermediate: same positions
            at(integral_constant<int, 2 * kPhases - 1>{});
            if constexpr (kPairedColumns) {
                // Last digit: register r is row x = r + 16 w'; after the
                // transpose lanes 0-31 hold row 2k, lanes 32-63 row 2k + 1,
                // of columns 2c and 2c + 1.
                static_assert(wl == LI, "the last digit holds the low four of eight row bits");
                const std::uint32_t l = threadIdx.x & 63u, h = l >> 5, w = t >> 6;
#pragma unroll
                for (int k = 0; k < kE / 2; ++k) {
                    float2 e = v[2 * k], o = v[2 * k + 1];
                    swap_halves(e, o);
                    const std::uint32_t x = (2u * std::uint32_t(k) + h) | (w << 4);
                    buffer_store<float4, kStoreAux>(make_float4(e.x, e.y, o.x, o.y), dst,
                                                    pair_column_bytes(a, tl, l, x));
                }
                return;
            }
            const std::uint32_t tb = natural_offset(a, tl, index<wl>(t, 0)) * 8u;
#pragma unroll
            for (int r = 0; r < kE; ++r) store_at(v[r], dst, tb, natural_offset(a, Tile{}, index<wl>(0, r)) * 8u);
            return;
        }
        if constexpr (kDirectStore) {
            static_assert(wl == 0, "registers hold tile positions 0-4");
            at(integral_constant<int, 2 * kPhases - 1>{});
            const std::uint32_t kt = brev(last_thread_index(t), LT) * 8u;
            if (a.scale == 1.0f) {
#pragma unroll
                for (int r = 0; r < kE; ++r) store_at(v[r], dst, kt, brev_const(std::uint32_t(r), LT) * 8u);
            } else {
#pragma unroll
                for (int r = 0; r < kE; ++r)
                    store_at(make_float2(v[r].x * a.scale, v[r].y * a.scale), dst, kt,
                             brev_const(std::uint32_t(r), LT) * 8u);
            }
            return;
        }
        // Final pass: bit-reversed positions -> natural order through LDS.
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kE; ++r) lds[L::split(index<wl>(t, 0), index<wl>(0, r))] = v[r];
        at(integral_constant<int, 2 * kPhases - 1>{});
        lds_barrier();
        if constexpr (kPairedStore) {
            store_pairs(a, t, lds, dst);
            return;
        }
        std::uint32_t it, ot;
        staged(a, tl, t, it, ot);
        // Unnormalised plans (scale 1) skip the products: a wave-uniform
        // branch over two copies of the store loop.
        if (a.scale == 1.0f) {
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                std::uint32_t ir, orr;
                staged(a, Tile{}, T * std::uint32_t(r), ir, orr);
                store_at(lds[L::split(it, ir)], dst, ot * 8u, orr * 8u);
            }
        } else {
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                std::uint32_t ir, orr;
                staged(a, Tile{}, T * std::uint32_t(r), ir, orr);
                const float2 x = lds[L::split(it, ir)];
                store_at(make_float2(x.x * a.scale, x.y * a.scale), dst, ot * 8u, orr * 8u);
            }
        }
    }

    // One-row tiles store pairs of neighbouring outputs, one 16-byte store per
    // lane: pair j = t + T r (r < kE / 2) holds outputs 2j and 2j + 1, read
    // from LDS at their tile indices (bit-reversed, or as they are for a
    // bit-reversed output order). The index of 2j splits into a thread part
    // (2t) and a register part (2 T r) over disjoint bits, and output 2j + 1
    // differs from it in one bit that is clear in both parts: the top one
    // after bit reversal, bit 0 otherwise.
    static constexpr bool kPairedStore = SINGLE && LI == 0;
    static __device__ __forceinline__ std::uint32_t pair_index(std::uint32_t g) {
        return (ORD & 2) != 0 ? g : brev(g, LT);
    }
    static __device__ __forceinline__ void store_pairs(const FftArgs& a, std::uint32_t t, const float2* lds,
                                                       __amdgpu_buffer_rsrc_t dst) {
        static_assert(L::kXor, "the thread / register split of a pair's index needs the XOR-linear image");
        constexpr std::uint32_t kSecond = (ORD & 2) != 0 ? 1u : 1u << (LT - 1);
        const std::uint32_t it = pair_index(2u * t), ot = 2u * t;
        // Unnormalised plans (scale 1) skip the products: a wave-uniform
        // branch over two copies of the store loop.
        if (a.scale == 1.0f) {
#pragma unroll
            for (int r = 0; r < kE / 2; ++r) {
                const std::uint32_t ir = pair_index(2u * T * std::uint32_t(r));
                const float2 x0 = lds[L::split(it, ir)], x1 = lds[L::split(it, ir | kSecond)];
                store2_at(x0, x1, dst, ot * 8u, 2u * T * std::uint32_t(r) * 8u);
            }
        } else {
#pragma unroll
            for (int r = 0; r < kE / 2; ++r) {
                const std::uint32_t ir = pair_index(2u * T * std::uint32_t(r));
                const float2 x0 = lds[L::split(it, ir)], x1 = lds[L::split(it, ir | kSecond)];
                store2_at(make_float2(x0.x * a.scale, x0.y * a.scale), make_float2(x1.x * a.scale, x1.y * a.scale),
                          dst, ot * 8u, 2u * T * std::uint32_t(r) * 8u);
            }
        }
    }

    // Final-store enumeration of element g (physical contiguity order): its
    // tile index i and its offset in the span. Both are sums over disjoint
    // bit fields of g (so g = t + T r splits into thread and register parts).
    static __device__ __forceinline__ void staged(const FftArgs& a, const Tile& tl, std::uint32_t g, std::uint32_t& i,
                                                  std::uint32_t& off) {
        if constexpr (SINGLE) {  // rows are transforms: in-row bit reversal, lanes along the row
            const std::uint32_t xp = g & ((1u << LT) - 1u), rr = g >> LT;
            // Bit-reversed output order is the DIF result's own order.
            i = ((ORD & 2) != 0 ? xp : brev(xp, LT)) | (rr << LT);
            off = (rr << LT) + xp;
        } else if constexpr ((ORD & 8) != 0) {  // tile rows bitrev(k0 + rr) land on rows k0 + rr
            const std::uint32_t xp = g & ((1u << LT) - 1u), rr = g >> LT;
            const std::uint32_t k0 = tl.row0 & ((1u << a.l1) - 1u);
            i = brev(xp, LT) | (rr << LT);
            off = ((k0 + rr) << LT) + xp;
        } else if constexpr ((ORD & 32) != 0) {  // bit-reversed output: rows go back where they were read
            const std::uint32_t xp = g & ((1u << LT) - 1u), rr = g >> LT;
            const std::uint32_t k0 = tl.row0 & ((1u << a.l1) - 1u);
            i = xp | (rr << LT);
            off = (brev(k0 + rr, a.l1) << LT) + xp;
        } else {  // grid transpose: tile rows are bitrev(k0 + rr) of one transform
            const std::uint32_t rr = g & ((1u << LI) - 1u), cp = g >> LI;
            const std::uint32_t k0 = tl.row0 & ((1u << a.l1) - 1u);
            i = brev(cp, LT) | (rr << LT);
            off = (cp << a.l1) + k0 + rr;
        }
    }

    // Persistent walk over tiles: the next tile's loads are issued before the
    // current tile is processed, and no global load sits between them and
    // their use (level-twiddle bases are fetched before the prefetch). When
    // the tile count and the grid are multiples of 8, each XCD (blocks are
    // dealt to the 8 XCDs round-robin) walks one contiguous range of tiles,
    // so tiles sharing cache lines meet in one L2.
    static __device__ void run(const FftArgs& a) {
        extern __shared__ float2 lds[];
        const std::uint32_t t = logical_thread(threadIdx.x);
        const std::uint32_t m = a.l1 + a.l2;
        const std::uint32_t grid = gridDim.x, b = blockIdx.x;
        const bool xcd = (a.tiles & 7u) == 0 && (grid & 7u) == 0;
        const std::uint32_t stride = xcd ? (grid >> 3) : grid;
        const std::uint32_t range_base = xcd ? (b & 7u) * (a.tiles >> 3) : 0u;
        const std::uint32_t range_end = xcd ? (a.tiles >> 3) : a.tiles;
        std::uint32_t pos = xcd ? (b >> 3) : b;
        if (pos >= range_end) return;
        Tile tl = decode(a, range_base + pos, m);
        float2 bs[3];
        if constexpr (!COL) {
            bases_of(bs, a, t, 0, m);  // row passes: the bases depend on the thread only
            // Finish the bases before the first tile's loads: registers of
            // their table loads would otherwise still be pending where the
            // tile loop begins, and the loop's waits (merged over its entry
            // and its back edge) would wait for the prefetch as well.
            if constexpr (kPrefetch) __builtin_amdgcn_sched_barrier(0);
        }
        float2 v[kE];
        load(a, tl, t, m, v);
        if constexpr (!kPrefetch) {  // one tile per workgroup (the grid covers every tile)
            if constexpr (COL) bases_of(bs, a, t, tl.c0, m);
            process(a, tl, t, m, v, bs, lds, [](auto) {});
            return;
        }
        // Two register buffers in turn (unrolled by two), so no tile is
        // copied between registers: a copy would make the wait for its loads
        // also wait for the prefetch issued after them.
        float2 w[kE];
        if constexpr (kDeep) {  // three buffers in turn, two tiles ahead
            Tile t1 = decode(a, range_base + pos + stride, m);
            load(a, t1, t, m, w, pos + stride < range_end);
            float2 x[kE];
            for (;;) {
                if (!step2(a, t, m, pos, stride, range_base, range_end, tl, t1, bs, v, w, x, lds)) break;
                if (!step2(a, t, m, pos, stride, range_base, range_end, tl, t1, bs, w, x, v, lds)) break;
                if (!step2(a, t, m, pos, stride, range_base, range_end, tl, t1, bs, x, v, w, lds)) break;
            }
            return;
        }
        for (;;) {
            if (!step(a, t, m, pos, stride, range_base, range_end, tl, bs, v, w, lds)) break;
            if (!step(a, t, m, pos, stride, range_base, range_end, tl, bs, w, v, lds)) break;
        }
    }
    // Column passes with 4-bit digits walk two tiles ahead: the tile after
    // `next` (already loading) is prefetched into a third buffer `far`, so a
    // workgroup keeps two tiles of loads in flight (123 VGPRs, within the
    // 128 of 4 waves per SIMD; C3a 141.0-141.5 -> 138.7 us, its first pass
    // reading from HBM). The row passes would spill with a third buffer, and
    // the 5-bit one-row tiles have no room for it.
    static constexpr bool kDeep = COL && DB == 4;
    // One tile of the depth-two walk (see step): prefetch the tile two ahead
    // into `far` in the same slices, process `cur`; `next` stays allocated
    // throughout, as `cur` does through its stores. Returns whether the
    // following tile exists; `tl_next` is the tile in `next`.
    static __device__ __forceinline__ bool step2(const FftArgs& a, std::uint32_t t, std::uint32_t m, std::uint32_t& pos,
                                                 std::uint32_t stride, std::uint32_t range_base,
                                                 std::uint32_t range_end, Tile& tl, Tile& tl_next, float2 (&bs)[3],
                                                 float2 (&cur)[kE], float2 (&next)[kE], float2 (&far)[kE], float2* lds) {
        std::uint32_t tt = t;
        asm volatile("" : "+v"(tt));
        const std::uint32_t following = pos + stride, ahead = pos + 2 * stride;
        const bool more = following < range_end, more2 = ahead < range_end;
        if constexpr (COL) bases_of(bs, a, tt, tl.c0, m);
        const Tile tf = decode(a, range_base + ahead, m);
        load<0, slice_end(0)>(a, tf, tt, m, far, more2);
        __builtin_amdgcn_sched_barrier(0);
        process(a, tl, tt, m, cur, bs, lds, [&](auto point) {
            constexpr int K = decltype(point)::value;
            if constexpr (slice_at(K)) {
                constexpr int S = slice_before(K) + 1;
                __builtin_amdgcn_sched_barrier(0);
                load<slice_end(S - 1), slice_end(S)>(a, tf, tt, m, far, more2);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
#pragma unroll
        for (int r = 0; r < kE; ++r) opaque(cur[r]);
#pragma unroll
        for (int r = 0; r < kE; ++r) opaque(next[r]);
        pos = following;
        tl = tl_next;
        tl_next = tf;
        return more;
    }

    // Hook points of process() that issue a prefetch slice: inside each
    // exchange, after this wave's LDS writes (measured against right after
    // each digit: C3a 150.3-150.6 -> 147.2-148.5 us, C3b 65.0-65.6 ->
    // 64.1-64.3 us; both sets: 148.2-148.6 / 64.2-64.5 us). Slice 0 goes out
    // before digit 0; slice S covers registers [slice_end(S - 1), slice_end(S)),
    // whole register pairs.
    static constexpr unsigned kSliceMask = kPhases == 2 ? 0b1010u : kPhases == 3 ? 0b101010u : 0b10101010u;
    static constexpr bool slice_at(int k) { return (kSliceMask >> k) & 1u; }
    static constexpr int slice_before(int k) {  // slices issued at hook points below k
        int c = 0;
        for (int j = 0; j < k; ++j) c += slice_at(j) ? 1 : 0;
        return c;
    }
    static constexpr int kSlices = 1 + slice_before(2 * kPhases);
    static constexpr int slice_end(int s) { return 2 * ((s + 1) * (kE / 2) / kSlices); }  // register pairs

    // One tile of the persistent walk: prefetch the next tile into `next`,
    // process the current one from `cur`. Returns whether a next tile exists.
    static __device__ __forceinline__ bool step(const FftArgs& a, std::uint32_t t, std::uint32_t m, std::uint32_t& pos,
                                                std::uint32_t stride, std::uint32_t range_base,
                                                std::uint32_t range_end, Tile& tl, float2 (&bs)[3],
                                                float2 (&cur)[kE], float2 (&next)[kE], float2* lds) {
        // Per-thread addresses depend on t only; hiding t from the optimiser
        // here keeps them from being hoisted out of the loop (and held in
        // registers across it).
        std::uint32_t tt = t;
        asm volatile("" : "+v"(tt));
        const std::uint32_t following = pos + stride;
        const bool more = following < range_end;
        if constexpr (COL) bases_of(bs, a, tt, tl.c0, m);
        // The prefetch is issued even past the last tile (as empty-range
        // loads): a branch around it would leave the compiler's wait for
        // `cur` merging a path without the prefetch, and it would then wait
        // for the prefetch too.
        const Tile tn = decode(a, range_base + following, m);
        // The prefetch goes out in kPhases + 1 slices: the first before digit
        // 0, one inside each exchange (the last in the final store's), so a
        // tile's loads do not all queue in the address unit at once (all
        // before digit 0: C3b 70.4 us, C3a 156.5 us; sliced: 64.1 / 147.2 us). No instruction moves across the slice
        // boundaries, so every use of `cur` comes after the first slice is
        // issued: the wait for `cur` then counts the prefetch as younger and
        // does not wait for it (or for the previous tile's stores).
        load<0, slice_end(0)>(a, tn, tt, m, next, more);
        __builtin_amdgcn_sched_barrier(0);
        process(a, tl, tt, m, cur, bs, lds, [&](auto point) {
            constexpr int K = decltype(point)::value;
            if constexpr (slice_at(K)) {
                constexpr int S = slice_before(K) + 1;
                __builtin_amdgcn_sched_barrier(0);
                load<slice_end(S - 1), slice_end(S)>(a, tn, tt, m, next, more);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
        // Keep `cur`'s registers allocated through the stores: otherwise the
        // stores take their data from them, and the next prefetch into them
        // would first wait for those stores.
#pragma unroll
        for (int r = 0; r < kE; ++r) opaque(cur[r]);
        pos = following;
        tl = tn;
        return more;
    }
};

template <int LT, int LI, bool COL, bool SINGLE, bool INV, int ORD>
__global__ __launch_bounds__(1 << (LT + LI - pass_digit_bits(LT + LI, SINGLE, ORD)))
__attribute__((amdgpu_waves_per_eu(pass_digit_bits(LT + LI, SINGLE, ORD) == 5 ? 2 : 4))) void fft_pass_kernel(FftArgs a) {
    FftPass<LT, LI, COL, SINGLE, INV, ORD>::run(a);
}

using Launch = void (*)(const FftArgs&, hipStream_t);

struct Key {
    int lt, li;
    bool col, single, inv;
    int ord = 0;
    bool operator<(const Key& o) const {
        return std::tie(lt, li, col, single, inv, ord) < std::tie(o.lt, o.li, o.col, o.single, o.inv, o.ord);
    }
};

// Prefetching passes run a persistent grid: as many workgroups as can be
// resident (occupancy of this kernel with its LDS), at most one per tile, a
// multiple of 8 when larger. Other passes launch one workgroup per tile.
template <int LT, int LI, bool COL, bool SINGLE, bool INV, int ORD>
void launch(const FftArgs& a, hipStream_t stream) {
    constexpr std::uint32_t bytes =
        FftLds<COL, LT, LI, SINGLE, false, FftPass<LT, LI, COL, SINGLE, INV, ORD>::DB>::kWords * sizeof(float2);
    constexpr int threads = int(FftPass<LT, LI, COL, SINGLE, INV, ORD>::T);
    static const std::uint64_t resident = [] {
        const void* fn = reinterpret_cast<const void*>(&fft_pass_kernel<LT, LI, COL, SINGLE, INV, ORD>);
        if (bytes > 65536 && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)) != hipSuccess)
            (void)hipGetLastError();
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, bytes) != hipSuccess || per_cu < 1) {
            (void)hipGetLastError();
            per_cu = 1;
        }
        return std::uint64_t(per_cu) * std::uint64_t(device_cu_count());
    }();
    std::uint64_t grid = a.tiles;
    if (FftPass<LT, LI, COL, SINGLE, INV, ORD>::kPrefetch) {
        grid = std::min<std::uint64_t>(grid, resident);
        if (grid > 8) grid &= ~std::uint64_t{7};
    }
    hipLaunchKernelGGL((fft_pass_kernel<LT, LI, COL, SINGLE, INV, ORD>), dim3(unsigned(grid)), dim3(threads), bytes, stream, a);
}

std::map<Key, Launch>& registry() {
    static std::map<Key, Launch> table;
    return table;
}

template <int LT, int LI, bool COL, bool SINGLE>
void add() {
    registry()[Key{LT, LI, COL, SINGLE, false}] = &launch<LT, LI, COL, SINGLE, false, 0>;
    registry()[Key{LT, LI, COL, SINGLE, true}] = &launch<LT, LI, COL, SINGLE, true, 0>;
    if constexpr (SINGLE) {  // bit-reversed logical orders of one-pass tiles
        registry()[Key{LT, LI, COL, SINGLE, false, 1}] = &launch<LT, LI, COL, SINGLE, false, 1>;
        registry()[Key{LT, LI, COL, SINGLE, true, 1}] = &launch<LT, LI, COL, SINGLE, true, 1>;
        registry()[Key{LT, LI, COL, SINGLE, false, 2}] = &launch<LT, LI, COL, SINGLE, false, 2>;
        registry()[Key{LT, LI, COL, SINGLE, true, 2}] = &launch<LT, LI, COL, SINGLE, true, 2>;
        registry()[Key{LT, LI, COL, SINGLE, false, 3}] = &launch<LT, LI, COL, SINGLE, false, 3>;
        registry()[Key{LT, LI, COL, SINGLE, true, 3}] = &launch<LT, LI, COL, SINGLE, true, 3>;
    }
    if constexpr (!COL && !SINGLE) {  // final row passes writing the bit-reversed order
        registry()[Key{LT, LI, COL, SINGLE, false, 32}] = &launch<LT, LI, COL, SINGLE, false, 32>;
        registry()[Key{LT, LI, COL, SINGLE, true, 32}] = &launch<LT, LI, COL, SINGLE, true, 32>;
    }
}

// Shapes: one pass for m <= 14 (2^12-point tiles, 2^13 / 2^14 for m = 13,
// 14); two passes with 2^14-point tiles over l1 = m / 2 high bits (column
// tiles) and l2 = m - l1 low bits (row tiles). The even split keeps both the
// column reads and the transposing row stores in segments of 2^(14 - m/2)
// elements (32 bytes at m = 24); a column-heavier split would leave the
// transposing store with single-element segments.
constexpr int single_li(int m) { return m < 12 ? 12 - m : 0; }
constexpr int split_l1(int m) { return m / 2; }
constexpr int col_lines(int l1, int l2) { return 14 - l1 < l2 ? 14 - l1 : l2; }
constexpr int row_lines(int l1, int l2) { return 14 - l2 < l1 ? 14 - l2 : l1; }
template <int M>
void add_two() {
    constexpr int l1 = split_l1(M), l2 = M - l1;
    add<l1, col_lines(l1, l2), true, false>();
    add<l2, row_lines(l1, l2), false, false>();
}

// Row passes over natural-order rows with the transposing store, tiles of
// 2^14 points (2^(14 - LT) rows, at least 4 so the transposed segments are
// 32 bytes or longer).
template <int LT>
void add_rows_natural() {
    registry()[Key{LT, 14 - LT, false, false, false, 4}] = &launch<LT, 14 - LT, false, false, false, 4>;
    registry()[Key{LT, 14 - LT, false, false, true, 4}] = &launch<LT, 14 - LT, false, false, true, 4>;
}

// Rank-2 blocks: column passes of 2^LT points over whole 2^14-point tiles,
// and rows written back in natural order in 2^12-point tiles (a quarter of
// the LDS each, so four workgroups per CU overlap one another's loads and
// butterflies where the rows of 2^9 points and more have no prefetching walk).
template <int LT>
void add_rank2_rows() {
    registry()[Key{LT, 12 - LT, false, false, false, 8}] = &launch<LT, 12 - LT, false, false, false, 8>;
    registry()[Key{LT, 12 - LT, false, false, true, 8}] = &launch<LT, 12 - LT, false, false, true, 8>;
}

void register_all() {
    add<1, single_li(1), false, true>();
    add<2, single_li(2), false, true>();
    add<3, single_li(3), false, true>();
    add<4, single_li(4), false, true>();
    add<5, single_li(5), false, true>();
    add<6, single_li(6), false, true>();
    add<7, single_li(7), false, true>();
    add<8, single_li(8), false, true>();
    add<9, single_li(9), false, true>();
    add<10, single_li(10), false, true>();
    add<11, single_li(11), false, true>();
    add<12, single_li(12), false, true>();
    add<13, 0, false, true>();
    add<14, 0, false, true>();
    for (bool inv : {false, true}) {
        registry()[Key{13, 0, false, true, inv, 16}] = inv ? &launch<13, 0, false, true, true, 16>
                                                           : &launch<13, 0, false, true, false, 16>;
        registry()[Key{14, 0, false, true, inv, 16}] = inv ? &launch<14, 0, false, true, true, 16>
                                                           : &launch<14, 0, false, true, false, 16>;
    }
    add_two<15>();
    add_two<16>();
    add_two<17>();
    add_two<18>();
    add_two<19>();
    add_two<20>();
    add_two<21>();
    add_two<22>();
    add_two<23>();
    add_two<24>();
    add_rows_natural<4>();
    add_rows_natural<5>();
    add_rows_natural<6>();
    add_rows_natural<7>();
    add_rows_natural<8>();
    add_rows_natural<9>();
    add_rows_natural<10>();
    add_rows_natural<11>();
    add_rows_natural<12>();
    add<4, 10, true, false>();
    add<5, 9, true, false>();
    add<6, 8, true, false>();
    add_rank2_rows<8>();
    add_rank2_rows<9>();
    add_rank2_rows<10>();
    add_rank2_rows<11>();
    add_rank2_rows<12>();
}

Launch lookup(const Key& k) {
    static std::once_flag once;
    std::call_once(once, register_all);
    auto it = registry().find(k);
    return it == registry().end() ? nullptr : it->second;
}

Launch find(const Key& k) {
    const Launch fn = lookup(k);
    if (fn == nullptr) throw NotSupported("FFT pass shape has no gfx950 kernel");
    return fn;
}

// The final row pass's order flag: 32 for a bit-reversed output order.
int row_ord(const Request& r) { return r.output_bit_reversed ? 32 : 0; }

// A two-pass split l1 + l2 = m whose column and row kernels both exist.
bool split_available(int m, int l1, bool inverse, int ord = 0) {
    const int l2 = m - l1;
    return l1 >= 1 && l2 >= 1 && l1 <= 14 && l2 <= 14 &&
           lookup(Key{l1, col_lines(l1, l2), true, false, inverse}) != nullptr &&
           lookup(Key{l2, row_lines(l1, l2), false, false, inverse, ord}) != nullptr;
}

constexpr const char* kTwoPassName = "fft-c64-two-pass-r16";

std::string two_pass_name(int m, int l1) {
    if (l1 == split_l1(m)) return kTwoPassName;
    return std::string(kTwoPassName) + "-" + std::to_string(l1) + "x" + std::to_string(m - l1);
}

// Column bits of a two-pass variant name, or -1 when the name is not one.
int parse_split(int m, const std::string& name) {
    if (name == kTwoPassName) return split_l1(m);
    const std::string prefix = std::string(kTwoPassName) + "-";
    if (name.compare(0, prefix.size(), prefix) != 0) return -1;
    unsigned a = 0, b = 0;
    char tail = 0;
    if (std::sscanf(name.c_str() + prefix.size(), "%ux%u%c", &a, &b, &tail) != 2) return -1;
    return int(a + b) == m && two_pass_name(m, int(a)) == name ? int(a) : -1;
}

// Three-pass lowering a + b + c = m (top, middle, low index bits): a column
// pass over the top a bits (2^(b + c) columns), the column pass of the
// batched 2^(b + c)-point transforms over the middle b bits (its level
// twiddles are those of the full transform: a DIF digit's twiddle depends
// only on the bits below it), and the row pass of a (a + b) x c split. Every
// pass moves segments of 2^min(14 - bits, ...) elements (512 bytes at
// 8 + 8 + 8), where the two-pass 12 + 12 split moves 32-byte segments.
bool split3_available(int m, int a, int b, bool inverse, int ord = 0) {
    const int c = m - a - b;
    return a >= 1 && b >= 1 && c >= 1 && a <= 14 && b <= 14 && c <= 14 &&
           lookup(Key{a, col_lines(a, b + c), true, false, inverse}) != nullptr &&
           lookup(Key{b, col_lines(b, c), true, false, inverse}) != nullptr &&
           lookup(Key{c, row_lines(a + b, c), false, false, inverse, ord}) != nullptr;
}

std::string three_pass_name(int m, int a, int b) {
    return "fft-c64-three-pass-r16-" + std::to_string(a) + "x" + std::to_string(b) + "x" + std::to_string(m - a - b);
}

// Top and middle bits of a three-pass name, or false.
bool parse_split3(int m, const std::string& name, int& a, int& b) {
    const std::string prefix = "fft-c64-three-pass-r16-";
    if (name.compare(0, prefix.size(), prefix) != 0) return false;
    unsigned x = 0, y = 0, z = 0;
    char tail = 0;
    if (std::sscanf(name.c_str() + prefix.size(), "%ux%ux%u%c", &x, &y, &z, &tail) != 3) return false;
    a = int(x);
    b = int(y);
    return int(x + y + z) == m && three_pass_name(m, a, b) == name;
}

// The static model's three-pass choice: from 2^23 points, where the
// two-pass split's segments drop to 32 or 64 bytes (measured on MI355X:
// 2^24 x 1 in 171 us against 199 us, 2^23 x 2 in 164 us against 188 us),
// a = m / 3 top bits and half the rest in the middle.
bool default_three_pass(int m, bool inverse, int& a, int& b, int ord = 0) {
    if (m < 23) return false;
    a = m / 3;
    b = (m - a) / 2;
    return split3_available(m, a, b, inverse, ord);
}

// Level-twiddle tables of a 2^log_len-point transform: A[k] = w^(4096 k),
// B[k] = w^k, w = exp(-+2 pi i / 2^log_len), from double.
void upload_twiddles(DeviceBuffer& a, DeviceBuffer& b, int log_len, bool inverse) {
    std::vector<float2> ta(4096), tb(4096);
    const double sign = inverse ? 1.0 : -1.0;
    const double n = std::ldexp(1.0, log_len);
    for (int k = 0; k < 4096; ++k) {
        const double fa = std::fmod(4096.0 * k, n), fb = std::fmod(double(k), n);
        ta[k] = make_float2(float(std::cos(2 * M_PI * fa / n)), float(sign * std::sin(2 * M_PI * fa / n)));
        tb[k] = make_float2(float(std::cos(2 * M_PI * fb / n)), float(sign * std::sin(2 * M_PI * fb / n)));
    }
    a.upload(ta);
    b.upload(tb);
}

// Name suffix of a one-pass plan with bit-reversed logical orders.
std::string order_suffix(const Request& r) {
    return std::string(r.input_bit_reversed ? "-bitrev-in" : "") + (r.output_bit_reversed ? "-bitrev-out" : "");
}

class FftExecutor final : public Executor {
  public:
    // split: column bits of a two-pass lowering (0: one pass); mid > 0: the
    // middle bits of a three-pass lowering with `split` top bits; radix16: a
    // one-pass tile of 2^13 / 2^14 points with 4-bit digits.
    FftExecutor(const Request& r, int split, int mid = 0, bool radix16 = false) : r_(r) {
        const std::uint32_t m = r.log_n;
        supported(m >= 1 && m <= 24, "complex FFT lengths above 2^24 are not yet lowered for gfx950");
        upload_twiddles(twa_, twb_, int(m), r.inverse);
        const float scale = r.normalize ? 1.0f / float(r.n) : 1.0f;
        require(r.batch <= 0xffffffffull, "FFT batch exceeds 2^32 transforms");
        FftArgs base{};
        base.twa = twa_.as<float2>();
        base.twb = twb_.as<float2>();
        base.scale = scale;
        const std::uint64_t in_pitch = r.pitched ? r.in_batch_stride : r.n;
        const std::uint64_t out_pitch = r.pitched ? r.out_batch_stride : r.n;
        if (mid > 0) {
            const std::uint32_t ta = std::uint32_t(split), tm = std::uint32_t(mid), tl = m - ta - tm;
            upload_twiddles(sub_twa_, sub_twb_, int(tm + tl), r.inverse);
            const int a_li = col_lines(int(ta), int(tm + tl));
            const int b_li = col_lines(int(tm), int(tl));
            const int c_li = row_lines(int(ta + tm), int(tl));
            const std::uint64_t a_tiles = r.batch << (tm + tl - a_li);
            const std::uint64_t b_tiles = (r.batch << ta) << (tl - b_li);
            const std::uint64_t c_tiles = r.batch << (ta + tm - c_li);
            require(a_tiles <= 0xffffffffull && b_tiles <= 0xffffffffull && c_tiles <= 0xffffffffull,
                    "FFT batch exceeds the grid");
            Step sa{find(Key{int(ta), a_li, true, false, r.inverse}), base, false, true};
            sa.args.l1 = ta;
            sa.args.l2 = tm + tl;
            sa.args.rows = unsigned(r.batch << ta);
            sa.args.tiles = unsigned(a_tiles);
            sa.args.scale = 1.0f;
            sa.args.in_pitch = in_pitch;
            sa.args.out_pitch = r.n;
            // The middle pass sees 2^top batched transforms of 2^(mid + low)
            // points, in place in the workspace, with their own tables.
            Step sb{find(Key{int(tm), b_li, true, false, r.inverse}), base, true, true};
            sb.args.twa = sub_twa_.as<float2>();
            sb.args.twb = sub_twb_.as<float2>();
            sb.args.l1 = tm;
            sb.args.l2 = tl;
            sb.args.rows = unsigned((r.batch << ta) << tm);
            sb.args.tiles = unsigned(b_tiles);
            sb.args.scale = 1.0f;
            sb.args.in_pitch = sb.args.out_pitch = std::uint64_t{1} << (tm + tl);
            Step sc{find(Key{int(tl), c_li, false, false, r.inverse, row_ord(r)}), base, true, false};
            sc.args.l1 = ta + tm;
            sc.args.l2 = tl;
            sc.args.rows = unsigned(r.batch << (ta + tm));
            sc.args.tiles = unsigned(c_tiles);
            sc.args.in_pitch = r.n;
            sc.args.out_pitch = out_pitch;
            steps_ = {sa, sb, sc};
            workspace_ = static_cast<std::size_t>(r.batch << m) * sizeof(float2);
            algorithm = three_pass_name(int(m), split, mid);
        } else if (split == 0) {
            const int li = single_li(int(m));
            const std::uint64_t tiles = (r.batch + (1ull << li) - 1) >> li;
            const int ord = (r.input_bit_reversed ? 1 : 0) | (r.output_bit_reversed ? 2 : 0) | (radix16 ? 16 : 0);
            Step s{find(Key{int(m), li, false, true, r.inverse, ord}), base, false, false};
            s.args.l1 = 0;
            s.args.l2 = m;
            s.args.rows = unsigned(r.batch);
            s.args.tiles = unsigned(tiles);
            s.args.in_pitch = in_pitch;
            s.args.out_pitch = out_pitch;
            steps_.push_back(s);
            algorithm = m >= 13 && !radix16 ? "fft-c64-resident-r32" : "fft-c64-resident-r16";
        } else {
            const std::uint32_t l1 = std::uint32_t(split), l2 = m - l1;
            const int col_li = col_lines(int(l1), int(l2));
            const int row_li = row_lines(int(l1), int(l2));
            const std::uint64_t col_tiles = r.batch << (l2 - col_li);
            const std::uint64_t row_tiles = r.batch << (l1 - row_li);
            require(col_tiles <= 0xffffffffull && row_tiles <= 0xffffffffull, "FFT batch exceeds the grid");
            Step a{find(Key{int(l1), col_li, true, false, r.inverse}), base, false, true};
            a.args.l1 = l1;
            a.args.l2 = l2;
            a.args.rows = unsigned(r.batch << l1);
            a.args.tiles = unsigned(col_tiles);
            a.args.scale = 1.0f;
            a.args.in_pitch = in_pitch;
            a.args.out_pitch = r.n;  // the workspace is packed
            Step b{find(Key{int(l2), row_li, false, false, r.inverse, row_ord(r)}), base, true, false};
            b.args.l1 = l1;
            b.args.l2 = l2;
            b.args.rows = unsigned(r.batch << l1);
            b.args.tiles = unsigned(row_tiles);
            b.args.in_pitch = r.n;
            b.args.out_pitch = out_pitch;
            steps_ = {a, b};
            workspace_ = static_cast<std::size_t>(r.batch << m) * sizeof(float2);
            algorithm = two_pass_name(int(m), int(l1));
        }
        algorithm += order_suffix(r);
        if (r.pitched) algorithm += "-pitched";
        reason = "decimation in frequency: in-register radix-16 codelets (radix-32 for one-pass 2^13 and 2^14), "
                 "level twiddles from two 4096-entry tables, LDS-staged bit-reversal (and grid transpose) on the "
                 "final store";
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("operator", "fft")
            .field("algorithm", algorithm)
            .field("log_n", m)
            .field("batch", r.batch)
            .field("direction", r.inverse ? "inverse" : "forward")
            .field("passes", unsigned(steps_.size()))
            .field("column_bits", unsigned(split))
            .field("middle_bits", unsigned(mid))
            .field("workspace_bytes", std::uint64_t(workspace_))
            .end_object();
        mapping_json = w.str();
    }
    std::size_t workspace_bytes() const override { return workspace_; }
    void execute(const void* in, void* out, void* ws, hipStream_t stream) override {
        require(steps_.size() < 2 || ws != nullptr, "two-pass FFT needs a workspace");
        for (const auto& s : steps_) {
            FftArgs a = s.args;
            a.in = static_cast<const float2*>(s.reads_ws ? ws : in);
            a.out = static_cast<float2*>(s.writes_ws ? ws : out);
            s.fn(a, stream);
            hip_check(hipGetLastError(), "FFT pass launch");
        }
    }

  private:
    struct Step {
        Launch fn;
        FftArgs args;
        bool reads_ws, writes_ws;
    };
    Request r_;
    DeviceBuffer twa_, twb_, sub_twa_, sub_twb_;
    std::vector<Step> steps_;
    std::size_t workspace_ = 0;
};

}  // namespace

std::unique_ptr<Executor> make_fft_executor(const Request& r) {
    const int m = int(r.log_n);
    supported(m >= 1 && m <= 24, "complex FFT lengths above 2^24 are not yet lowered for gfx950");
    require(!r.pitched || single_li(m) == 0, "pitched FFT rows need n >= 2^12 (one transform per tile)");
    require(!r.input_bit_reversed || m <= 14, "bit-reversed FFT input is native to one-pass lengths only");
    // Order and pitch suffixes ride on every candidate name.
    std::string variant = r.variant;
    const std::string suffix = order_suffix(r) + (r.pitched ? "-pitched" : "");
    if (!variant.empty() && !suffix.empty()) {
        supported(variant.size() > suffix.size() &&
                      variant.compare(variant.size() - suffix.size(), suffix.size(), suffix) == 0,
                  "'" + r.variant + "' is not a lowering of this FFT");
        variant.resize(variant.size() - suffix.size());
    }
    if (m <= 14) {
        // 2^13 / 2^14 points: radix-32 tiles by default, radix-16 by name
        // (natural orders only).
        const bool radix16 = m >= 13 && variant == "fft-c64-resident-r16";
        supported(variant.empty() || radix16 || variant == (m >= 13 ? "fft-c64-resident-r32" : "fft-c64-resident-r16"),
                  "'" + r.variant + "' is not a lowering of this FFT");
        supported(!radix16 || !(r.input_bit_reversed || r.output_bit_reversed),
                  "radix-16 tiles of 2^13 / 2^14 points take natural orders only");
        return std::make_unique<FftExecutor>(r, 0, 0, radix16);
    }
    int top = 0, mid = 0;
    if (variant.empty() && default_three_pass(m, r.inverse, top, mid, row_ord(r)))
        return std::make_unique<FftExecutor>(r, top, mid);
    if (parse_split3(m, variant, top, mid)) {
        supported(split3_available(m, top, mid, r.inverse, row_ord(r)),
                  "'" + r.variant + "' is not a lowering of this FFT");
        return std::make_unique<FftExecutor>(r, top, mid);
    }
    const int split = variant.empty() ? split_l1(m) : parse_split(m, variant);
    supported(split > 0 && split_available(m, split, r.inverse, row_ord(r)),
              "'" + r.variant + "' is not a lowering of this FFT");
    return std::make_unique<FftExecutor>(r, split);
}

namespace {

// FFTs of the rows of row-major 2^l1 x 2^l2 blocks, each block's result
// written transposed (2^l2 x 2^l1): one row pass over natural-order rows.
class FftRowsTransposedExecutor final : public Executor {
  public:
    FftRowsTransposedExecutor(const Request& r, std::uint32_t l1, Launch fn) : fn_(fn) {
        const std::uint32_t l2 = r.log_n;
        const int li = 14 - int(l2);
        // The row kernel forms level twiddles as powers of the 2^(l1 + l2)-th
        // root (w^(j << (m - h)) = the 2^h-th root's j-th power).
        upload_twiddles(twa_, twb_, int(l1 + l2), r.inverse);
        const std::uint64_t blocks = r.batch >> l1;
        const std::uint64_t tiles = blocks << (l1 - std::uint32_t(li));
        require(tiles <= 0xffffffffull && r.batch <= 0xffffffffull, "FFT batch exceeds the grid");
        args_ = FftArgs{};
        args_.twa = twa_.as<float2>();
        args_.twb = twb_.as<float2>();
        args_.l1 = l1;
        args_.l2 = l2;
        args_.rows = unsigned(r.batch);
        args_.tiles = unsigned(tiles);
        args_.scale = r.normalize ? 1.0f / float(r.n) : 1.0f;
        args_.in_pitch = args_.out_pitch = std::uint64_t{1} << (l1 + l2);
        algorithm = "fft-c64-rows-transposed-r16";
        reason = "row transforms of 2^" + std::to_string(l1) + " x 2^" + std::to_string(l2) +
                 " blocks with the transposing store of the two-pass row kernel";
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("operator", "fft")
            .field("algorithm", algorithm)
            .field("log_n", l2)
            .field("block_rows_log", l1)
            .field("blocks", blocks)
            .field("direction", r.inverse ? "inverse" : "forward")
            .end_object();
        mapping_json = w.str();
    }
    void execute(const void* in, void* out, void*, hipStream_t stream) override {
        FftArgs a = args_;
        a.in = static_cast<const float2*>(in);
        a.out = static_cast<float2*>(out);
        fn_(a, stream);
        hip_check(hipGetLastError(), "FFT pass launch");
    }

  private:
    Launch fn_;
    FftArgs args_{};
    DeviceBuffer twa_, twb_;
};

// Rank-2 FFTs of row-major 2^l0 x 2^l1 blocks (r.n = 2^(l0 + l1) points per
// block, r.batch blocks): the axis-0 transform as one or two column passes
// over each block (the low l1 bits of their column index number
// independent transforms, FftArgs::cbits), then the rows: each row pass tile
// gathers rows from the column passes' bit-reversed axis-0 order and writes
// them back transformed, in natural order. Every pass reads and writes whole
// segments of 2^(14 - t) columns or whole rows, where the transposing row
// passes of the same blocks move 2^(14 - l1)-element segments.
class FftRank2ColumnsExecutor final : public Executor {
  public:
    FftRank2ColumnsExecutor(const Request& r, std::uint32_t l0, std::uint32_t ta, std::uint32_t tb) {
        const std::uint32_t l1 = r.log_n - l0;
        upload_twiddles(twa_, twb_, int(r.log_n), r.inverse);
        FftArgs base{};
        base.twa = twa_.as<float2>();
        base.twb = twb_.as<float2>();
        base.scale = 1.0f;
        const std::uint64_t n = r.n;
        // First column pass: the top ta bits of axis 0, columns = the rest of
        // the block (tb axis-0 bits, then l1 bits that are not transformed).
        {
            const int li = 14 - int(ta);
            Step s{find(Key{int(ta), li, true, false, r.inverse}), base, false, true};
            s.args.l1 = ta;
            s.args.l2 = tb + l1;
            s.args.cbits = l1;
            s.args.rows = unsigned(r.batch << ta);
            s.args.tiles = unsigned(r.batch << (tb + l1 - std::uint32_t(li)));
            s.args.in_pitch = s.args.out_pitch = n;
            steps_.push_back(s);
        }
        if (tb > 0) {
            // Second column pass, in place: 2^ta transforms of 2^tb points per
            // block, each over 2^l1 columns; its own tables (level twiddles
            // of a 2^(tb + l1)-point span).
            upload_twiddles(sub_twa_, sub_twb_, int(tb + l1), r.inverse);
            const int li = 14 - int(tb);
            Step s{find(Key{int(tb), li, true, false, r.inverse}), base, true, true};
            s.args.twa = sub_twa_.as<float2>();
            s.args.twb = sub_twb_.as<float2>();
            s.args.l1 = tb;
            s.args.l2 = l1;
            s.args.cbits = l1;
            s.args.rows = unsigned((r.batch << ta) << tb);
            s.args.tiles = unsigned((r.batch << ta) << (l1 - std::uint32_t(li)));
            s.args.in_pitch = s.args.out_pitch = std::uint64_t{1} << (tb + l1);
            steps_.push_back(s);
        }
        {
            const int li = 12 - int(l1);
            Step s{find(Key{int(l1), li, false, false, r.inverse, 8}), base, true, false};
            s.args.l1 = l0;
            s.args.l2 = l1;
            s.args.rows = unsigned(r.batch << l0);
            s.args.tiles = unsigned(r.batch << (l0 - std::uint32_t(li)));
            s.args.scale = r.normalize ? 1.0f / float(n) : 1.0f;
            s.args.in_pitch = s.args.out_pitch = n;
            steps_.push_back(s);
        }
        workspace_ = static_cast<std::size_t>(r.batch * n) * sizeof(float2);
        algorithm = "fft-c64-rank2-columns-r16";
        reason = "axis 0 (2^" + std::to_string(l0) + ") as " + (tb > 0 ? "two column passes" : "one column pass") +
                 " over each block, then the 2^" + std::to_string(l1) + "-point rows, stored in natural order";
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("operator", "fft")
            .field("algorithm", algorithm)
            .field("log_n", r.log_n)
            .field("axis0_bits", l0)
            .field("column_passes", tb > 0 ? 2u : 1u)
            .field("blocks", r.batch)
            .field("direction", r.inverse ? "inverse" : "forward")
            .field("workspace_bytes", std::uint64_t(workspace_))
            .end_object();
        mapping_json = w.str();
    }
    std::size_t workspace_bytes() const override { return workspace_; }
    void execute(const void* in, void* out, void* ws, hipStream_t stream) override {
        require(ws != nullptr, "a rank-2 column plan needs its workspace");
        for (const auto& s : steps_) {
            FftArgs a = s.args;
            a.in = static_cast<const float2*>(s.reads_ws ? ws : in);
            a.out = static_cast<float2*>(s.writes_ws ? ws : out);
            s.fn(a, stream);
            hip_check(hipGetLastError(), "FFT pass launch");
        }
    }

  private:
    struct Step {
        Launch fn;
        FftArgs args;
        bool reads_ws, writes_ws;
    };
    DeviceBuffer twa_, twb_, sub_twa_, sub_twb_;
    std::vector<Step> steps_;
    std::size_t workspace_ = 0;
};

}  // namespace

bool fft_rows_transposed_available(const Request& r, std::uint32_t l1) {
    const int l2 = int(r.log_n);
    // Level-twiddle tables reach 2^24-th roots (so l1 + l2 <= 24, which also
    // keeps a block's byte offsets in 32 bits).
    return l2 >= 4 && l2 <= 12 && int(l1) >= 14 - l2 && l1 + std::uint32_t(l2) <= 24 &&
           (r.batch & ((std::uint64_t{1} << l1) - 1)) == 0 &&
           lookup(Key{l2, 14 - l2, false, false, r.inverse, 4}) != nullptr;
}

std::unique_ptr<Executor> make_fft_rows_transposed(const Request& r, std::uint32_t l1) {
    if (!fft_rows_transposed_available(r, l1)) return nullptr;
    const int l2 = int(r.log_n);
    return std::make_unique<FftRowsTransposedExecutor>(r, l1, lookup(Key{l2, 14 - l2, false, false, r.inverse, 4}));
}

// The column-pass split of axis 0 (ta top bits, then tb; tb = 0 for one
// pass), or false where no kernels cover the shape: rows of 2^8 .. 2^12
// points (whole 2^14-point row tiles within a block), blocks of at most 2^24
// points (the level-twiddle tables' reach), and axis 0 in one column pass of
// 4 .. 8 bits or two: the second over tb >= 14 - l1 bits (its 2^(14 - tb)
// columns within the 2^l1 of a row), the first over the rest, each within
// 4 .. 8 bits.
bool rank2_columns_split(const Request& r, std::uint32_t l0, std::uint32_t& ta, std::uint32_t& tb) {
    const std::uint32_t m = r.log_n;
    if (l0 < 4 || l0 >= m) return false;
    const std::uint32_t l1 = m - l0;
    if (l1 < 8 || l1 > 12 || m > 24 || l0 < 14 - l1) return false;
    ta = l0;
    tb = 0;
    if (l0 > 8) {
        tb = std::max(l0 / 2, 14 - l1);
        ta = l0 - tb;
        if (tb > 8 || ta < 4 || ta > 8) return false;
    }
    return r.batch <= (0xffffffffull >> l0);
}

bool fft_rank2_columns_available(const Request& r, std::uint32_t l0) {
    std::uint32_t ta = 0, tb = 0;
    return rank2_columns_split(r, l0, ta, tb);
}

std::unique_ptr<Executor> make_fft_rank2_columns(const Request& r, std::uint32_t l0) {
    std::uint32_t ta = 0, tb = 0;
    if (!rank2_columns_split(r, l0, ta, tb)) return nullptr;
    return std::make_unique<FftRank2ColumnsExecutor>(r, l0, ta, tb);
}

// One-pass lengths have one lowering; two-pass lengths add the neighbouring
// column / row splits whose kernels exist.
std::vector<std::string> fft_candidates(const Request& r) {
    const int m = int(r.log_n);
    const std::string suffix = order_suffix(r) + (r.pitched ? "-pitched" : "");
    if (m <= 14) {
        std::vector<std::string> names{std::string(m >= 13 ? "fft-c64-resident-r32" : "fft-c64-resident-r16") + suffix};
        if (m >= 13 && !(r.input_bit_reversed || r.output_bit_reversed))
            names.push_back("fft-c64-resident-r16" + suffix);
        return names;
    }
    std::vector<std::string> names;
    int top = 0, mid = 0;
    const int ord = row_ord(r);
    const bool three = default_three_pass(m, r.inverse, top, mid, ord);
    if (three) names.push_back(three_pass_name(m, top, mid) + suffix);
    if (split_available(m, split_l1(m), r.inverse, ord)) names.push_back(two_pass_name(m, split_l1(m)) + suffix);
    for (int l1 : {split_l1(m) - 1, split_l1(m) + 1, split_l1(m) - 2, split_l1(m) + 2})
        if (split_available(m, l1, r.inverse, ord)) names.push_back(two_pass_name(m, l1) + suffix);
    // Three passes from 2^18: splits within one bit of m / 3 per pass.
    if (m >= 18)
        for (int a = m / 3 - 1; a <= m / 3 + 1; ++a)
            for (int b = m / 3 - 1; b <= m / 3 + 1; ++b)
                if (std::abs(m - a - b - m / 3) <= 1 && split3_available(m, a, b, r.inverse, ord) &&
                    !(three && a == top && b == mid))
                    names.push_back(three_pass_name(m, a, b) + suffix);
    return names;
}

}  // namespace cbw
