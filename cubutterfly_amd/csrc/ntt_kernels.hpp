// Device code of the NTT engine: the templated pass kernel, Shoup arithmetic
// and the registry of instantiated pass shapes. Included by ntt.hip (host side)
// and by the ntt_u{32,64}_{lazy,strict}.hip translation units, which
// instantiate the kernels in parallel builds.
#pragma once

#include <hip/hip_runtime.h>

#include "ntt_engine.hpp"

#include <map>
#include <tuple>

namespace cbw {
namespace ntt_detail {

constexpr int kLE = 4;
constexpr int kE = 1 << kLE;

template <class W>
struct alignas(2 * sizeof(W)) TwPair {
    W w, wp;
};

template <class W>
struct DeviceDomain {
    W q, q2, rwp;         // modulus, 2q, floor(2^k / q) (Shoup factor of 1)
    TwPair<W> ninv;       // n^-1 with its Shoup factor
    TwPair<W> last;       // Tinv[1] * n^-1 (final inverse stage)
    std::uint64_t tw;     // offset of this domain's table (entries 1..n-1) in PassArgs::tw
};

template <class W>
struct PassArgs {
    const W* in;
    W* out;
    const DeviceDomain<W>* domains;
    const TwPair<W>* tw;               // all domains' twiddle tables, concatenated
    const std::uint32_t* poly_domain;  // per polynomial (null: domain 0)
    const std::uint64_t* in_off;       // per polynomial word offset (null: p << log n)
    const std::uint64_t* out_off;
    std::uint32_t l1, l2;  // high / low index bits of the two-pass split (l1 = 0: one pass)
    std::uint32_t polys, tiles;
    std::uint32_t reduce_input;
};

__device__ __forceinline__ std::uint32_t mulhi(std::uint32_t a, std::uint32_t b) { return __umulhi(a, b); }
__device__ __forceinline__ std::uint64_t mulhi(std::uint64_t a, std::uint64_t b) { return __umul64hi(a, b); }

// x - m if x >= m else x (x < 2m).
__device__ __forceinline__ std::uint32_t csub(std::uint32_t x, std::uint32_t m) { return min(x, x - m); }
__device__ __forceinline__ std::uint64_t csub(std::uint64_t x, std::uint64_t m) { return x >= m ? x - m : x; }

template <class W>
__device__ __forceinline__ W shoup(W a, W w, W wp, W q) {
    return a * w - mulhi(a, wp) * q;  // [0, 2q) for any a
}

template <class W, bool LAZY>
__device__ __forceinline__ void ct_butterfly(W& x, W& y, TwPair<W> t, W q, W q2) {
    if constexpr (LAZY) {  // x, y in [0, 4q)
        const W u = csub(x, q2);
        const W v = shoup(y, t.w, t.wp, q);
        x = u + v;
        y = u - v + q2;
    } else {  // x, y in [0, 2q)
        const W u = csub(x, q);
        const W v = csub(shoup(y, t.w, t.wp, q), q);
        x = u + v;
        y = u - v + q;
    }
}

template <class W, bool LAZY>
__device__ __forceinline__ void gs_butterfly(W& x, W& y, TwPair<W> t, W q, W q2) {
    if constexpr (LAZY) {  // x, y in [0, 2q)
        const W u = x, v = y;
        x = csub(u + v, q2);
        y = shoup(u - v + q2, t.w, t.wp, q);
    } else {
        const W u = csub(x, q), v = csub(y, q);
        x = u + v;
        y = shoup(u - v + q, t.w, t.wp, q);
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
    x = shoup(u + v, d.ninv.w, d.ninv.wp, d.q);
    y = shoup(u - v + span, d.last.w, d.last.wp, d.q);
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ std::uint32_t brev(std::uint32_t x, std::uint32_t bits) {
    return bits ? __brev(x) >> (32 - bits) : 0u;
}

// Tile index of (thread t, register r) when registers span tile bits [S, S+4).
template <int S>
__device__ __forceinline__ std::uint32_t phase_index(std::uint32_t t, std::uint32_t r) {
    const std::uint32_t lo = t & ((1u << S) - 1u);
    return lo | (r << S) | ((t >> S) << (S + kLE));
}

// Padded / swizzled LDS image of a tile (bank-conflict avoidance for the
// phase layouts and for the lane-over-line staged transposes).
template <bool COL, int LT, int LI>
struct Lds {
    static constexpr std::uint32_t kWords =
        COL ? (1u << LT) * ((1u << LI) + 1u) : (1u << LI) * ((1u << LT) + (1u << LT >> 4) + 1u);
    static __device__ __forceinline__ std::uint32_t addr(std::uint32_t i) {
        if constexpr (COL) {
            const std::uint32_t cc = i & ((1u << LI) - 1u), x = i >> LI;
            return x * ((1u << LI) + 1u) + (cc ^ ((x >> 3) & ((1u << LI) - 1u)));
        } else {
            const std::uint32_t x = i & ((1u << LT) - 1u), rr = i >> LT;
            return rr * ((1u << LT) + (1u << LT >> 4) + 1u) + x + (x >> 4);
        }
    }
};

// Transform-relative window start of phase P.
template <int LT, bool CT, int P>
constexpr int window_start() {
    if constexpr (CT) {
        return LT - kLE * (P + 1) > 0 ? LT - kLE * (P + 1) : 0;
    } else {
        return kLE * P < LT - kLE ? kLE * P : (LT - kLE > 0 ? LT - kLE : 0);
    }
}

template <class W, bool LAZY, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE>
struct Pass {
    static constexpr int LB = LT + LI;
    static constexpr std::uint32_t T = 1u << (LB - kLE);
    static constexpr int kPhases = (LT + kLE - 1) / kLE;
    static constexpr bool kFirst = SINGLE || (COL == CT);
    static constexpr bool kLast = SINGLE || (COL != CT);
    // Rows of a permuted two-pass ROW tile are bitrev(k0 + rr).
    static constexpr bool kPermRows = !COL && !SINGLE && (PIN || POUT);
    using L = Lds<COL, LT, LI>;

    template <int P>
    static constexpr int tile_window() {
        return (COL ? LI : 0) + window_start<LT, CT, P>();
    }

    struct Tile {
        std::uint32_t poly;  // COL / two-pass ROW: the polynomial
        std::uint32_t c0;    // COL: first column
        std::uint32_t k0;    // ROW: first row (or bit-reversed row index)
        std::uint32_t l1, l2;
    };

    static __device__ __forceinline__ std::uint64_t base(const std::uint64_t* off, std::uint32_t p,
                                                         std::uint32_t log_n) {
        return off ? off[p] : std::uint64_t(p) << log_n;
    }

    // Logical row of line rr in a ROW tile.
    static __device__ __forceinline__ std::uint32_t row_of(const Tile& tl, std::uint32_t rr) {
        if constexpr (SINGLE) return 0;
        else if constexpr (kPermRows) return brev(tl.k0 + rr, tl.l1);
        else return tl.k0 + rr;
    }

    // Physical word (relative to the polynomial base) of tile element i, natural side.
    static __device__ __forceinline__ std::uint64_t natural_word(const Tile& tl, std::uint32_t i) {
        if constexpr (COL) {
            const std::uint32_t cc = i & ((1u << LI) - 1u), x = i >> LI;
            return tl.c0 + cc + (std::uint64_t(x) << tl.l2);
        } else {
            const std::uint32_t x = i & ((1u << LT) - 1u), rr = i >> LT;
            return (std::uint64_t(row_of(tl, rr)) << tl.l2) + x;
        }
    }

    // Staged (permuted) enumeration: element g of the tile in physical
    // contiguity order -> (tile index, polynomial, word within polynomial).
    static __device__ __forceinline__ void permuted(const Tile& tl, std::uint32_t g, std::uint32_t& i,
                                                    std::uint32_t& poly, std::uint64_t& word) {
        if constexpr (COL) {  // each column is a contiguous bit-reversed block of 2^l1 words
            const std::uint32_t rp = g & ((1u << LT) - 1u), cc = g >> LT;
            i = cc | (brev(rp, LT) << LI);
            poly = tl.poly;
            word = (std::uint64_t(brev(tl.c0 + cc, tl.l2)) << tl.l1) + rp;
        } else if constexpr (SINGLE) {  // in-row bit reversal, rows are polynomials
            const std::uint32_t xp = g & ((1u << LT) - 1u), rr = g >> LT;
            i = brev(xp, LT) | (rr << LT);
            poly = tl.poly + rr;
            word = xp;
        } else {  // rows bitrev(k0 + rr): lanes over rr are contiguous words
            const std::uint32_t rr = g & ((1u << LI) - 1u), cp = g >> LI;
            i = brev(cp, LT) | (rr << LT);
            poly = tl.poly;
            word = (std::uint64_t(cp) << tl.l1) + tl.k0 + rr;
        }
    }

    static __device__ __forceinline__ std::uint32_t poly_of(const Tile& tl, std::uint32_t i) {
        if constexpr (SINGLE) return tl.poly + (i >> LT);
        else return tl.poly;
    }

    template <int P>
    static __device__ __forceinline__ void stages(W (&v)[kE], const Tile& tl, std::uint32_t t,
                                                  const DeviceDomain<W>& d, const TwPair<W>* __restrict__ table) {
        constexpr int ws = window_start<LT, CT, P>();
        constexpr int tw0 = tile_window<P>();
        // Transform index and twiddle prefix of register 0 (window bits clear).
        // The prefix is 1 for columns and 2^l1 + row for rows; the row is the
        // same for all registers whenever LT >= 4 (and 0 for one-pass tiles).
        const std::uint32_t i0 = phase_index<tw0>(t, 0);
        const std::uint32_t x0 = COL ? (i0 >> LI) : (i0 & ((1u << LT) - 1u));
        const std::uint32_t prefix = COL ? 1u : ((1u << tl.l1) + row_of(tl, i0 >> LT));
        const std::uint32_t head = (prefix << LT) | x0;
#pragma unroll
        for (int s = 0; s < kLE; ++s) {
            // CT walks bits high -> low, GS low -> high; skip bits of other phases.
            const int k = CT ? (ws + kLE - 1 - s) : (ws + s);
            const bool mine = CT ? (k < LT - kLE * P && k >= 0) : (k >= kLE * P && k < LT);
            if (!mine || k >= LT) continue;
            const int jb = k - ws;
            // Group g (register bits above jb) uses twiddle (head >> (k+1)) + g;
            // register bits beyond the transform (LT < 4) do not index it.
            const std::uint32_t gmask = (1u << (LT - 1 - k)) - 1u;
            const TwPair<W>* __restrict__ tk = table + (head >> (k + 1));
            const bool scale_stage = kLast && !CT && k == LT - 1;
#pragma unroll
            for (int g = 0; g < (1 << (kLE - 1 - jb)); ++g) {
                TwPair<W> tw{};
                if (!scale_stage) tw = tk[std::uint32_t(g) & gmask];
#pragma unroll
                for (int lo = 0; lo < (1 << jb); ++lo) {
                    const int r = (g << (jb + 1)) | lo;
                    const int r2 = r | (1 << jb);
                    if constexpr (CT) {
                        ct_butterfly<W, LAZY>(v[r], v[r2], tw, d.q, d.q2);
                    } else if (scale_stage) {
                        gs_scale_butterfly<W, LAZY>(v[r], v[r2], d);
                    } else {
                        gs_butterfly<W, LAZY>(v[r], v[r2], tw, d.q, d.q2);
                    }
                }
            }
        }
    }

    template <int FROM, int TO>
    static __device__ __forceinline__ void exchange(W (&v)[kE], W* lds, std::uint32_t t) {
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kE; ++r) lds[L::addr(phase_index<FROM>(t, r))] = v[r];
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kE; ++r) v[r] = lds[L::addr(phase_index<TO>(t, r))];
    }

    static __device__ __forceinline__ Tile decode(const PassArgs<W>& a, std::uint32_t tile) {
        Tile tl{};
        tl.l1 = a.l1;
        tl.l2 = a.l2;
        if constexpr (COL) {
            const std::uint32_t shift = a.l2 - LI;
            tl.poly = tile >> shift;
            tl.c0 = (tile & ((1u << shift) - 1u)) << LI;
        } else if constexpr (SINGLE) {
            tl.poly = tile << LI;
        } else {
            const std::uint32_t shift = a.l1 - LI;
            tl.poly = tile >> shift;
            tl.k0 = (tile & ((1u << shift) - 1u)) << LI;
        }
        return tl;
    }

    // Word address and validity of register r's input element.
    static __device__ __forceinline__ void input_word(const PassArgs<W>& a, const Tile& tl, std::uint32_t t, int r,
                                                      std::uint64_t& where, bool& valid) {
        const std::uint32_t log_n = a.l1 + a.l2;
        std::uint32_t i, p;
        std::uint64_t word;
        if constexpr (PIN) {
            permuted(tl, t + T * r, i, p, word);
        } else {
            i = phase_index<tile_window<0>()>(t, r);
            p = poly_of(tl, i);
            word = natural_word(tl, i);
        }
        valid = !SINGLE || p < a.polys;
        where = (valid ? base(a.in_off, SINGLE ? p : tl.poly, log_n) : 0) + word;
    }

    // Issue the 16 loads of a tile (raw words; reduction happens later).
    static __device__ __forceinline__ void load_tile(const PassArgs<W>& a, const Tile& tl, std::uint32_t t,
                                                     W (&v)[kE]) {
        std::uint64_t where[kE];
        bool valid[kE];
#pragma unroll
        for (int r = 0; r < kE; ++r) input_word(a, tl, t, r, where[r], valid[r]);
#pragma unroll
        for (int r = 0; r < kE; ++r) v[r] = valid[r] ? a.in[where[r]] : W(0);
    }

    static __device__ __forceinline__ void process(const PassArgs<W>& a, const Tile& tl, std::uint32_t t, W (&v)[kE],
                                                   W* lds) {
        const std::uint32_t log_n = a.l1 + a.l2;
        // One domain per tile (the planner keeps mixed-domain tiles apart).
        const std::uint32_t dom = a.poly_domain ? a.poly_domain[tl.poly] : 0u;
        const DeviceDomain<W> d = a.domains[dom];
        // Kernel-argument pointers are known to address global memory, so the
        // twiddle gathers compile to global (not FLAT) loads.
        const TwPair<W>* __restrict__ table = a.tw + d.tw;
        if (kFirst && a.reduce_input) {
#pragma unroll
            for (int r = 0; r < kE; ++r) v[r] = shoup(v[r], W(1), d.rwp, d.q);
        }
        if constexpr (PIN) {
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                std::uint32_t i, p;
                std::uint64_t word;
                permuted(tl, t + T * r, i, p, word);
                lds[L::addr(i)] = v[r];
            }
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kE; ++r) v[r] = lds[L::addr(phase_index<tile_window<0>()>(t, r))];
        }

        stages<0>(v, tl, t, d, table);
        if constexpr (kPhases > 1) {
            exchange<tile_window<0>(), tile_window<1>()>(v, lds, t);
            stages<1>(v, tl, t, d, table);
        }
        if constexpr (kPhases > 2) {
            exchange<tile_window<1>(), tile_window<2>()>(v, lds, t);
            stages<2>(v, tl, t, d, table);
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
        const std::uint64_t out_tile = SINGLE ? 0 : base(a.out_off, tl.poly, log_n);
        std::uint64_t where[kE];
        bool valid[kE];
        if constexpr (POUT) {
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kE; ++r) lds[L::addr(phase_index<wl>(t, r))] = v[r];
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                std::uint32_t i, p;
                std::uint64_t word;
                permuted(tl, t + T * r, i, p, word);
                v[r] = lds[L::addr(i)];
                valid[r] = !SINGLE || p < a.polys;
                where[r] = (SINGLE ? (valid[r] ? base(a.out_off, p, log_n) : 0) : out_tile) + word;
            }
        } else {
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                const std::uint32_t i = phase_index<wl>(t, r);
                const std::uint32_t p = poly_of(tl, i);
                valid[r] = !SINGLE || p < a.polys;
                where[r] = (SINGLE ? (valid[r] ? base(a.out_off, p, log_n) : 0) : out_tile) + natural_word(tl, i);
            }
        }
#pragma unroll
        for (int r = 0; r < kE; ++r)
            if (valid[r]) a.out[where[r]] = v[r];
    }

    // Persistent walk over tiles: the next tile's loads are issued before the
    // current tile is processed. When the tile count and the grid are
    // multiples of 8, each XCD (blocks are dealt to the 8 XCDs round-robin)
    // walks one contiguous range of tiles, so tiles sharing cache lines and
    // twiddle rows meet in the same L2.
    static __device__ void run(const PassArgs<W>& a) {
        __shared__ W lds[L::kWords];
        const std::uint32_t t = threadIdx.x;
        const std::uint32_t grid = gridDim.x, b = blockIdx.x;
        const bool xcd = (a.tiles & 7u) == 0 && (grid & 7u) == 0;
        const std::uint32_t per_xcd = a.tiles >> 3, stride = xcd ? (grid >> 3) : grid;
        const std::uint32_t first = xcd ? (b >> 3) : b;  // position within this block's range
        const std::uint32_t range_base = xcd ? (b & 7u) * per_xcd : 0u;
        const std::uint32_t range_end = xcd ? per_xcd : a.tiles;

        std::uint32_t pos = first;
        if (pos >= range_end) return;
        Tile tl = decode(a, range_base + pos);
        W v[kE];
        load_tile(a, tl, t, v);
        for (;;) {
            const std::uint32_t next = pos + stride;
            const bool more = next < range_end;
            Tile tn{};
            W nv[kE];
            if (more) {
                tn = decode(a, range_base + next);
                load_tile(a, tn, t, nv);
            }
            process(a, tl, t, v, lds);
            if (!more) break;
            pos = next;
            tl = tn;
#pragma unroll
            for (int r = 0; r < kE; ++r) v[r] = nv[r];
        }
    }
};

template <class W, bool LAZY, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE>
__global__ __launch_bounds__(1 << (LT + LI - kLE)) void ntt_pass_kernel(PassArgs<W> a) {
    Pass<W, LAZY, LT, LI, COL, CT, PIN, POUT, SINGLE>::run(a);
}

// ---- launcher registry -----------------------------------------------------

template <class W>
using PassLaunch = void (*)(const PassArgs<W>&, unsigned grid, hipStream_t);

struct PassKey {
    bool lazy;
    int lt, li;
    bool col, ct, pin, pout, single;
    bool operator<(const PassKey& o) const {
        return std::tie(lazy, lt, li, col, ct, pin, pout, single) <
               std::tie(o.lazy, o.lt, o.li, o.col, o.ct, o.pin, o.pout, o.single);
    }
};

template <class W, bool LAZY, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE>
void launch_pass(const PassArgs<W>& a, unsigned grid, hipStream_t stream) {
    hipLaunchKernelGGL((ntt_pass_kernel<W, LAZY, LT, LI, COL, CT, PIN, POUT, SINGLE>), dim3(grid),
                       dim3(1u << (LT + LI - kLE)), 0, stream, a);
}

// One table per word type, filled once by the per-arithmetic translation units.
template <class W>
std::map<PassKey, PassLaunch<W>>& registry();
template <>
std::map<PassKey, PassLaunch<std::uint32_t>>& registry<std::uint32_t>();
template <>
std::map<PassKey, PassLaunch<std::uint64_t>>& registry<std::uint64_t>();

template <class W, bool LAZY, int LT, int LI, bool COL, bool CT, bool PIN, bool POUT, bool SINGLE>
void add() {
    registry<W>()[PassKey{LAZY, LT, LI, COL, CT, PIN, POUT, SINGLE}] =
        &launch_pass<W, LAZY, LT, LI, COL, CT, PIN, POUT, SINGLE>;
}

// Boundary-permutation variants of one pass shape: a first pass may permute
// its input, a last pass its output.
template <class W, bool LAZY, int LT, int LI, bool COL, bool CT, bool SINGLE>
void add_variants() {
    constexpr bool first = SINGLE || (COL == CT);
    constexpr bool last = SINGLE || (COL != CT);
    add<W, LAZY, LT, LI, COL, CT, false, false, SINGLE>();
    if constexpr (first) add<W, LAZY, LT, LI, COL, CT, true, false, SINGLE>();
    if constexpr (last) add<W, LAZY, LT, LI, COL, CT, false, true, SINGLE>();
    if constexpr (first && last) add<W, LAZY, LT, LI, COL, CT, true, true, SINGLE>();
}

template <class W, bool LAZY, int LT, int LB>
void add_single() {
    add_variants<W, LAZY, LT, LB - LT, false, true, true>();
    add_variants<W, LAZY, LT, LB - LT, false, false, true>();
}

// Two-pass split used by the planner: l1 = min(8, log n / 2) high bits.
constexpr int split_l1(int log_n) { return log_n / 2 < 8 ? log_n / 2 : 8; }
template <int LB>
constexpr int row_li(int l1, int l2) { return l1 < LB - l2 ? l1 : LB - l2; }

template <class W, bool LAZY, int LOG_N, int LB, int COL_LI>
void add_two_pass() {
    constexpr int l1 = split_l1(LOG_N), l2 = LOG_N - l1;
    constexpr int rli = row_li<LB>(l1, l2);
    add_variants<W, LAZY, l1, COL_LI, true, true, false>();
    add_variants<W, LAZY, l1, COL_LI, true, false, false>();
    add_variants<W, LAZY, l2, rli, false, true, false>();
    add_variants<W, LAZY, l2, rli, false, false, false>();
}

// Word-size specific shapes: 4 KiWord tiles; columns of 64 B (u32) / 128 B (u64).
template <class W, bool LAZY>
void register_all() {
    constexpr int LB = 12;
    constexpr int COL_LI = sizeof(W) == 4 ? 4 : 4;
    add_single<W, LAZY, 1, LB>();
    add_single<W, LAZY, 2, LB>();
    add_single<W, LAZY, 3, LB>();
    add_single<W, LAZY, 4, LB>();
    add_single<W, LAZY, 5, LB>();
    add_single<W, LAZY, 6, LB>();
    add_single<W, LAZY, 7, LB>();
    add_single<W, LAZY, 8, LB>();
    add_single<W, LAZY, 9, LB>();
    add_single<W, LAZY, 10, LB>();
    add_single<W, LAZY, 11, LB>();
    add_single<W, LAZY, 12, LB>();
    add_two_pass<W, LAZY, 13, LB, COL_LI>();
    add_two_pass<W, LAZY, 14, LB, COL_LI>();
    add_two_pass<W, LAZY, 15, LB, COL_LI>();
    add_two_pass<W, LAZY, 16, LB, COL_LI>();
    add_two_pass<W, LAZY, 17, LB, COL_LI>();
    add_two_pass<W, LAZY, 18, LB, COL_LI>();
    add_two_pass<W, LAZY, 19, LB, COL_LI>();
    add_two_pass<W, LAZY, 20, LB, COL_LI>();
}


void register_u32_lazy();
void register_u32_strict();
void register_u64_lazy();
void register_u64_strict();

}  // namespace ntt_detail
}  // namespace cbw
