// FWHT kernels for gfx950: FP32 storage, and FP16 storage with FP32 compute
// and one final RNE narrowing (the reference's final-storage contract,
// src/butterfly.cu:1452-1470, 1882-1897).
//
// Bit exactness. Each output is a fixed binary tree of fp32 additions, and the
// tree depends on the ORDER in which index bits are butterflied. The reference
// CPU oracle and its stage-ordered GPU kernels process bits 0, 1, ..., log n - 1
// (src/butterfly_reference.cpp:349-369, src/stage_pipeline.cuh:573-680), so
// these kernels do the same: phase p butterflies bits [4p, 4p+4) entirely in
// registers, and between phases the block regroups its data through LDS so the
// next four bits become register bits. Same butterflies, same order, same
// roundings -- independent of how bits are mapped to lanes and waves.
//
// Layout in one workgroup: the block owns 2^LB consecutive elements (whole
// rows; 2^(LB - log n) rows when n is small). In phase p, thread t register r
// holds element  lo(t) | r << 4p | hi(t) << (4p + 4), lo/hi being t's bits
// below/above 4p. Phase 0 is "16 consecutive elements per thread", so loads
// (and the FP16 stores) are 16-byte vector accesses. The LDS image is padded
// with one word per 16 (addr = i + i/16), which makes the phase-0 row writes
// and the strided phase-1 reads conflict-free across a wave's 64 lanes.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "buffer.hpp"
#include "json.hpp"
#include "planner.hpp"

#include <algorithm>
#include <utility>

namespace cbw {
namespace {

constexpr int kLE = 4;  // log2 registers per thread per phase (radix-16 phases)
constexpr int kE = 1 << kLE;

// Phase P's register window starts at bit 4P, clamped so it ends inside the
// block (when LB is not a multiple of 4 the last window overlaps the previous
// one; only its new bits are butterflied).
template <int P, int LB>
constexpr int window_start() {
    return P * kLE < LB - kLE ? P * kLE : LB - kLE;
}

template <int P, int LB>
__device__ __forceinline__ unsigned phase_index(unsigned t, unsigned r) {
    constexpr unsigned lo_bits = window_start<P, LB>();
    const unsigned lo = t & ((1u << lo_bits) - 1u);
    const unsigned hi = t >> lo_bits;
    return lo | (r << lo_bits) | (hi << (lo_bits + kLE));
}

__device__ __forceinline__ unsigned lds_addr(unsigned i) { return i + (i >> kLE); }

template <int P, int LOG_N, int LB>
__device__ __forceinline__ void register_stages(float (&v)[kE]) {
    constexpr int s = window_start<P, LB>();
#pragma unroll
    for (int j = 0; j < kLE; ++j) {
        if (s + j >= P * kLE && s + j < LOG_N) {
            const int d = 1 << j;
#pragma unroll
            for (int r = 0; r < kE; ++r) {
                if ((r & d) == 0) {
                    const float a = v[r];
                    const float b = v[r + d];
                    v[r] = a + b;
                    v[r + d] = a - b;
                }
            }
        }
    }
}

// Workgroup barrier for LDS traffic only: each wave drains its own LDS
// operations, then meets the others. Unlike __syncthreads() it does not wait
// for outstanding global loads, so the next tile's prefetch stays in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int FROM, int TO, int LB>
__device__ __forceinline__ void exchange(float (&v)[kE], float* lds, unsigned t) {
    lds_barrier();  // earlier readers of the LDS image (this or the previous tile) are done
#pragma unroll
    for (int r = 0; r < kE; ++r) lds[lds_addr(phase_index<FROM, LB>(t, r))] = v[r];
    lds_barrier();
#pragma unroll
    for (int r = 0; r < kE; ++r) v[r] = lds[lds_addr(phase_index<TO, LB>(t, r))];
}

// ---- storage adapters ----------------------------------------------------

// FP32 results stored straight from the last phase (one element per lane,
// a wave covering 256 consecutive bytes) use nontemporal stores: each output
// is written once and not read again, and C1 measured 25.7 -> 20.9 us on
// MI355X. So do the 32-register kernel's runs (wide_store_run). The
// 16-register kernel's 16-byte vector stores, 32 bytes apart across the
// lanes, keep the default policy, where the hint measured slower (C5b 50.2
// -> 55.3 us; regrouped through LDS into 1 KiB per wave instruction, 51.7-
// 52.2 against 51.1-53.8 us).

// 16 bytes at byte offset `off` of a buffer resource.
__device__ __forceinline__ uint4 load_b128(__amdgpu_buffer_rsrc_t r, unsigned off) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
    return make_uint4(x[0], x[1], x[2], x[3]);
}

// The first radix-2 stage straight from one packed fp16 pair (lo = the even
// element, hi = the odd one): s = lo + hi, d = lo - hi in fp32. Both halves
// widen to fp32 exactly and v_fma_mix_f32 computes lo * 1.0 + (+-hi) with a
// single fp32 rounding, so s and d equal the fp32 sum and difference of the
// widened values bit for bit, in one instruction each instead of three.
__device__ __forceinline__ void f16x2_sum_diff(unsigned w, float& s, float& d) {
    asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(s) : "v"(w));
    asm("v_fma_mix_f32 %0, %1, 1.0, -%1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(w));
}

// Two fp32 values narrowed to one packed fp16 pair, round to nearest even
// (v_cvt_pk_f16_f32: the same rounding as two __float2half_rn).
__device__ __forceinline__ unsigned pack_f16x2(float lo, float hi) {
    return __builtin_bit_cast(unsigned, __floats2half2_rn(lo, hi));
}

struct F32Io {
    using T = float;
    // 16 consecutive floats at byte offset `off` of a tile's buffer.
    static __device__ __forceinline__ void load16(__amdgpu_buffer_rsrc_t r, unsigned off, float (&v)[kE]) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 x = load_b128(r, off + 16u * k);
            v[4 * k + 0] = __uint_as_float(x.x);
            v[4 * k + 1] = __uint_as_float(x.y);
            v[4 * k + 2] = __uint_as_float(x.z);
            v[4 * k + 3] = __uint_as_float(x.w);
        }
    }
    // Full path: 16 consecutive floats = four 16-byte loads.
    static __device__ __forceinline__ void load16(const float* p, float (&v)[kE]) {
        const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 x = q[k];
            v[4 * k + 0] = x.x;
            v[4 * k + 1] = x.y;
            v[4 * k + 2] = x.z;
            v[4 * k + 3] = x.w;
        }
    }
    static __device__ __forceinline__ void store16(float* p, const float (&v)[kE]) {
        float4* q = reinterpret_cast<float4*>(p);
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    }
    static __device__ __forceinline__ float load1(const float* p) { return *p; }
    static __device__ __forceinline__ void store1(float* p, float x) { __builtin_nontemporal_store(x, p); }
};

struct F16Io {
    using T = __half;
    static __device__ __forceinline__ void load16(__amdgpu_buffer_rsrc_t r, unsigned off, float (&v)[kE]) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint4 x = load_b128(r, off + 16u * k);
            const unsigned w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * k + 2 * j + 0] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[j] & 0xffffu)));
                v[8 * k + 2 * j + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[j] >> 16)));
            }
        }
    }
    static __device__ __forceinline__ void load16(const __half* p, float (&v)[kE]) {
        const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint4 x = q[k];
            const unsigned w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * k + 2 * j + 0] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[j] & 0xffffu)));
                v[8 * k + 2 * j + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[j] >> 16)));
            }
        }
    }
    static __device__ __forceinline__ void store16(__half* p, const float (&v)[kE]) {
        uint4* q = reinterpret_cast<uint4*>(p);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            unsigned w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack_f16x2(v[8 * k + 2 * j], v[8 * k + 2 * j + 1]);
            q[k] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    static __device__ __forceinline__ float load1(const __half* p) { return __half2float(*p); }
    static __device__ __forceinline__ void store1(__half* p, float x) { *p = __float2half_rn(x); }
};

// A workgroup owns tiles of 2^LB consecutive elements (2^(LB-LOG_N) whole
// rows) and walks tiles blockIdx.x, blockIdx.x + gridDim.x, ...; the next
// tile's loads are issued before the current tile is processed, so HBM reads
// overlap the register/LDS phases.
// `norm` is 1 or 1/n (normalised inverse), `scale` the FP16 output scale; the
// two products are applied in this order, as the reference's finalize and
// narrowing kernel do. Multiplying by 1.0f is exact, so unused factors are 1.

// Element-wise load of a tile that ends past `total` (zeros there).
template <int LB, class Io>
__device__ __forceinline__ void load_partial(const typename Io::T* __restrict__ input, std::uint64_t base,
                                             std::uint64_t total, unsigned t, float (&v)[kE]) {
#pragma unroll
    for (int r = 0; r < kE; ++r) {
        const std::uint64_t i = base + t * kE + r;
        v[r] = i < total ? Io::load1(input + i) : 0.0f;
    }
}

// A full tile's 16 elements per thread through a buffer over the tile;
// `valid` false gives an empty buffer, so the loads return zeros without
// touching memory (keeps the prefetch below unconditional).
template <int LB, class Io>
__device__ __forceinline__ void load_full(const typename Io::T* __restrict__ input, std::uint64_t tile, bool valid,
                                          unsigned t, float (&v)[kE]) {
    constexpr unsigned kBytes = (1u << LB) * unsigned(sizeof(typename Io::T));
    const __amdgpu_buffer_rsrc_t r = make_rsrc(input + (tile << LB), valid ? kBytes : 0u);
    Io::load16(r, t * kE * unsigned(sizeof(typename Io::T)), v);
}

// Hides a value from the optimiser (no code). Applied to the scaled fp32
// result before the FP16 narrowing, it keeps the two roundings of the
// contract (fp32 product, then RNE to fp16): the backend would otherwise fuse
// product and narrowing into one mixed-precision FMA with a single rounding.
__device__ __forceinline__ void opaque(float& x) { asm volatile("" : "+v"(x)); }

// Where transform_store puts tile element i: packed rows (element base + i,
// `full`: the tile lies inside `total`) ...
template <class Io>
struct PackedOut {
    typename Io::T* output;
    std::uint64_t base, total;
    bool full;
    __device__ __forceinline__ void one(unsigned i, float y) const {
        const std::uint64_t k = base + i;
        if (full || k < total) Io::store1(output + k, y);
    }
    __device__ __forceinline__ void sixteen(unsigned t, const float (&x)[kE]) const {
        if (full) {
            Io::store16(output + base + t * kE, x);
            return;
        }
#pragma unroll
        for (int r = 0; r < kE; ++r) {
            const std::uint64_t k = base + t * kE + r;
            if (k < total) Io::store1(output + k, x[r]);
        }
    }
};

// ... or pitched rows: element (row, column) of the tile at row * pitch +
// column from the tile's first row, rows past `rows` absent.
template <int LOG_N, class Io>
struct PitchedOut {
    typename Io::T* output;
    std::uint64_t pitch;
    unsigned rows;
    __device__ __forceinline__ void one(unsigned i, float y) const {
        const unsigned row = i >> LOG_N;
        if (row < rows) Io::store1(output + row * pitch + (i & ((1u << LOG_N) - 1u)), y);
    }
    __device__ __forceinline__ void sixteen(unsigned t, const float (&x)[kE]) const {
        const unsigned i = t * kE, row = i >> LOG_N;
        if (row < rows) Io::store16(output + row * pitch + (i & ((1u << LOG_N) - 1u)), x);
    }
};

// y = (x * norm) * scale, each product rounded to fp32, as the reference's
// finalize and narrowing kernels apply them; a factor of exactly 1 is
// skipped (x * 1 = x), by a uniform branch on the kernel arguments. The
// results are then hidden from the optimiser, so a product is not fused
// with the FP16 narrowing into one rounding.
template <int N>
__device__ __forceinline__ void finalize(float (&v)[N], float norm, float scale) {
    if (norm != 1.0f) {
#pragma unroll
        for (int r = 0; r < N; ++r) v[r] = v[r] * norm;
    }
    if (scale != 1.0f) {
#pragma unroll
        for (int r = 0; r < N; ++r) v[r] = v[r] * scale;
    }
#pragma unroll
    for (int r = 0; r < N; ++r) opaque(v[r]);
}

// The butterflies of one tile and its store through `out`.
template <int LOG_N, int LB, class Io, class Out>
__device__ __forceinline__ void transform_store(float (&v)[kE], float* lds, unsigned t, const Out& out, float norm,
                                                float scale) {
    constexpr int kPhases = (LOG_N + kLE - 1) / kLE;
    constexpr int kLast = kPhases - 1;
    // Store straight from the last phase when its lanes cover >= 64
    // consecutive elements; otherwise regroup to 16-per-thread vectors.
    constexpr bool kDirectStore = kPhases > 1 && window_start<kLast, LB>() >= 6;
    register_stages<0, LOG_N, LB>(v);
    if constexpr (kPhases > 1) {
        exchange<0, 1, LB>(v, lds, t);
        register_stages<1, LOG_N, LB>(v);
    }
    if constexpr (kPhases > 2) {
        exchange<1, 2, LB>(v, lds, t);
        register_stages<2, LOG_N, LB>(v);
    }
    if constexpr (kPhases > 3) {
        exchange<2, 3, LB>(v, lds, t);
        register_stages<3, LOG_N, LB>(v);
    }
    // The products land in new registers (not in `v`), so the caller can keep
    // `v` free of pending store data (see the tile loop).
    if constexpr (kDirectStore) {
        float y[kE];
#pragma unroll
        for (int r = 0; r < kE; ++r) y[r] = v[r];
        finalize<kE>(y, norm, scale);
#pragma unroll
        for (int r = 0; r < kE; ++r) out.one(phase_index<kLast, LB>(t, r), y[r]);
    } else {
        if constexpr (kPhases > 1) exchange<kLast, 0, LB>(v, lds, t);
        float x[kE];
#pragma unroll
        for (int r = 0; r < kE; ++r) x[r] = v[r];
        finalize<kE>(x, norm, scale);
        out.sixteen(t, x);
    }
}

template <int LOG_N, int LB, class Io>
__global__ __launch_bounds__(1 << (LB - kLE)) void fwht_resident_kernel(const typename Io::T* __restrict__ input,
                                                                        typename Io::T* output,
                                                                        std::uint64_t total, float norm,
                                                                        float scale, unsigned tiles) {
    constexpr unsigned kBlock = 1u << LB;
    __shared__ float lds[kBlock + (kBlock >> kLE)];
    const unsigned t = threadIdx.x;
    const unsigned grid = gridDim.x;
    const unsigned full_tiles = static_cast<unsigned>(total >> LB);
    unsigned tile = blockIdx.x;

    // Full tiles: two register buffers in turn. Each step issues the next
    // tile's loads (empty-range loads past the last one, so the issue is
    // unconditional), then transforms the current tile. A branch around the
    // prefetch, or a copy between buffers, would make the compiler's wait for
    // the current tile also wait for the prefetch.
    auto step = [&](float (&cur)[kE], float (&nxt)[kE]) -> bool {
        const unsigned following = tile + grid;
        const bool more = following < full_tiles;
        load_full<LB, Io>(input, following, more, t, nxt);
        __builtin_amdgcn_sched_barrier(0);  // the prefetch is issued before any use of `cur`
        transform_store<LOG_N, LB, Io>(cur, lds, t, PackedOut<Io>{output, std::uint64_t(tile) << LB, total, true},
                                       norm, scale);
        // Keep `cur`'s registers allocated through the stores, so no store
        // takes its data from them: the prefetch into them two steps on would
        // otherwise first wait for those stores.
#pragma unroll
        for (int r = 0; r < kE; ++r) opaque(cur[r]);
        tile = following;
        return more;
    };
    if (tile < full_tiles) {
        float a[kE], b[kE];
        load_full<LB, Io>(input, tile, true, t, a);
        for (;;) {
            if (!step(a, b)) break;
            if (!step(b, a)) break;
        }
    }
    // A last, partial tile goes to the workgroup whose walk reaches it.
    if (full_tiles < tiles && full_tiles % grid == blockIdx.x) {
        const std::uint64_t base = std::uint64_t(full_tiles) << LB;
        float v[kE];
        load_partial<LB, Io>(input, base, total, t, v);
        transform_store<LOG_N, LB, Io>(v, lds, t, PackedOut<Io>{output, base, total, false}, norm, scale);
    }
}

// Pitched rows: row k of the input at input + k * in_pitch, of the output at
// output + k * out_pitch (elements; both 16-byte multiples, n >= 16, so a
// thread's 16 consecutive elements stay in one row and load as 16-byte
// vectors). Tiles are 2^(LB - LOG_N) rows, walked as in the packed kernel;
// each tile's loads go through a buffer ending after its last row, so the
// last, partial tile reads zeros for its missing rows and skips their stores.
template <int LOG_N, int LB, class Io>
__global__ __launch_bounds__(1 << (LB - kLE)) void fwht_pitched_kernel(const typename Io::T* __restrict__ input,
                                                                       typename Io::T* output, std::uint64_t rows,
                                                                       std::uint64_t in_pitch,
                                                                       std::uint64_t out_pitch, float norm,
                                                                       float scale, unsigned tiles) {
    static_assert(LOG_N >= kLE, "a thread's 16 elements lie in one row");
    using T = typename Io::T;
    constexpr unsigned kBlock = 1u << LB;
    constexpr unsigned kRows = 1u << (LB - LOG_N);
    constexpr unsigned kMask = (1u << LOG_N) - 1u;
    __shared__ float lds[kBlock + (kBlock >> kLE)];
    const unsigned t = threadIdx.x;
    const unsigned grid = gridDim.x;
    const unsigned full_tiles = static_cast<unsigned>(rows / kRows);
    const auto span = [&](std::uint64_t n_rows) {
        return static_cast<std::uint32_t>(((n_rows - 1) * in_pitch + (kMask + 1)) * sizeof(T));
    };
    const std::uint32_t in_off =
        static_cast<std::uint32_t>((((t * kE) >> LOG_N) * in_pitch + ((t * kE) & kMask)) * sizeof(T));
    const std::uint32_t full_span = span(kRows);
    const auto load = [&](unsigned tile, std::uint32_t bytes, float (&v)[kE]) {
        Io::load16(make_rsrc(input + std::uint64_t(tile) * kRows * in_pitch, bytes), in_off, v);
    };
    unsigned tile = blockIdx.x;
    auto step = [&](float (&cur)[kE], float (&nxt)[kE]) -> bool {
        const unsigned following = tile + grid;
        const bool more = following < full_tiles;
        load(following, more ? full_span : 0u, nxt);
        __builtin_amdgcn_sched_barrier(0);
        transform_store<LOG_N, LB, Io>(
            cur, lds, t, PitchedOut<LOG_N, Io>{output + std::uint64_t(tile) * kRows * out_pitch, out_pitch, kRows},
            norm, scale);
#pragma unroll
        for (int r = 0; r < kE; ++r) opaque(cur[r]);
        tile = following;
        return more;
    };
    if (tile < full_tiles) {
        float a[kE], b[kE];
        load(tile, full_span, a);
        for (;;) {
            if (!step(a, b)) break;
            if (!step(b, a)) break;
        }
    }
    if (full_tiles < tiles && full_tiles % grid == blockIdx.x) {
        const unsigned present = static_cast<unsigned>(rows - std::uint64_t(full_tiles) * kRows);
        float v[kE];
        load(full_tiles, span(present), v);
        transform_store<LOG_N, LB, Io>(
            v, lds, t,
            PitchedOut<LOG_N, Io>{output + std::uint64_t(full_tiles) * kRows * out_pitch, out_pitch, present}, norm,
            scale);
    }
}

// ---- 32 registers per thread, one row per tile (2^11 .. 2^15 points) -------
//
// Thread t holds 32 elements. Phase 0 butterflies element bits 0-4 (t's 32
// consecutive elements), phase 1 bits 5-9, phase 2 bits 10 .. log n - 1. The
// registers of phase 2 also carry element bits 0 .. P-1 (P = 15 - log n)
// without butterflying them, so each thread ends with 2^(5-P) runs of 2^P
// consecutive results and stores each run as one 4- to 64-byte vector: no
// 2-byte scatter at the end, and still two LDS exchanges. A row of 2^14
// points takes 512 threads and a 67.6 KB LDS image, 2^15 points 1024
// threads and 132 KB (gfx950 gives a workgroup up to 160 KB); at 2^15 the
// phase-2 registers carry no low bits and each result leaves on its own
// (consecutive across the lanes). Same stages in the
// same order as the 16-register kernel, so results are bit-identical.
// LDS image: one pad word per 32 (addr = i + i/32), which leaves every
// 32-lane group of all four exchange accesses on 32 distinct banks (checked
// by enumeration for log n = 11 .. 15), with per-thread bases and
// compile-time register offsets.
constexpr int kLW = 5;
constexpr int kW = 1 << kLW;

__device__ __forceinline__ constexpr unsigned wide_lds_addr(unsigned i) { return i + (i >> kLW); }

template <int LOG_N>
struct WideMap {
    static constexpr int kP = kLW - (LOG_N - 10);  // passenger bits of phase 2
    static __device__ __forceinline__ constexpr unsigned i0(unsigned t, unsigned r) { return (t << kLW) | r; }
    static __device__ __forceinline__ constexpr unsigned i1(unsigned t, unsigned r) {
        return (t & 31u) | (r << 5) | ((t >> 5) << 10);
    }
    static __device__ __forceinline__ constexpr unsigned i2(unsigned t, unsigned r) {
        return (r & ((1u << kP) - 1u)) | (t << kP) | ((r >> kP) << 10);
    }
    // LDS word of element I(t, r): each map is a sum over disjoint bit
    // fields of t and r, and so is wide_lds_addr (i / 32 of disjoint fields is
    // the sum of their parts), so the word is a per-thread base plus a
    // compile-time register offset that folds into the LDS instruction.
    template <unsigned (*I)(unsigned, unsigned)>
    static __device__ __forceinline__ unsigned lds_word(unsigned t, int r) {
        return wide_lds_addr(I(t, 0u)) + wide_lds_addr(I(0u, unsigned(r)));
    }
};

// Radix-2 stages on register bits [LO, HI), lowest first.
template <int LO, int HI, int N>
__device__ __forceinline__ void wide_stages(float (&v)[N]) {
#pragma unroll
    for (int j = LO; j < HI; ++j) {
        const int d = 1 << j;
#pragma unroll
        for (int r = 0; r < N; ++r) {
            if ((r & d) == 0) {
                const float a = v[r];
                const float b = v[r + d];
                v[r] = a + b;
                v[r + d] = a - b;
            }
        }
    }
}

// A tile's 32 elements per thread as raw 32-bit words (fp16 pairs stay
// packed until the tile is processed, so the prefetch buffer is 16 words).
template <class Io>
constexpr int wide_words() {
    return kW * int(sizeof(typename Io::T)) / 4;
}

template <class Io>
__device__ __forceinline__ void wide_load(__amdgpu_buffer_rsrc_t r, unsigned off, unsigned (&w)[wide_words<Io>()]) {
#pragma unroll
    for (int k = 0; k < wide_words<Io>() / 4; ++k) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off + 16u * k), 0, 0);
        w[4 * k + 0] = x[0];
        w[4 * k + 1] = x[1];
        w[4 * k + 2] = x[2];
        w[4 * k + 3] = x[3];
    }
}

// The raw words as 32 fp32 elements with the first stage (register bit 0)
// already applied; for fp16 each word is that stage's pair.
template <class Io>
__device__ __forceinline__ void wide_unpack_first_stage(const unsigned (&w)[wide_words<Io>()], float (&v)[kW]) {
    if constexpr (sizeof(typename Io::T) == 4) {
#pragma unroll
        for (int r = 0; r < kW; ++r) v[r] = __uint_as_float(w[r]);
        wide_stages<0, 1>(v);
    } else {
#pragma unroll
        for (int k = 0; k < kW / 2; ++k) f16x2_sum_diff(w[k], v[2 * k], v[2 * k + 1]);
    }
}

// Stores `run` consecutive results (run * sizeof(T) bytes: 2, 4, 8, 16, 32 or 64)
// at byte offset `off` of the tile's output buffer, nontemporal: a wave's
// store instruction covers 512 bytes or more of consecutive output, written
// once (C5a 49.1-49.7 -> 47.2-47.6 us).
template <class Io, int RUN>
__device__ __forceinline__ void wide_store_run(__amdgpu_buffer_rsrc_t r, unsigned off, const float* x) {
    if constexpr (RUN * sizeof(typename Io::T) == 2) {  // one FP16 result (2^15-point rows)
        __builtin_amdgcn_raw_buffer_store_b16(__half_as_ushort(__float2half_rn(x[0])), r, static_cast<int>(off), 0,
                                              2);
    } else {
        constexpr int kWords = RUN * int(sizeof(typename Io::T)) / 4;
        unsigned w[kWords];
#pragma unroll
        for (int k = 0; k < kWords; ++k) {
            if constexpr (sizeof(typename Io::T) == 4) {
                w[k] = __float_as_uint(x[k]);
            } else {
                w[k] = pack_f16x2(x[2 * k], x[2 * k + 1]);
            }
        }
        using V4 = __attribute__((ext_vector_type(4))) unsigned;
        using V2 = __attribute__((ext_vector_type(2))) unsigned;
        if constexpr (kWords == 1) {  // one FP32 result, or FP16 runs of 2 (2^14-point rows)
            __builtin_amdgcn_raw_buffer_store_b32(w[0], r, static_cast<int>(off), 0, 2);
        } else if constexpr (kWords == 2) {
            __builtin_amdgcn_raw_buffer_store_b64(V2{w[0], w[1]}, r, static_cast<int>(off), 0, 2);
        } else {
#pragma unroll
            for (int k = 0; k < kWords / 4; ++k)
                __builtin_amdgcn_raw_buffer_store_b128(V4{w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]}, r,
                                                       static_cast<int>(off + 16u * k), 0, 2);
        }
    }
}

// One row per tile, rows at input + k * in_pitch / output + k * out_pitch
// (elements; packed rows have pitch n). Tiles blockIdx.x, + gridDim.x, ...;
// WALK: the next tile's loads are issued before the current tile's
// butterflies (for grids smaller than the row count); without it each tile
// is loaded when its turn comes, which needs no second register buffer.
// WALK for FP16 storage only: with 32-bit words the two prefetch buffers and
// the exchange registers exceed 128 VGPRs and spill. FP32 rows take the
// one-tile form (a MEASURE candidate: C1 29.5 against 23.9 us for the
// 16-register kernel).
template <int LOG_N, class Io, bool WALK>
__global__ __launch_bounds__(1 << (LOG_N - kLW), 4) void fwht_wide_kernel(const typename Io::T* __restrict__ input,
                                                                      typename Io::T* output, unsigned rows,
                                                                      std::uint64_t in_pitch,
                                                                      std::uint64_t out_pitch, float norm,
                                                                      float scale) {
    static_assert(LOG_N >= 11 && LOG_N <= 15, "phase 2 covers 1 to 5 bits");
    using T = typename Io::T;
    using M = WideMap<LOG_N>;
    constexpr unsigned kN = 1u << LOG_N;
    constexpr unsigned kBytes = kN * unsigned(sizeof(T));
    constexpr int kRun = 1 << M::kP;
    __shared__ float lds[kN + (kN >> kLW)];
    const unsigned t = threadIdx.x;
    const unsigned grid = gridDim.x;
    const unsigned in_off = t * kW * unsigned(sizeof(T));
    const unsigned out_off = (t << M::kP) * unsigned(sizeof(T));
    unsigned tile = blockIdx.x;

    // `v` arrives with register bit 0 butterflied (wide_unpack_first_stage).
    auto transform = [&](float (&v)[kW], unsigned row) {
        wide_stages<1, kLW>(v);
        lds_barrier();  // readers of the previous tile's image are done
#pragma unroll
        for (int r = 0; r < kW; ++r) lds[M::template lds_word<M::i0>(t, r)] = v[r];
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kW; ++r) v[r] = lds[M::template lds_word<M::i1>(t, r)];
        wide_stages<0, kLW>(v);
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kW; ++r) lds[M::template lds_word<M::i1>(t, r)] = v[r];
        lds_barrier();
#pragma unroll
        for (int r = 0; r < kW; ++r) v[r] = lds[M::template lds_word<M::i2>(t, r)];
        wide_stages<M::kP, kLW>(v);
        finalize<kW>(v, norm, scale);
        const __amdgpu_buffer_rsrc_t dst = make_rsrc(output + std::uint64_t(row) * out_pitch, kBytes);
#pragma unroll
        for (int g = 0; g < kW / kRun; ++g)
            wide_store_run<Io, kRun>(dst, out_off + (unsigned(g) << 10) * unsigned(sizeof(T)), v + g * kRun);
    };
    auto load = [&](unsigned row, bool valid, unsigned (&w)[wide_words<Io>()]) {
        wide_load<Io>(make_rsrc(input + std::uint64_t(row) * in_pitch, valid ? kBytes : 0u), in_off, w);
    };
    // Two raw buffers in turn, the prefetch issued unconditionally (an empty
    // range past the last tile), as in the 16-register kernel.
    auto step = [&](unsigned (&cur)[wide_words<Io>()], unsigned (&nxt)[wide_words<Io>()]) -> bool {
        const unsigned following = tile + grid;
        const bool more = following < rows;
        load(following, more, nxt);
        __builtin_amdgcn_sched_barrier(0);
        float v[kW];
        wide_unpack_first_stage<Io>(cur, v);
        transform(v, tile);
        // `cur` stays allocated through the stores (see the 16-register kernel).
#pragma unroll
        for (int k = 0; k < wide_words<Io>(); ++k) asm volatile("" : "+v"(cur[k]));
        tile = following;
        return more;
    };
    if constexpr (WALK) {
        if (tile < rows) {
            unsigned a[wide_words<Io>()], b[wide_words<Io>()];
            load(tile, true, a);
            for (;;) {
                if (!step(a, b)) break;
                if (!step(b, a)) break;
            }
        }
    } else {
        for (; tile < rows; tile += grid) {
            unsigned w[wide_words<Io>()];
            load(tile, true, w);
            float v[kW];
            wide_unpack_first_stage<Io>(w, v);
            transform(v, tile);
        }
    }
}

template <int LOG_N, class Io, bool WALK>
void launch_wide(const void* in, void* out, std::uint64_t rows, std::uint64_t in_pitch, std::uint64_t out_pitch,
                 float norm, float scale, unsigned grid, hipStream_t stream) {
    hipLaunchKernelGGL((fwht_wide_kernel<LOG_N, Io, WALK>), dim3(grid), dim3(1u << (LOG_N - kLW)), 0, stream,
                       static_cast<const typename Io::T*>(in), static_cast<typename Io::T*>(out),
                       static_cast<unsigned>(rows), in_pitch, out_pitch, norm, scale);
}

// ---- 32 registers per thread, short rows (2^7 and 2^8 points) ----------------
//
// A workgroup of 128 threads owns a tile of 4096 elements, 2^(12 - log n)
// whole rows. Phase 0: thread t holds the 32 consecutive elements from 32 t
// and butterflies element bits 0-4. Phase 1 (one LDS exchange): registers
// hold element bits 5 .. log n - 1 (register bits kP .. 4) and, below them,
// element bits 0 .. kP - 1 as passengers (kP = 10 - log n), so each thread
// butterflies the remaining bits and ends with runs of 2^kP consecutive
// results (8 or 16 bytes) that leave as vector stores; the thread bits are
// element bits kP .. 4 and the row. Same stages in the same order as the
// other kernels, so results are bit-identical.
// LDS image: the low five word bits XORed with word bits 5-9 rotated right
// by log n - 5 (a bijection, linear over bits), which puts every 32-lane
// group of both exchange accesses on 32 distinct banks.
template <int LOG_N>
struct ShortMap {
    static constexpr int kP = 10 - LOG_N;  // passenger bits of phase 1
    static constexpr int kB1 = LOG_N - 5;  // butterfly bits of phase 1
    static __device__ __forceinline__ constexpr unsigned lds_word(unsigned i) {
        const unsigned hi = (i >> 5) & 31u;
        const unsigned rot = ((hi >> kB1) | (hi << (5 - kB1))) & 31u;
        return i ^ rot;
    }
    // Phase 1: element of (thread t, register r), split into thread and
    // register parts over disjoint bits.
    static __device__ __forceinline__ constexpr unsigned i1_thread(unsigned t) {
        return ((t & ((1u << kB1) - 1u)) << kP) | ((t >> kB1) << LOG_N);
    }
    static __device__ __forceinline__ constexpr unsigned i1_register(unsigned r) {
        return (r & ((1u << kP) - 1u)) | ((r >> kP) << 5);
    }
};

// Rows at input + k * in_pitch / output + k * out_pitch (elements; packed
// rows have pitch n); rows past `rows` are absent (the buffer range drops
// their accesses; every access lies in one row). One tile per workgroup.
template <int LOG_N, class Io>
__global__ __launch_bounds__(128) void fwht_short_kernel(const typename Io::T* __restrict__ input,
                                                         typename Io::T* output, unsigned rows,
                                                         std::uint64_t in_pitch, std::uint64_t out_pitch,
                                                         float norm, float scale) {
    static_assert(LOG_N >= 7 && LOG_N <= 8, "the lengths this lowering is offered for");
    using T = typename Io::T;
    using M = ShortMap<LOG_N>;
    constexpr unsigned kN = 1u << LOG_N;
    constexpr unsigned kRows = 1u << (12 - LOG_N);
    constexpr unsigned kB = sizeof(T);
    constexpr int kRun = 1 << M::kP;
    __shared__ float lds[4096];
    const unsigned t = threadIdx.x;
    const std::uint64_t row0 = std::uint64_t(blockIdx.x) * kRows;
    const unsigned present = unsigned(min(std::uint64_t(kRows), rows - row0));
    auto span = [&](const T* base, std::uint64_t pitch) {
        return make_rsrc(base + row0 * pitch, unsigned(((present - 1u) * pitch + kN) * kB));
    };
    // Phase 0: elements 32 t .. 32 t + 31 = row t >> (log n - 5), columns from
    // (t mod 2^(log n - 5)) * 32.
    const unsigned row = t >> M::kB1, col = (t & ((1u << M::kB1) - 1u)) << kLW;
    unsigned w[wide_words<Io>()];
    wide_load<Io>(span(input, in_pitch), unsigned((row * in_pitch + col) * kB), w);
    float v[kW];
    wide_unpack_first_stage<Io>(w, v);
    wide_stages<1, kLW>(v);
    const unsigned base0 = M::lds_word(t << kLW);
#pragma unroll
    for (int r = 0; r < kW; ++r) lds[base0 ^ unsigned(r)] = v[r];
    lds_barrier();
    const unsigned base1 = M::lds_word(M::i1_thread(t));
#pragma unroll
    for (int r = 0; r < kW; ++r) v[r] = lds[base1 ^ M::lds_word(M::i1_register(unsigned(r)))];
    wide_stages<M::kP, kLW>(v);
    finalize<kW>(v, norm, scale);
    // Run g: register bits kP .. 4 = g, element row (t >> kB1), column
    // ((t mod 2^kB1) << kP) + (g << 5).
    const __amdgpu_buffer_rsrc_t dst = span(output, out_pitch);
    const unsigned out_row = t >> M::kB1, out_col = (t & ((1u << M::kB1) - 1u)) << M::kP;
#pragma unroll
    for (int g = 0; g < kW / kRun; ++g)
        wide_store_run<Io, kRun>(dst, unsigned((out_row * out_pitch + out_col + (unsigned(g) << 5)) * kB),
                                 v + g * kRun);
}

template <int LOG_N, class Io>
void launch_short(const void* in, void* out, std::uint64_t rows, std::uint64_t in_pitch, std::uint64_t out_pitch,
                  float norm, float scale, unsigned grid, hipStream_t stream) {
    hipLaunchKernelGGL((fwht_short_kernel<LOG_N, Io>), dim3(grid), dim3(128), 0, stream,
                       static_cast<const typename Io::T*>(in), static_cast<typename Io::T*>(out),
                       static_cast<unsigned>(rows), in_pitch, out_pitch, norm, scale);
}

// ---- 64 elements per lane, no LDS (rows of 2^5 .. 2^8 points) --------------
//
// A wave owns 4096 consecutive elements (4096 / n rows) and each lane 64 of
// them: four runs of 16 consecutive elements. Element index bits:
//   0-3   register bits 0-3 (position in the run),
//   4, 5  lane bits 4, 5 (the run's quarter of a 64-element line),
//   6, 7  register bits 4, 5 (which of the lane's four lines),
//   8-11  lane bits 0-3.
// So each 16-byte load or store instruction touches 16 lines of 128 bytes
// (as many as the 16-register kernel's), and the bits a row of <= 256 points
// butterflies are register bits or lane bits 4 and 5. gfx950's lane-swap
// instructions exchange those two lane bits with register bits
// (v_permlane16_swap: lane bit 4, v_permlane32_swap: lane bit 5; each swaps a
// register pair's values between lane halves, a 2 x 2 transpose): after
// register bits 0-3 are butterflied, bit 4 is swapped into register bit 0 and
// bit 5 into register bit 1, each butterflied there, then bits 6 and 7 in
// register bits 4 and 5, and the two swaps are undone for the stores. No
// LDS, no barrier, the waves are independent. Same stages in the same order
// (bits 0, 1, ..., log n - 1) as the other kernels, so results are
// bit-identical.
constexpr int kLaneLog = 6;
constexpr int kLaneRegs = 1 << kLaneLog;
constexpr int kLaneTileLog = kLaneLog + 6;  // elements per wave
constexpr int kLaneWaves = 4;               // waves per workgroup

// Element (within the wave's 4096) of lane l's register 0, and of register r
// of lane 0: the index is their sum (disjoint bit fields).
__device__ __forceinline__ unsigned lane_element(unsigned l) {
    return (((l >> 4) & 3u) << 4) | ((l & 15u) << 8);
}
constexpr unsigned register_element(unsigned r) { return (r & 15u) | ((r >> 4) << 6); }

// Exchanges register bit RB with lane bit LANE_BIT (4 or 5) in every register
// pair that differs in bit RB: afterwards the pair is indexed by the old lane
// bit and the lane bit by the old register bit.
template <int LANE_BIT, int RB, int N>
__device__ __forceinline__ void swap_lane_bit(float (&v)[N]) {
    static_assert(LANE_BIT == 4 || LANE_BIT == 5, "gfx950 swaps lane bits 4 and 5");
#pragma unroll
    for (int r = 0; r < N; ++r) {
        if ((r >> RB) & 1) continue;
        const int p = r | (1 << RB);
        const auto s = LANE_BIT == 5 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v[r]), __float_as_uint(v[p]),
                                                                        false, false)
                                     : __builtin_amdgcn_permlane16_swap(__float_as_uint(v[r]), __float_as_uint(v[p]),
                                                                        false, false);
        v[r] = __uint_as_float(s[0]);
        v[p] = __uint_as_float(s[1]);
    }
}

// Byte offset of element e of the wave's rows at pitch `pitch` (elements):
// row e >> log n, column e mod n. Additive over disjoint bit fields of e.
template <int LOG_N, int B>
__device__ __forceinline__ unsigned lane_offset(unsigned e, std::uint64_t pitch) {
    return unsigned(((e >> LOG_N) * pitch + (e & ((1u << LOG_N) - 1u))) * B);
}

// Rows of a tile (4096 / n rows, one wave) at input + row * pitch (elements;
// packed rows have pitch n); rows past `rows` are absent (the buffer range
// drops their accesses, and every 16-byte access lies in one row). Wave w of
// the grid takes tile w. (A persistent grid, each wave walking tiles with the
// next tile's loads in flight, measured slower: C5b 57.4-58.8 us against
// 54.2 us.)
template <int LOG_N, class Io>
__global__ __launch_bounds__(64 * kLaneWaves) void fwht_lane_kernel(const typename Io::T* __restrict__ input,
                                                                    typename Io::T* output, unsigned rows,
                                                                    std::uint64_t in_pitch,
                                                                    std::uint64_t out_pitch, float norm,
                                                                    float scale) {
    static_assert(LOG_N >= 5 && LOG_N <= 8, "bits 4 and 5 are the lane bits swapped in");
    using T = typename Io::T;
    constexpr unsigned kN = 1u << LOG_N;
    constexpr unsigned kRowsPerWave = 1u << (kLaneTileLog - LOG_N);
    constexpr unsigned kB = sizeof(T);
    constexpr int kPerAccess = 16 / int(kB);  // elements per 16-byte access
    constexpr int kWords = kLaneRegs * int(kB) / 4;
    const unsigned lane = threadIdx.x & 63u;
    const unsigned tiles = (rows + kRowsPerWave - 1u) / kRowsPerWave;
    const unsigned tile = uniform(blockIdx.x * unsigned(kLaneWaves) + (threadIdx.x >> 6));
    if (tile >= tiles) return;
    const unsigned le = lane_element(lane);
    const unsigned in_base = lane_offset<LOG_N, kB>(le, in_pitch);
    const unsigned out_base = lane_offset<LOG_N, kB>(le, out_pitch);
    // Buffer over the tile's existing rows.
    const std::uint64_t row0 = std::uint64_t(tile) * kRowsPerWave;
    const unsigned present = unsigned(min(std::uint64_t(kRowsPerWave), rows - row0));
    auto span = [&](const T* base, std::uint64_t pitch) {
        return make_rsrc(base + row0 * pitch, unsigned(((present - 1u) * pitch + kN) * kB));
    };
    // Raw words of the lane's 64 elements, 16 bytes per access, registers in order.
    unsigned w[kWords];
    const __amdgpu_buffer_rsrc_t src = span(input, in_pitch);
#pragma unroll
    for (int a = 0; a < kLaneRegs / kPerAccess; ++a) {
        const unsigned off = in_base + lane_offset<LOG_N, kB>(register_element(unsigned(a * kPerAccess)), in_pitch);
        const auto x = __builtin_amdgcn_raw_buffer_load_b128(src, static_cast<int>(off), 0, 0);
        w[4 * a + 0] = x[0];
        w[4 * a + 1] = x[1];
        w[4 * a + 2] = x[2];
        w[4 * a + 3] = x[3];
    }
    float v[kLaneRegs];
    if constexpr (kB == 4) {
#pragma unroll
        for (int r = 0; r < kLaneRegs; ++r) v[r] = __uint_as_float(w[r]);
        wide_stages<0, 1>(v);
    } else {
#pragma unroll
        for (int k = 0; k < kLaneRegs / 2; ++k) f16x2_sum_diff(w[k], v[2 * k], v[2 * k + 1]);
    }
    wide_stages<1, 4>(v);    // element bits 1-3
    swap_lane_bit<4, 0>(v);  // register bit 0 <- element bit 4
    wide_stages<0, 1>(v);
    if constexpr (LOG_N >= 6) {
        swap_lane_bit<5, 1>(v);  // register bit 1 <- element bit 5
        wide_stages<1, 2>(v);
    }
    if constexpr (LOG_N >= 7) wide_stages<4, LOG_N - 2>(v);  // element bits 6, 7 in register bits 4, 5
    if constexpr (LOG_N >= 6) swap_lane_bit<5, 1>(v);
    swap_lane_bit<4, 0>(v);
    finalize<kLaneRegs>(v, norm, scale);
    const __amdgpu_buffer_rsrc_t dst = span(output, out_pitch);
    using V4 = __attribute__((ext_vector_type(4))) unsigned;
#pragma unroll
    for (int a = 0; a < kLaneRegs / kPerAccess; ++a) {
        unsigned o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * a + j;
            if constexpr (kB == 4) o[j] = __float_as_uint(v[e]);
            else o[j] = pack_f16x2(v[2 * e], v[2 * e + 1]);
        }
        const unsigned off = out_base + lane_offset<LOG_N, kB>(register_element(unsigned(a * kPerAccess)), out_pitch);
        __builtin_amdgcn_raw_buffer_store_b128(V4{o[0], o[1], o[2], o[3]}, dst, static_cast<int>(off), 0, 0);
    }
}

template <int LOG_N, class Io>
void launch_lanes(const void* in, void* out, std::uint64_t rows, std::uint64_t in_pitch, std::uint64_t out_pitch,
                  float norm, float scale, unsigned grid, hipStream_t stream) {
    hipLaunchKernelGGL((fwht_lane_kernel<LOG_N, Io>), dim3(grid), dim3(64 * kLaneWaves), 0, stream,
                       static_cast<const typename Io::T*>(in), static_cast<typename Io::T*>(out),
                       static_cast<unsigned>(rows), in_pitch, out_pitch, norm, scale);
}

using Launch = void (*)(const void*, void*, std::uint64_t, float, float, unsigned, hipStream_t);

template <int LOG_N, class Io>
constexpr int block_log() {
    return LOG_N <= 12 ? 12 : LOG_N;
}

template <int LOG_N, class Io>
void launch_resident(const void* in, void* out, std::uint64_t total, float norm, float scale, unsigned grid,
                     hipStream_t stream) {
    constexpr int LB = block_log<LOG_N, Io>();
    const std::uint64_t tiles = (total + (1ull << LB) - 1) >> LB;
    hipLaunchKernelGGL((fwht_resident_kernel<LOG_N, LB, Io>), dim3(grid), dim3(1u << (LB - kLE)), 0, stream,
                       static_cast<const typename Io::T*>(in), static_cast<typename Io::T*>(out), total, norm,
                       scale, static_cast<unsigned>(tiles));
}

using PitchedLaunch = void (*)(const void*, void*, std::uint64_t, std::uint64_t, std::uint64_t, float, float,
                               unsigned, hipStream_t);

template <int LOG_N, class Io>
void launch_pitched(const void* in, void* out, std::uint64_t rows, std::uint64_t in_pitch, std::uint64_t out_pitch,
                    float norm, float scale, unsigned grid, hipStream_t stream) {
    constexpr int LB = block_log<LOG_N, Io>();
    constexpr std::uint64_t kRows = std::uint64_t{1} << (LB - LOG_N);
    const std::uint64_t tiles = (rows + kRows - 1) / kRows;
    hipLaunchKernelGGL((fwht_pitched_kernel<LOG_N, LB, Io>), dim3(grid), dim3(1u << (LB - kLE)), 0, stream,
                       static_cast<const typename Io::T*>(in), static_cast<typename Io::T*>(out), rows, in_pitch,
                       out_pitch, norm, scale, static_cast<unsigned>(tiles));
}

template <class Io, int... L>
PitchedLaunch pitched_table_entry(int log_n, std::integer_sequence<int, L...>) {
    PitchedLaunch table[] = {launch_pitched<L + kLE, Io>...};
    return table[log_n - kLE];
}

template <class Io, int... L>
Launch resident_table_entry(int log_n, std::integer_sequence<int, L...>) {
    Launch table[] = {nullptr, launch_resident<L + 1, Io>...};
    return table[log_n];
}

constexpr int kMaxResidentLog = 13;

template <class Io>
Launch resident_launcher(int log_n) {
    if (log_n < 1 || log_n > kMaxResidentLog) return nullptr;
    return resident_table_entry<Io>(log_n, std::make_integer_sequence<int, kMaxResidentLog>{});
}

template <class Io>
PitchedLaunch pitched_launcher(int log_n) {
    if (log_n < kLE || log_n > kMaxResidentLog) return nullptr;
    return pitched_table_entry<Io>(log_n, std::make_integer_sequence<int, kMaxResidentLog - kLE + 1>{});
}

// Workgroups of the walking 32-register kernel resident on the device at once.
template <int LOG_N, class Io>
unsigned wide_resident() {
    static const unsigned resident = [] {
        int per_cu = 0;
        const void* fn = reinterpret_cast<const void*>(&fwht_wide_kernel<LOG_N, Io, true>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 1 << (LOG_N - kLW), 0) != hipSuccess ||
            per_cu < 1) {
            (void)hipGetLastError();
            per_cu = 1;
        }
        return unsigned(per_cu) * unsigned(device_cu_count());
    }();
    return resident;
}

struct WideLaunch {
    PitchedLaunch launch = nullptr;  // one tile per workgroup's turn
    PitchedLaunch walk = nullptr;    // with next-tile prefetch
    unsigned (*resident)() = nullptr;
    explicit operator bool() const { return launch != nullptr; }
};

template <int... L>
WideLaunch wide_table_entry(int log_n, std::integer_sequence<int, L...>) {
    WideLaunch table[] = {WideLaunch{launch_wide<L + 11, F16Io, false>, launch_wide<L + 11, F16Io, true>,
                                     wide_resident<L + 11, F16Io>}...};
    return table[log_n - 11];
}
// FP32 rows: no walking variant (two 32-word prefetch buffers spill).
template <int... L>
WideLaunch wide_table_entry_f32(int log_n, std::integer_sequence<int, L...>) {
    WideLaunch table[] = {WideLaunch{launch_wide<L + 11, F32Io, false>, nullptr, nullptr}...};
    return table[log_n - 11];
}

// The 32-register kernel: rows of 2^11 .. 2^15 points (FP16, and FP32 without
// the walking form), row count within 32 bits.
// For FP16 rows of 2^7 and 2^8 points, the short-row form of the same
// lowering (fwht_short_kernel: 4096-element tiles of whole rows, one LDS
// exchange, a tile's pitched span within 31-bit byte offsets), without a
// persistent variant. At 2^6 points its 32-byte runs leave as two 16-byte
// stores with 16-byte gaps across the lanes, and it measured 64 us against
// 47 us for C5b's volume; it is not offered there.
WideLaunch wide_launcher(const Request& r) {
    if (r.batch > 0xffffffffull) return {};
    if (!r.fp16_final) {
        if (r.log_n < 11 || r.log_n > kMaxFwhtRowLog) return {};
        return wide_table_entry_f32(int(r.log_n), std::make_integer_sequence<int, kMaxFwhtRowLog - 10>{});
    }
    if (r.log_n >= 7 && r.log_n <= 8) {
        const std::uint64_t rows_per_tile = std::uint64_t{1} << (12 - r.log_n);
        const std::uint64_t pitch = r.pitched ? std::max(r.in_batch_stride, r.out_batch_stride) : r.n;
        if (rows_per_tile * pitch * 2 >= (std::uint64_t{1} << 31)) return {};
        return WideLaunch{r.log_n == 7 ? launch_short<7, F16Io> : launch_short<8, F16Io>, nullptr, nullptr};
    }
    if (r.log_n < 11 || r.log_n > kMaxFwhtRowLog) return {};
    return wide_table_entry(int(r.log_n), std::make_integer_sequence<int, kMaxFwhtRowLog - 10>{});
}

template <class Io, int... L>
PitchedLaunch lane_table_entry(int log_n, std::integer_sequence<int, L...>) {
    PitchedLaunch table[] = {launch_lanes<L + 5, Io>...};
    return table[log_n - 5];
}

// The 64-elements-per-lane kernel: rows of 2^5 .. 2^8 points, row count
// within 32 bits, a wave's pitched span within 31-bit byte offsets.
PitchedLaunch lane_launcher(const Request& r) {
    if (r.log_n < 5 || r.log_n > 8 || r.batch > 0xffffffffull) return nullptr;
    if (r.pitched) {
        const std::uint64_t rows_per_wave = std::uint64_t{1} << (kLaneTileLog - r.log_n);
        const std::uint64_t pitch = std::max(r.in_batch_stride, r.out_batch_stride);
        const std::uint64_t bytes = r.fp16_final ? 2 : 4;
        if (rows_per_wave * pitch * bytes >= (std::uint64_t{1} << 31)) return nullptr;
    }
    return r.fp16_final ? lane_table_entry<F16Io>(int(r.log_n), std::make_integer_sequence<int, 4>{})
                        : lane_table_entry<F32Io>(int(r.log_n), std::make_integer_sequence<int, 4>{});
}

// Kernel families of the FWHT lowerings.
enum class FwhtKind { Resident, Wide, WidePersistent, Lanes };

class FwhtExecutor final : public Executor {
  public:
    // Resident: the 16-register kernels (`launch` packed, `pitched` pitched
    // rows); Wide: the 32-register kernel, one tile per workgroup's turn;
    // WidePersistent: its grid sized to the resident workgroups, each walking
    // rows with next-row prefetch; Lanes: 64 elements per lane, no LDS, one
    // tile per wave.
    FwhtExecutor(const Request& r, FwhtKind kind, Launch launch, PitchedLaunch pitched, PitchedLaunch rows_kernel,
                 unsigned resident)
        : r_(r), launch_(launch), pitched_(pitched), rows_kernel_(rows_kernel) {
        norm_ = r.normalize ? 1.0f / static_cast<float>(r.n) : 1.0f;
        scale_ = r.fp16_final ? r.output_scale : 1.0f;
        const std::uint64_t total = r.n * r.batch;
        std::uint64_t tiles = 0, tile_elements = 0, lds = 0;
        unsigned threads = 0, regs = 0, phases = 0;
        if (kind == FwhtKind::Lanes) {
            const std::uint64_t rows_per_wave = std::uint64_t{1} << (kLaneTileLog - int(r.log_n));
            tiles = (r.batch + rows_per_wave - 1) / rows_per_wave;  // one per wave
            tile_elements = std::uint64_t{1} << kLaneTileLog;
            threads = 64u * kLaneWaves;
            regs = kLaneRegs;
            phases = 1;
            grid_ = static_cast<unsigned>(std::min<std::uint64_t>((tiles + kLaneWaves - 1) / kLaneWaves,
                                                                  0x7fffffffull));
            reason = "64 elements per lane (" + std::to_string(threads) +
                     " threads, each wave on its own 4096 elements): bits 0-3 in registers, bit 4 through "
                     "v_permlane16_swap" +
                     std::string(r.log_n >= 6 ? ", bit 5 through v_permlane32_swap" : "") +
                     std::string(r.log_n >= 7 ? ", bits 6+ in registers" : "") + ", no LDS";
        } else {
            const bool wide = kind != FwhtKind::Resident;
            const bool short_rows = wide && r.log_n < 11;  // fwht_short_kernel: 4096-element tiles
            const int lb = short_rows ? 12 : wide ? static_cast<int>(r.log_n) : r.log_n <= 12 ? 12 : static_cast<int>(r.log_n);
            const std::uint64_t rows_per_tile = std::uint64_t{1} << (lb - int(r.log_n));
            tiles = pitched_ || wide ? (r.batch + rows_per_tile - 1) / rows_per_tile
                                     : (total + (1ull << lb) - 1) >> lb;
            tile_elements = std::uint64_t{1} << lb;
            const int regs_log = wide ? kLW : kLE;
            threads = 1u << (lb - regs_log);
            regs = 1u << regs_log;
            phases = short_rows ? 2u : wide ? 3u : unsigned((r.log_n + kLE - 1) / kLE);
            lds = short_rows ? 4096ull * 4 : ((1u << lb) + ((1u << lb) >> regs_log)) * 4ull;
            // Grid: one workgroup per tile (measured at least as fast as a
            // persistent, occupancy-sized grid for every BASELINE shape once
            // the kernel's prefetch overlapped), capped at the launch limit;
            // the kernel walks any tiles beyond the grid with next-tile
            // prefetch.
            grid_ = static_cast<unsigned>(std::min<std::uint64_t>(tiles, 0x7fffffffull));
            if (kind == FwhtKind::WidePersistent) grid_ = std::min(grid_, resident);
            reason = short_rows
                         ? "whole rows resident in one workgroup (128 threads x 32 registers, phases of bits 0-4 "
                           "and 5+, the second carrying the low element bits so results leave as 8- to 32-byte "
                           "vectors, one swizzled LDS exchange)"
                     : wide ? "one row per workgroup (" + std::to_string(threads) +
                                  " threads x 32 registers, phases of bits 0-4, 5-9 and 10+, the last carrying the low "
                                  "element bits so results leave as 8- to 64-byte vectors)"
                            : "whole rows resident in one workgroup (" + std::to_string(threads) +
                                  " threads x 16 registers, padded LDS exchange)";
            reason += std::string(grid_ < tiles ? ", persistent grid with next-tile prefetch" : "");
        }
        require(tiles <= 0xffffffffull, "FWHT batch exceeds the tile index range");
        reason += "; stage order bits 0..log n-1";
        algorithm = name(r, kind);
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("operator", "fwht")
            .field("algorithm", algorithm)
            .field("log_n", r.log_n)
            .field("batch", r.batch)
            .field("tile_elements", tile_elements)
            .field("tiles", tiles)
            .field("grid", grid_)
            .field("threads_per_block", threads)
            .field("registers_per_thread", regs)
            .field("phases", phases)
            .field("lds_bytes", lds)
            .field("input_pitch", r.pitched ? r.in_batch_stride : r.n)
            .field("output_pitch", r.pitched ? r.out_batch_stride : r.n)
            .end_object();
        mapping_json = w.str();
    }
    static std::string name(const Request& r, FwhtKind kind) {
        const char* family = kind == FwhtKind::Lanes      ? "lanes-r64"
                             : kind == FwhtKind::Resident ? "resident-r16"
                             : kind == FwhtKind::Wide     ? "resident-r32"
                                                          : "resident-r32-persistent";
        return std::string(r.fp16_final ? "fwht-fp16-fp32-" : "fwht-fp32-") + family + (r.pitched ? "-pitched" : "");
    }
    void execute(const void* in, void* out, void*, hipStream_t stream) override {
        if (rows_kernel_)
            rows_kernel_(in, out, r_.batch, r_.pitched ? r_.in_batch_stride : r_.n,
                         r_.pitched ? r_.out_batch_stride : r_.n, norm_, scale_, grid_, stream);
        else if (pitched_)
            pitched_(in, out, r_.batch, r_.in_batch_stride, r_.out_batch_stride, norm_, scale_, grid_, stream);
        else
            launch_(in, out, r_.n * r_.batch, norm_, scale_, grid_, stream);
        hip_check(hipGetLastError(), "FWHT launch");
    }

  private:
    Request r_;
    Launch launch_;
    PitchedLaunch pitched_;
    PitchedLaunch rows_kernel_;  // the 32-register or the lane kernel (packed or pitched rows)
    float norm_ = 1.0f, scale_ = 1.0f;
    unsigned grid_ = 1;
};

// The lowerings of a request, default first. Default: the 32-register kernel
// for FP16 rows of 2^11 to 2^13 points and FP32 rows of 2^13 points (three
// LDS phases where the 16-register kernel takes four at 2^13), the
// 16-register kernel elsewhere. Measured, 2^24 elements per call, HIP events:
// FP16 2^11 15.3 against 17.6 us, 2^12 14.0 / 17.4, 2^13 15.0 / 22.3; FP32
// 2^13 24.2 / 34.1, but FP32 2^12 28.5 / 22.9 and 2^11 54.4 / 22.8. The
// others are MEASURE candidates and explicit choices.
std::vector<FwhtKind> fwht_kinds(const Request& r) {
    std::vector<FwhtKind> kinds;
    if (r.log_n <= kMaxResidentLog) kinds.push_back(FwhtKind::Resident);
    if (const WideLaunch wide = wide_launcher(r)) {
        // Rows of 2^14 and 2^15 points have only the 32-register kernels.
        const bool first = r.log_n > kMaxResidentLog || (r.log_n >= 11 && (r.fp16_final || r.log_n == 13));
        kinds.insert(first ? kinds.begin() : kinds.end(), FwhtKind::Wide);
        if (wide.walk) kinds.push_back(FwhtKind::WidePersistent);
    }
    if (lane_launcher(r)) kinds.push_back(FwhtKind::Lanes);
    return kinds;
}

}  // namespace

std::unique_ptr<Executor> make_fwht_executor(const Request& r) {
    supported(r.log_n <= kMaxResidentLog || wide_launcher(r),
              "FWHT lengths above 2^" + std::to_string(kMaxFwhtRowLog) + " run as factored plans");
    supported(!r.allow_mma || r.fp16_final, "MFMA Hadamard blocks require FP16 storage");
    // ALLOW_FP16_MMA permits the MFMA Hadamard-block kernel but does not make
    // it the default: the stage-ordered VALU kernels are bit-exact and, on
    // MI355X, faster at both QuaRot shapes (sustained, 16384 x 4096: 45.4
    // against 49.0 us; 524288 x 128: 47.6 against 48.4 us). The reference
    // likewise keeps its native selection unless a calibrated MMA profile
    // wins (src/mapping_selector.cpp:13-44). The MFMA kernel is taken by name
    // (EXPLICIT) or when MEASURE times it fastest.
    const bool mfma = r.allow_mma && fwht_mfma_covers(r);
    if (r.variant == fwht_mfma_name()) {
        supported(r.allow_mma, "'" + r.variant + "' needs the ALLOW_FP16_MMA arithmetic policy");
        supported(mfma, "'" + r.variant + "' covers packed FP16 rows of 2 to 4096 points only");
        return make_fwht_mfma_executor(r);
    }
    const Launch launch = r.fp16_final ? resident_launcher<F16Io>(r.log_n) : resident_launcher<F32Io>(r.log_n);
    require(launch != nullptr || r.log_n > kMaxResidentLog, "FWHT length has no launcher");
    PitchedLaunch pitched = nullptr;
    if (r.pitched && r.log_n <= kMaxResidentLog) {
        pitched = r.fp16_final ? pitched_launcher<F16Io>(r.log_n) : pitched_launcher<F32Io>(r.log_n);
        require(pitched != nullptr, "pitched FWHT rows need n >= 16");
    }
    const std::vector<FwhtKind> kinds = fwht_kinds(r);
    FwhtKind kind = kinds.front();
    if (!r.variant.empty()) {
        std::string available;
        bool found = false;
        for (FwhtKind k : kinds) {
            available += (available.empty() ? "" : ", ") + FwhtExecutor::name(r, k);
            if (FwhtExecutor::name(r, k) == r.variant) {
                kind = k;
                found = true;
            }
        }
        supported(found, "'" + r.variant + "' is not a lowering of this FWHT (available: " + available + ")");
    }
    const WideLaunch wide = wide_launcher(r);
    PitchedLaunch rows_kernel = nullptr;
    unsigned resident = 0;
    if (kind == FwhtKind::Wide) rows_kernel = wide.launch;
    if (kind == FwhtKind::WidePersistent) {
        rows_kernel = wide.walk;
        resident = wide.resident();
    }
    if (kind == FwhtKind::Lanes) rows_kernel = lane_launcher(r);
    auto e = std::make_unique<FwhtExecutor>(r, kind, launch, kind == FwhtKind::Resident ? pitched : nullptr,
                                            rows_kernel, resident);
    if (r.allow_mma && !mfma)
        e->reason += "; ALLOW_FP16_MMA requested, but the MFMA Hadamard-block kernel covers packed rows of 2 to 4096 "
                     "points only: stage-ordered VALU kernel used";
    else if (r.allow_mma && r.variant.empty())
        e->reason += "; ALLOW_FP16_MMA requested: stage-ordered VALU kernel kept as the default (bit-exact, and "
                     "faster than the MFMA Hadamard-block kernel on MI355X); " + fwht_mfma_name() +
                     " is available by name or MEASURE, with a different accumulation order (up to one fp16 ulp "
                     "from the stage-ordered result, beyond the 2e-3 bound where |y| >= 4)";
    return e;
}

std::vector<std::string> fwht_candidates(const Request& r) {
    Request v = r;
    v.variant.clear();
    make_fwht_executor(v);  // the default lowering exists (throws NotSupported otherwise)
    std::vector<std::string> names;
    for (FwhtKind k : fwht_kinds(r)) names.push_back(FwhtExecutor::name(r, k));
    if (r.allow_mma && fwht_mfma_covers(r)) names.push_back(fwht_mfma_name());
    return names;
}

}  // namespace cbw
