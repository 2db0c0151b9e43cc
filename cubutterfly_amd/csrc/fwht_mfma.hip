// FP16 FWHT through MFMA 16 x 16 Hadamard blocks (the ALLOW_FP16_MMA policy,
// reference include/cubutterfly/cubutterfly.h:86-90): FP16 storage, FP32
// accumulation, one final RNE narrowing after the output scale -- the
// final-storage contract of src/butterfly.cu:1452-1470, 1882-1897 -- for rows
// of 2 .. 4096 points.
//
// H(2^m) = H(2^a) (x) H(2^b) (x) ... for the Sylvester matrix, so the
// transform factors into one 16 x 16 block contraction per 4-bit group of the
// element index. A wave owns a tile of 4096 consecutive elements, index
// e = i2 * 256 + i1 * 16 + i0 (whole rows: the row bits sit above bit m - 1).
// Per block of fixed i2 (16 blocks per tile):
//
//   1. Contraction along i0 on the matrix cores: A[i1][i0] is the fp16 input
//      itself (v_mfma_f32_16x16x16_f16 wants lane l to supply A[l % 16]
//      [4 (l / 16) + j], which is 4 consecutive halves, one 8-byte load), B is
//      the 16 x 16 block M0 = I (x) H(2^t0) (t0 transform bits in the group).
//      The fp32 result D0[i1][k0] lands in lane l as rows 4 (l / 16) + r,
//      column l % 16.
//   2. Contraction along i1 on the matrix cores: the transposed block D0^T
//      has lane l supplying D0^T[l % 16][4 (l / 16) + j] = D0[4 (l / 16) + j]
//      [l % 16] -- exactly lane l's accumulator registers, so no data moves
//      between lanes. The fp32 values enter the fp16 operand as an exact-ish
//      split, D0 / 16 = hi + lo (two fp16 parts, 22 significant bits; the
//      1/16 keeps |hi| below the fp16 range for any fp16 input), and
//      D1 = 16 (hi M1 + lo M1) accumulates both products in fp32.
//   3. Bits 8 .. 11 (i2), when they are transform bits: after all 16 blocks
//      each lane holds, for its four (k0, k1), the 16 values over i2 -- a
//      radix-2 transform in registers (VALU, fp32, bits in stage order).
//
// The output element (k2, k1, k0) of lane l, register r is k2 * 256 +
// (l % 16) * 16 + 4 (l / 16) + r: four consecutive halves. Blocks move in
// pairs, one 16-byte access per lane each way, with one v_permlane16_swap per
// dword to trade the halves of neighbouring 16-lane groups. No LDS is used.
// Accumulation order differs from the radix-2 stage order of the STRICT
// kernels, so results can differ from them by one fp16 ulp where a value sits
// near a rounding boundary; this lowering is taken only when the caller names
// it (or MEASURE picks it) under the ALLOW_FP16_MMA policy.
//
// Rows stay independent. The block matrices I (x) H(2^t) hold zeros for the
// element pairs of different rows (rows shorter than 16 points in the first
// contraction, 32..128-point rows in the second), and on the matrix cores
// inf * 0 and NaN * 0 are NaN, so one non-finite input would turn outputs of
// its neighbouring rows into NaN (the hi / lo split would also turn an inf
// into NaN, inf - inf). A wave whose tile holds any non-finite input
// therefore runs the radix-2 stages on the VALU instead, in stage order, with
// lane exchanges for the index bits held across lanes: every row of such a
// tile is then bit-identical to the stage-ordered kernels and the oracle.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "buffer.hpp"
#include "json.hpp"
#include "planner.hpp"

namespace cbw {
namespace {

using half4 = __attribute__((ext_vector_type(4))) _Float16;
using pk16 = __attribute__((ext_vector_type(2))) __fp16;  // v_cvt_pkrtz_f16_f32 result
using float4v = __attribute__((ext_vector_type(4))) float;

constexpr int kTileLog = 12;         // elements per wave tile
constexpr int kWavesPerBlock = 4;    // tiles per workgroup
constexpr int kMaxLog = kTileLog;    // longest row this lowering covers

// Lane l's B operand of the 16 x 16 block I (x) H(2^t): B[k][j] for
// k = 4 (l / 16) + 0..3 and j = l % 16. Entries are 0 or +-1 (exact in fp16).
__device__ __forceinline__ half4 hadamard_block(unsigned lane, int t) {
    const unsigned j = lane & 15u, k0 = 4u * (lane >> 4);
    const unsigned low = (1u << t) - 1u;
    half4 b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned k = k0 + unsigned(q);
        const bool same_block = (k & ~low) == (j & ~low);
        const bool negative = __popc(k & j & low) & 1u;
        b[q] = same_block ? (negative ? _Float16(-1.0f) : _Float16(1.0f)) : _Float16(0.0f);
    }
    return b;
}

// Hides a value from the optimiser (no code): keeps the fp32 product and the
// fp16 narrowing two separate roundings.
__device__ __forceinline__ void opaque(float& x) { asm volatile("" : "+v"(x)); }

// y = (x * norm) * scale rounded to fp32 twice, then one RNE narrowing.
__device__ __forceinline__ unsigned short narrow(float x, float norm, float scale) {
    float y = (x * norm) * scale;
    opaque(y);
    return __half_as_ushort(__float2half_rn(y));
}

// The tile's transform for a wave that holds a non-finite input: radix-2
// stages over element bits 0 .. LOG_N - 1 in order, fp32, each pair (x at
// the lower index, y at the upper) -> (x + y, x - y) as the oracle forms
// them. Lane l holds a[i2][j] = element i2 * 256 + (l % 16) * 16 +
// 4 (l / 16) + j: element bits 0-1 are register bits (j), bits 2-3 lane
// bits 4-5, bits 4-7 lane bits 0-3, bits 8-11 register bits (i2). Results
// leave in the input's own layout. The tile is loaded again here, so that no
// input register stays live into this path: the common path keeps its own
// allocation and this one spills what does not fit.
// This path needs about 200 VGPRs where the MFMA path needs 120 (rows of
// more than 256 points, which hold all 64 results for the register stages)
// or 96 (shorter rows), and the kernel's allocation covers both: the kernel
// therefore asks for four waves per SIMD (at most 128 VGPRs) or five (at most
// 96; C5b 48.1 -> 47.7 us), so what does not fit spills here, in the path
// that only tiles holding inf or NaN take. Scheduling barriers after
// each group of four lane exchanges keep the compiler from hoisting all 64
// of a stage at once.
template <int LOG_N>
__device__ __forceinline__ void stage_ordered_tile(__amdgpu_buffer_rsrc_t src, unsigned lane, unsigned lane_bytes,
                                                   __amdgpu_buffer_rsrc_t dst, float norm, float scale) {
    using U2 = __attribute__((ext_vector_type(2))) unsigned;
    // A fresh copy of the lane offset: addresses derived from it are computed
    // here, not shared with (and kept live from) the common path.
    asm volatile("" : "+v"(lane_bytes));
    float v[16][4];
#pragma unroll
    for (int i2 = 0; i2 < 16; ++i2) {
        const U2 raw = __builtin_amdgcn_raw_buffer_load_b64(src, int(lane_bytes + 512u * unsigned(i2)), 0, 0);
        const half4 a = __builtin_bit_cast(half4, raw);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i2][j] = float(a[j]);
    }
#pragma unroll
    for (int b = 0; b < LOG_N; ++b) {
        if (b < 2 || b >= 8) {  // both elements of a pair in this lane's registers
            const int dj = b < 2 ? 1 << b : 0, di = b >= 8 ? 1 << (b - 8) : 0;
#pragma unroll
            for (int i2 = 0; i2 < 16; ++i2)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if ((i2 & di) || (j & dj)) continue;
                    const float x = v[i2][j], y = v[i2 + di][j + dj];
                    v[i2][j] = x + y;
                    v[i2 + di][j + dj] = x - y;
                }
        } else {  // the partner lies in lane l ^ m; the upper lane keeps x - y
            const int m = b < 4 ? 16 << (b - 2) : 1 << (b - 4);
            const bool upper = (lane & unsigned(m)) != 0u;
#pragma unroll
            for (int i2 = 0; i2 < 16; ++i2) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float other = __shfl_xor(v[i2][j], m);
                    v[i2][j] = upper ? other - v[i2][j] : v[i2][j] + other;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#pragma unroll
    for (int i2 = 0; i2 < 16; ++i2) {
        const U2 packed = {unsigned(narrow(v[i2][0], norm, scale)) | (unsigned(narrow(v[i2][1], norm, scale)) << 16),
                           unsigned(narrow(v[i2][2], norm, scale)) | (unsigned(narrow(v[i2][3], norm, scale)) << 16)};
        __builtin_amdgcn_raw_buffer_store_b64(packed, dst, int(lane_bytes + 512u * unsigned(i2)), 0, 0);
    }
}

// Waves per SIMD: 4 where the register stages hold all 64 results, 5 for
// rows of up to 256 points.
constexpr int mfma_waves_per_simd(int log_n) { return log_n <= 8 ? 5 : 4; }

template <int LOG_N>
__global__ __launch_bounds__(64 * kWavesPerBlock) __attribute__((amdgpu_waves_per_eu(mfma_waves_per_simd(LOG_N))))
void fwht_mfma_kernel(const __half* __restrict__ input, __half* output, std::uint64_t total, float norm, float scale) {
    constexpr int t0 = LOG_N < 4 ? LOG_N : 4;                        // transform bits among 0..3
    constexpr int t1 = LOG_N <= 4 ? 0 : (LOG_N < 8 ? LOG_N - 4 : 4);  // among 4..7
    constexpr int t2 = LOG_N <= 8 ? 0 : LOG_N - 8;                    // among 8..11
    const unsigned lane = threadIdx.x & 63u;
    // The wave's tile, read back into scalar registers: the compiler treats
    // threadIdx.x >> 6 as divergent, and a buffer resource built from it sat
    // in vector registers, which wrapped every load and store in a
    // readfirstlane loop.
    const std::uint64_t tile = uniform(std::uint64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6));
    const std::uint64_t first = tile << kTileLog;
    if (first >= total) return;  // whole wave: no tile here
    // The tile's span (the last tile of a batch may be partial: the range
    // check zero-fills its loads and drops its stores past the data).
    const std::uint64_t left = total - first;
    const unsigned bytes = unsigned((left < (1u << kTileLog) ? left : (1u << kTileLog)) * sizeof(__half));
    const __amdgpu_buffer_rsrc_t src = make_rsrc(input + first, bytes);
    const __amdgpu_buffer_rsrc_t dst = make_rsrc(output + first, bytes);
    // Element offset of lane l's four halves within block i2: i1 = l % 16,
    // i0 = 4 (l / 16) .. +3 on the way in; k1 = l % 16, k0 likewise out.
    const unsigned lane_bytes = ((lane & 15u) * 16u + 4u * (lane >> 4)) * unsigned(sizeof(__half));

    const half4 m0 = hadamard_block(lane, t0);
    const half4 m1 = hadamard_block(lane, t1 > 0 ? t1 : 1);

    using U2 = __attribute__((ext_vector_type(2))) unsigned;
    using U4 = __attribute__((ext_vector_type(4))) unsigned;
    // Blocks 2p and 2p + 1 move together as one 16-byte access per lane
    // (1 KiB of consecutive elements per wave instruction): lanes of even
    // 16-lane groups g take elements 4g .. 4g + 7 of block 2p's 16-element
    // row l % 16, lanes of odd groups elements 4 (g - 1) .. 4 (g - 1) + 7 of
    // block 2p + 1's, and v_permlane16_swap (registers indexed by the old
    // lane bit 4 afterwards) trades the halves that belong to the other
    // group. Rows of 8 or more points keep every 16-byte access inside or
    // outside the tile's range; shorter ones load 8 bytes per block.
    const unsigned pair_bytes = (lane_bytes & ~15u) + 512u * ((lane >> 4) & 1u);
    half4 a[16];
    if constexpr (LOG_N >= 3) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const U4 raw = __builtin_amdgcn_raw_buffer_load_b128(src, int(pair_bytes + 1024u * unsigned(p)), 0, 0);
            const auto s0 = __builtin_amdgcn_permlane16_swap(raw[0], raw[2], false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(raw[1], raw[3], false, false);
            a[2 * p] = __builtin_bit_cast(half4, U2{s0[0], s1[0]});
            a[2 * p + 1] = __builtin_bit_cast(half4, U2{s0[1], s1[1]});
        }
    } else {
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
            const U2 raw = __builtin_amdgcn_raw_buffer_load_b64(src, int(lane_bytes + 512u * i2), 0, 0);
            a[i2] = __builtin_bit_cast(half4, raw);
        }
    }
    // Any inf or NaN in the wave's tile (exponent field all ones, i.e. a
    // half whose magnitude bits are 0x7c00 or more), from the per-half
    // maxima of the magnitude bits (a tree of packed 16-bit maxima): such a
    // tile runs the stage-ordered VALU transform instead, so rows stay
    // independent. (Deciding after the contractions, to overlap this with the
    // matrix cores, kept the inputs live across them and measured slower.)
    using u16x2 = __attribute__((ext_vector_type(2))) unsigned short;
    u16x2 mag[16];
#pragma unroll
    for (int i2 = 0; i2 < 16; ++i2) {
        const U2 raw = __builtin_bit_cast(U2, a[i2]);
        mag[i2] = __builtin_elementwise_max(__builtin_bit_cast(u16x2, raw[0] & 0x7fff7fffu),
                                            __builtin_bit_cast(u16x2, raw[1] & 0x7fff7fffu));
    }
#pragma unroll
    for (int span = 8; span >= 1; span >>= 1)
#pragma unroll
        for (int i2 = 0; i2 < span; ++i2) mag[i2] = __builtin_elementwise_max(mag[i2], mag[i2 + span]);
    const bool special = mag[0][0] >= 0x7c00u || mag[0][1] >= 0x7c00u;
    if (uniform(unsigned(__any(int(special)))) != 0u) {  // wave-uniform, and read into a scalar register so
                                                          // the compiler branches rather than masking both paths
        stage_ordered_tile<LOG_N>(src, lane, lane_bytes, dst, norm, scale);
        return;
    }

    float v[16][4];
#pragma unroll
    for (int i2 = 0; i2 < 16; ++i2) {
        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
        float4v d = __builtin_amdgcn_mfma_f32_16x16x16f16(a[i2], m0, zero, 0, 0, 0);
        if constexpr (t1 > 0) {
            // D0 / 16 = hi + lo; D1 = 16 (hi + lo) M1.
            float s[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = d[r] * 0.0625f;
            const pk16 h01 = __builtin_amdgcn_cvt_pkrtz(s[0], s[1]);
            const pk16 h23 = __builtin_amdgcn_cvt_pkrtz(s[2], s[3]);
            const pk16 l01 = __builtin_amdgcn_cvt_pkrtz(s[0] - float(h01[0]), s[1] - float(h01[1]));
            const pk16 l23 = __builtin_amdgcn_cvt_pkrtz(s[2] - float(h23[0]), s[3] - float(h23[1]));
            const U2 hi_bits = {__builtin_bit_cast(unsigned, h01), __builtin_bit_cast(unsigned, h23)};
            const U2 lo_bits = {__builtin_bit_cast(unsigned, l01), __builtin_bit_cast(unsigned, l23)};
            const half4 hi = __builtin_bit_cast(half4, hi_bits);
            const half4 lo = __builtin_bit_cast(half4, lo_bits);
            d = __builtin_amdgcn_mfma_f32_16x16x16f16(hi, m1, zero, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x16f16(lo, m1, d, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[i2][r] = d[r] * 16.0f;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) v[i2][r] = d[r];
        }
    }
    // Bits 8 .. 8 + t2 - 1 across the 16 blocks, in stage order.
#pragma unroll
    for (int b = 0; b < t2; ++b) {
        const int dist = 1 << b;
#pragma unroll
        for (int i2 = 0; i2 < 16; ++i2) {
            if ((i2 & dist) == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float x = v[i2][r], y = v[i2 + dist][r];
                    v[i2][r] = x + y;
                    v[i2 + dist][r] = x - y;
                }
            }
        }
    }
    if constexpr (t1 > 0) {
        // Blocks 2p and 2p + 1 leave as one 16-byte nontemporal store per
        // lane, the load's exchange run backwards: each output is written
        // once, and a wave instruction writes 1 KiB of consecutive output.
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            unsigned w[2][2];
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int d = 0; d < 2; ++d)
                    w[q][d] = unsigned(narrow(v[2 * p + q][2 * d], norm, scale)) |
                              (unsigned(narrow(v[2 * p + q][2 * d + 1], norm, scale)) << 16);
            const auto s0 = __builtin_amdgcn_permlane16_swap(w[0][0], w[1][0], false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(w[0][1], w[1][1], false, false);
            __builtin_amdgcn_raw_buffer_store_b128(U4{s0[0], s1[0], s0[1], s1[1]}, dst,
                                                   int(pair_bytes + 1024u * unsigned(p)), 0, 2);
        }
    } else {
        // Rows of <= 16 points: no second contraction, so lane l holds D0
        // rows i1 = 4 (l / 16) + r at column k0 = l % 16, 16 elements apart.
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const unsigned e = 256u * k2 + 16u * (4u * (lane >> 4) + unsigned(r)) + (lane & 15u);
                __builtin_amdgcn_raw_buffer_store_b16(narrow(v[k2][r], norm, scale), dst, int(e * sizeof(__half)), 0,
                                                      0);
            }
        }
    }
}

using MfmaLaunch = void (*)(const void*, void*, std::uint64_t, float, float, unsigned, hipStream_t);

template <int LOG_N>
void launch_mfma(const void* in, void* out, std::uint64_t total, float norm, float scale, unsigned grid,
                 hipStream_t stream) {
    hipLaunchKernelGGL(fwht_mfma_kernel<LOG_N>, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream,
                       static_cast<const __half*>(in), static_cast<__half*>(out), total, norm, scale);
}

template <int... L>
MfmaLaunch mfma_entry(int log_n, std::integer_sequence<int, L...>) {
    static constexpr MfmaLaunch table[] = {&launch_mfma<L + 1>...};
    return table[log_n - 1];
}

class FwhtMfmaExecutor final : public Executor {
  public:
    FwhtMfmaExecutor(const Request& r, MfmaLaunch launch) : r_(r), launch_(launch) {
        norm_ = r.normalize ? 1.0f / static_cast<float>(r.n) : 1.0f;
        scale_ = r.output_scale;
        total_ = r.n * r.batch;
        const std::uint64_t tiles = (total_ + (1ull << kTileLog) - 1) >> kTileLog;
        const std::uint64_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
        require(blocks <= 0x7fffffffull, "FWHT batch exceeds the MFMA lowering's grid");
        grid_ = static_cast<unsigned>(blocks);
        algorithm = fwht_mfma_name();
        reason = "MFMA 16x16 Hadamard blocks (v_mfma_f32_16x16x16_f16, fp32 accumulation; fp32 intermediates enter "
                 "the second contraction as hi + lo fp16 parts), bits 8+ butterflied in registers; one 4096-element "
                 "tile per wave, no LDS; accumulation order differs from the radix-2 stage order, so an output can "
                 "differ from the stage-ordered result by one fp16 ulp (beyond 2e-3 where |y| >= 4); tiles holding "
                 "inf or NaN run the stage-ordered radix-2 stages instead, keeping rows independent";
        const int t0 = r.log_n < 4 ? int(r.log_n) : 4;
        const int t1 = r.log_n <= 4 ? 0 : (r.log_n < 8 ? int(r.log_n) - 4 : 4);
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("operator", "fwht")
            .field("algorithm", algorithm)
            .field("log_n", r.log_n)
            .field("batch", r.batch)
            .field("tile_elements", std::uint64_t{1} << kTileLog)
            .field("tiles", tiles)
            .field("grid", grid_)
            .field("threads_per_block", 64u * kWavesPerBlock)
            .field("mfma_per_tile", 16u * (t1 > 0 ? 3u : 1u))
            .field("contraction_bits", unsigned(t0 + t1))
            .field("register_bits", unsigned(r.log_n > 8 ? r.log_n - 8 : 0))
            .field("lds_bytes", 0u)
            .end_object();
        mapping_json = w.str();
    }
    void execute(const void* in, void* out, void*, hipStream_t stream) override {
        launch_(in, out, total_, norm_, scale_, grid_, stream);
        hip_check(hipGetLastError(), "FWHT MFMA launch");
    }

  private:
    Request r_;
    MfmaLaunch launch_;
    float norm_ = 1.0f, scale_ = 1.0f;
    std::uint64_t total_ = 0;
    unsigned grid_ = 1;
};

}  // namespace

std::string fwht_mfma_name() { return "fwht-fp16-mfma16"; }

bool fwht_mfma_covers(const Request& r) {
    return r.fp16_final && !r.pitched && r.log_n >= 1 && r.log_n <= kMaxLog;
}

std::unique_ptr<Executor> make_fwht_mfma_executor(const Request& r) {
    supported(fwht_mfma_covers(r), "the MFMA Hadamard-block FWHT covers packed FP16 rows of 2 to 4096 points");
    return std::make_unique<FwhtMfmaExecutor>(r, mfma_entry(int(r.log_n), std::make_integer_sequence<int, kMaxLog>{}));
}

}  // namespace cbw
