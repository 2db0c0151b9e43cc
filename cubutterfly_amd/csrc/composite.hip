// Rank-2 and higher transforms composed from batched rank-1 plans (the
// reference's rank-two lowering, src/c_api.cpp:5231-5327, and its generic
// axis schedule, src/c_api.cpp:623-672, 5163-5219).
//
// Axes are transformed innermost first. Before each axis plan a batched
// tiled transpose moves that axis to the innermost (contiguous) position, so
// every axis plan is an ordinary packed batched rank-1 plan; after the last
// axis further transposes restore the original axis order. A batched
// transpose of G blocks of R x C elements covers every such move: the axes
// before the moved one form the blocks, the moved axis the rows, the axes
// after it the columns.
//
// A rank-2 FFT whose axes the row kernel's transposing store covers runs as
// two row passes instead: the rows of each 2^n0 x 2^n1 block transformed and
// stored transposed, then the rows of the transposed block, stored back in
// the original order (two HBM round trips where the transposes take four).
// The transposing store writes segments of 2^(14 - n) elements for rows of
// 2^n points; where an axis has 2^11 points or more (segments under 128
// bytes) the block runs instead as column passes over axis 0 and a row pass
// over axis 1 that stores whole rows (every segment 512 bytes or longer).
// Either lowering can be named (EXPLICIT) where its kernels cover the shape.
//
// FWHT needs none of this: the Sylvester Hadamard matrix of n0 * n1 points
// is the Kronecker product H(n0) (x) H(n1), and the innermost-first axis
// order applies the stages from the lowest index bit to the highest, which is
// the rank-1 stage order. A rank-N FWHT whose point count a single rank-1
// plan covers therefore runs as that one plan, bit-identically (the inverse
// with normalisation keeps the per-axis composition, whose per-axis 1/n
// scaling rounds differently in the subnormal range). Longer FWHTs, and
// rank-N ones normalised per axis, run the innermost axis as one packed row
// plan (at least 64 points) and every other axis, lowest bits first, as
// in-place column passes of at most 2^7 rows held in registers: the same
// stages in the same order, with no transposes. A rank-1 FWHT beyond 2^15
// points is factored into such axes and divides by n once, in its last pass.
//
// Strided sides and bit-reversed logical orders are handled as in the
// rank-1 semantic boundary: an N-dimensional gather into packed natural
// order first, an N-dimensional scatter last. A packed natural side is read
// or written directly by the first or last step.
//
// The zero-extended embedding (any rank, reference src/c_api.cpp:5231-5245,
// 5312-5325) runs the power-of-two transform of each axis's next power of
// two: the forward input side (logical extents) is gathered with zeros in
// the padding, the inverse output side keeps the first logical-extent
// elements of each axis.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <numeric>

#include "json.hpp"
#include "planner.hpp"

namespace cbw {
namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kTile = 64;  // transpose tile edge (elements)

inline std::size_t align16(std::size_t bytes) { return (bytes + 15) & ~std::size_t{15}; }

// dst[g][c][r] = src[g][r][c] for G blocks of 2^log_rows x 2^log_cols
// elements. Each workgroup moves 64 x 64 tiles through LDS: reads run along
// the source rows and writes along the destination rows, 64 consecutive
// elements per wave. The row pitch of 65 elements keeps the column-wise LDS
// reads on distinct banks.
template <class T>
__global__ __launch_bounds__(kThreads) void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                             std::uint64_t tiles, std::uint32_t log_rows,
                                                             std::uint32_t log_cols) {
    __shared__ T tile[kTile][kTile + 1];
    const std::uint32_t tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
    const std::uint64_t rows = std::uint64_t{1} << log_rows, cols = std::uint64_t{1} << log_cols;
    const std::uint32_t lr = log_rows > 6 ? log_rows - 6 : 0, lc = log_cols > 6 ? log_cols - 6 : 0;
    for (std::uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const std::uint64_t c0 = (t & ((std::uint64_t{1} << lc) - 1)) * kTile;
        const std::uint64_t r0 = ((t >> lc) & ((std::uint64_t{1} << lr) - 1)) * kTile;
        const std::uint64_t block = (t >> (lc + lr)) << (log_rows + log_cols);
        const T* s = src + block;
        T* d = dst + block;
        {
            const std::uint64_t c = c0 + tx;
#pragma unroll
            for (unsigned k = 0; k < kTile; k += kThreads / kTile) {
                const std::uint64_t r = r0 + ty + k;
                if (r < rows && c < cols) tile[ty + k][tx] = s[(r << log_cols) + c];
            }
        }
        __syncthreads();
        {
            const std::uint64_t r = r0 + tx;
#pragma unroll
            for (unsigned k = 0; k < kTile; k += kThreads / kTile) {
                const std::uint64_t c = c0 + ty + k;
                if (r < rows && c < cols) d[(c << log_rows) + r] = tile[tx][ty + k];
            }
        }
        __syncthreads();
    }
}

// One side of an N-dimensional layout: element (b, i_0 .. i_{rank-1}) of the
// packed natural buffer (power-of-two extents 2^log_extent[a]) is element
// b * batch_stride + sum_a r_a(i_a) * stride[a] of the side, r_a the
// log_extent[a]-bit reversal where bit a of `reversed` is set, else the
// identity. Elements with some i_a >= extent[a] (the side's own extent,
// shorter under the zero-extended embedding) are absent from the side: the
// gather reads them as zero, the scatter drops them.
struct NdSide {
    std::uint32_t rank = 0;
    std::uint32_t reversed = 0;
    std::uint32_t log_extent[kMaxRank] = {};
    std::uint64_t extent[kMaxRank] = {};
    std::uint64_t stride[kMaxRank] = {};
    std::uint64_t batch_stride = 0;
};

template <class T, bool GATHER>
__global__ __launch_bounds__(kThreads) void nd_boundary_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                               std::uint64_t count, NdSide side) {
    for (std::uint64_t linear = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; linear < count;
         linear += std::uint64_t(gridDim.x) * kThreads) {
        std::uint64_t rest = linear, physical = 0;
        bool present = true;
        for (int a = int(side.rank) - 1; a >= 0; --a) {
            const std::uint32_t l = side.log_extent[a];
            std::uint64_t i = rest & ((std::uint64_t{1} << l) - 1);
            rest >>= l;
            present = present && i < side.extent[a];
            if ((side.reversed >> a) & 1u) i = __brevll(i) >> (64u - l);
            physical += i * side.stride[a];
        }
        physical += rest * side.batch_stride;
        if constexpr (GATHER) dst[linear] = present ? src[physical] : T{};
        else if (present) dst[physical] = src[linear];
    }
}

template <class T>
void launch_transpose(const void* src, void* dst, std::uint64_t groups, std::uint32_t log_rows,
                      std::uint32_t log_cols, hipStream_t stream) {
    const std::uint32_t lr = log_rows > 6 ? log_rows - 6 : 0, lc = log_cols > 6 ? log_cols - 6 : 0;
    const std::uint64_t tiles = groups << (lr + lc);
    const std::uint64_t blocks = std::min<std::uint64_t>(tiles, std::uint64_t{1} << 20);
    hipLaunchKernelGGL((transpose_kernel<T>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                       static_cast<const T*>(src), static_cast<T*>(dst), tiles, log_rows, log_cols);
    hip_check(hipGetLastError(), "composite transpose launch");
}

template <class T>
void launch_nd_boundary(bool gather, const void* src, void* dst, std::uint64_t count, const NdSide& side,
                        hipStream_t stream) {
    const std::uint64_t blocks = std::min<std::uint64_t>((count + kThreads - 1) / kThreads, 65536);
    if (gather)
        hipLaunchKernelGGL((nd_boundary_kernel<T, true>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                           static_cast<const T*>(src), static_cast<T*>(dst), count, side);
    else
        hipLaunchKernelGGL((nd_boundary_kernel<T, false>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                           static_cast<const T*>(src), static_cast<T*>(dst), count, side);
    hip_check(hipGetLastError(), "composite gather / scatter launch");
}

// y = x * scale rounded to FP32, then to FP16 (round to nearest even). The
// empty asm keeps the two roundings apart: without it the compiler fuses the
// product and the narrowing into one v_fma_mixlo_f16, a single rounding of
// the exact product, which differs from the contract for scales that are not
// powers of two.
__device__ __forceinline__ __half narrow_scaled(float x, float scale) {
    float y = x * scale;
    asm volatile("" : "+v"(y));
    return __float2half_rn(y);
}

// FWHT stages over the row bits of G blocks of 2^LOG_L rows x 2^log_cols
// columns (row pitch 2^log_cols elements): for each block and column, the
// values x[i] of rows i = 0 .. 2^LOG_L - 1 go through the stages of bit 0,
// 1, ..., LOG_L - 1 of i (pairs i, i + h -> a + b, a - b), then are
// multiplied by `scale` where `apply_scale` is set. Each lane holds VEC
// consecutive columns of all the rows in registers, so one load instruction
// of a wave covers 64 * VEC consecutive elements of a row; no LDS and no
// barriers. A lane writes exactly the elements it read, so src == dst is
// allowed (no __restrict__). NARROW: the results leave as FP16,
// narrow_scaled(x, out_scale), at the same element offsets of `dst` (the
// FP32 promotion's final narrowing, fused into its last pass).
constexpr std::uint32_t kMaxColumnBits = 7;  // rows * VEC <= 128 registers of data

template <int VEC>
struct ColumnVector;
template <>
struct ColumnVector<1> {
    using type = float;
};
template <>
struct ColumnVector<2> {
    using type = float __attribute__((ext_vector_type(2)));
};
template <>
struct ColumnVector<4> {
    using type = float __attribute__((ext_vector_type(4)));
};

template <int VEC>
struct HalfVector;
template <>
struct HalfVector<1> {
    using type = unsigned short;
};
template <>
struct HalfVector<2> {
    using type = unsigned short __attribute__((ext_vector_type(2)));
};
template <>
struct HalfVector<4> {
    using type = unsigned short __attribute__((ext_vector_type(4)));
};

template <int LOG_L, int VEC, bool NARROW>
__global__ __launch_bounds__(kThreads) void fwht_columns_kernel(const float* src, void* dst, std::uint64_t vectors,
                                                                std::uint32_t log_cols, float scale, int apply_scale,
                                                                float out_scale) {
    constexpr int L = 1 << LOG_L;
    constexpr std::uint32_t kLogVec = VEC == 4 ? 2 : VEC == 2 ? 1 : 0;
    using V = typename ColumnVector<VEC>::type;
    const std::uint64_t v = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (v >= vectors) return;
    const std::uint32_t log_vectors = log_cols - kLogVec;  // column vectors per row
    const std::uint64_t block = v >> log_vectors;
    const std::uint64_t base = (block << (LOG_L + log_cols)) + ((v & ((std::uint64_t{1} << log_vectors) - 1)) << kLogVec);
    V x[L];
#pragma unroll
    for (int i = 0; i < L; ++i) x[i] = *reinterpret_cast<const V*>(src + base + (std::uint64_t(i) << log_cols));
#pragma unroll
    for (int h = 1; h < L; h <<= 1) {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            if ((i & h) == 0) {
                const V a = x[i], b = x[i + h];
                x[i] = a + b;
                x[i + h] = a - b;
            }
        }
    }
    if (apply_scale) {
#pragma unroll
        for (int i = 0; i < L; ++i) x[i] = x[i] * scale;
    }
    if constexpr (NARROW) {
        using H = typename HalfVector<VEC>::type;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            H h;
            if constexpr (VEC == 1) {
                h = __half_as_ushort(narrow_scaled(x[i], out_scale));
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) h[k] = __half_as_ushort(narrow_scaled(x[i][k], out_scale));
            }
            __builtin_nontemporal_store(
                h, reinterpret_cast<H*>(static_cast<unsigned short*>(dst) + base + (std::uint64_t(i) << log_cols)));
        }
    } else {
#pragma unroll
        for (int i = 0; i < L; ++i)
            __builtin_nontemporal_store(
                x[i], reinterpret_cast<V*>(static_cast<float*>(dst) + base + (std::uint64_t(i) << log_cols)));
    }
}

template <int LOG_L, bool NARROW>
void launch_fwht_columns_rows(const float* src, void* dst, std::uint64_t count, std::uint32_t log_cols, int vec,
                              float scale, bool apply_scale, float out_scale, hipStream_t stream) {
    const std::uint64_t vectors = count >> (LOG_L + (vec == 4 ? 2 : vec == 2 ? 1 : 0));
    const std::uint64_t blocks = (vectors + kThreads - 1) / kThreads;
    require(blocks < (std::uint64_t{1} << 31), "FWHT column pass grid too large");
    const dim3 grid{unsigned(blocks)}, block{kThreads};
    if constexpr (LOG_L <= 5) {
        if (vec == 4) {
            hipLaunchKernelGGL((fwht_columns_kernel<LOG_L, 4, NARROW>), grid, block, 0, stream, src, dst, vectors,
                               log_cols, scale, int(apply_scale), out_scale);
            return;
        }
    }
    if constexpr (LOG_L <= 6) {
        if (vec == 2) {
            hipLaunchKernelGGL((fwht_columns_kernel<LOG_L, 2, NARROW>), grid, block, 0, stream, src, dst, vectors,
                               log_cols, scale, int(apply_scale), out_scale);
            return;
        }
    }
    hipLaunchKernelGGL((fwht_columns_kernel<LOG_L, 1, NARROW>), grid, block, 0, stream, src, dst, vectors, log_cols,
                       scale, int(apply_scale), out_scale);
}

template <bool NARROW>
void launch_fwht_columns_of(const float* src, void* dst, std::uint64_t count, std::uint32_t log_rows,
                            std::uint32_t log_cols, int vec, float scale, bool apply_scale, float out_scale,
                            hipStream_t stream) {
    switch (log_rows) {
        case 1: launch_fwht_columns_rows<1, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
        case 2: launch_fwht_columns_rows<2, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
        case 3: launch_fwht_columns_rows<3, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
        case 4: launch_fwht_columns_rows<4, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
        case 5: launch_fwht_columns_rows<5, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
        case 6: launch_fwht_columns_rows<6, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
        default: launch_fwht_columns_rows<7, NARROW>(src, dst, count, log_cols, vec, scale, apply_scale, out_scale, stream); break;
    }
}

// Column pass over `count` FP32 elements (G blocks of 2^log_rows x
// 2^log_cols), src == dst allowed; with `narrow_out`, the results go there as
// FP16 (narrow_scaled(x, out_scale)) instead. The widest vector both
// pointers' alignment and the register budget allow.
void launch_fwht_columns(const float* src, float* dst, std::uint64_t count, std::uint32_t log_rows,
                         std::uint32_t log_cols, float scale, bool apply_scale, hipStream_t stream,
                         __half* narrow_out = nullptr, float out_scale = 1.0f) {
    require(log_rows >= 1 && log_rows <= kMaxColumnBits && log_cols >= 6, "FWHT column pass shape");
    const auto s = reinterpret_cast<std::uintptr_t>(src);
    int vec = s % 16 == 0 ? 4 : s % 8 == 0 ? 2 : 1;
    if (narrow_out) {  // VEC halves per store
        const auto d = reinterpret_cast<std::uintptr_t>(narrow_out);
        vec = std::min(vec, d % 8 == 0 ? 4 : d % 4 == 0 ? 2 : 1);
    } else {
        const auto d = reinterpret_cast<std::uintptr_t>(dst);
        vec = std::min(vec, d % 16 == 0 ? 4 : d % 8 == 0 ? 2 : 1);
    }
    if (log_rows == 6) vec = std::min(vec, 2);
    if (log_rows == 7) vec = 1;
    if (narrow_out)
        launch_fwht_columns_of<true>(src, narrow_out, count, log_rows, log_cols, vec, scale, apply_scale, out_scale,
                                     stream);
    else
        launch_fwht_columns_of<false>(src, dst, count, log_rows, log_cols, vec, scale, apply_scale, 1.0f, stream);
    hip_check(hipGetLastError(), "FWHT column pass launch");
}

// One step of the schedule: an axis plan, a batched transpose moving one
// axis innermost, or an in-place FWHT column pass over some bits of an axis.
struct Step {
    bool transpose = false;
    std::size_t child = 0;                // axis plan index (transpose == false)
    std::uint32_t axis = 0;               // logical axis it transforms
    std::uint64_t groups = 0;             // transpose / columns: blocks, log2 rows / cols
    std::uint32_t log_rows = 0, log_cols = 0;
    bool columns = false;                 // FWHT column pass (in place)
    bool apply_scale = false;             // columns: times `scale` after the stages
    float scale = 1.0f;
};

class CompositeExecutor final : public Executor {
  public:
    // force: 0 the static rule (or the name an EXPLICIT request gives), 1 a
    // rank-2 FFT's column passes, 2 its transposing row passes.
    CompositeExecutor(const Request& r, bool flatten, Selection* sel, int force = 0) : r_(r) {
        const std::uint32_t rank = r.rank;
        std::vector<std::uint32_t> logs(rank);
        for (std::uint32_t a = 0; a < rank; ++a) logs[a] = log2_u64(r.extents[a]);
        direct_in_ = packed_natural(true);
        direct_out_ = packed_natural(false);
        in_side_ = side(true, logs);
        out_side_ = side(false, logs);
        std::vector<std::string> names;
        // A rank-2 FFT named explicitly as one of its two lowerings takes that
        // one (EXPLICIT); otherwise column passes from 2^11-point axes.
        const bool named = r.policy == CUBUTTERFLY_ALGORITHM_EXPLICIT;
        const bool want_columns = force == 1 || (named && r.explicit_algorithm.rfind("rank2-columns[", 0) == 0);
        const bool want_rows = force == 2 || (named && r.explicit_algorithm.rfind("rank2-transposing[", 0) == 0);
        if (!flatten && r.op == Op::Fft && rank == 2 && !want_rows &&
            (want_columns || std::max(logs[0], logs[1]) >= 11)) {
            // Axis 0 as column passes over each block, then the rows.
            auto cols = make_fft_rank2_columns(axis_request(r.n, r.batch), logs[0]);
            if (cols) {
                columns_ = true;
                children_.push_back(std::move(cols));
                steps_.push_back(Step{false, 0, 0, 0, 0, 0});
            }
        }
        if (!columns_ && !want_columns && !flatten && r.op == Op::Fft && rank == 2) {
            // Each axis as one row pass that stores its blocks transposed:
            // rows of the caller's layout, then rows of the transposed one,
            // which lands back in the original order. No transpose kernels.
            const std::uint64_t n0 = r.extents[0], n1 = r.extents[1];
            auto rows1 = make_fft_rows_transposed(axis_request(n1, r.batch * n0), logs[0]);
            auto rows0 = make_fft_rows_transposed(axis_request(n0, r.batch * n1), logs[1]);
            if (rows1 && rows0) {
                transposing_ = true;
                children_.push_back(std::move(rows1));
                children_.push_back(std::move(rows0));
                steps_.push_back(Step{false, 0, 1, 0, 0, 0});
                steps_.push_back(Step{false, 1, 0, 0, 0, 0});
            }
        }
        if (transposing_ || columns_) {
        } else if (flatten) {
            children_.push_back(plan_executor(axis_request(r.n, r.batch), sel));
            steps_.push_back(Step{false, 0, 0, 0, 0, 0});
        } else if (r.op == Op::Fwht && rank >= 2 && r.element_bytes == 4 && logs[rank - 1] >= 6) {
            // FWHT: the innermost axis as one packed row plan, then every
            // other axis, lowest bits first, as in-place column passes of at
            // most 2^7 rows over rows at least 64 elements long -- the
            // stages in index-bit order, no transposes. A factored rank-1
            // FWHT divides by n once, after its last stage (the reference's
            // rank-1 normalisation); a rank-N FWHT by each axis's extent
            // after that axis.
            fwht_columns_ = true;
            const bool normalise = r.inverse && r.normalize;
            Request rows = axis_request(r.extents[rank - 1], r.batch * (r.n / r.extents[rank - 1]));
            if (r.factored) rows.normalize = false;
            children_.push_back(plan_executor(rows, sel));
            Step first;
            first.axis = rank - 1;
            steps_.push_back(first);
            std::uint32_t log_cols = logs[rank - 1];
            for (std::uint32_t a = rank - 1; a-- > 0;) {
                const std::uint32_t bits = logs[a];
                const std::uint32_t chunks = (bits + kMaxColumnBits - 1) / kMaxColumnBits;
                std::uint32_t done = 0;
                for (std::uint32_t k = 0; k < chunks; ++k) {
                    Step s;
                    s.columns = true;
                    s.axis = a;
                    s.log_rows = (bits - done) / (chunks - k);  // balanced chunks
                    s.log_cols = log_cols + done;
                    s.groups = r.batch * (r.n >> (s.log_rows + s.log_cols));
                    done += s.log_rows;
                    if (normalise && done == bits && (!r.factored || a == 0)) {
                        s.apply_scale = true;
                        s.scale = static_cast<float>(1.0 / double(r.factored ? r.n : r.extents[a]));
                    }
                    steps_.push_back(s);
                }
                log_cols += bits;
            }
        } else {
            // Innermost axis first; each axis is first moved innermost.
            std::vector<std::uint32_t> order(rank);
            std::iota(order.begin(), order.end(), 0u);
            const auto move_innermost = [&](std::uint32_t axis) {
                const auto pos = std::size_t(std::find(order.begin(), order.end(), axis) - order.begin());
                if (pos + 1 == rank) return;
                Step s;
                s.transpose = true;
                s.groups = r.batch;
                for (std::size_t i = 0; i < pos; ++i) s.groups <<= logs[order[i]];
                s.log_rows = logs[axis];
                for (std::size_t i = pos + 1; i < rank; ++i) s.log_cols += logs[order[i]];
                steps_.push_back(s);
                order.erase(order.begin() + std::ptrdiff_t(pos));
                order.push_back(axis);
            };
            for (std::uint32_t k = 0; k < rank; ++k) {
                const std::uint32_t axis = rank - 1 - k;
                move_innermost(axis);
                const std::uint64_t e = r.extents[axis];
                children_.push_back(plan_executor(axis_request(e, r.batch * (r.n / e)), sel));
                Step s;
                s.child = children_.size() - 1;
                s.axis = axis;
                steps_.push_back(s);
            }
            for (std::uint32_t axis = 0; axis < rank; ++axis) move_innermost(axis);
        }
        for (const auto& c : children_) {
            if (!fwht_columns_) names.push_back(c->algorithm);
            child_ws_ = std::max(child_ws_, c->workspace_bytes());
        }
        if (fwht_columns_)
            for (const auto& s : steps_)
                names.push_back(s.columns ? "fwht-fp32-columns-l" + std::to_string(s.log_rows)
                                          : children_[s.child]->algorithm);
        std::string joined;
        for (std::size_t i = 0; i < names.size(); ++i) joined += (i ? "," : "") + names[i];
        algorithm = std::string(r.factored     ? "fwht-factored"
                                : rank == 1    ? "zero-extended"
                                : transposing_ ? "rank2-transposing"
                                : columns_     ? "rank2-columns"
                                : fwht_columns_ ? (rank == 2 ? "rank2-fwht-columns" : "rankN-fwht-columns")
                                : flatten      ? (rank == 2 ? "rank2-kronecker" : "rankN-kronecker")
                                               : (rank == 2 ? "rank2-transpose" : "rankN-composite")) +
                    "[" + joined + "]" + (direct_in_ ? "+direct-input" : "") + (direct_out_ ? "+direct-output" : "");
        reason = transposing_ ? "each axis one row pass with a transposing store (innermost axis first)"
                 : columns_   ? "axis 0 as column passes over each block, then the rows stored in natural order"
                 : fwht_columns_
                     ? "innermost axis one row plan, the other axes in-place column passes of at most 2^7 rows "
                       "(FWHT stages in index-bit order, no transposes)"
                 : flatten    ? "FWHT of the flattened point count: H(n0 n1) = H(n0) (x) H(n1), same stage order"
                              : "one batched rank-1 plan per axis, innermost first, tiled transposes between";
        if (r.embedding) reason += "; sides zero-extended to / cut from the power-of-two extents";
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("kind", "composition")
            .field("rank", rank)
            .field("lowering", transposing_ ? "transposing-rows"
                               : columns_   ? "columns-then-rows"
                               : fwht_columns_ ? "rows-then-columns"
                               : flatten    ? "kronecker"
                                            : "transpose")
            .field("zero_extended", r.embedding);
        w.begin_array("extents");
        for (auto e : r.extents) w.value(e);
        w.end_array();
        w.begin_array("input_extents");
        for (auto e : r.in_extents) w.value(e);
        w.end_array();
        w.begin_array("output_extents");
        for (auto e : r.out_extents) w.value(e);
        w.end_array();
        w.begin_array("schedule");
        for (const auto& s : steps_) {
            w.begin_object();
            if (s.columns) {
                w.field("step", "columns").field("axis", s.axis).field("blocks", s.groups)
                    .field("rows", std::uint64_t{1} << s.log_rows).field("cols", std::uint64_t{1} << s.log_cols)
                    .field("scale", s.apply_scale ? double(s.scale) : 1.0);
            } else if (s.transpose) {
                w.field("step", "transpose").field("blocks", s.groups).field("rows", std::uint64_t{1} << s.log_rows)
                    .field("cols", std::uint64_t{1} << s.log_cols);
            } else if (columns_) {
                w.field("step", "axes");
                w.begin_array("axes").value(0u).value(1u).end_array();
                w.key("child").value_raw(children_[s.child]->mapping_json);
            } else {
                w.field("step", "axis").field("axis", s.axis).key("child").value_raw(children_[s.child]->mapping_json);
            }
            w.end_object();
        }
        w.end_array();
        w.field("direct_input_boundary", direct_in_)
            .field("direct_output_boundary", direct_out_)
            .field("workspace_bytes", std::uint64_t(workspace_bytes()))
            .end_object();
        mapping_json = w.str();
    }

    // Ping-pong buffers of the packed data the schedule touches (0, 1 or 2):
    // the gather's target, then every step's destination but a direct last one.
    std::size_t buffers() const {
        std::size_t used = direct_in_ ? 0 : 1;
        int next = direct_in_ ? 0 : 1;
        for (std::size_t i = 0; i < steps_.size(); ++i) {
            if (steps_[i].columns) continue;  // in place
            if (i == last_moving() && direct_out_) break;
            used = std::max<std::size_t>(used, std::size_t(next) + 1);
            next ^= 1;
        }
        return used;
    }

    // The last step that writes a new buffer (the in-place column passes
    // after it run on its destination).
    std::size_t last_moving() const {
        std::size_t last = 0;
        for (std::size_t i = 0; i < steps_.size(); ++i)
            if (!steps_[i].columns) last = i;
        return last;
    }

    bool columns() const { return columns_; }
    bool transposing() const { return transposing_; }

    std::size_t workspace_bytes() const override {
        // The ping-pong buffers, then the largest child's workspace.
        return buffers() * align16(r_.data_bytes()) + align16(child_ws_);
    }

    void execute(const void* in, void* out, void* ws, hipStream_t stream) override {
        run(in, out, ws, stream, nullptr, 1.0f);
    }

    // Whether run() can narrow to FP16 in the last step: an FWHT whose
    // schedule ends with a column pass, on packed natural sides.
    bool narrows() const { return fwht_columns_ && direct_in_ && direct_out_ && steps_.back().columns; }

    // execute(); with `narrow`, the last column pass writes its results there
    // as FP16, narrow_scaled(x, out_scale), instead of to `out` (which the
    // earlier steps still use). Needs narrows().
    void run(const void* in, void* out, void* ws, hipStream_t stream, __half* narrow, float out_scale) {
        require(narrow == nullptr || narrows(), "FP16 narrowing needs a final FWHT column pass");
        const std::size_t bytes = align16(r_.data_bytes());
        const std::size_t ws_bytes = workspace_bytes();
        require(ws_bytes == 0 || ws != nullptr, "a composite plan needs its workspace");
        auto* base = static_cast<unsigned char*>(ws);
        unsigned char* buffer[2] = {base, base + bytes};
        void* child_ws = child_ws_ ? base + buffers() * bytes : nullptr;
        const std::uint64_t count = r_.n * r_.batch;

        // Ping-pong: the next destination is the buffer the current data is
        // not in (the caller's input counts as neither).
        int next = 0;
        const void* cur = in;
        void* cur_writable = nullptr;  // cur, once it is no longer the caller's input
        if (!direct_in_) {
            move(true, in, buffer[0], count, in_side_, stream);
            cur = cur_writable = buffer[0];
            next = 1;
        }
        const std::size_t last = last_moving();
        for (std::size_t i = 0; i < steps_.size(); ++i) {
            const auto& s = steps_[i];
            if (s.columns) {
                require(cur_writable != nullptr, "an FWHT column pass runs on a step's destination");
                const bool narrow_here = narrow != nullptr && i + 1 == steps_.size();
                launch_fwht_columns(static_cast<const float*>(cur_writable), static_cast<float*>(cur_writable),
                                    count, s.log_rows, s.log_cols, s.scale, s.apply_scale, stream,
                                    narrow_here ? narrow : nullptr, out_scale);
                continue;
            }
            void* dst = i == last && direct_out_ ? out : buffer[next];
            if (s.transpose) transpose(cur, dst, s, stream);
            else children_[s.child]->execute(cur, dst, child_ws, stream);
            cur = cur_writable = dst;
            next = dst == buffer[0] ? 1 : 0;
        }
        if (!direct_out_) move(false, cur, out, count, out_side_, stream);
    }

    // Whether a rank-2 FFT request has both lowerings (no device work).
    static bool both_rank2_lowerings(const Request& r) {
        const std::uint32_t l0 = log2_u64(r.extents[0]), l1 = log2_u64(r.extents[1]);
        return fft_rank2_columns_available(axis_request_of(r, r.n, r.batch), l0) &&
               fft_rows_transposed_available(axis_request_of(r, r.extents[1], r.batch * r.extents[0]), l0) &&
               fft_rows_transposed_available(axis_request_of(r, r.extents[0], r.batch * r.extents[1]), l1);
    }

  private:
    Request axis_request(std::uint64_t n, std::uint64_t batch) const { return axis_request_of(r_, n, batch); }
    static Request axis_request_of(const Request& r, std::uint64_t n, std::uint64_t batch) {
        Request c = r;
        c.rank = 1;
        c.extents.clear();
        c.in_strides.clear();
        c.out_strides.clear();
        c.in_reversed.clear();
        c.out_reversed.clear();
        c.embedding = false;
        c.factored = false;
        c.in_extents.clear();
        c.out_extents.clear();
        c.n = n;
        c.log_n = log2_u64(n);
        c.batch = batch;
        c.boundary = false;
        c.in_place = false;
        c.input_bit_reversed = c.output_bit_reversed = false;
        c.in_stride = c.out_stride = 1;
        c.in_batch_stride = c.out_batch_stride = n;
        c.policy = CUBUTTERFLY_ALGORITHM_DEFAULT;
        c.explicit_algorithm.clear();
        c.variant.clear();
        return c;
    }

    bool packed_natural(bool input) const {
        const auto& strides = input ? r_.in_strides : r_.out_strides;
        const auto& reversed = input ? r_.in_reversed : r_.out_reversed;
        const auto& side = input ? r_.in_extents : r_.out_extents;
        std::uint64_t expect = 1;
        for (std::size_t a = r_.rank; a-- > 0;) {
            if (strides[a] != expect || reversed[a] || side[a] != r_.extents[a]) return false;
            expect *= r_.extents[a];
        }
        return r_.batch == 1 || (input ? r_.in_batch_stride : r_.out_batch_stride) == r_.n;
    }

    NdSide side(bool input, const std::vector<std::uint32_t>& logs) const {
        NdSide s;
        s.rank = r_.rank;
        const auto& strides = input ? r_.in_strides : r_.out_strides;
        const auto& reversed = input ? r_.in_reversed : r_.out_reversed;
        const auto& side = input ? r_.in_extents : r_.out_extents;
        for (std::uint32_t a = 0; a < r_.rank; ++a) {
            s.log_extent[a] = logs[a];
            s.extent[a] = side[a];
            s.stride[a] = strides[a];
            if (reversed[a]) s.reversed |= 1u << a;
        }
        s.batch_stride = input ? r_.in_batch_stride : r_.out_batch_stride;
        return s;
    }

    void transpose(const void* src, void* dst, const Step& s, hipStream_t stream) const {
        switch (r_.element_bytes) {
            case 4: launch_transpose<std::uint32_t>(src, dst, s.groups, s.log_rows, s.log_cols, stream); break;
            case 8: launch_transpose<std::uint64_t>(src, dst, s.groups, s.log_rows, s.log_cols, stream); break;
            default: throw NotSupported("transpose element size has no gfx950 kernel");
        }
    }

    void move(bool gather, const void* src, void* dst, std::uint64_t count, const NdSide& side,
              hipStream_t stream) const {
        switch (r_.element_bytes) {
            case 4: launch_nd_boundary<std::uint32_t>(gather, src, dst, count, side, stream); break;
            case 8: launch_nd_boundary<std::uint64_t>(gather, src, dst, count, side, stream); break;
            default: throw NotSupported("boundary element size has no gfx950 kernel");
        }
    }

    Request r_;
    bool transposing_ = false, columns_ = false, fwht_columns_ = false;
    bool direct_in_ = false, direct_out_ = false;
    NdSide in_side_, out_side_;
    std::vector<std::unique_ptr<Executor>> children_;
    std::vector<Step> steps_;
    std::size_t child_ws_ = 0;
};

// FP16 final-storage FWHT rows of more than 2^15 points: the reference's
// FP32 promotion (src/butterfly.cu:1452-1470) -- the input widened into an
// FP32 buffer, the factored FP32 transform in place on it (with the
// inverse's 1/n), then y * scale rounded to FP32 and narrowed once to FP16
// (round to nearest even) -- which is the stage-ordered FP32 transform
// narrowed once, as the one-tile FP16 kernels compute it. The narrowing runs
// in the factored plan's last column pass, which stores FP16 straight to the
// output.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void widen_f16_kernel(const __half* __restrict__ src, float* __restrict__ dst,
                                                             std::uint64_t count) {
    const std::uint64_t step = std::uint64_t(gridDim.x) * kThreads;
    if constexpr (VEC) {  // 8 halves per 16-byte load, both sides 16-byte aligned
        for (std::uint64_t c = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; c < count / 8; c += step) {
            const uint4 raw = reinterpret_cast<const uint4*>(src)[c];
            const unsigned w[4] = {raw.x, raw.y, raw.z, raw.w};
            float f[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                f[2 * k] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[k] & 0xffffu)));
                f[2 * k + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[k] >> 16)));
            }
            reinterpret_cast<float4*>(dst)[2 * c] = make_float4(f[0], f[1], f[2], f[3]);
            reinterpret_cast<float4*>(dst)[2 * c + 1] = make_float4(f[4], f[5], f[6], f[7]);
        }
    } else {
        for (std::uint64_t i = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += step)
            dst[i] = __half2float(src[i]);
    }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void narrow_f16_kernel(const float* __restrict__ src, __half* __restrict__ dst,
                                                              std::uint64_t count, float scale) {
    const std::uint64_t step = std::uint64_t(gridDim.x) * kThreads;
    if constexpr (VEC) {
        for (std::uint64_t c = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; c < count / 8; c += step) {
            const float4 a = reinterpret_cast<const float4*>(src)[2 * c];
            const float4 b = reinterpret_cast<const float4*>(src)[2 * c + 1];
            const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            unsigned w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w[k] = unsigned(__half_as_ushort(narrow_scaled(f[2 * k], scale))) |
                       (unsigned(__half_as_ushort(narrow_scaled(f[2 * k + 1], scale))) << 16);
            reinterpret_cast<uint4*>(dst)[c] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else {
        for (std::uint64_t i = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += step)
            dst[i] = narrow_scaled(src[i], scale);
    }
}

class FwhtPromotedExecutor final : public Executor {
  public:
    FwhtPromotedExecutor(const Request& r, Selection* sel) : r_(r) {
        Request c = r;
        c.storage = CUBUTTERFLY_DATA_FP32;
        c.element_bytes = sizeof(float);
        c.fp16_final = false;
        c.allow_mma = false;
        c.output_scale = 1.0f;
        c.in_place = false;
        c.policy = CUBUTTERFLY_ALGORITHM_DEFAULT;
        c.explicit_algorithm.clear();
        c.variant.clear();
        factor_long_fwht(c);
        child_ = make_composite_executor(c, sel);
        auto* composite = dynamic_cast<CompositeExecutor*>(child_.get());
        fused_ = composite != nullptr && composite->narrows() ? composite : nullptr;
        f32_bytes_ = align16(c.data_bytes());
        algorithm = "fwht-fp16-promoted[" + child_->algorithm + "]";
        reason = "FP16 rows beyond one resident tile: widened to FP32, the factored FP32 transform, one final "
                 "narrowing of y * scale" + std::string(fused_ ? " (in the last column pass)" : "") +
                 "; child: " + child_->reason;
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("kind", "fp32-promotion")
            .field("operator", "fwht")
            .field("algorithm", algorithm)
            .field("log_n", r.log_n)
            .field("batch", r.batch)
            .field("fp32_buffer_bytes", std::uint64_t(f32_bytes_))
            .field("narrowing", fused_ ? "last-column-pass" : "separate-pass")
            .key("child")
            .value_raw(child_->mapping_json)
            .end_object();
        mapping_json = w.str();
    }

    std::size_t workspace_bytes() const override { return f32_bytes_ + child_->workspace_bytes(); }

    void execute(const void* in, void* out, void* ws, hipStream_t stream) override {
        require(ws != nullptr, "the FP32 promotion needs its workspace");
        auto* buffer = static_cast<float*>(ws);
        void* child_ws = child_->workspace_bytes() ? static_cast<unsigned char*>(ws) + f32_bytes_ : nullptr;
        const std::uint64_t count = r_.n * r_.batch;
        const bool vec = reinterpret_cast<std::uintptr_t>(in) % 16 == 0 && reinterpret_cast<std::uintptr_t>(out) % 16 == 0;
        const std::uint64_t work = vec ? count / 8 : count;
        const unsigned blocks = unsigned(std::min<std::uint64_t>((work + kThreads - 1) / kThreads, 65536));
        const auto* src = static_cast<const __half*>(in);
        auto* dst = static_cast<__half*>(out);
        if (vec)
            hipLaunchKernelGGL((widen_f16_kernel<true>), dim3(blocks), dim3(kThreads), 0, stream, src, buffer, count);
        else
            hipLaunchKernelGGL((widen_f16_kernel<false>), dim3(blocks), dim3(kThreads), 0, stream, src, buffer, count);
        hip_check(hipGetLastError(), "FP16 widening launch");
        if (fused_) {
            fused_->run(buffer, buffer, child_ws, stream, dst, r_.output_scale);
            return;
        }
        child_->execute(buffer, buffer, child_ws, stream);
        if (vec)
            hipLaunchKernelGGL((narrow_f16_kernel<true>), dim3(blocks), dim3(kThreads), 0, stream, buffer, dst, count,
                               r_.output_scale);
        else
            hipLaunchKernelGGL((narrow_f16_kernel<false>), dim3(blocks), dim3(kThreads), 0, stream, buffer, dst, count,
                               r_.output_scale);
        hip_check(hipGetLastError(), "FP16 narrowing launch");
    }

  private:
    Request r_;
    std::unique_ptr<Executor> child_;
    CompositeExecutor* fused_ = nullptr;  // child_, when it narrows in its last pass
    std::size_t f32_bytes_ = 0;
};

}  // namespace

std::unique_ptr<Executor> make_composite_executor(const Request& r, Selection* sel) {
    require(r.rank >= 1 && r.rank <= kMaxRank && r.extents.size() == r.rank &&
                (r.rank >= 2 || r.embedding || r.factored),
            "composite plans need rank 2 to 8, the zero-extended embedding or a factored FWHT");
    // A flattened FWHT is one rank-1 plan; it exists up to the resident length.
    const bool flatten = r.op == Op::Fwht && !(r.inverse && r.normalize) && r.log_n <= kMaxFwhtRowLog;
    // A rank-2 FFT with both lowerings: MEASURE times the two, DEFAULT
    // replays a selection-cache record of that choice (keyed by the extents
    // too), the static rule decides otherwise.
    if (!flatten && r.op == Op::Fft && r.rank == 2 && !r.embedding && sel != nullptr &&
        r.policy != CUBUTTERFLY_ALGORITHM_EXPLICIT &&
        (sel->policy == CUBUTTERFLY_ALGORITHM_MEASURE ||
         (sel->policy == CUBUTTERFLY_ALGORITHM_DEFAULT && !sel->cache_path.empty()))) {
        const std::string key = selection_key(r) + "|rank2-fft|" + std::to_string(r.extents[0]) + "x" +
                                std::to_string(r.extents[1]);
        if (sel->policy == CUBUTTERFLY_ALGORITHM_DEFAULT) {
            const std::string cached = lookup_cache(sel->cache_path, key);
            const int force = cached.rfind("rank2-columns[", 0) == 0       ? 1
                              : cached.rfind("rank2-transposing[", 0) == 0 ? 2
                                                                           : 0;
            if (force) {
                auto e = std::make_unique<CompositeExecutor>(r, flatten, sel, force);
                if (e->algorithm == cached) {
                    combine_source(*sel, CUBUTTERFLY_SELECTION_USER_CACHE);
                    note_selection(*sel, "replayed '" + cached + "' from the selection cache");
                    return e;
                }
                note_selection(*sel, "ignored cache record '" + cached + "' (not a lowering of this request)");
            }
        } else if (CompositeExecutor::both_rank2_lowerings(r)) {
            require_no_capture(*sel);
            auto cols = std::make_unique<CompositeExecutor>(r, flatten, sel, 1);
            auto rows = std::make_unique<CompositeExecutor>(r, flatten, sel, 2);
            if (cols->columns() && rows->transposing()) {
                std::vector<std::unique_ptr<Executor>> alternatives;
                alternatives.push_back(std::move(cols));
                alternatives.push_back(std::move(rows));
                const std::size_t best = measure_executors(r, key, alternatives, *sel);
                if (best < alternatives.size()) return std::move(alternatives[best]);
            }
        }
    }
    return std::make_unique<CompositeExecutor>(r, flatten, sel);
}

std::unique_ptr<Executor> make_long_fwht_executor(const Request& r, Selection* sel) {
    require(r.op == Op::Fwht && r.rank == 1 && r.log_n > kMaxFwhtRowLog && !r.boundary,
            "a packed rank-1 FWHT beyond one resident row");
    if (r.fp16_final) return std::make_unique<FwhtPromotedExecutor>(r, sel);
    Request f = r;
    factor_long_fwht(f);
    return make_composite_executor(f, sel);
}

}  // namespace cbw
