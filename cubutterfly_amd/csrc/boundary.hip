// Semantic boundary for strided sides and FWHT / FFT logical orders: gather
// the input into packed natural order, run the packed transform, scatter the
// result (the reference's boundary plan, src/c_api.cpp:3085-3130, 5064-5085,
// with its ordered gather / scatter, src/general_kernels.cu:30-54, 475-535).
// A side already packed in natural order is used by the packed transform
// directly.
//
// Element (b, j) of the packed buffer is element b * batch_stride +
// r(j) * stride of the strided side, r(j) = j, or the log2 n-bit reversal of j
// for a bit-reversed logical order. Each thread moves consecutive packed
// elements, so the packed side is coalesced; the strided side is as
// contiguous as its stride allows. Bit-reversed unit-stride rows of 2^10
// elements or more move through 32 x 32 LDS tiles, coalesced on both sides.
#include <hip/hip_runtime.h>

#include "json.hpp"
#include "planner.hpp"

namespace cbw {
namespace {

constexpr unsigned kThreads = 256;

template <class T, bool GATHER>
__global__ __launch_bounds__(kThreads) void boundary_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                            std::uint64_t count, std::uint32_t log_n,
                                                            std::uint64_t stride, std::uint64_t batch_stride,
                                                            bool reversed) {
    const std::uint64_t mask = (std::uint64_t{1} << log_n) - 1u;
    for (std::uint64_t linear = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; linear < count;
         linear += std::uint64_t(gridDim.x) * kThreads) {
        const std::uint64_t j = linear & mask;
        const std::uint64_t r = reversed ? (__brevll(j) >> (64u - log_n)) : j;
        const std::uint64_t physical = (linear >> log_n) * batch_stride + r * stride;
        if constexpr (GATHER) dst[linear] = src[physical];
        else dst[physical] = src[linear];
    }
}

// Unit stride in natural order (pitched rows): 16-byte chunks of a row,
// V = 16 / sizeof(element) elements each, both sides 16-byte aligned.
template <bool GATHER>
__global__ __launch_bounds__(kThreads) void pitched_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                           std::uint64_t chunks, std::uint32_t row_log,
                                                           std::uint64_t pitch) {
    const std::uint64_t mask = (std::uint64_t{1} << row_log) - 1u;
    for (std::uint64_t linear = std::uint64_t(blockIdx.x) * kThreads + threadIdx.x; linear < chunks;
         linear += std::uint64_t(gridDim.x) * kThreads) {
        const std::uint64_t physical = (linear >> row_log) * pitch + (linear & mask);
        if constexpr (GATHER) dst[linear] = src[physical];
        else dst[physical] = src[linear];
    }
}

// Bit reversal of rows of n = 2^m >= 2^10 elements at unit stride, through
// 32 x 32 tiles in LDS. Index j = hi 2^(m-5) + mid 2^5 + lo (hi, lo: 5 bits)
// maps to bitrev(j) = bitrev(lo) 2^(m-5) + bitrev(mid) 2^5 + bitrev(hi), so
// the elements of one (row, mid) tile are read as 32 runs of 32 consecutive
// elements (over lo) and written as 32 runs of 32 consecutive elements (over
// bitrev(hi)). The permutation is its own inverse, so gathers and scatters
// both use it: dst[d_base + p] = src[s_base + bitrev(p)] within each row,
// with the rows src_pitch / dst_pitch elements apart.
constexpr std::uint32_t kRevBits = 5, kRev = 1u << kRevBits;

template <class T>
__global__ __launch_bounds__(kThreads) void bitrev_rows_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                               std::uint64_t tiles, std::uint32_t log_n,
                                                               std::uint64_t src_pitch, std::uint64_t dst_pitch) {
    __shared__ T tile[kRev][kRev + 1];
    const std::uint32_t mid_bits = log_n - 2 * kRevBits;
    const std::uint64_t mids = std::uint64_t{1} << mid_bits;
    const std::uint32_t high_shift = log_n - kRevBits;
    for (std::uint64_t w = blockIdx.x; w < tiles; w += gridDim.x) {
        const std::uint64_t row = w >> mid_bits;
        const std::uint32_t mid = std::uint32_t(w & (mids - 1u));
        const std::uint32_t rmid = mid_bits ? __brev(mid) >> (32u - mid_bits) : 0u;
        const T* s = src + row * src_pitch + (std::uint64_t(mid) << kRevBits);
        T* d = dst + row * dst_pitch + (std::uint64_t(rmid) << kRevBits);
#pragma unroll
        for (std::uint32_t k = 0; k < kRev * kRev / kThreads; ++k) {
            const std::uint32_t e = threadIdx.x + k * kThreads, hi = e >> kRevBits, lo = e & (kRev - 1u);
            tile[hi][lo] = s[(std::uint64_t(hi) << high_shift) + lo];
        }
        __syncthreads();
#pragma unroll
        for (std::uint32_t k = 0; k < kRev * kRev / kThreads; ++k) {
            // Output run over bitrev(hi) = q in destination row bitrev(lo).
            const std::uint32_t e = threadIdx.x + k * kThreads, lo = e >> kRevBits, q = e & (kRev - 1u);
            const std::uint32_t rlo = __brev(lo) >> (32u - kRevBits), hi = __brev(q) >> (32u - kRevBits);
            d[(std::uint64_t(rlo) << high_shift) + q] = tile[hi][lo];
        }
        __syncthreads();
    }
}

template <class T>
void launch_boundary(bool gather, const void* src, void* dst, std::uint64_t count, std::uint32_t log_n,
                     std::uint64_t stride, std::uint64_t batch_stride, bool reversed, hipStream_t stream) {
    constexpr std::uint32_t kPerChunk = 16 / sizeof(T);
    if (reversed && stride == 1 && log_n >= 2 * kRevBits) {
        const std::uint64_t tiles = count >> (2 * kRevBits);
        const std::uint64_t blocks = std::min<std::uint64_t>(tiles, std::uint64_t{1} << 20);
        const std::uint64_t n = std::uint64_t{1} << log_n;
        hipLaunchKernelGGL((bitrev_rows_kernel<T>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                           static_cast<const T*>(src), static_cast<T*>(dst), tiles, log_n,
                           gather ? batch_stride : n, gather ? n : batch_stride);
        hip_check(hipGetLastError(), "boundary bit-reversal launch");
        return;
    }
    if (!reversed && stride == 1 && (std::uint64_t{1} << log_n) % kPerChunk == 0 && batch_stride % kPerChunk == 0 &&
        reinterpret_cast<std::uintptr_t>(src) % 16 == 0 && reinterpret_cast<std::uintptr_t>(dst) % 16 == 0) {
        const std::uint64_t chunks = count / kPerChunk;
        std::uint32_t row_log = log_n;
        for (std::uint32_t k = kPerChunk; k > 1; k >>= 1) --row_log;
        const std::uint64_t blocks = std::min<std::uint64_t>((chunks + kThreads - 1) / kThreads, 65536);
        if (gather)
            hipLaunchKernelGGL((pitched_kernel<true>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                               static_cast<const uint4*>(src), static_cast<uint4*>(dst), chunks, row_log,
                               batch_stride / kPerChunk);
        else
            hipLaunchKernelGGL((pitched_kernel<false>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                               static_cast<const uint4*>(src), static_cast<uint4*>(dst), chunks, row_log,
                               batch_stride / kPerChunk);
        hip_check(hipGetLastError(), "boundary gather / scatter launch");
        return;
    }
    const std::uint64_t blocks = std::min<std::uint64_t>((count + kThreads - 1) / kThreads, 65536);
    if (gather)
        hipLaunchKernelGGL((boundary_kernel<T, true>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                           static_cast<const T*>(src), static_cast<T*>(dst), count, log_n, stride, batch_stride,
                           reversed);
    else
        hipLaunchKernelGGL((boundary_kernel<T, false>), dim3(unsigned(blocks)), dim3(kThreads), 0, stream,
                           static_cast<const T*>(src), static_cast<T*>(dst), count, log_n, stride, batch_stride,
                           reversed);
    hip_check(hipGetLastError(), "boundary gather / scatter launch");
}

std::size_t align16(std::size_t bytes) { return (bytes + 15) & ~std::size_t{15}; }

class BoundaryExecutor final : public Executor {
  public:
    BoundaryExecutor(const Request& r, std::unique_ptr<Executor> child) : r_(r), child_(std::move(child)) {
        // A side that is already packed in natural order is read or written
        // by the packed plan itself: no gather or scatter for it.
        const auto packed = [&](std::uint64_t stride, std::uint64_t batch_stride, bool reversed) {
            return stride == 1 && !reversed && (r.batch == 1 || batch_stride == r.n);
        };
        direct_in_ = packed(r.in_stride, r.in_batch_stride, r.input_bit_reversed);
        direct_out_ = packed(r.out_stride, r.out_batch_stride, r.output_bit_reversed);
        algorithm = "semantic-boundary[" + child_->algorithm + "]";
        reason = "strided or reordered sides: gather to packed natural order, packed transform, scatter; child: " +
                 child_->reason;
        json::Writer w;
        w.begin_object()
            .field("schema_version", 1u)
            .field("kind", "semantic-boundary")
            .field("boundary", "gather-natural-child-scatter")
            .field("input_stride", r.in_stride)
            .field("input_batch_stride", r.in_batch_stride)
            .field("input_bit_reversed", r.input_bit_reversed)
            .field("output_stride", r.out_stride)
            .field("output_batch_stride", r.out_batch_stride)
            .field("output_bit_reversed", r.output_bit_reversed)
            .field("direct_input", direct_in_)
            .field("direct_output", direct_out_)
            .field("workspace_bytes", std::uint64_t(workspace_bytes()))
            .key("child")
            .value_raw(child_->mapping_json)
            .end_object();
        mapping_json = w.str();
    }
    std::size_t workspace_bytes() const override { return 2 * align16(r_.data_bytes()) + child_->workspace_bytes(); }
    void execute(const void* in, void* out, void* ws, hipStream_t stream) override {
        require(ws != nullptr, "a semantic-boundary plan needs its workspace");
        auto* first = static_cast<unsigned char*>(ws);
        auto* second = first + align16(r_.data_bytes());
        auto* child_ws = child_->workspace_bytes() ? second + align16(r_.data_bytes()) : nullptr;
        const std::uint64_t count = r_.n * r_.batch;
        // In place (in == out): a gathered input is consumed before the packed
        // plan writes `out`, and a scattered output is written after the
        // packed plan has read `in`.
        if (!direct_in_) move(true, in, first, count, r_.in_stride, r_.in_batch_stride, r_.input_bit_reversed, stream);
        child_->execute(direct_in_ ? in : first, direct_out_ ? out : second, child_ws, stream);
        if (!direct_out_)
            move(false, second, out, count, r_.out_stride, r_.out_batch_stride, r_.output_bit_reversed, stream);
    }

  private:
    void move(bool gather, const void* src, void* dst, std::uint64_t count, std::uint64_t stride,
              std::uint64_t batch_stride, bool reversed, hipStream_t stream) const {
        switch (r_.element_bytes) {
            case 2: launch_boundary<std::uint16_t>(gather, src, dst, count, r_.log_n, stride, batch_stride, reversed, stream); break;
            case 4: launch_boundary<std::uint32_t>(gather, src, dst, count, r_.log_n, stride, batch_stride, reversed, stream); break;
            case 8: launch_boundary<std::uint64_t>(gather, src, dst, count, r_.log_n, stride, batch_stride, reversed, stream); break;
            default: throw NotSupported("boundary element size has no gfx950 kernel");
        }
    }
    Request r_;
    std::unique_ptr<Executor> child_;
    bool direct_in_ = false, direct_out_ = false;
};

}  // namespace

std::unique_ptr<Executor> make_boundary_executor(const Request& r, Selection* sel) {
    Request child = r;
    child.boundary = false;
    child.in_place = false;
    child.input_bit_reversed = child.output_bit_reversed = false;
    child.in_stride = child.out_stride = 1;
    child.in_batch_stride = child.out_batch_stride = r.n;
    child.policy = CUBUTTERFLY_ALGORITHM_DEFAULT;
    child.explicit_algorithm.clear();
    child.variant.clear();
    return std::make_unique<BoundaryExecutor>(r, plan_executor(child, sel));
}

}  // namespace cbw
