// CPU-side transform descriptor behind cubutterflyDescriptor_t, and the
// normalised rank-1 request the gfx950 planner lowers.
#pragma once

#include "../../include/cubutterfly/cubutterfly.h"
#include "../../include/cubutterfly/cubutterfly_mi355x.h"
#include "common.hpp"

#include <string>
#include <vector>

// Default field values follow the reference descriptor
// (src/semantic_contract.hpp:11-41): FFT, COMPLEX_FP32, extents {256}, batch 1,
// normalised inverse, modulus 1152921504606584833 with 64-bit words.
struct cubutterflyDescriptor {
    cubutterflyOperator_t op = CUBUTTERFLY_OPERATOR_FFT;
    cubutterflyDataType_t storage = CUBUTTERFLY_DATA_COMPLEX_FP32;
    cubutterflyComputeType_t compute = CUBUTTERFLY_COMPUTE_FP32;
    cubutterflyDirection_t direction = CUBUTTERFLY_DIRECTION_FORWARD;
    cubutterflyPlacement_t placement = CUBUTTERFLY_PLACEMENT_OUT_OF_PLACE;
    cubutterflyLengthMode_t length_mode = CUBUTTERFLY_LENGTH_STANDARD;
    cubutterflyExecutionMode_t execution_mode = CUBUTTERFLY_EXECUTION_AUTO;
    cubutterflyFftTransformType_t fft_type = CUBUTTERFLY_FFT_C2C;
    double fft_output_scale = 1.0;
    double output_scale = 1.0;
    cubutterflyOutputRounding_t output_rounding = CUBUTTERFLY_ROUNDING_STAGE_STORAGE;
    cubutterflyArithmeticPolicy_t arithmetic_policy = CUBUTTERFLY_ARITHMETIC_STRICT;
    cubutterflyAlgorithmPolicy_t algorithm_policy = CUBUTTERFLY_ALGORITHM_DEFAULT;
    std::string explicit_algorithm;
    std::uint32_t rank = 1;
    std::vector<std::size_t> extents{256};
    std::vector<std::size_t> input_strides, output_strides;
    std::size_t input_batch_stride = 0, output_batch_stride = 0;
    std::size_t batch = 1;
    bool normalize_inverse = true;
    std::uint64_t modulus = 1152921504606584833ULL;
    std::uint32_t word_bits = 64;
    cubutterflyNttLayout_t input_ntt_layout = CUBUTTERFLY_NTT_LAYOUT_NATURAL;
    cubutterflyNttLayout_t output_ntt_layout = CUBUTTERFLY_NTT_LAYOUT_NATURAL;
    std::vector<std::vector<cubutterflyMatrix2x2_t>> stage_matrices{3};
    std::vector<cubutterflyLogicalOrder_t> input_orders, output_orders;
    // Extension (cubutterfly_mi355x.h): NTT ring and explicit psi.
    cubutterflyNttRing_t ring = CUBUTTERFLY_NTT_RING_CYCLIC;
    std::uint64_t psi = 0;
};

namespace cbw {

enum class Op { Fwht, Fft, Ntt };

// Highest executable rank (reference kGeneralMaxRank).
constexpr std::uint32_t kMaxRank = 8;
// Longest FWHT row one workgroup transforms in one pass (the 32-register
// kernel); longer rows factor into a row pass and column passes.
constexpr std::uint32_t kMaxFwhtRowLog = 15;

// A validated power-of-two request. Rank 1 is described by n, the strides
// and the orders below; rank 2 and above additionally by the per-axis
// vectors (outermost axis first), with n the points per transform.
struct Request {
    Op op = Op::Fwht;
    cubutterflyDataType_t storage = CUBUTTERFLY_DATA_FP32;
    std::uint32_t log_n = 0;
    std::uint64_t n = 0, batch = 0;
    bool inverse = false;
    bool normalize = false;      // FFT/FWHT 1/n on the inverse
    bool in_place = false;
    bool fp16_final = false;     // FP16 storage, FP32 compute, one final narrowing
    bool allow_mma = false;      // FP16 FWHT may use MFMA Hadamard blocks
    float output_scale = 1.0f;   // rounded to float as the reference does
    std::uint64_t modulus = 0;
    std::uint32_t word_bits = 0;
    bool negacyclic = false;
    std::uint64_t psi = 0;       // 0 = benchmark rule
    bool input_bit_reversed = false, output_bit_reversed = false;
    cubutterflyAlgorithmPolicy_t policy = CUBUTTERFLY_ALGORITHM_DEFAULT;
    std::string explicit_algorithm;
    // Rank-1 lowering to build, by algorithm name (empty: the static model's
    // choice). Set by the selection (explicit, cached or measured).
    std::string variant;
    std::size_t element_bytes = 0;
    // Normalised element and batch strides of each side (packed: 1 and n).
    std::uint64_t in_stride = 1, out_stride = 1, in_batch_stride = 0, out_batch_stride = 0;
    // The sides are strided, or carry FWHT / FFT logical orders: the plan
    // gathers, runs the packed natural-order transform and scatters.
    bool boundary = false;
    // Rows with a pitch (unit element stride; in/out_batch_stride apart)
    // that the transform kernels load and store directly, in place of a
    // boundary plan.
    bool pitched = false;
    // Rank >= 2: per-axis extents, element strides and bit-reversed orders of
    // each side (outermost axis first). Empty for rank 1.
    std::uint32_t rank = 1;
    std::vector<std::uint64_t> extents, in_strides, out_strides;
    std::vector<std::uint8_t> in_reversed, out_reversed;
    // Zero-extended embedding (any rank): `extents` are the executed
    // power-of-two extents, each side keeps its own (the logical extents on
    // the forward input and the inverse output).
    bool embedding = false;
    std::vector<std::uint64_t> in_extents, out_extents;
    // A rank-1 FWHT longer than one resident tile, factored into axes of at
    // most 2^12 points (rank and the vectors above describe the factors).
    bool factored = false;
    std::size_t data_bytes() const { return static_cast<std::size_t>(n * batch) * element_bytes; }
    // Bytes a side spans: the sum over axes of (extent - 1) stride, plus
    // (batch - 1) batch stride, plus one element.
    std::size_t span_bytes(bool input) const {
        const std::uint64_t bs = input ? in_batch_stride : out_batch_stride;
        std::uint64_t last = (batch - 1) * bs;
        if (extents.empty() || factored) {
            last += (n - 1) * (input ? in_stride : out_stride);
        } else {
            const auto& strides = input ? in_strides : out_strides;
            const auto& side = input ? in_extents : out_extents;
            for (std::size_t axis = 0; axis < side.size(); ++axis) last += (side[axis] - 1) * strides[axis];
        }
        return static_cast<std::size_t>(last + 1) * element_bytes;
    }
};

// Full semantic validation (std::invalid_argument), then the executable
// subset check (NotSupported). Mirrors the reference's normalize_descriptor
// rules for the fields this library accepts (src/semantic_contract.cpp:189-280).
void validate_descriptor(const cubutterflyDescriptor& d);
Request lower_request(const cubutterflyDescriptor& d);
// A natural-order FP32 FWHT request of more than 2^15 points as its factors
// (a resident row of 2^12 to 2^15 points, then axes of at most 2^7 points,
// lowest bits innermost).
void factor_long_fwht(Request& r);

std::string descriptor_json(const cubutterflyDescriptor& d);
cubutterflyDescriptor descriptor_from_json(const std::string& text);
std::string capabilities_json(const cubutterflyDescriptor& d);

}  // namespace cbw
