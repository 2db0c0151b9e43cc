// Descriptor validation, lowering to a rank-1 request, and JSON round trip.
#include "descriptor.hpp"

#include "json.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>
#include <unordered_set>

namespace cbw {
namespace {

template <class E>
void enum_range(E value, int maximum, const char* name) {
    require(static_cast<int>(value) >= 0 && static_cast<int>(value) <= maximum,
            std::string("unknown ") + name + " enumerator");
}

bool is_low(cubutterflyDataType_t s) {
    return s == CUBUTTERFLY_DATA_FP16 || s == CUBUTTERFLY_DATA_BF16 ||
           s == CUBUTTERFLY_DATA_COMPLEX_FP16 || s == CUBUTTERFLY_DATA_COMPLEX_BF16;
}

std::size_t storage_bytes(cubutterflyDataType_t s) {
    switch (s) {
        case CUBUTTERFLY_DATA_FP16:
        case CUBUTTERFLY_DATA_BF16: return 2;
        case CUBUTTERFLY_DATA_FP32:
        case CUBUTTERFLY_DATA_COMPLEX_FP16:
        case CUBUTTERFLY_DATA_COMPLEX_BF16:
        case CUBUTTERFLY_DATA_UINT32: return 4;
        case CUBUTTERFLY_DATA_FP64:
        case CUBUTTERFLY_DATA_COMPLEX_FP32:
        case CUBUTTERFLY_DATA_UINT64: return 8;
        case CUBUTTERFLY_DATA_COMPLEX_FP64: return 16;
    }
    return 0;
}

// Resolve the per-axis logical order of one side, folding the legacy
// rank-one NTT layout spelling into it (reference semantic_contract.cpp:246-262).
bool side_bit_reversed(const cubutterflyDescriptor& d, bool input) {
    const auto layout = input ? d.input_ntt_layout : d.output_ntt_layout;
    const auto& orders = input ? d.input_orders : d.output_orders;
    bool reversed = !orders.empty() && orders[0] == CUBUTTERFLY_ORDER_BIT_REVERSED;
    if (layout == CUBUTTERFLY_NTT_LAYOUT_BIT_REVERSED) {
        require(orders.empty() || orders[0] == CUBUTTERFLY_ORDER_BIT_REVERSED,
                "legacy bit reversal conflicts with explicit logical order");
        reversed = true;
    }
    return reversed;
}

// Normalised layout of one side: empty strides mean packed, a zero batch
// stride means the axis span (reference semantic_contract.cpp:104-123).
struct SideLayout {
    std::vector<std::size_t> strides;
    std::size_t batch_stride = 0;
};

std::size_t checked_mul(std::size_t a, std::size_t b) {
    require(b == 0 || a <= std::numeric_limits<std::size_t>::max() / b, "layout size overflows size_t");
    return a * b;
}
std::size_t checked_add(std::size_t a, std::size_t b) {
    require(a <= std::numeric_limits<std::size_t>::max() - b, "layout size overflows size_t");
    return a + b;
}

// Whether the addresses sum_k c_k s_k (0 <= c_k < n_k) of a layout repeat.
// Sorted by stride, a layout whose every stride clears the span of the
// smaller ones is one-to-one. Otherwise a pair (s_a, n_a), (s_b, n_b) with
// n_a - 1 >= s_b / g and n_b - 1 >= s_a / g (g = gcd) has the collision
// (s_b / g) s_a = (s_a / g) s_b. Small layouts are enumerated; larger ones
// with no such pair are accepted (as the reference's normaliser does,
// semantic_contract.cpp:55-103).
bool layout_overlaps(std::vector<std::pair<std::size_t, std::size_t>> dims) {
    std::sort(dims.begin(), dims.end());
    std::size_t covered = 1;
    bool nested = true;
    for (const auto& [stride, extent] : dims) {
        if (stride < covered) nested = false;
        covered = checked_add(covered, checked_mul(extent - 1, stride));
    }
    if (nested) return false;
    for (std::size_t a = 0; a < dims.size(); ++a)
        for (std::size_t b = a + 1; b < dims.size(); ++b) {
            const std::size_t g = std::gcd(dims[a].first, dims[b].first);
            if (dims[a].second - 1 >= dims[b].first / g && dims[b].second - 1 >= dims[a].first / g) return true;
        }
    std::size_t points = 1;
    for (const auto& dim : dims) {
        if (dim.second > 65536 / points) return false;
        points *= dim.second;
    }
    std::unordered_set<std::size_t> seen;
    for (std::size_t index = 0; index < points; ++index) {
        std::size_t rest = index, address = 0;
        for (const auto& [stride, extent] : dims) {
            address += (rest % extent) * stride;
            rest /= extent;
        }
        if (!seen.insert(address).second) return true;
    }
    return false;
}

std::size_t next_pow2(std::size_t n) {
    std::size_t p = 1;
    while (p < n) p = checked_mul(p, 2);
    return p;
}

// Extents of one side. The zero-extended embedding pads every axis to the
// next power of two on the forward output and the inverse input (reference
// semantic_contract.cpp:43-53).
std::vector<std::size_t> side_extents(const cubutterflyDescriptor& d, bool input) {
    std::vector<std::size_t> e = d.extents;
    if (d.length_mode == CUBUTTERFLY_LENGTH_ZERO_EXTENDED_EMBEDDING &&
        input == (d.direction == CUBUTTERFLY_DIRECTION_INVERSE))
        for (auto& n : e) n = next_pow2(n);
    return e;
}

SideLayout side_layout(const cubutterflyDescriptor& d, bool input) {
    const std::vector<std::size_t> extents = side_extents(d, input);
    SideLayout l;
    l.strides = input ? d.input_strides : d.output_strides;
    l.batch_stride = input ? d.input_batch_stride : d.output_batch_stride;
    if (l.strides.empty()) {
        l.strides.resize(d.rank);
        std::size_t stride = 1;
        for (std::size_t axis = d.rank; axis-- > 0;) {
            l.strides[axis] = stride;
            stride = checked_mul(stride, extents[axis]);
        }
    }
    require(l.strides.size() == d.rank, "one stride per axis is required");
    std::size_t span = 1;
    std::vector<std::pair<std::size_t, std::size_t>> dims;
    for (std::size_t axis = 0; axis < d.rank; ++axis) {
        require(l.strides[axis] > 0, "axis strides must be positive");
        span = checked_add(span, checked_mul(extents[axis] - 1, l.strides[axis]));
        if (extents[axis] > 1) dims.emplace_back(l.strides[axis], extents[axis]);
    }
    if (l.batch_stride == 0) l.batch_stride = span;
    checked_add(span, checked_mul(d.batch - 1, l.batch_stride));
    if (d.batch > 1) dims.emplace_back(l.batch_stride, d.batch);
    require(!layout_overlaps(dims), "descriptor layout overlaps");
    return l;
}

}  // namespace

void validate_descriptor(const cubutterflyDescriptor& d) {
    enum_range(d.op, 5, "operator");
    enum_range(d.storage, 9, "storage type");
    enum_range(d.compute, 4, "compute type");
    enum_range(d.direction, 1, "direction");
    enum_range(d.placement, 1, "placement");
    enum_range(d.length_mode, 1, "length mode");
    enum_range(d.execution_mode, 2, "execution mode");
    enum_range(d.fft_type, 2, "FFT transform type");
    enum_range(d.algorithm_policy, 2, "algorithm policy");
    enum_range(d.input_ntt_layout, 2, "NTT layout");
    enum_range(d.output_ntt_layout, 2, "NTT layout");
    enum_range(d.output_rounding, 1, "output rounding");
    enum_range(d.arithmetic_policy, 1, "arithmetic policy");
    enum_range(d.ring, 1, "NTT ring");
    require((d.algorithm_policy == CUBUTTERFLY_ALGORITHM_EXPLICIT) == !d.explicit_algorithm.empty(),
            "explicit selection policy and algorithm must be supplied together");
    require(d.rank > 0 && d.extents.size() == d.rank, "rank and shape mismatch");
    require(d.batch > 0, "batch must be positive");
    for (auto n : d.extents) require(n > 0, "extent must be positive");
    require(std::isfinite(d.fft_output_scale) && std::isfinite(d.output_scale),
            "output scales must be finite");
    const bool real = d.storage <= CUBUTTERFLY_DATA_FP64;
    const bool complex = d.storage >= CUBUTTERFLY_DATA_COMPLEX_FP16 && d.storage <= CUBUTTERFLY_DATA_COMPLEX_FP64;
    const bool integer = d.storage >= CUBUTTERFLY_DATA_UINT32;
    require(d.compute == CUBUTTERFLY_COMPUTE_NATIVE ||
                (integer ? (d.compute == CUBUTTERFLY_COMPUTE_UINT32 || d.compute == CUBUTTERFLY_COMPUTE_UINT64)
                         : (d.compute == CUBUTTERFLY_COMPUTE_FP32 || d.compute == CUBUTTERFLY_COMPUTE_FP64)),
            "compute domain is incompatible with storage");
    if (d.op == CUBUTTERFLY_OPERATOR_FFT) {
        require(d.fft_type == CUBUTTERFLY_FFT_C2C ? complex : real, "FFT transform and storage are incompatible");
    } else {
        require(d.fft_type == CUBUTTERFLY_FFT_C2C && d.fft_output_scale == 1.0, "FFT parameters require FFT operator");
        if (d.op == CUBUTTERFLY_OPERATOR_NTT) require(integer, "NTT requires integer storage");
    }
    if (d.op == CUBUTTERFLY_OPERATOR_NTT) {
        require(d.word_bits == (d.storage == CUBUTTERFLY_DATA_UINT32 ? 32u : 64u), "NTT word bits must match storage");
        require(d.modulus > 2 && (d.modulus & 1) &&
                    (d.word_bits == 64 || d.modulus <= std::numeric_limits<std::uint32_t>::max()),
                "invalid NTT modulus");
    } else {
        require(d.modulus == 1152921504606584833ULL && d.word_bits == 64, "modulus and word bits require NTT operator");
        require(d.input_ntt_layout == CUBUTTERFLY_NTT_LAYOUT_NATURAL &&
                    d.output_ntt_layout == CUBUTTERFLY_NTT_LAYOUT_NATURAL,
                "NTT layouts require NTT operator");
        require(d.ring == CUBUTTERFLY_NTT_RING_CYCLIC && d.psi == 0, "NTT ring requires NTT operator");
    }
    if (d.ring == CUBUTTERFLY_NTT_RING_CYCLIC) require(d.psi == 0, "psi requires the negacyclic ring");
    if (d.op != CUBUTTERFLY_OPERATOR_FFT && d.op != CUBUTTERFLY_OPERATOR_NTT &&
        d.length_mode == CUBUTTERFLY_LENGTH_STANDARD)
        for (auto n : d.extents) require(is_pow2(n), "butterfly extent must be a power of two");
    for (const auto* orders : {&d.input_orders, &d.output_orders}) {
        require(orders->empty() || orders->size() == d.rank, "one logical order per axis is required");
        for (auto o : *orders)
            require(o == CUBUTTERFLY_ORDER_NATURAL || o == CUBUTTERFLY_ORDER_BIT_REVERSED, "unknown logical order");
    }
    for (bool input : {true, false}) {
        const auto layout = input ? d.input_ntt_layout : d.output_ntt_layout;
        if (layout == CUBUTTERFLY_NTT_LAYOUT_BIT_REVERSED)
            require(d.rank == 1 && is_pow2(d.extents[0]), "legacy bit reversal requires rank-one power-of-two shape");
        (void)side_bit_reversed(d, input);
        const auto& orders = input ? d.input_orders : d.output_orders;
        const auto extents = side_extents(d, input);
        for (std::size_t axis = 0; axis < orders.size(); ++axis)
            if (orders[axis] == CUBUTTERFLY_ORDER_BIT_REVERSED)
                require(is_pow2(extents[axis]), "bit-reversed order requires a power-of-two extent");
    }
    (void)side_layout(d, true);
    (void)side_layout(d, false);
    // Epilogue contract (reference src/butterfly.cu:569-576): a non-unit output
    // scale or final-storage rounding needs FP16 FWHT with FP32 compute.
    if (d.output_scale != 1.0 || d.output_rounding == CUBUTTERFLY_ROUNDING_FINAL_STORAGE)
        require(d.op == CUBUTTERFLY_OPERATOR_FWHT && d.storage == CUBUTTERFLY_DATA_FP16 &&
                    d.compute == CUBUTTERFLY_COMPUTE_FP32 &&
                    d.output_rounding == CUBUTTERFLY_ROUNDING_FINAL_STORAGE,
                "output epilogue requires FP16 FWHT with FP32 final-storage rounding");
    if (d.arithmetic_policy == CUBUTTERFLY_ARITHMETIC_ALLOW_FP16_MMA)
        require(d.op == CUBUTTERFLY_OPERATOR_FWHT && d.storage == CUBUTTERFLY_DATA_FP16 && d.rank == 1,
                "FP16 MMA policy applies to rank-one FP16 FWHT only");
    for (std::size_t axis = 0; axis < d.stage_matrices.size(); ++axis)
        require(d.stage_matrices[axis].empty() ||
                    (axis < d.rank && d.op == CUBUTTERFLY_OPERATOR_STRUCTURED_2X2),
                "stage matrices require the structured operator within the rank");
}

// H(2^a) (x) H(2^b) (x) ... factors an FWHT beyond one resident tile into
// axes of at most 2^12 points, lowest index bits innermost, so the composite
// plan's innermost-first axis order is the rank-1 stage order (bits 0
// upward) and the result is bit-identical. The rank-1 element strides carry
// over to the factors; bit-reversed orders do not factor.
void factor_long_fwht(Request& r) {
    require(r.op == Op::Fwht && r.rank == 1 && !r.factored && !r.embedding && !r.fp16_final &&
                !r.input_bit_reversed && !r.output_bit_reversed,
            "only natural-order FP32 FWHT rows factor");
    // Innermost: one resident row of 2^12 points, or up to 2^15 where that
    // saves a pass; then axes of at most 2^7 points (one in-place column pass
    // each), as even as their count allows. 2^16 .. 2^22 points take two
    // passes, 2^23 .. 2^29 three.
    constexpr std::uint32_t kColumnBits = 7;
    const std::uint32_t outer = r.log_n - kMaxFwhtRowLog;
    const std::uint32_t passes = (outer + kColumnBits - 1) / kColumnBits;
    std::uint32_t inner = 12;
    while (r.log_n - inner > passes * kColumnBits) ++inner;
    std::vector<std::uint32_t> bits{inner};  // innermost first
    for (std::uint32_t k = 0, done = 0; k < passes; ++k) {
        bits.push_back((r.log_n - inner - done) / (passes - k));
        done += bits.back();
    }
    supported(bits.size() <= kMaxRank, "FWHT length exceeds the factored rank");
    r.factored = true;
    r.rank = std::uint32_t(bits.size());
    r.extents.assign(r.rank, 0);
    r.in_strides.assign(r.rank, 0);
    r.out_strides.assign(r.rank, 0);
    std::uint64_t below = 1;
    for (std::size_t k = 0; k < bits.size(); ++k) {
        const std::size_t axis = r.rank - 1 - k;
        r.extents[axis] = std::uint64_t{1} << bits[k];
        r.in_strides[axis] = r.in_stride * below;
        r.out_strides[axis] = r.out_stride * below;
        below <<= bits[k];
    }
    r.in_extents = r.out_extents = r.extents;
    r.in_reversed.assign(r.rank, 0);
    r.out_reversed.assign(r.rank, 0);
    r.boundary = r.pitched = false;
}

Request lower_request(const cubutterflyDescriptor& d) {
    validate_descriptor(d);
    supported(d.rank <= kMaxRank, "ranks above eight are not executable");
    const bool embedding = d.length_mode == CUBUTTERFLY_LENGTH_ZERO_EXTENDED_EMBEDDING;
    supported(d.execution_mode != CUBUTTERFLY_EXECUTION_XD, "XD execution requires a multidimensional descriptor");
    supported(d.fft_type == CUBUTTERFLY_FFT_C2C, "only C2C FFTs are executable");
    supported(d.input_ntt_layout != CUBUTTERFLY_NTT_LAYOUT_APPT_STATIC &&
                  d.output_ntt_layout != CUBUTTERFLY_NTT_LAYOUT_APPT_STATIC,
              "APPT static layouts are not executable");
    // Executed (physical) extents: the power-of-two embedding of each axis.
    std::vector<std::size_t> physical = d.extents;
    if (embedding)
        for (auto& e : physical) e = next_pow2(e);
    std::size_t n = 1;
    for (auto e : physical) {
        supported(is_pow2(e) && e >= 2, "only power-of-two lengths >= 2 are executable");
        n = checked_mul(n, e);
    }
    (void)checked_mul(checked_mul(n, d.batch), storage_bytes(d.storage));
    Request r;
    const SideLayout in = side_layout(d, true), out = side_layout(d, false);
    r.rank = d.rank;
    r.embedding = embedding;
    if (d.rank == 1 && !embedding) {
        r.in_stride = in.strides[0];
        r.out_stride = out.strides[0];
    } else {
        // Rank two and above, and the zero-extended embedding: per-axis
        // layout for the composite plan, which brings each axis innermost in
        // turn (reference src/c_api.cpp:4578-4600, 5231-5327) and pads / cuts
        // each side to its own extents.
        r.extents.assign(physical.begin(), physical.end());
        const auto in_ext = side_extents(d, true), out_ext = side_extents(d, false);
        r.in_extents.assign(in_ext.begin(), in_ext.end());
        r.out_extents.assign(out_ext.begin(), out_ext.end());
        r.in_strides.assign(in.strides.begin(), in.strides.end());
        r.out_strides.assign(out.strides.begin(), out.strides.end());
        for (bool input : {true, false}) {
            const auto& orders = input ? d.input_orders : d.output_orders;
            auto& reversed = input ? r.in_reversed : r.out_reversed;
            reversed.assign(d.rank, 0);
            for (std::size_t axis = 0; axis < orders.size(); ++axis)
                reversed[axis] = orders[axis] == CUBUTTERFLY_ORDER_BIT_REVERSED;
        }
    }
    r.in_batch_stride = in.batch_stride;
    r.out_batch_stride = out.batch_stride;
    r.n = n;
    r.log_n = log2_u64(n);
    r.batch = d.batch;
    r.inverse = d.direction == CUBUTTERFLY_DIRECTION_INVERSE;
    r.in_place = d.placement == CUBUTTERFLY_PLACEMENT_IN_PLACE;
    r.storage = d.storage;
    r.policy = d.algorithm_policy;
    r.explicit_algorithm = d.explicit_algorithm;
    r.input_bit_reversed = d.rank == 1 && !embedding && side_bit_reversed(d, true);
    r.output_bit_reversed = d.rank == 1 && !embedding && side_bit_reversed(d, false);
    r.element_bytes = storage_bytes(d.storage);
    // Strided sides, and FWHT / FFT logical orders, go through the semantic
    // boundary: gather to packed natural order, the packed transform,
    // scatter (reference src/c_api.cpp:2969-2993, 5064-5085). NTT orders on
    // packed sides are native to the NTT kernels.
    const auto packed = [&](std::size_t stride, std::size_t batch_stride) {
        return stride == 1 && (d.batch == 1 || batch_stride == n);
    };
    const bool strided = !packed(r.in_stride, r.in_batch_stride) || !packed(r.out_stride, r.out_batch_stride);
    // Rows with a pitch load and store in the transform kernels themselves.
    // FWHT: unit element stride, natural order, n >= 16 and
    // 16-byte pitches (a thread's 16-element vectors stay in one row and stay
    // aligned), a tile's row span below 2^31 bytes (32-bit lane offsets), and
    // no in-place pitch change (a tile's output would overlap rows that other
    // workgroups have yet to read).
    const auto pitch_ok = [&](std::uint64_t pitch) {
        const std::uint64_t rows_per_tile = n >= 4096 ? 1 : 4096 / n;
        return (pitch * r.element_bytes) % 16 == 0 &&
               ((rows_per_tile - 1) * pitch + n) * r.element_bytes < (std::uint64_t{1} << 31);
    };
    // NTT and FFT rows with a pitch, n >= 2^12: one transform per tile, each
    // at its own offset (NTT: the RNS engine's per-polynomial offsets; FFT:
    // a per-side transform pitch).
    const bool rows_pitched = d.rank == 1 && !embedding && strided && r.in_stride == 1 && r.out_stride == 1 &&
                              (!r.in_place || r.in_batch_stride == r.out_batch_stride);
    if (d.op == CUBUTTERFLY_OPERATOR_FWHT)
        r.pitched = rows_pitched && !r.input_bit_reversed && !r.output_bit_reversed && n >= 16 &&
                    pitch_ok(r.in_batch_stride) && pitch_ok(r.out_batch_stride);
    else if (d.op == CUBUTTERFLY_OPERATOR_NTT)
        r.pitched = rows_pitched && n >= 4096;
    else if (d.op == CUBUTTERFLY_OPERATOR_FFT)  // one transform per tile from 2^12 points
        r.pitched = rows_pitched && !r.input_bit_reversed && !r.output_bit_reversed && n >= 4096;
    // Logical orders: native to the NTT kernels, to one-pass FFTs (n <= 2^14)
    // on packed sides, and as a bit-reversed output to the final row pass of
    // longer FFTs; FWHT orders and bit-reversed input of longer FFTs use the
    // boundary.
    const bool reversed = r.input_bit_reversed || r.output_bit_reversed;
    const bool native_orders =
        d.op == CUBUTTERFLY_OPERATOR_NTT ||
        (d.op == CUBUTTERFLY_OPERATOR_FFT && (n <= (std::size_t{1} << 14) || !r.input_bit_reversed));
    r.boundary = d.rank == 1 && !embedding && !r.pitched && (strided || (reversed && !native_orders));
    switch (d.op) {
        case CUBUTTERFLY_OPERATOR_FWHT:
            r.op = Op::Fwht;
            r.normalize = r.inverse && d.normalize_inverse;
            if (d.storage == CUBUTTERFLY_DATA_FP16) {
                supported(d.compute == CUBUTTERFLY_COMPUTE_FP32 &&
                              d.output_rounding == CUBUTTERFLY_ROUNDING_FINAL_STORAGE,
                          "FP16 FWHT requires FP32 compute with final-storage rounding");
                supported(d.rank == 1 && !embedding, "FP16 FWHT is executable at rank one, standard length");
                r.fp16_final = true;
                r.output_scale = static_cast<float>(d.output_scale);
                r.allow_mma = d.arithmetic_policy == CUBUTTERFLY_ARITHMETIC_ALLOW_FP16_MMA;
            } else {
                supported(d.storage == CUBUTTERFLY_DATA_FP32 &&
                              (d.compute == CUBUTTERFLY_COMPUTE_NATIVE || d.compute == CUBUTTERFLY_COMPUTE_FP32),
                          "FWHT executes FP32 storage, or FP16 storage with FP32 compute");
            }
            break;
        case CUBUTTERFLY_OPERATOR_FFT:
            r.op = Op::Fft;
            r.normalize = r.inverse && d.normalize_inverse;
            supported(d.storage == CUBUTTERFLY_DATA_COMPLEX_FP32 &&
                          (d.compute == CUBUTTERFLY_COMPUTE_NATIVE || d.compute == CUBUTTERFLY_COMPUTE_FP32),
                      "FFT executes COMPLEX_FP32 storage with FP32 compute");
            supported(d.fft_output_scale == 1.0, "FFT output scale is not executable");
            break;
        case CUBUTTERFLY_OPERATOR_NTT: {
            r.op = Op::Ntt;
            r.normalize = r.inverse;  // modular inverse always multiplies by n^-1
            r.modulus = d.modulus;
            r.word_bits = d.word_bits;
            r.negacyclic = d.ring == CUBUTTERFLY_NTT_RING_NEGACYCLIC;
            supported(d.rank == 1 || !r.negacyclic, "the negacyclic ring is executable at rank one");
            r.psi = d.psi;
            supported(d.word_bits == 64 || d.modulus < (std::uint64_t{1} << 31),
                      "32-bit NTT words require modulus < 2^31");
            require(d.modulus < (std::uint64_t{1} << 63), "NTT modulus must be below 2^63");
            break;
        }
        default:
            throw NotSupported("operator has no MI355X lowering");
    }
    // FWHT beyond one resident row (2^15 points). Packed FP32 rows in
    // natural order factor here; FP16 rows (the FP32 promotion), strided
    // sides and bit-reversed orders are planned as rank-1 requests, the
    // orders and strides through the boundary (16-byte chunks for pitched
    // rows, LDS tiles for bit reversals), and factor when their packed FP32
    // transform is planned (factor_long_fwht). No kernel loads long rows at a
    // pitch.
    if (r.op == Op::Fwht && d.rank == 1 && !embedding && r.log_n > kMaxFwhtRowLog) {
        r.pitched = false;
        r.boundary = strided || reversed;
        if (!r.boundary && !r.fp16_final) factor_long_fwht(r);
    }
    return r;
}

// ---- JSON ----------------------------------------------------------------

std::string descriptor_json(const cubutterflyDescriptor& d) {
    json::Writer w;
    w.begin_object();
    w.field("schema", "cubutterfly-semantic-v1");
    w.field("operator", int(d.op)).field("storage", int(d.storage)).field("compute", int(d.compute));
    w.begin_array("shape");
    for (auto e : d.extents) w.value(std::uint64_t(e));
    w.end_array();
    w.field("batch", std::uint64_t(d.batch));
    w.field("inverse", int(d.direction)).field("normalize_inverse", d.normalize_inverse);
    w.field("placement", int(d.placement)).field("fft_type", int(d.fft_type));
    w.field("fft_output_scale", d.fft_output_scale).field("length_mode", int(d.length_mode));
    w.field("execution_mode", int(d.execution_mode));
    w.begin_array("input_strides");
    for (auto s : d.input_strides) w.value(std::uint64_t(s));
    w.end_array();
    w.begin_array("output_strides");
    for (auto s : d.output_strides) w.value(std::uint64_t(s));
    w.end_array();
    w.field("input_batch_stride", std::uint64_t(d.input_batch_stride));
    w.field("output_batch_stride", std::uint64_t(d.output_batch_stride));
    w.begin_array("input_orders");
    for (auto o : d.input_orders) w.value(int(o));
    w.end_array();
    w.begin_array("output_orders");
    for (auto o : d.output_orders) w.value(int(o));
    w.end_array();
    w.field("ntt_input_layout", int(d.input_ntt_layout)).field("ntt_output_layout", int(d.output_ntt_layout));
    w.field("modulus", d.modulus).field("word_bits", d.word_bits);
    w.field("output_scale", d.output_scale).field("output_rounding", int(d.output_rounding));
    w.field("arithmetic_policy", int(d.arithmetic_policy));
    w.field("algorithm_policy", int(d.algorithm_policy)).field("explicit_algorithm", d.explicit_algorithm);
    w.field("ntt_ring", int(d.ring)).field("ntt_psi", d.psi);
    w.end_object();
    return w.str();
}

cubutterflyDescriptor descriptor_from_json(const std::string& text) {
    const auto j = json::parse(text);
    require(j.is_object(), "descriptor JSON must be an object");
    static const char* allowed[] = {
        "schema", "operator", "storage", "compute", "shape", "batch", "inverse", "normalize_inverse",
        "placement", "fft_type", "fft_output_scale", "length_mode", "execution_mode", "input_strides",
        "output_strides", "input_batch_stride", "output_batch_stride", "input_orders", "output_orders",
        "ntt_input_layout", "ntt_output_layout", "modulus", "word_bits", "output_scale", "output_rounding",
        "arithmetic_policy", "algorithm_policy", "explicit_algorithm", "ntt_ring", "ntt_psi", "matrices"};
    for (const auto& m : j.members)
        require(std::find_if(std::begin(allowed), std::end(allowed),
                             [&](const char* a) { return m.first == a; }) != std::end(allowed),
                "unknown descriptor JSON field: " + m.first);
    require(j.at("schema").as_string("schema") == "cubutterfly-semantic-v1", "unsupported descriptor schema");
    cubutterflyDescriptor d;
    auto u = [&](const char* k, std::uint64_t fallback) {
        const auto* v = j.find(k);
        return v ? v->as_u64(k) : fallback;
    };
    auto list = [&](const char* k) {
        std::vector<std::uint64_t> out;
        if (const auto* v = j.find(k)) {
            require(v->is_array(), std::string(k) + " must be an array");
            for (const auto& item : v->items) out.push_back(item.as_u64(k));
        }
        return out;
    };
    d.op = cubutterflyOperator_t(u("operator", d.op));
    d.storage = cubutterflyDataType_t(u("storage", d.storage));
    d.compute = cubutterflyComputeType_t(u("compute", d.compute));
    auto shape = list("shape");
    require(!shape.empty(), "descriptor JSON shape must be nonempty");
    d.extents.assign(shape.begin(), shape.end());
    d.rank = std::uint32_t(d.extents.size());
    d.batch = u("batch", 1);
    d.direction = cubutterflyDirection_t(u("inverse", 0));
    if (const auto* v = j.find("normalize_inverse")) d.normalize_inverse = v->as_bool("normalize_inverse");
    d.placement = cubutterflyPlacement_t(u("placement", 0));
    d.fft_type = cubutterflyFftTransformType_t(u("fft_type", 0));
    if (const auto* v = j.find("fft_output_scale")) d.fft_output_scale = v->as_double("fft_output_scale");
    d.length_mode = cubutterflyLengthMode_t(u("length_mode", 0));
    d.execution_mode = cubutterflyExecutionMode_t(u("execution_mode", 0));
    for (auto s : list("input_strides")) d.input_strides.push_back(s);
    for (auto s : list("output_strides")) d.output_strides.push_back(s);
    d.input_batch_stride = u("input_batch_stride", 0);
    d.output_batch_stride = u("output_batch_stride", 0);
    for (auto o : list("input_orders")) d.input_orders.push_back(cubutterflyLogicalOrder_t(o));
    for (auto o : list("output_orders")) d.output_orders.push_back(cubutterflyLogicalOrder_t(o));
    d.input_ntt_layout = cubutterflyNttLayout_t(u("ntt_input_layout", 0));
    d.output_ntt_layout = cubutterflyNttLayout_t(u("ntt_output_layout", 0));
    if (const auto* v = j.find("modulus"); v && v->kind != json::Value::Kind::Null) d.modulus = v->as_u64("modulus");
    if (const auto* v = j.find("word_bits"); v && v->kind != json::Value::Kind::Null)
        d.word_bits = std::uint32_t(v->as_u64("word_bits"));
    if (const auto* v = j.find("output_scale")) d.output_scale = v->as_double("output_scale");
    d.output_rounding = cubutterflyOutputRounding_t(u("output_rounding", 0));
    d.arithmetic_policy = cubutterflyArithmeticPolicy_t(u("arithmetic_policy", 0));
    d.algorithm_policy = cubutterflyAlgorithmPolicy_t(u("algorithm_policy", 0));
    if (const auto* v = j.find("explicit_algorithm")) d.explicit_algorithm = v->as_string("explicit_algorithm");
    d.ring = cubutterflyNttRing_t(u("ntt_ring", 0));
    d.psi = u("ntt_psi", 0);
    if (const auto* v = j.find("matrices")) {
        require(v->is_array(), "matrices must be an array");
        for (const auto& axis : v->items) require(axis.is_array() && axis.items.empty(), "stage matrices are not executable");
    }
    validate_descriptor(d);
    return d;
}

std::string capabilities_json(const cubutterflyDescriptor& d) {
    validate_descriptor(d);
    json::Writer w;
    w.begin_object().field("schema", "cubutterfly-capabilities-v1").field("target", "gfx950");
    try {
        const auto r = lower_request(d);
        w.field("eligible", true).field("log_n", r.log_n).field("batch", r.batch);
    } catch (const NotSupported& e) {
        w.field("eligible", false).field("reason", std::string(e.what()));
    }
    w.end_object();
    return w.str();
}

}  // namespace cbw
