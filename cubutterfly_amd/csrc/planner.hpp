// gfx950 planner: lowers a validated request to one executor.
// Each kernel family exposes a factory; the factory chooses the radix, the
// stage split between passes and the register/LDS residency for CDNA4
// (64-wide wavefronts, 160 KB LDS per CU, 256 CUs in 8 XCDs).
#pragma once

#include "common.hpp"
#include "descriptor.hpp"

namespace cbw {

// Rank-1 kernel families. Each factory builds `r.variant` (one of its
// candidates' names) or, when that is empty, the static model's choice, and
// throws NotSupported for a name that is not a lowering of the request.
std::unique_ptr<Executor> make_fwht_executor(const Request& r);
std::unique_ptr<Executor> make_fft_executor(const Request& r);
std::unique_ptr<Executor> make_ntt_executor(const Request& r);
// Candidate lowerings of a rank-1 request, the static model's choice first.
std::vector<std::string> fwht_candidates(const Request& r);
// The MFMA Hadamard-block FP16 FWHT (ALLOW_FP16_MMA): its name, whether it
// covers a request (packed FP16 final-storage rows of 2 .. 4096 points) and
// its executor.
std::string fwht_mfma_name();
bool fwht_mfma_covers(const Request& r);
std::unique_ptr<Executor> make_fwht_mfma_executor(const Request& r);
// FFTs (r.log_n points) of the rows of row-major 2^l1 x 2^(r.log_n) blocks
// (r.batch rows in all), each block's result stored transposed; null where
// no kernel covers the shape.
std::unique_ptr<Executor> make_fft_rows_transposed(const Request& r, std::uint32_t l1);
// Rank-2 FFTs of row-major 2^l0 x 2^(r.log_n - l0) blocks (r.batch blocks of
// r.n points): axis 0 as column passes, then the rows in natural order; null
// where no kernel covers the shape.
std::unique_ptr<Executor> make_fft_rank2_columns(const Request& r, std::uint32_t l0);
// Whether those two factories would build a plan (no device work).
bool fft_rows_transposed_available(const Request& r, std::uint32_t l1);
bool fft_rank2_columns_available(const Request& r, std::uint32_t l0);
std::vector<std::string> fft_candidates(const Request& r);
std::vector<std::string> ntt_candidates(const Request& r);

// Plan-time selection state (reference src/c_api.cpp:1756-1901): the policy,
// the user selection cache and the stream MEASURE times on; `source` and
// `notes` accumulate over every rank-1 plan the request lowers to.
struct Selection {
    cubutterflyAlgorithmPolicy_t policy = CUBUTTERFLY_ALGORITHM_DEFAULT;
    std::string cache_path;
    hipStream_t stream = nullptr;
    cubutterflySelectionSource_t source = CUBUTTERFLY_SELECTION_STATIC_MODEL;
    std::string notes;
};
void combine_source(Selection& sel, cubutterflySelectionSource_t next);
// Appends a note to the plan's selection reason.
void note_selection(Selection& sel, const std::string& text);
// MEASURE's refusal on a capturing stream (NOT_SUPPORTED), to be called
// before any candidate is built: building allocates device tables.
void require_no_capture(const Selection& sel);
std::string selection_key(const Request& r);
std::string lookup_cache(const std::string& path, const std::string& key);
void store_cache(const std::string& path, const std::string& key, const std::string& algorithm);
std::unique_ptr<Executor> build_leaf(const Request& r);
// A packed rank-1 plan: explicit variant, cached record (DEFAULT), measured
// candidates (MEASURE) or the static model.
std::unique_ptr<Executor> select_leaf(const Request& r, Selection* sel);
// MEASURE between alternative executors of one request (MEASURE's timing
// protocol and scratch): records the fastest's name under `key` in the
// selection cache and returns its index, or built.size() when the scratch
// could not be allocated.
std::size_t measure_executors(const Request& r, const std::string& key,
                              const std::vector<std::unique_ptr<Executor>>& built, Selection& sel);

// Gather / packed child / scatter, for strided sides and FWHT / FFT orders.
std::unique_ptr<Executor> make_boundary_executor(const Request& r, Selection* sel);
// Rank >= 2 and the zero-extended embedding: one batched rank-1 plan per
// axis, innermost first, with tiled transposes bringing each axis innermost
// and the original order back; sides padded or cut to their own extents.
std::unique_ptr<Executor> make_composite_executor(const Request& r, Selection* sel);

// A packed rank-1 FWHT of more than 2^15 points: FP32 rows as the factored
// composite; FP16 final-storage rows through the FP32 promotion (widen, the
// factored FP32 plan narrowing in its last pass).
std::unique_ptr<Executor> make_long_fwht_executor(const Request& r, Selection* sel);

inline std::unique_ptr<Executor> plan_executor(const Request& r, Selection* sel = nullptr) {
    if (r.rank > 1 || r.embedding || r.factored) return make_composite_executor(r, sel);
    if (r.boundary) return make_boundary_executor(r, sel);
    if (r.op == Op::Fwht && r.log_n > kMaxFwhtRowLog) return make_long_fwht_executor(r, sel);
    return select_leaf(r, sel);
}

}  // namespace cbw
