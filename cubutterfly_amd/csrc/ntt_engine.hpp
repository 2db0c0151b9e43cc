// Batched multi-domain NTT engine for gfx950, shared by the cubutterfly.h NTT
// plans (one modulus, dense rows) and the RNS C ABI (one domain per limb,
// arbitrary per-polynomial word offsets).
//
// Algorithm: the merged-twist formulation of Longa and Naehrig ("Speeding up
// the NTT", CANS 2016). Forward: Cooley-Tukey butterflies, natural input,
// bit-reversed output, stage (m groups, bit b) twiddle T[m + i] = T[(n+j)>>(b+1)]
// with T[k] = psi^bitrev(k) (negacyclic) or w^(bitrev_s(i) n/2m) (cyclic), so
// the psi^j twist is folded into the butterflies. Inverse: Gentleman-Sande
// butterflies with the inverse table, bit-reversed input, natural output,
// times n^-1. Natural/bit-reversed boundaries are LDS-staged permutations of
// the first or last pass.
//
// Lengths up to 2^12 run in one pass (whole polynomials resident in a
// workgroup); up to 2^24 in two passes over the high and low index bits,
// each an in-register radix-16 / LDS-exchange core, with the intermediate in
// a workspace of polys * n words.
#pragma once

#include "common.hpp"

#include <string>
#include <vector>

namespace cbw {

struct NttDomain {
    std::uint64_t modulus = 0;
    std::uint64_t root = 0;  // forward ring root: psi (negacyclic) or w (cyclic)
};

struct NttPolynomial {
    std::uint32_t domain = 0;
    std::uint64_t input_offset = 0;   // words from the input pointer
    std::uint64_t output_offset = 0;  // words from the output pointer
};

struct NttEngineConfig {
    std::uint32_t word_bits = 32;
    std::uint32_t log_n = 0;
    bool negacyclic = false;
    bool inverse = false;
    bool input_bit_reversed = false;
    bool output_bit_reversed = false;
    bool reduce_input = true;  // reduce arbitrary words mod q on load
    bool force_strict = false; // fully reduced butterflies even where lazy ones fit
    bool barrett = false;      // Barrett products on canonical values (moduli below 2^(word bits - 2))
    bool wide_columns = false; // two-pass: 32-column tiles in the column pass (`-c32`)
    std::uint32_t split_high = 0;  // two-pass: high (column-pass) bits; 0 = the planner's split (`-h<l1>`)
    std::vector<NttDomain> domains;
    std::vector<NttPolynomial> polynomials;  // empty: `batch` dense rows of domain 0
    std::uint64_t batch = 0;
};

class NttEngine {
  public:
    explicit NttEngine(const NttEngineConfig& config);
    ~NttEngine();
    NttEngine(const NttEngine&) = delete;
    NttEngine& operator=(const NttEngine&) = delete;
    // Workspace bytes needed between the two passes (0 for one pass).
    std::size_t workspace_bytes() const;
    void execute(const void* input, void* output, void* workspace, hipStream_t stream) const;
    const std::string& algorithm() const { return algorithm_; }
    const std::string& mapping_json() const { return mapping_json_; }
    std::uint32_t passes() const;

  private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    std::string algorithm_, mapping_json_;
};

// Two-pass high-bit splits other than the planner's that have kernels at
// 2^log_n (the `-h<l1>` lowerings), empty elsewhere.
std::vector<std::uint32_t> ntt_other_splits(std::uint32_t log_n);

}  // namespace cbw
