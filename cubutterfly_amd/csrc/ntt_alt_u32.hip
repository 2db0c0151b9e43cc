// Instantiates the NTT pass shapes beyond the planner's static choice for
// u32 words, lazy and strict: the neighbouring splits of 2^15..2^17 (16- and
// 32-column tiles). They are candidates of MEASURE and RNS Prepare.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
namespace {
template <bool LAZY>
void register_alt() {
    add_split<std::uint32_t, LAZY, 15, 6>();
    add_split<std::uint32_t, LAZY, 15, 8>();
    add_split<std::uint32_t, LAZY, 16, 7>();
    add_split<std::uint32_t, LAZY, 16, 9>();
    add_split<std::uint32_t, LAZY, 17, 7>();
    add_split<std::uint32_t, LAZY, 17, 9>();
}
}  // namespace
void register_alt_u32() {
    register_alt<true>();
    register_alt<false>();
}
}  // namespace ntt_detail
}  // namespace cbw
