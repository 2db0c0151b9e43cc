// Instantiates the NTT pass kernels for u64 words, strict reduction.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
void register_u64_strict() { register_all<std::uint64_t, false>(); }
}  // namespace ntt_detail
}  // namespace cbw
