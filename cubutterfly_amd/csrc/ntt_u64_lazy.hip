// Instantiates the NTT pass kernels for u64 words, lazy reduction.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
void register_u64_lazy() { register_all<std::uint64_t, true>(); }
}  // namespace ntt_detail
}  // namespace cbw
