// Instantiates the NTT pass kernels for u32 words, lazy reduction.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
void register_u32_lazy() { register_all<std::uint32_t, true>(); }
}  // namespace ntt_detail
}  // namespace cbw
