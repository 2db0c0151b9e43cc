// Instantiates the NTT pass kernels for u32 words, strict reduction.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
void register_u32_strict() { register_all<std::uint32_t, false>(); }
}  // namespace ntt_detail
}  // namespace cbw
