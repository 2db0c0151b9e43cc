// Instantiates the NTT pass kernels for u32 words, Barrett arithmetic.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
void register_u32_barrett() { register_all<std::uint32_t, kBarrett>(); }
}  // namespace ntt_detail
}  // namespace cbw
