// Instantiates the NTT pass kernels for u64 words, Barrett arithmetic.
#include "ntt_kernels.hpp"

namespace cbw {
namespace ntt_detail {
void register_u64_barrett() { register_all<std::uint64_t, kBarrett>(); }
}  // namespace ntt_detail
}  // namespace cbw
