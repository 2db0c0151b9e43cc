// NTT kernels for gfx950 (lowering added in a later milestone).
#include <hip/hip_runtime.h>

#include "planner.hpp"

namespace cbw {
std::unique_ptr<Executor> make_ntt_executor(const Request&) {
    throw NotSupported("NTT is not yet lowered for gfx950");
}
}  // namespace cbw
