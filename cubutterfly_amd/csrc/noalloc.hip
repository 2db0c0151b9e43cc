// cubutterflyExecuteNoAlloc: cubutterflyExecute for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The plan's workspace -- the intermediate
// of two-pass NTT / FFT plans, the packed buffers of boundary and composite
// plans -- comes from `scratch`, a file-scope device array of kScratchBytes
// that each GPU holds from the library's load until the process ends, instead
// of the buffer bound with cubutterflyPlanSetWorkspace. Nothing here calls
// hipMalloc, hipFree or any allocating routine.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one
// device (two streams, or two host threads) race on it and must be ordered
// by the caller. No lowering needs the array to start at zero -- each plan
// writes every workspace word it later reads -- so it is never cleared, and
// it keeps the last call's contents.
#include "../../include/cubutterfly/cubutterfly_mi355x.h"
#include "common.hpp"

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

namespace cbw {
cubutterflyStatus_t guarded_call(void (*body)(void*), void* context) noexcept;
void execute_plan_with_workspace(cubutterflyHandle_t handle, cubutterflyPlan_t plan, const void* input, void* output,
                                 void* workspace, std::size_t capacity, const char* what);
}  // namespace cbw

namespace {

constexpr std::size_t kScratchBytes = std::size_t{CUBUTTERFLY_NOALLOC_SCRATCH_BYTES};
constexpr int kMaxDevices = 64;

// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> scratch_address[kMaxDevices];
std::mutex scratch_lookup;

// This device's copy of `scratch`, looked up on the first call with that
// device current.
void* device_scratch() {
    int device = -1;
    cbw::hip_check(hipGetDevice(&device), "hipGetDevice");
    cbw::require(device >= 0 && device < kMaxDevices, "device index beyond the no-allocation scratch table");
    void* ptr = scratch_address[device].load(std::memory_order_acquire);
    if (ptr) return ptr;
    std::lock_guard<std::mutex> lock(scratch_lookup);
    ptr = scratch_address[device].load(std::memory_order_relaxed);
    if (!ptr) {
        cbw::hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        cbw::require(ptr != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
        scratch_address[device].store(ptr, std::memory_order_release);
    }
    return ptr;
}

struct Call {
    cubutterflyHandle_t handle;
    cubutterflyPlan_t plan;
    const void* input;
    void* output;
};

void run(void* context) {
    const auto& c = *static_cast<const Call*>(context);
    cbw::execute_plan_with_workspace(c.handle, c.plan, c.input, c.output, device_scratch(), kScratchBytes,
                                     "the no-allocation scratch array (CUBUTTERFLY_NOALLOC_SCRATCH_BYTES)");
}

}  // namespace

extern "C" cubutterflyStatus_t cubutterflyExecuteNoAlloc(cubutterflyHandle_t handle, cubutterflyPlan_t plan,
                                                         const void* input, void* output) {
    Call call{handle, plan, input, output};
    return cbw::guarded_call(&run, &call);
}
