// Shared internals of libcubutterfly: error classes mapped to C ABI statuses,
// HIP error checks, the executor interface every lowering implements, and the
// plan-time modular arithmetic used to build twiddle tables.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace cbw {

// Exception classes; the C ABI firewall maps each to one status code
// (reference src/c_api.cpp:130-163 maps the same categories).
struct NotSupported : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void require(bool condition, const std::string& message) {
    if (!condition) throw std::invalid_argument(message);
}
inline void supported(bool condition, const std::string& message) {
    if (!condition) throw NotSupported(message);
}
// A failed HIP call becomes this library's error status. The runtime's
// last-error state is cleared first: the library reports the error itself,
// and a caller's next hipGetLastError (torch checks it after every call)
// must not see it again.
inline void hip_check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        (void)hipGetLastError();
        throw HipError(std::string(what) + ": " + hipGetErrorString(status));
    }
}

inline bool is_pow2(std::uint64_t n) { return n != 0 && (n & (n - 1)) == 0; }
inline std::uint32_t log2_u64(std::uint64_t n) {
    std::uint32_t l = 0;
    while ((std::uint64_t{1} << l) < n) ++l;
    return l;
}

// Device memory owned by a plan (twiddle tables). Allocated at plan creation,
// never during execution.
class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t bytes) { allocate(bytes); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept : ptr_(other.ptr_), bytes_(other.bytes_) {
        other.ptr_ = nullptr;
        other.bytes_ = 0;
    }
    ~DeviceBuffer() { release(); }
    void allocate(std::size_t bytes) {
        release();
        if (bytes == 0) return;
        if (hipMalloc(&ptr_, bytes) != hipSuccess) {
            ptr_ = nullptr;
            (void)hipGetLastError();  // reported as ALLOC_FAILED / a runtime status, not left for the caller
            throw std::bad_alloc();
        }
        bytes_ = bytes;
    }
    template <class T>
    void upload(const std::vector<T>& host) {
        allocate(host.size() * sizeof(T));
        if (bytes_) hip_check(hipMemcpy(ptr_, host.data(), bytes_, hipMemcpyHostToDevice), "table upload");
    }
    void release() noexcept {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
    }
    template <class T>
    T* as() const noexcept { return static_cast<T*>(ptr_); }
    std::size_t bytes() const noexcept { return bytes_; }

  private:
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

// A lowered rank-1 request. Every executable plan owns exactly one.
class Executor {
  public:
    virtual ~Executor() = default;
    virtual std::size_t workspace_bytes() const { return 0; }
    // Enqueue the transform; `workspace` is the caller-bound buffer (may be
    // null when workspace_bytes() == 0).
    virtual void execute(const void* input, void* output, void* workspace, hipStream_t stream) = 0;
    std::string algorithm;     // stable lowering name
    std::string reason;        // why the planner chose it
    std::string mapping_json;  // full execution mapping
};

// Compute units of the current device (256 on MI355X); falls back to 256 when
// no device is visible so plans can still be described on a CPU-only host.
int device_cu_count();

// ---- plan-time modular arithmetic (host only) ----------------------------
using u128 = unsigned __int128;
inline std::uint64_t mulmod(std::uint64_t a, std::uint64_t b, std::uint64_t q) {
    return static_cast<std::uint64_t>(static_cast<u128>(a) * b % q);
}
std::uint64_t powmod(std::uint64_t base, std::uint64_t exponent, std::uint64_t q);
bool is_prime_u64(std::uint64_t value);
// Smallest-candidate primitive 2^log_n-th root of unity (the reference rule,
// src/reference.cpp:564-582); throws when none exists.
std::uint64_t primitive_root_pow2(std::uint32_t log_n, std::uint64_t q);
// 2n-th root whose square is `root` (crypto_ntt_bench.cu:273-290).
std::uint64_t psi_for_root(std::uint32_t log_n, std::uint64_t q, std::uint64_t root);
inline std::uint64_t invmod(std::uint64_t a, std::uint64_t q) { return powmod(a, q - 2, q); }
inline std::uint64_t bit_reverse(std::uint64_t x, std::uint32_t bits) {
    std::uint64_t r = 0;
    for (std::uint32_t i = 0; i < bits; ++i, x >>= 1) r = (r << 1) | (x & 1);
    return r;
}

}  // namespace cbw
