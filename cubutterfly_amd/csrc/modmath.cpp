// Plan-time modular arithmetic: primality and the root-of-unity conventions the
// NTT plans share with the reference (so transforms agree bit for bit).
#include "common.hpp"

namespace cbw {

int device_cu_count() {
    int device = 0, count = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return 256;
    }
    return count;
}

std::uint64_t powmod(std::uint64_t base, std::uint64_t exponent, std::uint64_t q) {
    std::uint64_t acc = 1 % q;
    base %= q;
    for (; exponent; exponent >>= 1) {
        if (exponent & 1) acc = mulmod(acc, base, q);
        base = mulmod(base, base, q);
    }
    return acc;
}

// Deterministic Miller-Rabin for 64-bit integers with the 7-base witness set
// {2, 325, 9375, 28178, 450775, 9780504, 1795265022} (Jim Sinclair's set,
// exact for all n < 2^64), after trial division by the primes below 40.
bool is_prime_u64(std::uint64_t value) {
    if (value < 2) return false;
    for (std::uint64_t p : {2ull, 3ull, 5ull, 7ull, 11ull, 13ull, 17ull, 19ull, 23ull, 29ull, 31ull, 37ull})
        if (value % p == 0) return value == p;
    std::uint64_t d = value - 1;
    unsigned s = 0;
    while ((d & 1) == 0) d >>= 1, ++s;
    for (std::uint64_t a : {2ull, 325ull, 9375ull, 28178ull, 450775ull, 9780504ull, 1795265022ull}) {
        a %= value;
        if (a == 0) continue;
        std::uint64_t x = powmod(a, d, value);
        if (x == 1 || x == value - 1) continue;
        bool composite = true;
        for (unsigned r = 1; r < s && composite; ++r) {
            x = mulmod(x, x, value);
            if (x == value - 1) composite = false;
        }
        if (composite) return false;
    }
    return true;
}

// The reference picks the smallest c >= 2 (below 2^20) for which
// c^((q-1)/n) has exact multiplicative order n (src/reference.cpp:564-582);
// any other primitive root would give a different (equally valid) transform,
// so the same rule is required for bit-identical outputs.
std::uint64_t primitive_root_pow2(std::uint32_t log_n, std::uint64_t q) {
    require(log_n >= 1 && log_n <= 62, "NTT log_n must be in [1, 62]");
    require(is_prime_u64(q), "NTT modulus must be prime");
    const std::uint64_t n = std::uint64_t{1} << log_n;
    require((q - 1) % n == 0, "modulus - 1 must be divisible by the NTT length");
    const std::uint64_t cofactor = (q - 1) / n;
    for (std::uint64_t c = 2; c < (std::uint64_t{1} << 20); ++c) {
        const std::uint64_t w = powmod(c, cofactor, q);
        // Exact order n: w^n == 1 (false only when q | c) and w^(n/2) != 1.
        if (powmod(w, n, q) == 1 && powmod(w, n >> 1, q) != 1) return w;
    }
    throw std::runtime_error("no primitive power-of-two root found below 2^20");
}

// The crypto benchmark's negacyclic root: the default 2n-th root if it squares
// to `root`, else the smallest-candidate 2n-th root that does
// (benchmarks/crypto_ntt/crypto_ntt_bench.cu:273-290).
std::uint64_t psi_for_root(std::uint32_t log_n, std::uint64_t q, std::uint64_t root) {
    require(log_n + 1 <= 62, "negacyclic root order overflows");
    const std::uint64_t order = std::uint64_t{1} << (log_n + 1);
    require((q - 1) % order == 0, "negacyclic NTT requires 2n | modulus - 1");
    const std::uint64_t first = primitive_root_pow2(log_n + 1, q);
    if (mulmod(first, first, q) == root) return first;
    const std::uint64_t cofactor = (q - 1) / order;
    for (std::uint64_t c = 2; c < (std::uint64_t{1} << 20); ++c) {
        const std::uint64_t psi = powmod(c, cofactor, q);
        if (powmod(psi, order, q) == 1 && powmod(psi, order >> 1, q) != 1 &&
            mulmod(psi, psi, q) == root)
            return psi;
    }
    throw std::runtime_error("no 2n-th root squares to the cyclic plan root");
}

}  // namespace cbw
