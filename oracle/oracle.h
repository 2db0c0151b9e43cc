/*
 * CPU oracle for the butterfly execution path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C, the CPU reference algorithms that
 * cuButterfly 0.9.3 uses to check its own GPU kernels. It is the checker, never
 * the thing measured or shipped: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product library
 * (cubutterfly_amd/libcubutterfly.so) never links or calls it.
 *
 * Every function cites the reference file:line it follows. How each function
 * is pinned (golden vectors, closed forms, brute force) is listed in
 * tests/test_oracle.py; functions with no such check would be marked
 * "parity unpinned" here -- there are none.
 *
 * Conventions: all lengths are powers of two; status 0 = success, -1 = invalid
 * argument. "threads" splits independent rows over POSIX threads (<=0 means 1).
 */
#ifndef CUBUTTERFLY_ORACLE_H
#define CUBUTTERFLY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- FWHT --------------------------------------------------------------- */
/* reference_fwht<float> (src/butterfly_reference.cpp:349-369): radix-2 stages
 * half = 1, 2, ..., n/2 in that order; optional x *= 1/n for normalised
 * inverse. */
int cbo_fwht_f32(float* values, uint64_t n, int inverse, int normalize);
int cbo_fwht_f32_batch(float* values, uint64_t n, uint64_t batch, int inverse,
                       int normalize, int threads);

/* IEEE binary16 conversions. f32->f16 is round-to-nearest-even with
 * overflow to infinity (the semantics of __float2half_rn used at
 * src/butterfly.cu:64). */
uint16_t cbo_f32_to_f16_rne(float value);
float cbo_f16_to_f32(uint16_t bits);

/* FP16 storage / FP32 compute / final-storage rounding contract
 * (src/butterfly.cu:1452-1470 plan, :1882-1897 execute, :53-68 conversion;
 * test oracle tests/test_fwht_final_storage.py:28-40): widen each fp16 input,
 * run the fp32 FWHT above, multiply by (float)scale, narrow once with RNE. */
int cbo_fwht_f16_final_batch(const uint16_t* input, uint16_t* output,
                             uint64_t n, uint64_t batch, float scale,
                             int inverse, int normalize, int threads);

/* ---- complex FFT -------------------------------------------------------- */
/* reference_fft(std::vector<Complex32>&) (src/butterfly_reference.cpp:392-433):
 * in-place bit reversal, then radix-2 DIT with twiddles cos/sin(+-pi*k/half)
 * evaluated in double per butterfly, the product b*w formed in double and
 * rounded to float once, a +- v in float. Interleaved (re, im) storage. */
int cbo_fft_c64(float* values, uint64_t n, int inverse, int normalize);
int cbo_fft_c64_batch(float* values, uint64_t n, uint64_t batch, int inverse,
                      int normalize, int threads);

/* ---- modular arithmetic and root conventions ---------------------------- */
uint64_t cbo_mod_mul(uint64_t a, uint64_t b, uint64_t q);
/* mod_pow (src/reference.cpp:506-520). */
uint64_t cbo_mod_pow(uint64_t base, uint64_t exponent, uint64_t q);
/* is_prime: trial division + deterministic Miller-Rabin
 * (src/reference.cpp:522-562). */
int cbo_is_prime(uint64_t value);
/* find_primitive_power_of_two_root (src/reference.cpp:564-582): smallest
 * candidate c in [2, 2^20) such that c^((q-1)/n) has exact order n = 2^log_n.
 * Returns 0 when the arguments are invalid or no root is found. */
uint64_t cbo_find_primitive_root(uint32_t log_n, uint64_t q);
/* find_psi_for_root (benchmarks/crypto_ntt/crypto_ntt_bench.cu:273-290): the
 * default 2n-th root when its square is `root`, else the smallest-candidate
 * 2n-th root whose square is `root`. Returns 0 on failure. */
uint64_t cbo_find_psi(uint32_t log_n, uint64_t q, uint64_t root);

/* ---- NTT ---------------------------------------------------------------- */
/* reference_ntt (src/reference.cpp:584-630): cyclic DIT, natural in/out,
 * omega = cbo_find_primitive_root(log n, q) (inverse: omega^-1, then x n^-1). */
int cbo_ntt_cyclic(uint64_t* values, uint64_t n, uint64_t q, int inverse);
int cbo_ntt_cyclic_batch(uint64_t* values, uint64_t n, uint64_t batch,
                         uint64_t q, int inverse, int threads);

/* expected_transform with the negacyclic channel of the crypto benchmark
 * (benchmarks/crypto_ntt/crypto_ntt_bench.cu:292-323 make_channel,
 * :454-508 independent_ntt, :510-528 expected_transform). Forward: twist by
 * psi^j, then the cyclic forward NTT. Inverse: cyclic inverse NTT (x n^-1),
 * then twist by psi^-j. Natural order on both sides. */
int cbo_ntt_negacyclic_batch(const uint64_t* input, uint64_t* output,
                             uint64_t n, uint64_t batch, uint64_t q,
                             int inverse, int threads);

/* RNS reference (tests/test_rns_ntt.cu:62-111): order-aware, one polynomial of
 * n = 2^log_n words. `root` is the FORWARD ring root (psi for negacyclic,
 * omega for cyclic), as in the RNS JSON config. */
int cbo_rns_reference(const uint64_t* input, uint64_t* output, uint32_t log_n,
                      uint64_t q, uint64_t root, int negacyclic, int inverse,
                      int input_bit_reversed, int output_bit_reversed);
/* Polynomial p of `count` contiguous polynomials uses domain p. */
int cbo_rns_batch(const uint64_t* input, uint64_t* output, uint32_t log_n,
                  const uint64_t* moduli, const uint64_t* roots, uint64_t count,
                  int negacyclic, int inverse, int input_bit_reversed,
                  int output_bit_reversed, int threads);

#ifdef __cplusplus
}
#endif
#endif
