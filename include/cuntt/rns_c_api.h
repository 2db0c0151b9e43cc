/*
 * rns_c_api.h -- multi-limb (RNS) word64 NTT C ABI.
 *
 * Drop-in replacement for cuButterfly 0.9.3's include/cuntt/rns_c_api.h:1-40:
 * same symbols, arguments and status codes (0 success, 1 invalid argument or
 * state, 2 runtime failure; thread-local error text valid until the next call;
 * no C++ exception escapes). The config JSON is the reference schema
 * (src/rns_tuning.cpp:114-150): schema_version 1, log_n, inverse, ring,
 * input_order, output_order, domains [{modulus, root}], polynomials
 * [{domain, input_offset, output_offset}]; unknown fields are rejected.
 * Roots describe the FORWARD transform (psi for negacyclic, w for cyclic).
 */
#ifndef CUNTT_RNS_C_API_H
#define CUNTT_RNS_C_API_H

#include <stddef.h>
#include <stdint.h>

#define CUBUTTERFLY_RNS_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cubutterflyRnsPlanOpaque* cubutterflyRnsPlan;

/* reference rns_c_api.h:16 */
CUBUTTERFLY_RNS_API const char* cubutterflyRnsLastError(void);
/* Parses and validates the config, builds per-limb tables (reference :17). */
CUBUTTERFLY_RNS_API int cubutterflyRnsCreate(const char* config_json, cubutterflyRnsPlan* result);
/* placement: 0 separate buffers, 1 in place. policy: 0 prefer, 1 require,
 * 2 refresh the cache record in cache_directory (empty disables writes).
 * Call once, outside graph capture and timing. `stream` is a hipStream_t.
 * (reference :18-23) */
CUBUTTERFLY_RNS_API int cubutterflyRnsPrepare(cubutterflyRnsPlan plan, int placement,
                                              const char* cache_directory, int policy,
                                              unsigned repetitions, void* stream);
/* Asynchronous, allocation-free; canonical residues in and out; input/output
 * aliasing must match the prepared placement (reference :24-29). */
CUBUTTERFLY_RNS_API int cubutterflyRnsExecute(cubutterflyRnsPlan plan, const uint64_t* input,
                                              uint64_t* output, void* stream);
/* Two-call query: buffer == NULL stores the required size (with NUL) in
 * *bytes (reference :30-33). */
CUBUTTERFLY_RNS_API int cubutterflyRnsInfoJson(cubutterflyRnsPlan plan, char* buffer, size_t* bytes);
CUBUTTERFLY_RNS_API int cubutterflyRnsDestroy(cubutterflyRnsPlan plan);

#ifdef __cplusplus
}
#endif
#endif /* CUNTT_RNS_C_API_H */
