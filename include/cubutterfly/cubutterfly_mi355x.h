/*
 * cubutterfly_mi355x.h -- extensions of the public C ABI.
 *
 * cuButterfly's public descriptor only expresses the cyclic NTT. Its
 * negacyclic single-prime transform exists only as a composition in the crypto
 * benchmark: a psi^j twist kernel, then a cyclic cuntt::Plan, and for the
 * inverse the cyclic inverse followed by a psi^-j twist
 * (reference benchmarks/crypto_ntt/crypto_ntt_bench.cu:552-612 twist kernels,
 * :715-730 launch_channel, :292-323 make_channel). This setter makes that
 * composition a property of the plan, so the twist is fused into the first
 * (forward) or last (inverse) pass instead of costing an extra HBM round trip.
 */
#ifndef CUBUTTERFLY_MI355X_H
#define CUBUTTERFLY_MI355X_H

#include "cubutterfly.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum cubutterflyNttRing {
    CUBUTTERFLY_NTT_RING_CYCLIC = 0,     /* X_k = sum_j x_j w^(jk) (default) */
    CUBUTTERFLY_NTT_RING_NEGACYCLIC = 1  /* X_k = sum_j x_j psi^j w^(jk), w = psi^2 */
} cubutterflyNttRing_t;

/* Selects the NTT ring. For NEGACYCLIC, `psi` is the primitive 2n-th root of
 * unity; 0 selects it as the crypto benchmark does (find_psi_for_root,
 * crypto_ntt_bench.cu:273-290): the smallest-candidate 2n-th root whose square
 * is the plan's cyclic root w. A nonzero psi must have exact order 2n and
 * then defines w = psi^2. The forward transform twists by psi^j before the
 * cyclic NTT; the inverse applies the cyclic inverse (x n^-1) and then psi^-j.
 * `psi` must be 0 for CYCLIC. Validated at plan creation. No counterpart in
 * the reference's public ABI; replaces the benchmark-side composition above. */
CUBUTTERFLYAPI cubutterflyStatus_t cubutterflySetNttRing(cubutterflyDescriptor_t descriptor,
                                                        cubutterflyNttRing_t ring,
                                                        uint64_t psi);

/* Bytes of the library-owned device array that cubutterflyExecuteNoAlloc
 * uses as the plan's workspace: 32 MiB, held by each GPU the library runs on
 * until the process ends. */
#define CUBUTTERFLY_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* cubutterflyExecute without any device allocation and without the workspace
 * bound by cubutterflyPlanSetWorkspace: the plan's workspace is carved from a
 * static device array of CUBUTTERFLY_NOALLOC_SCRATCH_BYTES per GPU instead.
 * No counterpart in the reference's ABI; it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). A plan whose PlanGetWorkspaceSize exceeds the array is
 * rejected with INVALID_VALUE before any work is queued; plans without a
 * workspace run exactly as with cubutterflyExecute. Same pointer, placement,
 * stream and asynchrony rules as cubutterflyExecute. All calls on one GPU
 * share that GPU's array: calls that may overlap on one device (other
 * streams, other host threads) race on it and must be serialised by the
 * caller. */
CUBUTTERFLYAPI cubutterflyStatus_t cubutterflyExecuteNoAlloc(cubutterflyHandle_t handle,
                                                            cubutterflyPlan_t plan,
                                                            const void* input,
                                                            void* output);

#ifdef __cplusplus
}
#endif
#endif /* CUBUTTERFLY_MI355X_H */
