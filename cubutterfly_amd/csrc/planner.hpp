// gfx950 planner: lowers a validated request to one executor.
// Each kernel family exposes a factory; the factory chooses the radix, the
// stage split between passes and the register/LDS residency for CDNA4
// (64-wide wavefronts, 160 KB LDS per CU, 256 CUs in 8 XCDs).
#pragma once

#include "common.hpp"
#include "descriptor.hpp"

namespace cbw {

std::unique_ptr<Executor> make_fwht_executor(const Request& r);
std::unique_ptr<Executor> make_fft_executor(const Request& r);
std::unique_ptr<Executor> make_ntt_executor(const Request& r);
// Gather / packed child / scatter, for strided sides and FWHT / FFT orders.
std::unique_ptr<Executor> make_boundary_executor(const Request& r);
// Rank >= 2: one batched rank-1 plan per axis, innermost first, with tiled
// transposes bringing each axis innermost and the original order back.
std::unique_ptr<Executor> make_composite_executor(const Request& r);

inline std::unique_ptr<Executor> plan_executor(const Request& r) {
    if (r.rank > 1) return make_composite_executor(r);
    if (r.boundary) return make_boundary_executor(r);
    switch (r.op) {
        case Op::Fwht: return make_fwht_executor(r);
        case Op::Fft: return make_fft_executor(r);
        case Op::Ntt: return make_ntt_executor(r);
    }
    throw NotSupported("operator has no MI355X lowering");
}

}  // namespace cbw
