// Buffer-resource access for the gfx950 kernels: a wave-uniform base and
// byte range (the hardware drops stores and zero-fills loads past the range),
// 32-bit per-lane offsets, an optional wave-uniform scalar offset and the
// instruction's cache-policy bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cbw {

constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer, gfx9 family

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, std::uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             kBufferWord3);
}

// byte_off: per-lane offset; scalar_off: a wave-uniform offset carried in
// the instruction's scalar operand (outside the range check: callers use it
// only where every access lies inside the resource's range). T is a 4- or
// 8-byte type. AUX: the instruction's cache-policy bits.
template <class T, int AUX = 0>
__device__ __forceinline__ T buffer_load(__amdgpu_buffer_rsrc_t r, std::uint32_t byte_off, std::uint32_t scalar_off = 0) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte elements");
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(
            T, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(byte_off), static_cast<int>(scalar_off), AUX));
    } else {
        return __builtin_bit_cast(
            T, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(byte_off), static_cast<int>(scalar_off), AUX));
    }
}

// AUX: the instruction's cache-policy bits. T is a 4-, 8- or 16-byte type.
//
// A buffer store of more than 8 bytes needs one wait state before an
// instruction that overwrites its data VGPRs; the GCN rule the compiler
// follows exempts stores whose scalar offset is an SGPR, so for those it
// emits none (`buffer_store_dwordx4 v[4:7], v30, s[0:3], s8 offen` directly
// followed by `v_mul_f32 v7, ...`). On gfx950 such stores wrote overwritten
// values: wrong results, no fault. 16-byte stores therefore carry their
// scalar part in the lane offset (the scalar operand is the constant 0, and
// the compiler keeps the wait state); 4- and 8-byte stores are not affected.
template <class T, int AUX = 0>
__device__ __forceinline__ void buffer_store(T x, __amdgpu_buffer_rsrc_t r, std::uint32_t byte_off,
                                             std::uint32_t scalar_off = 0) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8 || sizeof(T) == 16, "4-, 8- or 16-byte elements");
    if constexpr (sizeof(T) == 4) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(std::uint32_t, x), r, static_cast<int>(byte_off),
                                              static_cast<int>(scalar_off), AUX);
    } else if constexpr (sizeof(T) == 16) {
        using V4 = __attribute__((ext_vector_type(4))) std::uint32_t;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(V4, x), r, static_cast<int>(byte_off + scalar_off),
                                               0, AUX);
    } else {
        using V2 = __attribute__((ext_vector_type(2))) std::uint32_t;
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(V2, x), r, static_cast<int>(byte_off),
                                              static_cast<int>(scalar_off), AUX);
    }
}

// Wave-uniform copies (readfirstlane returns int: go through uint32 so the
// low half of a 64-bit value is not sign-extended).
__device__ __forceinline__ std::uint32_t uniform(std::uint32_t x) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
}
__device__ __forceinline__ std::uint64_t uniform(std::uint64_t x) {
    return (std::uint64_t(uniform(std::uint32_t(x >> 32))) << 32) | std::uint64_t(uniform(std::uint32_t(x)));
}

}  // namespace cbw
