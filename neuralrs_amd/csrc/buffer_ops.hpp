// Vector types and raw buffer loads shared by the matrix-core kernels.
#pragma once

#include "nrs_internal.hpp"

namespace nrs {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor format).
// A buffer load whose byte offset is >= bytes returns zero in hardware, so a
// gathered operand needs neither a branch nor a select for its padding: out
// of range elements use kOutOfRange. The host keeps gathered tensors at most
// 2 GiB so every valid offset is below kOutOfRange.
constexpr int kOutOfRange = (int)0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0,
                                             (int)(bytes < 0x80000000ll ? bytes : 0x80000000ll),
                                             0x00020000);
}

__device__ __forceinline__ float buffer_load1(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}

__device__ __forceinline__ f32x2 buffer_load2(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
}

__device__ __forceinline__ f32x4 buffer_load4(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

}  // namespace nrs
