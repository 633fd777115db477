// Shared device helpers for the gfx950 kernels of libmemforge_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "memforge_hip.h"

namespace mf {

// Records the HIP error of the last failed launch on this thread.
void set_last_hip_error(int err);

// Checks the launch that was just enqueued; returns MF_OK or MF_ERR_HIP.
int check_launch();

// ---------------------------------------------------------------- dtypes
__host__ __device__ inline int dtype_size(int dt) { return dt == MF_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == MF_F32 || dt == MF_F16 || dt == MF_BF16; }

// bf16 <-> fp32 with the rounding torch uses (round to nearest even, NaN kept
// quiet), so a converting copy is bit-identical to tensor.to(torch.bfloat16).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
    return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)b);
    return (float)h;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

template <int DT>
__device__ __forceinline__ float bits_to_f32(uint32_t b) {
    if constexpr (DT == MF_BF16) return bf16_bits_to_f32(b);
    else if constexpr (DT == MF_F16) return f16_bits_to_f32(b);
    else return __uint_as_float(b);
}
template <int DT>
__device__ __forceinline__ uint32_t f32_to_bits(float f) {
    if constexpr (DT == MF_BF16) return f32_to_bf16_bits(f);
    else if constexpr (DT == MF_F16) return f32_to_f16_bits(f);
    else return __float_as_uint(f);
}

// ------------------------------------------------------------ wave helpers
// Reductions over the four 16-lane groups of a wave (lanes l, l^16, l^32,
// l^48) in registers, with gfx950's lane-swap instructions instead of an LDS
// permute. With both operands equal to x, v_permlane16_swap returns
// (x.g0, x.g0, x.g2, x.g2) and (x.g1, x.g1, x.g3, x.g3) -- each lane's
// xor-16 pair -- and v_permlane32_swap likewise each lane's xor-32 pair.
// The maxima use the NaN-propagating maximum (one v_maximum3_f32, no
// operand canonicalisation), as a softmax over a NaN score is NaN anyway.
__device__ __forceinline__ float fmax_prop(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float group_max4(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmax_prop(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmax_prop(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum4(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace mf
