// pm_common.h — device helpers shared by the delta-rule kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pm {

// bf16 is carried as its 16-bit pattern; widening to fp32 is exact.
__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t x) { return bf16_to_f32(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float x) { return f32_to_bf16(x); }

// x plus the value DPP control CTRL selects, in the 16-lane rows ROW_MASK enables
// (other rows, and lanes whose source is outside their row, add 0).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add_rows(float x) {
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}
// Sum over each 16-lane row without LDS, every lane of the row ending with the same
// bits: quad_perm [1,0,3,2] and [2,3,0,1], then row_half_mirror and row_mirror.
__device__ __forceinline__ float row16_sum(float x) {
    x = dpp_add_rows<0xB1, 0xF>(x);
    x = dpp_add_rows<0x4E, 0xF>(x);
    x = dpp_add_rows<0x141, 0xF>(x);
    return dpp_add_rows<0x140, 0xF>(x);
}
// Sum over the wave's 64 lanes without LDS, valid in lanes 48-63: row sums, then
// row_bcast:15 adds row 2's total to row 3 and row_bcast:31 adds rows 0-1's.
__device__ __forceinline__ float wave_sum_row3(float x) {
    x = row16_sum(x);
    x = dpp_add_rows<0x142, 0xA>(x);
    return dpp_add_rows<0x143, 0xC>(x);
}
// Inclusive prefix sum over the wave's 64 lanes without LDS: row_shr 1, 2, 4, 8
// inside each row, then row_bcast:15 adds row 0's (row 2's) total to row 1 (row 3),
// and row_bcast:31 adds rows 0-1's total to rows 2 and 3.
__device__ __forceinline__ float wave_prefix_sum(float x) {
    x = dpp_add_rows<0x111, 0xF>(x);
    x = dpp_add_rows<0x112, 0xF>(x);
    x = dpp_add_rows<0x114, 0xF>(x);
    x = dpp_add_rows<0x118, 0xF>(x);
    x = dpp_add_rows<0x142, 0xA>(x);
    return dpp_add_rows<0x143, 0xC>(x);
}

}  // namespace pm
