// pm_rec.h — device helpers of the per-token (VALU) recurrence kernels: the
// forward (delta_recurrent.hip) and the backward's checkpoint pass
// (delta_bwd.hip).  A workgroup of kRecThreads threads owns a group of
// columns of S; thread (el, r) holds rows [r*RPT, r*RPT + RPT) of its column,
// and the RS row slices of a column are adjacent lanes of one 16-lane DPP row.
#pragma once

#include "pm_common.h"

namespace pm {

constexpr int kRecSteps = 16;     // tokens per staged block
constexpr int kRecThreads = 256;  // threads per workgroup

// x plus the value of the lane selected by a DPP control inside each 16-lane row
// (old = 0 and full masks, so the permute folds into one v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    const int xi = __float_as_int(x);
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, xi, CTRL, 0xF, 0xF, false));
}
// Sums over the RS adjacent lanes that hold one column (RS a power of two <= 16,
// aligned to RS inside a 16-lane row), for two values at once.  Each step adds the
// same two values on both partner lanes, so every lane of the group ends with the
// same bits.
template <int RS>
__device__ __forceinline__ void col_sum2(float& a, float& b) {
    if constexpr (RS >= 2) a = dpp_add<0xB1>(a), b = dpp_add<0xB1>(b);    // lane ^ 1
    if constexpr (RS >= 4) a = dpp_add<0x4E>(a), b = dpp_add<0x4E>(b);    // lane ^ 2
    if constexpr (RS >= 8) a = dpp_add<0x141>(a), b = dpp_add<0x141>(b);  // 7 - i in each 8
    if constexpr (RS >= 16) a = dpp_add<0x140>(a), b = dpp_add<0x140>(b); // 15 - i
}
template <int RS>
__device__ __forceinline__ float col_sum(float a) {
    if constexpr (RS >= 2) a = dpp_add<0xB1>(a);
    if constexpr (RS >= 4) a = dpp_add<0x4E>(a);
    if constexpr (RS >= 8) a = dpp_add<0x141>(a);
    if constexpr (RS >= 16) a = dpp_add<0x140>(a);
    return a;
}
// Sum over aligned groups of N adjacent lanes (N a power of two <= 64), every lane
// of a group ending with the same bits: DPP inside 16-lane rows (col_sum), then
// one lane permute per doubling beyond 16.
template <int N>
__device__ __forceinline__ float lane_sum(float x) {
    x = col_sum<(N < 16 ? N : 16)>(x);
    if constexpr (N >= 32) x += __shfl_xor(x, 16);
    if constexpr (N >= 64) x += __shfl_xor(x, 32);
    return x;
}

// Dot products of row slices with a column slice, one accumulator each.  The
// recurrence kernels are bound by VALU issue (wave64 FP32 at 4 cycles an
// instruction), so the adds that would join split accumulators cost more
// than the shorter dependent chains save.
template <int RPT>
__device__ __forceinline__ float row_dot(const float (&a)[RPT], const float (&s)[RPT]) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) acc = fmaf(a[i], s[i], acc);
    return acc;
}
template <int RPT>
__device__ __forceinline__ void row_dot2(const float (&a)[RPT], const float (&b)[RPT], const float (&s)[RPT],
                                        float& da, float& db) {
    float x = 0.f, y = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        x = fmaf(a[i], s[i], x);
        y = fmaf(b[i], s[i], y);
    }
    da = x;
    db = y;
}

// Four consecutive elements of a q or k row as loaded, converted only when
// written to LDS (so the loads stay in flight across a token loop).  With
// vec, one 16-byte (fp32) or 8-byte (bf16, two packed pairs in w[0..1])
// load; otherwise up to four element loads.  Elements past the row are 0.
template <typename InT>
struct Raw4;
template <>
struct Raw4<float> {
    float x[4];
    __device__ __forceinline__ void load(const float* p, int n, bool vec) {
        if (vec) {
            if (n > 0) {
                const float4 t = *reinterpret_cast<const float4*>(p);
                x[0] = t.x, x[1] = t.y, x[2] = t.z, x[3] = t.w;
            } else {
                x[0] = x[1] = x[2] = x[3] = 0.f;
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) x[c] = c < n ? p[c] : 0.f;
        }
    }
    __device__ __forceinline__ void get(float (&y)[4], bool) const {
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = x[c];
    }
};
template <>
struct Raw4<uint16_t> {
    uint32_t w[4];
    __device__ __forceinline__ void load(const uint16_t* p, int n, bool vec) {
        if (vec) {
            if (n > 0) {
                const uint2 t = *reinterpret_cast<const uint2*>(p);
                w[0] = t.x, w[1] = t.y;
            } else {
                w[0] = w[1] = 0u;
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) w[c] = c < n ? p[c] : 0u;
        }
    }
    __device__ __forceinline__ void get(float (&y)[4], bool vec) const {
        if (vec) {
            y[0] = __uint_as_float(w[0] << 16), y[1] = __uint_as_float(w[0] & 0xffff0000u);
            y[2] = __uint_as_float(w[1] << 16), y[3] = __uint_as_float(w[1] & 0xffff0000u);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) y[c] = __uint_as_float(w[c] << 16);
        }
    }
};

// LDS floats of one staging buffer: k and q rows [kRecSteps][RS * (RPT + 4)],
// v and the outputs [kRecSteps][CW], and per token {beta, q.k, alpha, 0}.
template <int RPT, int RS>
struct RecGeo {
    static constexpr int CW = kRecThreads / RS;  // columns per workgroup
    static constexpr int DP = RS * RPT;          // padded row length
    static constexpr int SL = RPT + 4;           // LDS stride of a row slice
    static constexpr int DPL = RS * SL;          // LDS row length
    static constexpr int BUF = 2 * kRecSteps * DPL + 2 * kRecSteps * CW + 4 * kRecSteps;
    static constexpr size_t BYTES = 2 * BUF * sizeof(float);
};

}  // namespace pm
