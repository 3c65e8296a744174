// mfma_probe.hip — test-only check of the MFMA operand/accumulator lane
// layouts the chunked kernel relies on (built to tests/hip/libmfma_probe.so).
//
// One wave computes C = A B with the layout assumptions of delta_chunked.hip:
//   16x16x32: A lane l -> row l%16, B lane l -> column l%16, lane group
//             g = l/16 slot s <-> contraction index 4g+s (s<4), 16+4g+(s-4);
//   16x16x16: same with slot s <-> 4g+s;
//   both:     accumulator lane l, element i -> C[4(l/16)+i][l%16];
//   16x16x4 fp32: A lane l -> A[l%16][l/16], B lane l -> B[l/16][l%16], accumulator alike.
// The host compares C with a NumPy product; any wrong assumption shows.
//
// dpp_probe runs the DPP lane reductions of pm_common.h / pm_rec.h on one
// wave's 64 values: out[64 j + lane] for j = 0 prefix sum, 1 row16_sum,
// 2 wave_sum_row3, 3..8 lane_sum<2, 4, 8, 16, 32, 64>.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pm_common.h"
#include "pm_rec.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ void probe32(const uint16_t* A, const uint16_t* B, float* C) {
    const int l = threadIdx.x, r = l % 16, g = l / 16;
    bf16x8_t a, b;
    for (int s = 0; s < 8; ++s) {
        const int kk = (s < 4) ? 4 * g + s : 16 + 4 * g + (s - 4);
        a[s] = __builtin_bit_cast(__bf16, A[r * 32 + kk]);  // A 16x32 row-major
        b[s] = __builtin_bit_cast(__bf16, B[kk * 16 + r]);  // B 32x16 row-major
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
    for (int i = 0; i < 4; ++i) C[(4 * g + i) * 16 + r] = acc[i];
}

__global__ void probe16(const uint16_t* A, const uint16_t* B, float* C) {
    const int l = threadIdx.x, r = l % 16, g = l / 16;
    bf16x4_t a, b;
    for (int s = 0; s < 4; ++s) {
        const int kk = 4 * g + s;
        a[s] = __builtin_bit_cast(__bf16, A[r * 16 + kk]);  // A 16x16
        b[s] = __builtin_bit_cast(__bf16, B[kk * 16 + r]);  // B 16x16
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
    for (int i = 0; i < 4; ++i) C[(4 * g + i) * 16 + r] = acc[i];
}

// 16x16x4 fp32 (the fp32 chunked forward): A lane l -> A[l%16][l/16], B lane l ->
// B[l/16][l%16], accumulator as above.
__global__ void probe4f32(const float* A, const float* B, float* C) {
    const int l = threadIdx.x, r = l % 16, g = l / 16;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[r * 4 + g], B[g * 16 + r], acc, 0, 0, 0);
    for (int i = 0; i < 4; ++i) C[(4 * g + i) * 16 + r] = acc[i];
}

extern "C" int mfma_probe_f32(const float* a, const float* b, float* c) {
    hipLaunchKernelGGL(probe4f32, dim3(1), dim3(64), 0, 0, a, b, c);
    if (hipGetLastError() != hipSuccess) return 1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : 2;
}

extern "C" int mfma_probe(const uint16_t* a32, const uint16_t* b32, float* c32,
                          const uint16_t* a16, const uint16_t* b16, float* c16) {
    hipLaunchKernelGGL(probe32, dim3(1), dim3(64), 0, 0, a32, b32, c32);
    hipLaunchKernelGGL(probe16, dim3(1), dim3(64), 0, 0, a16, b16, c16);
    if (hipGetLastError() != hipSuccess) return 1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : 2;
}

__global__ void dpp_probe_kernel(const float* x, float* out) {
    const int l = threadIdx.x;
    const float v = x[l];
    out[l] = pm::wave_prefix_sum(v);
    out[64 + l] = pm::row16_sum(v);
    out[128 + l] = pm::wave_sum_row3(v);
    out[192 + l] = pm::lane_sum<2>(v);
    out[256 + l] = pm::lane_sum<4>(v);
    out[320 + l] = pm::lane_sum<8>(v);
    out[384 + l] = pm::lane_sum<16>(v);
    out[448 + l] = pm::lane_sum<32>(v);
    out[512 + l] = pm::lane_sum<64>(v);
}

// x: 64 floats, out: 9 x 64 floats (device pointers).
extern "C" int dpp_probe(const float* x, float* out) {
    hipLaunchKernelGGL(dpp_probe_kernel, dim3(1), dim3(64), 0, 0, x, out);
    if (hipGetLastError() != hipSuccess) return 1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : 2;
}
